"""The reference's ``fwd_layer(h, lw, pos, kv, kv_pos)``
(rtl/vc707/host/gen_smollm_blockfp_full.py:261-293) with its own argument
types, computed by the fused layer kernels of libbfp.so.

The caller owns everything, as in the reference: ``lw`` is a dict of
``(m, e)`` weight tuples in quantize_W's layout plus BFP-exact float64
gammas, and ``kv`` is ``{'k', 'v'}`` float64 arrays of shape
(MAX_CTX, H_KV, HD) that the call updates in place at ``kv_pos``
(full.py:270-272).  ``pos`` (the RoPE position) and ``kv_pos`` (the cache
slot; attention runs over slots 0..kv_pos) are independent, as the
reference's single-layer harness drives them
(gen_smollm_blockfp_bfp.py:42-43,332-344).

Each call:
  1. finds (or makes) a one-layer device context holding ``lw``'s weights,
     keyed by the dims and a content hash of the weight arrays, so a model's
     layers are uploaded once (up to ``CACHE_LAYERS`` distinct layers);
  2. encodes h, and the cache rows 0..kv_pos-1 that differ from what the
     context already holds, into BFP tiles on the device
     (``bfp_tile_encode_f64_d``: the values the reference holds are decoded
     tiles, and the encoding keeps them exactly).  The context keeps a host
     copy of the rows it holds; rows equal to it are not sent again, so a
     decode loop that passes the same ``kv`` step after step uploads only
     what it did not get from the device (nothing, in the reference's loop);
  3. runs the layer (``bfp_layer_step_kv``), reads cache row kv_pos back
     (decoded on the device) into ``kv`` and returns the decoded output.

Per call this still compares rows 0..kv_pos-1 on the host, hashes the
weights (to find the context; about 0.5 ms for a SmolLM2 layer) and
synchronises with the device; bulk decodes belong on ``BfpModel.decode``,
which keeps everything on the device.

Errors follow the reference's: an ``IndexError`` for a kv_pos outside the
cache (numpy's indexing error in full.py:271), ``ValueError`` for shapes
the reference's reshapes would reject or for inputs that are not BFP
values (the reference only ever passes decoded tiles).
"""
from __future__ import annotations

from collections import OrderedDict

import numpy as np

from .dims import Dims

CACHE_LAYERS = 64
_MATS = ("Wq", "Wk", "Wv", "Wo", "Wg", "Wu", "Wd")
_CTX: "OrderedDict[tuple, object]" = OrderedDict()


def _hasher():
    try:
        import xxhash
        return xxhash.xxh3_128()
    except ImportError:            # same bits, slower
        import hashlib
        return hashlib.blake2b(digest_size=16)


def _weights(lw):
    out = {}
    for name in _MATS:
        m, e = lw[name]
        m = np.ascontiguousarray(np.asarray(m, dtype=np.int16))
        e = np.ascontiguousarray(np.asarray(e, dtype=np.int8))
        if m.ndim != 3 or m.shape[2] != 16 or e.shape != m.shape[:2]:
            raise ValueError(f"lw[{name!r}]: bad BFP shapes {m.shape} / {e.shape}")
        out[name] = (m, e)
    for name in ("g1", "g2"):
        out[name] = np.ascontiguousarray(np.asarray(lw[name], dtype=np.float64).reshape(-1))
    return out


def _dims(w, kv_k) -> Dims:
    D = w["Wq"][0].shape[0]
    KV = w["Wk"][0].shape[0]
    FFN = w["Wg"][0].shape[0]
    if kv_k.ndim != 3:
        raise ValueError(f"kv['k'] must be (MAX_CTX, H_KV, HD), got {kv_k.shape}")
    max_ctx, h_kv, hd = kv_k.shape
    if hd == 0 or D % hd or h_kv * hd != KV:
        raise ValueError(f"kv shape {kv_k.shape} does not match Wk's {KV} rows / D={D}")
    expect = {"Wq": (D, D), "Wk": (KV, D), "Wv": (KV, D), "Wo": (D, D), "Wg": (FFN, D),
              "Wu": (FFN, D), "Wd": (D, FFN)}
    for name, (r, c) in expect.items():
        m = w[name][0]
        if m.shape[0] != r or m.shape[1] * 16 != c:
            raise ValueError(f"lw[{name!r}] is {m.shape[0]}x{m.shape[1] * 16}, expected {r}x{c}")
    for name in ("g1", "g2"):
        if w[name].size != D:
            raise ValueError(f"lw[{name!r}] has {w[name].size} values, expected {D}")
    return Dims(D=D, H_Q=D // hd, H_KV=h_kv, HD=hd, FFN=FFN, NL=1, MAX_CTX=max_ctx,
                VOCAB=16).check()


def _context(w, d: Dims):
    from . import api
    from .model import BfpModel
    h = _hasher()
    for name in _MATS:
        h.update(memoryview(w[name][0]).cast("B"))
        h.update(memoryview(w[name][1]).cast("B"))
    for name in ("g1", "g2"):
        h.update(memoryview(w[name]).cast("B"))
    key = (d, h.digest())
    gm = _CTX.get(key)
    if gm is not None:
        _CTX.move_to_end(key)
        return gm
    gm = BfpModel(d)
    for name in _MATS:
        gm.load_tensor(name, 0, m=w[name][0], e=w[name][1])
    for name in ("g1", "g2"):
        m, e = api.tile_encode(w[name])
        gm.load_tensor(name, 0, m=m, e=e)
    # host copy of the cache rows the device holds: rows 0.._kv_n-1 equal it
    gm._kv_k = np.zeros((d.MAX_CTX, d.KV), np.float64)
    gm._kv_v = np.zeros((d.MAX_CTX, d.KV), np.float64)
    gm._kv_n = 0
    _CTX[key] = gm
    while len(_CTX) > CACHE_LAYERS:
        _CTX.popitem(last=False)[1].close()
    return gm


def clear_cache():
    """Release the device contexts of every layer seen so far."""
    while _CTX:
        _CTX.popitem()[1].close()


def fwd_layer(h, lw, pos, kv, kv_pos):
    """full.py:261-293; see the module docstring."""
    from . import api
    w = _weights(lw)
    kk, vv = kv["k"], kv["v"]
    if not (isinstance(kk, np.ndarray) and isinstance(vv, np.ndarray)):
        raise TypeError("kv['k'] and kv['v'] must be numpy arrays (they are updated in place)")
    d = _dims(w, kk)
    if vv.shape != kk.shape:
        raise ValueError(f"kv['v'] {vv.shape} differs from kv['k'] {kk.shape}")
    pos, kv_pos = int(pos), int(kv_pos)
    if not 0 <= kv_pos < d.MAX_CTX:
        raise IndexError(f"kv_pos {kv_pos} is out of bounds for a cache of {d.MAX_CTX} positions")
    if pos < 0:
        raise ValueError(f"pos {pos} is negative")
    hm, he = api.tile_encode(np.asarray(h, dtype=np.float64).reshape(-1))
    if hm.size != d.D:
        raise ValueError(f"h has {hm.size} values, expected {d.D}")
    gm = _context(w, d)
    if kv_pos > 0:
        kf = kk[:kv_pos].reshape(kv_pos, d.KV)
        vf = vv[:kv_pos].reshape(kv_pos, d.KV)
        n = min(kv_pos, gm._kv_n)
        r0 = n
        if n:
            diff = np.flatnonzero(((kf[:n] != gm._kv_k[:n]) | (vf[:n] != gm._kv_v[:n])).any(axis=1))
            r0 = int(diff[0]) if diff.size else n
        if r0 < kv_pos:
            gm.kv_io_f64(0, 0, r0, kv_pos - r0, k=kf[r0:], v=vf[r0:])
            gm._kv_k[r0:kv_pos] = kf[r0:]
            gm._kv_v[r0:kv_pos] = vf[r0:]
            # rows past kv_pos are unchanged on the device, and in the copy
            gm._kv_n = max(gm._kv_n, kv_pos)
    om, oe, _ = gm.layer_step_bfp(0, pos, hm.reshape(1, -1), he.reshape(1, -1), kv_pos=kv_pos)
    k_new, v_new = gm.kv_io_f64(0, 0, kv_pos, 1)
    kk[kv_pos] = k_new.reshape(kk.shape[1:])
    vv[kv_pos] = v_new.reshape(vv.shape[1:])
    gm._kv_k[kv_pos] = k_new.reshape(-1)
    gm._kv_v[kv_pos] = v_new.reshape(-1)
    if gm._kv_n >= kv_pos:
        gm._kv_n = max(gm._kv_n, kv_pos + 1)
    return api.tile_decode(om[0], oe[0])
