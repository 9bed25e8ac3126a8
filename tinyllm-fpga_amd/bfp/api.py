"""The reference simulator's function set, computed on the MI355X.

Drop-in names and argument meanings of
rtl/vc707/host/gen_smollm_blockfp_full.py (full.py): numpy in, numpy out.
Every function here runs the HIP kernels of libbfp.so; PyTorch only
provides device memory and the current stream.  Shape errors raise
ValueError where the reference would fail its reshape/assert.
"""
from __future__ import annotations

import numpy as np

from . import _dev
from ._lib import call

TILE = 16


def _flat_f64(v):
    a = np.ascontiguousarray(np.asarray(v, dtype=np.float64).reshape(-1))
    if a.size % TILE:
        raise ValueError(f"length {a.size} is not a multiple of {TILE}")
    return a


def tile_quantize(v):
    """full.py:90-97 -> (m int16 (n/16, 16), e int8 (n/16,))."""
    a = _flat_f64(v)
    n = a.size
    dv = _dev.to_dev(a)
    m = _dev.empty(n, "int16")
    e = _dev.empty(n // TILE, "int8")
    call("bfp_tile_quantize_f64_d", _dev.ptr(dv), n, _dev.ptr(m), _dev.ptr(e), _dev.stream())
    return _dev.to_host(m).reshape(-1, TILE), _dev.to_host(e)


def tile_decode(m_int, e_int):
    """full.py:100-102 -> flat float64 (exact)."""
    m = np.ascontiguousarray(np.asarray(m_int, dtype=np.int16).reshape(-1))
    e = np.ascontiguousarray(np.asarray(e_int, dtype=np.int8).reshape(-1))
    if m.size != e.size * TILE:
        raise ValueError(f"{m.size} mantissas vs {e.size} exponents")
    dm, de = _dev.to_dev(m), _dev.to_dev(e)
    v = _dev.empty(m.size, "float64")
    call("bfp_tile_decode_d", _dev.ptr(dm), _dev.ptr(de), m.size, _dev.ptr(v), _dev.stream())
    return _dev.to_host(v)


def fp_quantize_vec(v):
    """full.py:105-107."""
    return tile_decode(*tile_quantize(v))


def tile_encode(v, strict=True):
    """The BFP tiles of float64 values that are already BFP (decoded tiles,
    as the reference's arrays hold them): tile_decode(*tile_encode(v)) == v.
    Equal to tile_quantize except for the raw form of a tile whose largest
    magnitude is the mantissa -32768, which tile_quantize would re-round.
    strict: raise ValueError when v holds a value that is not BFP-exact."""
    a = _flat_f64(v)
    n = a.size
    dv = _dev.to_dev(a)
    m = _dev.empty(n, "int16")
    e = _dev.empty(n // TILE, "int8")
    flag = _dev.zeros(1, "int32")
    call("bfp_tile_encode_f64_d", _dev.ptr(dv), n, _dev.ptr(m), _dev.ptr(e), _dev.ptr(flag),
         _dev.stream())
    if strict and int(_dev.to_host(flag)[0]):
        raise ValueError("values are not BFP tiles (16 int16 mantissas sharing an exponent)")
    return _dev.to_host(m).reshape(-1, TILE), _dev.to_host(e)


# ------------------------------------------------------------ float64 leaf ops
def rmsnorm_fp(x, gamma, eps=1e-5):
    """full.py:236-238: fp_quantize_vec((x*gamma) / np.sqrt(np.mean(x*x) + eps))."""
    xa, ga = _flat_f64(x), _flat_f64(gamma)
    if xa.size != ga.size:
        raise ValueError(f"x has {xa.size} values, gamma {ga.size}")
    dx, dg = _dev.to_dev(xa), _dev.to_dev(ga)
    y = _dev.empty(xa.size, "float64")
    call("bfp_rmsnorm_fp_d", _dev.ptr(dx), _dev.ptr(dg), xa.size, 1, float(eps), _dev.ptr(y),
         _dev.stream())
    return _dev.to_host(y)


def silu_fp(x):
    """full.py:241-242: fp_quantize_vec(x / (1.0 + np.exp(-x)))."""
    xa = _flat_f64(x)
    dx = _dev.to_dev(xa)
    y = _dev.empty(xa.size, "float64")
    call("bfp_silu_fp_d", _dev.ptr(dx), xa.size, _dev.ptr(y), _dev.stream())
    return _dev.to_host(y)


def softmax_fp(x):
    """full.py:245-247: e = np.exp(x - x.max()); e / e.sum() (float64)."""
    xa = np.ascontiguousarray(np.asarray(x, dtype=np.float64).reshape(-1))
    if xa.size == 0:
        raise ValueError("softmax of an empty vector")
    dx = _dev.to_dev(xa)
    y = _dev.empty(xa.size, "float64")
    call("bfp_softmax_fp_d", _dev.ptr(dx), xa.size, 1, _dev.ptr(y), _dev.stream())
    return _dev.to_host(y)


def rope_fp(x, pos, base=10000.0):
    """full.py:250-258 on one 64-wide head (or several, each rotated on its
    own): out[j] = a*c - b*s, out[j+32] = b*c + a*s, then fp_quantize_vec."""
    xa = np.ascontiguousarray(np.asarray(x, dtype=np.float64).reshape(-1))
    if xa.size % 64 or xa.size == 0:
        raise ValueError(f"rope_fp works on heads of 64 values, got {xa.size}")
    cs = np.empty(64, np.float64)
    call("bfp_rope_cos_sin", int(pos), 64, float(base), cs.ctypes.data)
    dx, dc = _dev.to_dev(xa), _dev.to_dev(cs)
    y = _dev.empty(xa.size, "float64")
    call("bfp_rope_fp_d", _dev.ptr(dx), xa.size // 64, _dev.ptr(dc), _dev.ptr(y), _dev.stream())
    return _dev.to_host(y)


def fwd_layer(h, lw, pos, kv, kv_pos):
    """full.py:261-293 with the reference's own arguments: ``lw`` a dict of
    (m, e) weight tuples 'Wq'..'Wd' (quantize_W layout) and BFP-exact float64
    gammas 'g1', 'g2'; ``kv`` {'k', 'v'} float64 arrays (MAX_CTX, H_KV, HD),
    updated in place at ``kv_pos``.  RoPE at ``pos``, attention over slots
    0..kv_pos.  Returns the float64 layer output.  See bfp.layer."""
    from .layer import fwd_layer as _fwd
    return _fwd(h, lw, pos, kv, kv_pos)


def quantize_W(W):
    """full.py:110-119: row-wise tile quantisation -> (m (out, in/16, 16),
    e (out, in/16))."""
    W = np.asarray(W)
    if W.ndim != 2 or W.shape[1] % TILE:
        raise ValueError(f"bad weight shape {W.shape}")
    n_out, n_in = W.shape
    m, e = tile_quantize(W.astype(np.float64))
    return m.reshape(n_out, n_in // TILE, TILE), e.reshape(n_out, n_in // TILE)


class PackedMatrix:
    """A BFP weight matrix resident in HBM in the kernels' layout."""

    def __init__(self, W_m, W_e):
        W_m = np.ascontiguousarray(np.asarray(W_m, dtype=np.int16))
        W_e = np.ascontiguousarray(np.asarray(W_e, dtype=np.int8))
        if W_m.ndim != 3 or W_m.shape[2] != TILE or W_e.shape != W_m.shape[:2]:
            raise ValueError(f"bad BFP weight shapes {W_m.shape} / {W_e.shape}")
        self.n_out, nt, _ = W_m.shape
        self.n_in = nt * TILE
        if self.n_out % 16:
            raise ValueError(f"n_out={self.n_out} is not a multiple of 16")
        dm, de = _dev.to_dev(W_m), _dev.to_dev(W_e)
        self.P_m = _dev.empty(W_m.size, "int16")
        self.P_e = _dev.empty(W_e.size, "int8")
        call("bfp_pack_d", _dev.ptr(dm), _dev.ptr(de), self.n_out, self.n_in,
             _dev.ptr(self.P_m), _dev.ptr(self.P_e), _dev.stream())

    @classmethod
    def from_float(cls, W):
        """quantize_W on the device from a float32 matrix."""
        self = cls.__new__(cls)
        W = np.ascontiguousarray(np.asarray(W, dtype=np.float32))
        self.n_out, self.n_in = W.shape
        if self.n_out % 16 or self.n_in % TILE:
            raise ValueError(f"bad weight shape {W.shape}")
        dW = _dev.to_dev(W)
        self.P_m = _dev.empty(W.size, "int16")
        self.P_e = _dev.empty(W.size // TILE, "int8")
        call("bfp_quantize_pack_f32_d", _dev.ptr(dW), self.n_out, self.n_in,
             _dev.ptr(self.P_m), _dev.ptr(self.P_e), _dev.stream())
        return self

    def unpack(self):
        m = _dev.empty(self.n_out * self.n_in, "int16")
        e = _dev.empty(self.n_out * self.n_in // TILE, "int8")
        call("bfp_unpack_d", _dev.ptr(self.P_m), _dev.ptr(self.P_e), self.n_out, self.n_in,
             _dev.ptr(m), _dev.ptr(e), _dev.stream())
        nt = self.n_in // TILE
        return _dev.to_host(m).reshape(self.n_out, nt, TILE), _dev.to_host(e).reshape(self.n_out, nt)

    def matvec_bfp(self, x_m, x_e, waves=0):
        """y = W x in BFP: returns (y_m (out,) int16, y_e (out/16,) int8)."""
        x_m = np.ascontiguousarray(np.asarray(x_m, dtype=np.int16).reshape(-1))
        x_e = np.ascontiguousarray(np.asarray(x_e, dtype=np.int8).reshape(-1))
        if x_m.size != self.n_in or x_e.size != self.n_in // TILE:
            raise ValueError(f"x has {x_m.size} mantissas / {x_e.size} exponents, "
                             f"matrix expects {self.n_in}")
        dxm, dxe = _dev.to_dev(x_m), _dev.to_dev(x_e)
        ym = _dev.empty(self.n_out, "int16")
        ye = _dev.empty(self.n_out // TILE, "int8")
        call("bfp_matvec_d", _dev.ptr(self.P_m), _dev.ptr(self.P_e), self.n_out, self.n_in, 1,
             0, 0, _dev.ptr(dxm), _dev.ptr(dxe), 0, _dev.ptr(ym), _dev.ptr(ye), 0, int(waves),
             _dev.stream())
        return _dev.to_host(ym), _dev.to_host(ye)


def matvec_bfp(x_m, x_e, W_m, W_e):
    """matvec_hw_golden with BFP output: (y_m (out,), y_e (out/16,))."""
    return PackedMatrix(W_m, W_e).matvec_bfp(x_m, x_e)


def matvec_hw_golden(x_m, x_e, W_m, W_e):
    """full.py:217-233: float64 output (the decoded BFP result)."""
    ym, ye = matvec_bfp(x_m, x_e, W_m, W_e)
    return tile_decode(ym, ye)


def embed_lookup(lu_m, lu_e, ids, vocab=None):
    """The FPGA's embedding lookup: narrow BFP rows of token `ids` from an
    EMBED_LU table (gen_smollm_blockfp_ddr.py:203-216), gathered on the
    device.  lu_m (V, D) int16, lu_e (V, R) int8 with R >= D/16 (the image
    pads exponent rows to 64 bytes); `vocab` (default V) bounds the valid
    ids, and an id outside [0, vocab) gives the zero tile (m 0, e -127).
    Returns (m (n, D) int16, e (n, D/16) int8)."""
    def host(a, t):   # contiguous and writable (torch.from_numpy wants both)
        a = np.ascontiguousarray(np.asarray(a, dtype=t))
        return a if a.flags.writeable else a.copy()
    lu_m, lu_e, ids = host(lu_m, np.int16), host(lu_e, np.int8), host(ids, np.int32).reshape(-1)
    if lu_m.ndim != 2 or lu_e.ndim != 2 or lu_e.shape[0] != lu_m.shape[0]:
        raise ValueError(f"bad table shapes {lu_m.shape} / {lu_e.shape}")
    V, D = lu_m.shape
    vocab = V if vocab is None else int(vocab)
    if not 0 < vocab <= V or D % TILE or lu_e.shape[1] < D // TILE:
        raise ValueError(f"bad table: vocab {vocab}, shapes {lu_m.shape} / {lu_e.shape}")
    n = ids.size
    om, oe = _dev.empty(max(n, 1) * D, "int16"), _dev.empty(max(n, 1) * (D // TILE), "int8")
    if n:
        dm, de, di = _dev.to_dev(lu_m), _dev.to_dev(lu_e), _dev.to_dev(ids)
        call("bfp_embed_gather_d", _dev.ptr(dm), _dev.ptr(de), vocab, D, lu_e.shape[1],
             _dev.ptr(di), n, _dev.ptr(om), _dev.ptr(oe), _dev.stream())
    return (_dev.to_host(om)[:n * D].reshape(n, D),
            _dev.to_host(oe)[:n * (D // TILE)].reshape(n, D // TILE))
