"""numpy-vectorised restatement of the reference simulator -- TEST
INFRASTRUCTURE ONLY (same import rule as ``oracle/bfp_sim.py``: tests/,
smoke() and bench.py's CPU baseline legs).

The same semantics as ``oracle/bfp_sim.py`` (which follows
``rtl/vc707/host/gen_smollm_blockfp_full.py`` line for line), with the
reference's Python loops replaced by whole-array numpy:

* ``quantize_W`` (full.py:110-119): one ``tile_quantize`` over every tile of
  the matrix instead of a loop over rows (tile_quantize is elementwise per
  tile, so the bits are the same);
* attention (full.py:273-283): all H_Q heads and all kv_pos+1 positions at
  once instead of 9*(kv_pos+1) ``np.dot`` calls and vector adds:
  - scores: ``np.dot(q, K[t])`` is OpenBLAS's SkylakeX ``ddot``: four
    8-lane FMA accumulators over the two 32-element halves, folded
    (l, l+4), ((a0+a1)+a2)+a3, then (s0+s2)+(s1+s3).  q and K[t] are BFP
    values, so every product q[j]*K[t,j] is exact in float64 (a product of
    two int16 mantissas times a power of two) and each FMA is one rounded
    add; the whole order is reproduced with elementwise array operations;
  - softmax: the reference's per-head ``softmax_fp`` on each row of a
    (H_Q, n) array (``e.sum(axis=1)`` is numpy's pairwise sum per row);
  - AV: ``attn[h] += p[t] * V[t]`` in ascending t from 0.0 is
    ``np.add.accumulate`` (cumsum) over t of the rounded products, with a
    zero row first;
* RoPE (full.py:250-258): the (cos, sin) of a position are computed once
  with ``math`` (as the reference evaluates them) and applied to all heads
  at once.

``tests/test_oracle_vec.py`` pins it bit for bit against ``bfp_sim`` on
config 1, on the reference-written config-3 prefix and on random BFP
score inputs against ``np.dot`` itself.  It is a CPU baseline (the
"numpy-vectorised version" of the reference), never the product.
"""
from __future__ import annotations

import math

import numpy as np

from . import bfp_sim as sim
from .bfp_sim import Dims, fp_quantize_vec, matvec_hw_golden, tile_quantize

TILE = 16


def quantize_W(W):
    """full.py:110-119 without the row loop."""
    n_out, n_in = W.shape
    assert n_in % TILE == 0
    m, e = tile_quantize(np.asarray(W, dtype=np.float64))
    return m.reshape(n_out, n_in // TILE, TILE), e.reshape(n_out, n_in // TILE)


_ROPE = {}


def rope_cs(pos, hd=64, base=10000.0):
    """(cos, sin) arrays of the hd/2 angles of full.py:253-254, evaluated
    with math.* exactly as the reference does; cached per position."""
    key = (pos, hd, base)
    cs = _ROPE.get(key)
    if cs is None:
        c = np.empty(hd // 2)
        s = np.empty(hd // 2)
        for j in range(hd // 2):
            th = sim.rope_angle(j, pos, hd, base)
            c[j] = math.cos(th)
            s[j] = math.sin(th)
        cs = _ROPE[key] = (c, s)
    return cs


def rope_heads(x, pos, hd=64):
    """rope_fp on every hd-wide head of x (n_heads*hd,), vectorised."""
    c, s = rope_cs(pos, hd)
    h2 = hd // 2
    xh = x.reshape(-1, hd)
    a, b = xh[:, :h2], xh[:, h2:]
    out = np.empty_like(xh)
    out[:, :h2] = a * c - b * s
    out[:, h2:] = b * c + a * s
    return fp_quantize_vec(out.reshape(-1))   # tiles of 16 never cross a head


def ddot64_bfp(q, K):
    """np.dot(q, K[t]) for every row t of K (n, 64), for BFP-valued q and K:
    OpenBLAS's SkylakeX ddot order with exact products (see the module
    docstring)."""
    P = K * q                                  # (n, 64), exact products
    acc = (P[:, :32] + 0.0) + P[:, 32:]        # fma(x[32+j], y[32+j], fma(x[j], y[j], 0.0))
    a = acc.reshape(-1, 4, 8)                  # accumulator r, lane l
    f = a[:, :, :4] + a[:, :, 4:]              # 512 -> 256 fold: (n, 4, 4)
    s = ((f[:, 0] + f[:, 1]) + f[:, 2]) + f[:, 3]   # (n, 4)
    return (s[:, 0] + s[:, 2]) + (s[:, 1] + s[:, 3])


def softmax_rows(S):
    """softmax_fp (full.py:245-247) of every row of S."""
    e = np.exp(S - S.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def attention(q, kv, kv_pos, dims: Dims):
    """full.py:273-283 over all heads at once: returns attn (D,) before its
    fp_quantize_vec."""
    HD, H_Q, H_KV = dims.HD, dims.H_Q, dims.H_KV
    grp = H_Q // H_KV
    n = kv_pos + 1
    inv = math.sqrt(HD)
    qh = q.reshape(H_Q, HD)
    S = np.empty((H_Q, n))
    for hq in range(H_Q):
        S[hq] = ddot64_bfp(qh[hq], kv["k"][:n, hq // grp]) / inv
    P = softmax_rows(S)
    attn = np.empty((H_Q, HD))
    for hq in range(H_Q):
        prod = P[hq][:, None] * kv["v"][:n, hq // grp]          # (n, HD), rounded products
        acc = np.add.accumulate(np.concatenate([np.zeros((1, HD)), prod]), axis=0)
        attn[hq] = acc[-1]
    return attn.reshape(-1)


def fwd_layer(h, lw, pos, kv, kv_pos, dims: Dims = Dims()):
    """full.py:261-293 with the vectorised attention and RoPE."""
    HD, H_Q, H_KV = dims.HD, dims.H_Q, dims.H_KV
    n1 = sim.rmsnorm_fp(h, lw["g1"])
    n1_m, n1_e = tile_quantize(n1)
    q = matvec_hw_golden(n1_m, n1_e, *lw["Wq"])
    k = matvec_hw_golden(n1_m, n1_e, *lw["Wk"])
    v = matvec_hw_golden(n1_m, n1_e, *lw["Wv"])
    q = rope_heads(q, pos, HD)
    k = rope_heads(k, pos, HD)
    kv["k"][kv_pos] = k.reshape(H_KV, HD)
    kv["v"][kv_pos] = v.reshape(H_KV, HD)
    attn = fp_quantize_vec(attention(q, kv, kv_pos, dims))
    a_m, a_e = tile_quantize(attn)
    o = matvec_hw_golden(a_m, a_e, *lw["Wo"])
    h1 = fp_quantize_vec(h + o)
    n2 = sim.rmsnorm_fp(h1, lw["g2"])
    n2_m, n2_e = tile_quantize(n2)
    g = matvec_hw_golden(n2_m, n2_e, *lw["Wg"])
    u = matvec_hw_golden(n2_m, n2_e, *lw["Wu"])
    mlp = fp_quantize_vec(sim.silu_fp(g) * u)
    mlp_m, mlp_e = tile_quantize(mlp)
    d = matvec_hw_golden(mlp_m, mlp_e, *lw["Wd"])
    return fp_quantize_vec(h1 + d)


def build_model(fm) -> sim.Model:
    """bfp_sim.build_model with the vectorised quantize_W."""
    layers = []
    for lw in fm.layers:
        q = {name: quantize_W(np.asarray(lw[name]).astype(np.float64))
             for name in ("Wq", "Wk", "Wv", "Wo", "Wg", "Wu", "Wd")}
        q["g1"] = fp_quantize_vec(np.asarray(lw["g1"]).astype(np.float64))
        q["g2"] = fp_quantize_vec(np.asarray(lw["g2"]).astype(np.float64))
        layers.append(q)
    d = fm.dims
    dims = Dims(d.D, d.H_Q, d.H_KV, d.HD, d.FFN, d.NL, d.MAX_CTX, d.VOCAB)
    return sim.Model(dims, layers, np.asarray(fm.embed).astype(np.float64),
                     fp_quantize_vec(np.asarray(fm.norm_w).astype(np.float64)))


def decode(model: sim.Model, prompt, n_gen, max_ctx=None, on_layer=None):
    """The golden-token loop of full.py:426-443 (bfp_sim.decode) over the
    vectorised layer."""
    dims = model.dims
    ids = [int(t) for t in prompt]
    n_ctx = max_ctx if max_ctx is not None else max(dims.MAX_CTX, len(ids) + n_gen)
    kv = [sim.new_kv(dims, n_ctx) for _ in range(dims.NL)]
    generated = list(ids)
    for step in range(len(ids) + n_gen):
        tid = ids[step] if step < len(ids) else generated[-1]
        h = model.embed_row_q(tid)
        for li in range(dims.NL):
            h = fwd_layer(h, model.layers[li], pos=step, kv=kv[li], kv_pos=step, dims=dims)
            if on_layer is not None:
                on_layer(step, li, h)
        if step >= len(ids) - 1:
            nid = sim.head_argmax(h, model.norm_w_q, model.embed)
            if step >= len(ids):
                generated.append(nid)
    return generated
