"""How far the float64 stages of BASELINE config 1 are from a 16-bit
rounding decision.

Some float64 results of the reference depend on library internals the GPU
does not reproduce bit for bit: numpy's SIMD exp, and BLAS summation orders
on other hosts.  Those differ by a few ulps at most, and a few ulps can change
a BFP mantissa only when the float64 value sits that close to a
round-half-even boundary of the 16-bit re-quantisation (or to a power of two,
for the tile exponent).  This test recomputes the pre-quantisation float64
values of the inexact stages -- RMSNorm, RoPE, attention, SiLU -- on the
config-1 inputs and measures that distance.
"""
import math

import numpy as np

from oracle import bfp_sim as sim


def _margins(v):
    """(min distance to a mantissa rounding boundary, in ulps of the scaled
    value; min relative distance of a tile max to a power of two)."""
    v = np.asarray(v, dtype=np.float64).reshape(-1, 16)
    m, e = sim.tile_quantize(v)
    sc = v * np.power(2.0, 15 - e.astype(np.float64))[:, None]
    nz = sc != 0
    dist = np.abs((sc - np.floor(sc)) - 0.5)
    ulp = np.spacing(np.abs(sc))
    mant = (dist[nz] / ulp[nz]).min()
    amax = np.abs(v).max(axis=1)
    amax = amax[amax > 0]
    lg = np.log2(amax)
    expo = np.abs(amax / np.power(2.0, np.round(lg)) - 1.0).min()
    return mant, expo


def test_config1_rounding_margins():
    from bfp import Dims, synth
    d = Dims(NL=1, MAX_CTX=16, VOCAB=256)
    fm = synth.make_model(d, seed=1)
    om = sim.build_model(fm)
    lw = om.layers[0]
    xs = synth.make_layer_inputs(d, 8, seed=1)
    kv = sim.new_kv(om.dims, d.MAX_CTX)
    worst_m, worst_e = np.inf, np.inf
    for p in range(8):
        h = sim.fp_quantize_vec(xs[p])
        dump = {}
        sim.fwd_layer(h, lw, pos=p, kv=kv, kv_pos=p, dims=om.dims, dump=dump)
        pre = {}
        pre["n1"] = h * lw["g1"] / np.sqrt(np.mean(h * h) + 1e-5)
        n1m, n1e = sim.tile_quantize(dump["N1"])
        q = sim.matvec_hw_golden(n1m, n1e, *lw["Wq"])
        rot = []
        for hq in range(d.H_Q):
            x = q[hq * 64:(hq + 1) * 64]
            out = np.empty(64)
            for j in range(32):
                th = sim.rope_angle(j, p, 64)
                c, s = math.cos(th), math.sin(th)
                out[j] = x[j] * c - x[j + 32] * s
                out[j + 32] = x[j + 32] * c + x[j] * s
            rot.append(out)
        pre["rope_q"] = np.concatenate(rot)
        attn = np.zeros(d.D)
        qd = dump["Q"]
        for hq in range(d.H_Q):
            g = hq // (d.H_Q // d.H_KV)
            sc = np.array([float(np.dot(qd[hq * 64:(hq + 1) * 64], kv["k"][t, g])) / 8.0
                           for t in range(p + 1)])
            pr = sim.softmax_fp(sc)
            for t in range(p + 1):
                attn[hq * 64:(hq + 1) * 64] += pr[t] * kv["v"][t, g]
        pre["attn"] = attn
        h1 = dump["H1"]
        pre["n2"] = h1 * lw["g2"] / np.sqrt(np.mean(h1 * h1) + 1e-5)
        gv = dump["G"]
        pre["silu"] = gv / (1.0 + np.exp(-gv))
        for k, v in pre.items():
            mm, ee = _margins(v)
            worst_m, worst_e = min(worst_m, mm), min(worst_e, ee)
    print(f"min mantissa margin {worst_m:.0f} ulps, min exponent margin {worst_e:.3g}")
    # a few-ulp float64 difference cannot change any BFP output of config 1
    assert worst_m > 64
    assert worst_e > 1e-12


def test_long_context_rounding_margins():
    """The same measure for one SmolLM2-shaped layer at the end of config
    4's range (positions 2040-2047, attention over up to 2048 cached rows):
    the attention output is a 2048-term float64 sum, so this is where a
    one-ulp difference in np.exp could first reach a BFP mantissa."""
    from bfp import Dims, synth
    d = Dims(NL=1, MAX_CTX=2048, VOCAB=256)
    om = sim.build_model(synth.make_model(d, seed=2))
    lw = om.layers[0]
    rng = np.random.default_rng(2)
    kv = sim.new_kv(om.dims, 2048)
    for t in range(2040):
        kv["k"][t] = sim.fp_quantize_vec(rng.standard_normal(d.KV) * 0.5).reshape(d.H_KV, d.HD)
        kv["v"][t] = sim.fp_quantize_vec(rng.standard_normal(d.KV) * 0.5).reshape(d.H_KV, d.HD)
    worst = np.inf
    for p in range(2040, 2048):
        h = sim.fp_quantize_vec(rng.standard_normal(d.D))
        dump = {}
        sim.fwd_layer(h, lw, pos=p, kv=kv, kv_pos=p, dims=om.dims, dump=dump)
        attn = np.zeros(d.D)
        for hq in range(d.H_Q):
            g = hq // (d.H_Q // d.H_KV)
            qh = dump["Q"][hq * 64:(hq + 1) * 64]
            sc = np.array([float(np.dot(qh, kv["k"][t, g])) / 8.0 for t in range(p + 1)])
            pr = sim.softmax_fp(sc)
            for t in range(p + 1):
                attn[hq * 64:(hq + 1) * 64] += pr[t] * kv["v"][t, g]
        mm, _ = _margins(attn)
        worst = min(worst, mm)
    print(f"long context: min attention mantissa margin {worst:.0f} ulps")
    assert worst > 64
