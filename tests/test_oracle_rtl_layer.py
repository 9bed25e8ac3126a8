"""CPU checks of the composed RTL-exact layer restated in
oracle/bfp_rtl.py:rtl_fwd_layer (the per-op RTL goldens wired in the order
of rtl/vc707/src/smollm/smollm_layer_bfp.sv:1603-2600).

The reference's own acceptance test for that layer
(rtl/vc707/sim/tb_smollm_layer_bfp.sv:132-175) compares it with the float
layer: every mantissa within 256 LSB and every tile exponent within 1.  The
composition must meet that bound against sim A's fwd_layer at SmolLM2
shapes while the attention window is one tile (kv_pos <= 15); a wiring
mistake (wrong KV group, transposed V, a dropped re-tile or exponent term)
breaks it by orders of magnitude.  Beyond 15 the RTL's AV reads only
positions 0..15 (:2139-2180), which a second check pins directly."""
import numpy as np
import pytest

from oracle import bfp_rtl as rtl
from oracle import bfp_sim as sim

FULL = dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, NL=1, MAX_CTX=24, VOCAB=256)
TINY = dict(D=128, H_Q=2, H_KV=1, HD=64, FFN=256, NL=1, MAX_CTX=24, VOCAB=256)


def _model(cfg, seed):
    from bfp import Dims, synth
    d = Dims(**cfg)
    return d, sim.build_model(synth.make_model(d, seed=seed))


def test_shr8_is_the_8bit_requant_shift():
    """requant_mant holds the shift in `logic signed [7:0]`
    (smollm_layer_bfp.sv:1390-1395)."""
    assert rtl.shr8(-5, 10, 9) == -3          # -5 >>> 1
    assert rtl.shr8(12345, 10, -5) == 0       # shift 15 -> 12345 >> 15 == 0
    assert rtl.shr8(-1, 20, 4) == 0           # shift 16 -> 0
    assert rtl.shr8(777, 10, -128) == 777     # 138 wraps to -118: unshifted
    assert rtl.shr8(777, 127, -1) == 777      # 128 wraps to -128
    assert rtl.shr8(777, 127, 0) == 0         # 127 stays positive: >= 16


def test_config1_within_the_testbench_bound():
    """Config 1 (8 positions, KV growing) at SmolLM2 shapes: the composition
    against sim A's float layer, with the testbench's tolerances."""
    from bfp import synth
    d, om = _model(FULL, 1)
    xs = synth.make_layer_inputs(d, 8, seed=1)
    tabs = rtl.RtlTables()
    kvr = rtl.rtl_kv_cache(d.MAX_CTX, d.H_KV * d.HD)
    kvs = sim.new_kv(d, d.MAX_CTX)
    for p in range(8):
        h = sim.fp_quantize_vec(xs[p])
        hm, he = sim.tile_quantize(h)
        om_, oe_ = rtl.rtl_fwd_layer(hm.reshape(-1), he, om.layers[0], p, p, kvr, tabs, d)
        wm, we = sim.tile_quantize(sim.fwd_layer(h, om.layers[0], p, kvs, p, d))
        dm = np.abs(om_.astype(np.int64) - wm.reshape(-1))
        de = np.abs(oe_.astype(np.int64) - we)
        assert de.max() <= 1 and dm.max() <= 256, (p, int(dm.max()), int(de.max()))
        assert dm.max() > 0      # a different arithmetic, not the float layer


def test_attention_reads_sixteen_positions():
    """At kv_pos >= 16 the attention output does not depend on V's
    mantissas at positions >= 16 (the AV tile is t = 0..15); their
    exponents still enter the pre-shift maximum."""
    d, om = _model(TINY, 3)
    rng = np.random.default_rng(0)
    tabs = rtl.RtlTables()
    kv = rtl.rtl_kv_cache(d.MAX_CTX, d.HD)
    for p in range(20):
        hm, he = sim.tile_quantize(rng.standard_normal(d.D))
        rtl.rtl_fwd_layer(hm.reshape(-1), he, om.layers[0], p, p, kv, tabs, d)
    hm, he = sim.tile_quantize(rng.standard_normal(d.D))
    outs = []
    for trial in range(2):
        k2 = {k: v.copy() for k, v in kv.items()}
        if trial:
            k2["v_m"][16:20] = rng.integers(-32768, 32768, size=k2["v_m"][16:20].shape)
        st = {}
        rtl.rtl_fwd_layer(hm.reshape(-1), he, om.layers[0], 20, 20, k2, tabs, d, stages=st)
        outs.append(st["ATTN"])
    assert (outs[0][0] == outs[1][0]).all() and (outs[0][1] == outs[1][1]).all()
    # and the window does read position 15
    k3 = {k: v.copy() for k, v in kv.items()}
    k3["v_m"][15] = -k3["v_m"][15]
    st = {}
    rtl.rtl_fwd_layer(hm.reshape(-1), he, om.layers[0], 20, 20, k3, tabs, d, stages=st)
    assert (st["ATTN"][0] != outs[0][0]).any()
