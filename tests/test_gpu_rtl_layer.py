"""GPU parity of the composed RTL-exact layer (bfp_rtl_layer_step, the
engines of rtl/vc707/src/smollm/smollm_layer_bfp.sv:1603-2600 in its FSM
order) against oracle/bfp_rtl.py:rtl_fwd_layer: all 13 stages and the
output bit for bit, at SmolLM2 shapes across the 16-position attention
tile, with RoPE position and KV slot apart, and on a second layer."""
import numpy as np
import pytest

from oracle import bfp_rtl as rtl
from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

FULL = dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, NL=1, MAX_CTX=24, VOCAB=256)
TINY = dict(D=128, H_Q=2, H_KV=1, HD=64, FFN=256, NL=2, MAX_CTX=40, VOCAB=256)
NAMES = ("N1", "Q", "K", "V", "ATTN", "O", "H1", "N2", "G", "U", "MLP", "D", "HOUT")


def _setup(cfg, seed):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=seed)
    gm = BfpModel(d)
    gm.load_fp32(fm)
    return d, sim.build_model(fm), gm


def _run(d, om, gm, layer, steps, seed):
    """steps: (pos, kv_pos) pairs run in order on one sequence."""
    rng = np.random.default_rng(seed)
    tabs = rtl.RtlTables()
    kv = rtl.rtl_kv_cache(d.MAX_CTX, d.H_KV * d.HD)
    for pos, kv_pos in steps:
        hm, he = sim.tile_quantize(rng.standard_normal(d.D))
        want = {}
        wm, we = rtl.rtl_fwd_layer(hm.reshape(-1), he, om.layers[layer], pos, kv_pos, kv, tabs, d,
                                   stages=want)
        om_, oe_, st = gm.rtl_layer_step(layer, pos, hm, he, kv_pos=kv_pos, dump=True)
        for name in NAMES:
            assert (st[name][1] == want[name][1]).all(), f"pos {pos}: stage {name} exponents"
            assert (st[name][0] == want[name][0]).all(), f"pos {pos}: stage {name} mantissas"
        assert (om_ == wm).all() and (oe_ == we).all(), f"pos {pos}: output"


def test_rtl_layer_smollm_shapes(gpu):
    d, om, gm = _setup(FULL, 1)
    print("[rtl layer] SmolLM2 shapes, positions 0..19", flush=True)
    _run(d, om, gm, 0, [(p, p) for p in range(20)], seed=1)
    gm.close()


def test_rtl_layer_pos_apart_from_slot_second_layer(gpu):
    d, om, gm = _setup(TINY, 2)
    print("[rtl layer] tiny, layer 1, pos != kv_pos", flush=True)
    _run(d, om, gm, 1, [(100 + 7 * p, p) for p in range(34)] + [(2047, 34)], seed=2)
    gm.close()


def test_rtl_layer_rejects_out_of_range(gpu):
    from bfp._lib import BfpError
    d, om, gm = _setup(TINY, 3)
    hm, he = sim.tile_quantize(np.ones(d.D))
    for pos, kv_pos in ((2048, 0), (-1, 0), (0, d.MAX_CTX), (0, -1)):
        with pytest.raises(BfpError):
            gm.rtl_layer_step(0, pos, hm, he, kv_pos=kv_pos)
    with pytest.raises(BfpError):
        gm.rtl_layer_step(2, 0, hm, he)
    gm.close()
