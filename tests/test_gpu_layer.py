"""GPU parity of one decoder layer against the oracle's
fwd_layer (oracle/bfp_sim.py restating
rtl/vc707/host/gen_smollm_blockfp_full.py:261-293): every one of the 13
stage outputs, bit for bit, at positions 0..7 with the KV cache growing."""
import numpy as np
import pytest

from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

SMALL = dict(D=64, H_Q=1, H_KV=1, HD=64, FFN=128, NL=1, MAX_CTX=16, VOCAB=256)
MID = dict(D=192, H_Q=3, H_KV=1, HD=64, FFN=256, NL=1, MAX_CTX=16, VOCAB=256)
FULL = dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, NL=1, MAX_CTX=16, VOCAB=256)
# a KV capacity above 512: the long-context attention form (four workgroups
# per head, each dumping its own 16-dimension tile of the attention output)
FULL_LONG = dict(FULL, MAX_CTX=600)


def _setup(cfg, seed, max_batch=1):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=seed)
    om = sim.build_model(fm)
    gm = BfpModel(d, max_batch=max_batch)
    gm.load_fp32(fm)
    return d, om, gm


def _check_stages(stages, dump, b, pos, tag):
    for name in sim.STAGES:
        wm, we = sim.tile_quantize(dump[name])
        gm_, ge_ = stages[name]
        assert (ge_[b] == we).all(), f"{tag} pos {pos}: stage {name} exponents differ"
        assert (gm_[b] == wm.reshape(-1)).all(), f"{tag} pos {pos}: stage {name} mantissas differ"


@pytest.mark.parametrize("cfg", [SMALL, MID, FULL, FULL_LONG], ids=["small", "mid", "full", "full-long"])
def test_layer_8_positions(gpu, cfg):
    d, om, gm = _setup(cfg, seed=1)
    print(f"[layer] dims {cfg}", flush=True)
    from bfp import synth
    xs = synth.make_layer_inputs(d, 8, seed=1)
    kv = sim.new_kv(om.dims, d.MAX_CTX)
    for p in range(8):
        h = sim.fp_quantize_vec(xs[p])
        dump = {}
        want = sim.fwd_layer(h, om.layers[0], pos=p, kv=kv, kv_pos=p, dims=om.dims, dump=dump)
        hm, he = sim.tile_quantize(h)
        out_m, out_e, st = gm.layer_step_bfp(0, p, hm.reshape(1, -1), he.reshape(1, -1), dump=True)
        _check_stages(st, dump, 0, p, str(cfg["D"]))
        # the returned tile is the raw quantisation: its values are the reference's
        assert (sim.tile_decode(out_m[0].reshape(-1, 16), out_e[0]) == want).all()
    gm.close()


def test_layer_batched_sequences(gpu):
    """Three independent sequences in one launch: each matches its own
    oracle run (own KV cache)."""
    d, om, gm = _setup(MID, seed=2, max_batch=3)
    rng = np.random.default_rng(5)
    kvs = [sim.new_kv(om.dims, d.MAX_CTX) for _ in range(3)]
    for p in range(5):
        hs = [sim.fp_quantize_vec(rng.standard_normal(d.D) * (1 + b)) for b in range(3)]
        q = [sim.tile_quantize(h) for h in hs]
        hm = np.stack([x[0].reshape(-1) for x in q])
        he = np.stack([x[1] for x in q])
        out_m, out_e, st = gm.layer_step_bfp(0, p, hm, he, dump=True)
        for b in range(3):
            dump = {}
            sim.fwd_layer(hs[b], om.layers[0], pos=p, kv=kvs[b], kv_pos=p, dims=om.dims, dump=dump)
            _check_stages(st, dump, b, p, f"seq{b}")
    gm.close()


@pytest.mark.parametrize("cfg,batch", [(MID, 5), (FULL, 6), (MID, 9), (MID, 33), (FULL, 40),
                                       (FULL_LONG, 9)],
                         ids=["mid-b5", "full-b6", "mfma-mid-b9", "mfma-mid-b33", "mfma-full-b40",
                              "mfma-full-long-b9"])
def test_layer_multi_sequence_path(gpu, cfg, batch):
    """Batches of 4 or more run the multi-sequence kernels (separate norm,
    weight chunks reused across a group of sequences), from 8 on with the
    tile sums on the int8 matrix cores in blocks of 16 sequences (9: one
    partial block; 33: a last block of one sequence): every stage of every
    sequence still equals its own oracle run."""
    d, om, gm = _setup(cfg, seed=7, max_batch=batch)
    rng = np.random.default_rng(9)
    kvs = [sim.new_kv(om.dims, d.MAX_CTX) for _ in range(batch)]
    for p in range(4):
        hs = [sim.fp_quantize_vec(rng.standard_normal(d.D) * (0.5 + b)) for b in range(batch)]
        q = [sim.tile_quantize(h) for h in hs]
        hm = np.stack([x[0].reshape(-1) for x in q])
        he = np.stack([x[1] for x in q])
        out_m, out_e, st = gm.layer_step_bfp(0, p, hm, he, dump=True)
        for b in range(batch):
            dump = {}
            sim.fwd_layer(hs[b], om.layers[0], pos=p, kv=kvs[b], kv_pos=p, dims=om.dims, dump=dump)
            _check_stages(st, dump, b, p, f"seq{b}")
    gm.close()


def test_fwd_layer_float_api(gpu):
    """The reference-named float64 entry point."""
    d, om, gm = _setup(SMALL, seed=3)
    kv = sim.new_kv(om.dims, d.MAX_CTX)
    rng = np.random.default_rng(0)
    for p in range(3):
        h = sim.fp_quantize_vec(rng.standard_normal(d.D))
        want = sim.fwd_layer(h, om.layers[0], pos=p, kv=kv, kv_pos=p, dims=om.dims)
        got = gm.fwd_layer(h, 0, p)
        assert (got == want).all()
    # RoPE position and cache slot apart: slot 2 is overwritten
    want = sim.fwd_layer(h, om.layers[0], pos=3, kv=kv, kv_pos=2, dims=om.dims)
    assert (gm.fwd_layer(h, 0, 3, kv_pos=2) == want).all()
    gm.close()


def test_second_context_keeps_lds_limit(gpu):
    """A context made after a larger one of the same attention form must
    not lower the kernel's dynamic-LDS limit under the first: the first
    still runs at a position past the second's capacity, and matches the
    oracle."""
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d1 = Dims(NL=1, MAX_CTX=2048, VOCAB=256)
    fm = synth.make_model(d1, seed=41)
    om = sim.build_model(fm)
    big = BfpModel(d1)
    big.load_fp32(fm)
    small = BfpModel(Dims(NL=1, MAX_CTX=600, VOCAB=256))
    rng = np.random.default_rng(41)
    kv = sim.new_kv(om.dims, 2048)
    h = sim.fp_quantize_vec(rng.standard_normal(d1.D))
    want = sim.fwd_layer(h, om.layers[0], pos=1500, kv=kv, kv_pos=1500, dims=om.dims)
    hm, he = sim.tile_quantize(h)
    om_, oe_, _ = big.layer_step_bfp(0, 1500, hm.reshape(1, -1), he.reshape(1, -1))
    assert (sim.tile_decode(om_[0].reshape(-1, 16), oe_[0]) == want).all()
    small.close()
    big.close()
