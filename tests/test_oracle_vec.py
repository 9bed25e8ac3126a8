"""Pins of the numpy-vectorised restatement (oracle/bfp_vec.py) against the
line-faithful one (oracle/bfp_sim.py) and against numpy/BLAS itself: it is
the second CPU baseline, so it must compute the same bits."""
import hashlib

import numpy as np
import pytest

from oracle import bfp_sim as sim
from oracle import bfp_vec as vec
from refcases import GOLDEN


def test_ddot_emulation_vs_np_dot():
    """The vectorised score equals np.dot(q, K[t]) on BFP values (exact
    products), including spread exponents and signed zeros."""
    rng = np.random.default_rng(31)
    for scale in (1e-3, 1.0, 300.0):
        q = sim.fp_quantize_vec(rng.standard_normal(64) * scale)
        K = sim.fp_quantize_vec(rng.standard_normal((200, 64)).reshape(-1) *
                                np.repeat(np.exp(rng.standard_normal(800) * 3), 16)).reshape(200, 64)
        K[5] = 0.0
        K[6, :32] = -0.0
        got = vec.ddot64_bfp(q, K)
        want = np.array([float(np.dot(q, K[t])) for t in range(200)])
        assert (got == want).all() and (np.signbit(got) == np.signbit(want)).all()


def test_quantize_w_vs_row_loop():
    rng = np.random.default_rng(32)
    W = (rng.standard_normal((96, 576)) * 0.02).astype(np.float32).astype(np.float64)
    a, b = vec.quantize_W(W), sim.quantize_W(W)
    assert (a[0] == b[0]).all() and (a[1] == b[1]).all()


@pytest.mark.parametrize("max_ctx,positions", [(16, range(8)), (600, [0, 1, 517])])
def test_layer_vs_faithful(max_ctx, positions):
    """Config 1's layer (and a long-context one) with the KV cache growing:
    every output and the cache equal the line-faithful oracle's."""
    from bfp import Dims, synth
    d = Dims(NL=1, MAX_CTX=max_ctx, VOCAB=256)
    fm = synth.make_model(d, seed=1)
    om = sim.build_model(fm)
    xs = synth.make_layer_inputs(d, 8, seed=1)
    kv_a = sim.new_kv(om.dims, max_ctx)
    rng = np.random.default_rng(33)
    for t in range(max(positions)):       # a filled cache below the probed positions
        kv_a["k"][t] = sim.fp_quantize_vec(rng.standard_normal(d.KV)).reshape(d.H_KV, d.HD)
        kv_a["v"][t] = sim.fp_quantize_vec(rng.standard_normal(d.KV)).reshape(d.H_KV, d.HD)
    kv_b = {k: v.copy() for k, v in kv_a.items()}
    for i, p in enumerate(positions):
        h = sim.fp_quantize_vec(xs[i % 8])
        a = sim.fwd_layer(h, om.layers[0], pos=p, kv=kv_a, kv_pos=p, dims=om.dims)
        b = vec.fwd_layer(h, om.layers[0], pos=p, kv=kv_b, kv_pos=p, dims=om.dims)
        assert (a == b).all(), p
        assert (kv_a["k"] == kv_b["k"]).all() and (kv_a["v"] == kv_b["v"]).all()


def test_config1_vs_reference():
    from bfp import Dims, synth
    f = np.load(GOLDEN / "ref_layer_cfg1.npz")
    d = Dims(NL=1, MAX_CTX=16, VOCAB=256)
    fm = synth.make_model(d, seed=int(f["seed"]))
    om = vec.build_model(fm)
    xs = synth.make_layer_inputs(d, 8, seed=int(f["seed"]))
    kv = sim.new_kv(om.dims, d.MAX_CTX)
    for p in range(8):
        out = vec.fwd_layer(sim.fp_quantize_vec(xs[p]), om.layers[0], pos=p, kv=kv, kv_pos=p,
                            dims=om.dims)
        m, e = sim.tile_quantize(out)
        assert (m.reshape(-1) == f["hout_m"][p]).all() and (e == f["hout_e"][p]).all(), p


def test_config3_prefix_vs_reference():
    """The first 12 steps of the reference's config-3 run (30 layers)."""
    from bfp import Dims, synth
    f = np.load(GOLDEN / "ref_decode_cfg3.npz")
    prompt = [int(t) for t in f["prompt"]]
    d = Dims(MAX_CTX=len(prompt) + len(f["tokens"]))
    om = vec.build_model(synth.make_model(d, seed=int(f["seed"])))
    digests, cur = [], []

    def on_layer(step, li, h):
        m, e = sim.tile_quantize(h)
        cur.append((m.reshape(-1), e))
        if li == d.NL - 1:
            hh = hashlib.sha256()
            for mm, ee in cur:
                hh.update(mm.astype(np.int16).tobytes())
                hh.update(ee.astype(np.int8).tobytes())
            digests.append(hh.hexdigest())
            cur.clear()

    toks = vec.decode(om, prompt, 4, max_ctx=d.MAX_CTX, on_layer=on_layer)
    assert list(toks[len(prompt):]) == [int(t) for t in f["tokens"][:4]]
    assert digests == [str(x) for x in f["digests"][:12]]
