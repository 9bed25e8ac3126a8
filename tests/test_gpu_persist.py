"""GPU: the persistent batch-1 decode (one launch, stages
handing over through device-coherent memory) against the per-stage graph
path and the oracle -- tokens and every layer's output at every step, bit
for bit, for every attention form (context capacities 32, 200, 300, 600),
at SmolLM2's width, under both loop policies and across repeated decodes
on one context (the hand-off words are re-armed per launch)."""
import numpy as np
import pytest

from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

TINY = dict(D=128, H_Q=2, H_KV=1, HD=64, FFN=256, NL=2, MAX_CTX=32, VOCAB=512)


def _setup(cfg, seed):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=seed)
    gm = BfpModel(d)
    gm.load_fp32(fm)
    return d, fm, gm


def _both(gm, prompt, n_gen, **kw):
    tp, hp = gm.decode(prompt[None, :], n_gen, hist=True, **kw)
    assert gm.decode_path() == "persist"
    tg, hg = gm.decode(prompt[None, :], n_gen, hist=True, persist=False, **kw)
    assert gm.decode_path() == "graph"
    return (tp, hp), (tg, hg)


def _same(a, b):
    (tp, (hpm, hpe)), (tg, (hgm, hge)) = a, b
    steps = hpm.shape[1]
    bad = [s for s in range(steps) if not ((hpm[0, s] == hgm[0, s]).all() and (hpe[0, s] == hge[0, s]).all())]
    assert not bad, f"layer outputs differ at steps {bad[:8]}"
    assert (tp == tg).all()


@pytest.mark.parametrize("max_ctx", [32, 200, 300, 600],
                         ids=["half-wave-128", "lane-split-256", "per-thread-512", "long-form"])
def test_persist_equals_graph_every_form(gpu, max_ctx):
    cfg = dict(TINY, MAX_CTX=max_ctx)
    d, fm, gm = _setup(cfg, seed=21)
    from bfp import synth
    prompt = synth.make_prompt(d, 6, seed=21)
    n_gen = max_ctx - 6
    print(f"[persist] capacity {max_ctx}", flush=True)
    p, g = _both(gm, prompt, n_gen)
    _same(p, g)
    gm.close()


def test_persist_against_oracle(gpu):
    """The persistent path alone against the oracle (no graph in the loop)."""
    d, fm, gm = _setup(TINY, seed=22)
    from bfp import synth
    om = sim.build_model(fm)
    prompt = synth.make_prompt(d, 5, seed=22)
    steps = 5 + 20
    hm_w = np.zeros((steps, d.NL, d.D), np.int16)
    he_w = np.zeros((steps, d.NL, d.D // 16), np.int8)

    def on_layer(step, li, h):
        m, e = sim.tile_quantize(h)
        hm_w[step, li] = m.reshape(-1)
        he_w[step, li] = e

    want = sim.decode(om, prompt, 20, on_layer=on_layer)[5:]
    toks, (hm, he) = gm.decode(prompt[None, :], 20, hist=True)
    assert gm.decode_path() == "persist"
    assert (hm[0] == hm_w).all() and (he[0] == he_w).all()
    assert list(toks[0]) == list(want)
    gm.close()


@pytest.mark.parametrize("max_ctx", [40, 560], ids=["short", "long-form"])
def test_persist_full_width(gpu, max_ctx):
    """D = 576, 9 heads over 3 KV groups, FFN 1536: the shapes of BASELINE
    configs 3-5 (2 layers), both attention families."""
    cfg = dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, NL=2, MAX_CTX=max_ctx, VOCAB=1024)
    d, fm, gm = _setup(cfg, seed=23)
    from bfp import synth
    prompt = synth.make_prompt(d, 8, seed=23)
    print(f"[persist] full width, capacity {max_ctx}", flush=True)
    p, g = _both(gm, prompt, max_ctx - 8)
    _same(p, g)
    gm.close()


def test_persist_rtl_loop(gpu):
    d, fm, gm = _setup(TINY, seed=24)
    from bfp import synth
    om = sim.build_model(fm)
    prompt = synth.make_prompt(d, 4, seed=24)
    toks, _ = gm.decode(prompt[None, :], 9, rtl_loop=True)
    assert gm.decode_path() == "persist"
    assert list(toks[0]) == sim.decode_rtl_loop(om, prompt, 9)
    gm.close()


def test_persist_repeated_and_single_token(gpu):
    """Decodes back to back on one context give the same result (the tags
    restart from zero each launch), and a one-token prompt (the head from
    step 0, step 1 re-feeding the prompt) matches the graph path."""
    d, fm, gm = _setup(TINY, seed=25)
    from bfp import synth
    prompt = synth.make_prompt(d, 3, seed=25)
    a = gm.decode(prompt[None, :], 12, hist=True)
    b = gm.decode(prompt[None, :], 7, hist=True)      # shorter: a different step count
    c = gm.decode(prompt[None, :], 12, hist=True)
    _same(a, c)
    assert (b[0][0] == a[0][0][:7]).all()
    p, g = _both(gm, np.array([5]), 6)
    _same(p, g)
    gm.close()


def test_persist_step_times(gpu):
    d, fm, gm = _setup(TINY, seed=26)
    from bfp import synth
    prompt = synth.make_prompt(d, 4, seed=26)
    gm.decode(prompt[None, :], 8)
    st = gm.step_times_ms()
    total, gen = gm.decode_time_ms()
    assert st.shape == (12,) and (st > 0).all()
    assert 0 < gen <= total and abs(st[4:].sum() - gen) < 1e-3 * max(gen, 1.0) + 1e-3
    gm.close()


@pytest.mark.parametrize("max_ctx", [40, 600], ids=["short", "long-form"])
def test_persist_trace(gpu, max_ctx):
    """A traced decode (stage stamps, BFP_DECODE_TRACE) gives the untraced
    tokens and layer outputs, and the Q|K|V role's stamps follow its own
    order at every (step, layer): input ready, RMSNorm, matvec, q|k|v
    stored, then attention job 0's phases (q|k|v in and RoPE, scores,
    softmax, AV chains) and its output stored; the head's three stamps are
    ordered at every step that ran it."""
    cfg = dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, NL=2, MAX_CTX=max_ctx, VOCAB=1024)
    d, fm, gm = _setup(cfg, seed=27)
    from bfp import synth
    prompt = synth.make_prompt(d, 8, seed=27)
    n_gen = 24
    want = gm.decode(prompt[None, :], n_gen, hist=True)
    got = gm.decode(prompt[None, :], n_gen, hist=True, trace=True)
    assert gm.decode_path() == "persist"
    _same(got, want)
    lay, head = gm.decode_trace()
    steps = 8 + n_gen
    assert lay.shape == (steps, d.NL, 20) and head.shape == (steps, 3)
    order = [0, 10, 11, 1, 2, 16, 17, 18, 19, 3]
    for s in range(steps):
        for li in range(d.NL):
            v = lay[s, li, order].astype(np.int64)
            assert (v > 0).all() and (np.diff(v) >= 0).all(), (s, li, v)
        if s >= 7:   # sim A's loop runs the head from step n_prompt - 1 on
            assert (head[s] > 0).all() and (np.diff(head[s].astype(np.int64)) >= 0).all(), s
    gm.close()
