"""GPU parity of the decode head and the autoregressive driver against the
oracle (full.py:411-443): token ids and every layer's output at every step,
bit for bit, graph-replayed and directly launched, batch 1 and batched."""
import numpy as np
import pytest

from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

TINY = dict(D=128, H_Q=2, H_KV=1, HD=64, FFN=256, NL=2, MAX_CTX=32, VOCAB=512)


def _setup(cfg, seed, max_batch=1):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=seed)
    om = sim.build_model(fm)
    gm = BfpModel(d, max_batch=max_batch)
    gm.load_fp32(fm)
    return d, om, gm


def _oracle_decode(om, prompt, n_gen):
    d = om.dims
    steps = len(prompt) + n_gen
    hm = np.zeros((steps, d.NL, d.D), np.int16)
    he = np.zeros((steps, d.NL, d.D // 16), np.int8)

    def on_layer(step, li, h):
        m, e = sim.tile_quantize(h)
        hm[step, li] = m.reshape(-1)
        he[step, li] = e

    toks = sim.decode(om, prompt, n_gen, on_layer=on_layer)
    return toks[len(prompt):], hm, he


def test_head_argmax_and_logits(gpu):
    d, om, gm = _setup(TINY, seed=4, max_batch=4)
    rng = np.random.default_rng(1)
    hs = [sim.fp_quantize_vec(rng.standard_normal(d.D) * s) for s in (0.5, 1.0, 3.0, 10.0)]
    q = [sim.tile_quantize(h) for h in hs]
    am, lg = gm.head(np.stack([x[0].reshape(-1) for x in q]), np.stack([x[1] for x in q]),
                     logits=True)
    same = total = 0
    worst = 0.0
    for b, h in enumerate(hs):
        want = sim.head_logits(h, om.norm_w_q, om.embed)
        # Both sides sum the same D exact-operand products in different
        # orders (the kernel's fixed 16-lane tree, numpy's BLAS dgemv), so
        # each is within gamma_D * sum|h_n,i * E_j,i| of the exact dot
        # product (Higham, Accuracy and Stability of Numerical Algorithms,
        # eq. 3.5: gamma_n = n u / (1 - n u), u = 2^-53), and the two within
        # twice that.  A dropped or doubled term exceeds it by orders of
        # magnitude.
        hn = (h / np.sqrt(np.mean(h * h) + 1e-5)) * om.norm_w_q
        u = 2.0 ** -53
        gam = d.D * u / (1 - d.D * u)
        bound = 2 * gam * (np.abs(hn) @ np.abs(om.embed).T)
        err = np.abs(lg[b] - want)
        assert (err <= bound).all(), float((err / bound).max())
        worst = max(worst, float((err / bound).max()))
        same += int((lg[b] == want).sum())
        total += want.size
        assert am[b] == int(np.argmax(want))
    print(f"head logits vs numpy's h_normed @ embed.T: {same}/{total} bit-equal, "
          f"largest error {worst:.3g} of the bound")
    gm.close()


def test_head_batched_equals_single_d576(gpu):
    """The batched head (k_head_norm + k_head_gemv, D = 576: the exact-width
    variant) over 20 sequences -- one full LDS group of 16 and a partial
    one -- equals the single-sequence head bit for bit (same summation
    order per logit), and the oracle to rounding."""
    cfg = dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, NL=1, MAX_CTX=8, VOCAB=1024)
    d, om, gm = _setup(cfg, seed=9, max_batch=20)
    rng = np.random.default_rng(9)
    hs = [sim.fp_quantize_vec(rng.standard_normal(d.D) * (0.3 + 0.2 * b)) for b in range(20)]
    q = [sim.tile_quantize(h) for h in hs]
    am, lg = gm.head(np.stack([x[0].reshape(-1) for x in q]), np.stack([x[1] for x in q]),
                     logits=True)
    for b in (0, 7, 15, 16, 19):
        a1, l1 = gm.head(q[b][0].reshape(1, -1), q[b][1].reshape(1, -1), logits=True)
        assert (lg[b].view(np.int64) == l1[0].view(np.int64)).all(), b
        assert am[b] == a1[0]
        want = sim.head_logits(hs[b], om.norm_w_q, om.embed)
        assert np.allclose(lg[b], want, rtol=1e-13, atol=1e-13)
        assert am[b] == int(np.argmax(want))
    gm.close()


@pytest.mark.parametrize("D,vocab", [(576, 4176), (128, 512), (192, 1040)],
                         ids=["d576-ragged", "d128", "d192"])
def test_head_sequence_lanes_equal_single(gpu, D, vocab):
    """The batched head with sequences on the lanes (k_head_seq, batches of
    32 and more) over 70 sequences -- a full lane group of 64 and a partial
    one -- equals the single-sequence head bit for bit, logits and argmax.
    The vocabulary leaves a short last workgroup (4176 rows in 32-row
    workgroups).  Tied logits: rows 5 and 9 (one workgroup) hold the same
    vector V and rows 3 and 40 (two workgroups) hold -V, scaled so that for
    most sequences one of the two ties holds the largest logit: the argmax is
    then the tie's first row."""
    from bfp import Dims, synth
    from bfp.model import BfpModel
    H = D // 64
    cfg = dict(D=D, H_Q=H, H_KV=1, HD=64, FFN=2 * D, NL=1, MAX_CTX=8, VOCAB=vocab)
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=31)
    V = fm.embed[7].copy() * np.float32(60.0)
    fm.embed[5] = V
    fm.embed[9] = V
    fm.embed[3] = -V
    fm.embed[40] = -V
    gm = BfpModel(d, max_batch=70)
    gm.load_fp32(fm)
    rng = np.random.default_rng(31)
    hs = [sim.fp_quantize_vec(rng.standard_normal(d.D) * (0.3 + 0.01 * b)) for b in range(70)]
    q = [sim.tile_quantize(h) for h in hs]
    am, lg = gm.head(np.stack([x[0].reshape(-1) for x in q]), np.stack([x[1] for x in q]),
                     logits=True)
    n_tie = 0
    for b in range(70):
        a1, l1 = gm.head(q[b][0].reshape(1, -1), q[b][1].reshape(1, -1), logits=True)
        assert (lg[b].view(np.int64) == l1[0].view(np.int64)).all(), b
        assert am[b] == a1[0] == int(np.argmax(lg[b])), b     # np.argmax: first index
        if lg[b][am[b]] in (lg[b][5], lg[b][3]):
            assert am[b] in (3, 5), (b, am[b])
            n_tie += 1
    assert n_tie >= 40, n_tie
    gm.close()


@pytest.mark.parametrize("D,vocab", [(576, 4176), (128, 512), (192, 1040)],
                         ids=["d576-ragged", "d128", "d192"])
def test_head_bounded_equals_full(gpu, D, vocab):
    """The bounded head (an exact int16 dot product brackets every logit;
    only the 16-row blocks that can hold the largest one get float64
    logits) returns the argmax of the full float64 head, first index on
    ties, over 70 sequences (a group of 64 and a ragged one) and a
    vocabulary whose last workgroup is short.  The embedding holds exact ties
    within and across blocks (rows 5, 9; 3, 40 = -(5)), rows one float32 ulp
    apart (100, 101, in two sequences' lead), zero rows (200-215, a whole
    block, and 300) and rows of very different scales."""
    from bfp import Dims, synth
    from bfp.model import BfpModel
    H = D // 64
    cfg = dict(D=D, H_Q=H, H_KV=1, HD=64, FFN=2 * D, NL=1, MAX_CTX=8, VOCAB=vocab)
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=37)
    E = fm.embed
    V = E[7].copy() * np.float32(60.0)
    E[5] = V
    E[9] = V
    E[3] = -V
    E[40] = -V
    E[100] = E[11] * np.float32(55.0)
    E[101] = np.nextafter(E[100], np.float32(np.inf))
    E[200:216] = 0.0
    E[300] = 0.0
    E[400] *= np.float32(1e-30)
    E[401] *= np.float32(4.0)
    E[402] *= np.float32(1e-5)
    gm = BfpModel(d, max_batch=70)
    gm.load_fp32(fm)
    rng = np.random.default_rng(37)
    hs = [sim.fp_quantize_vec(rng.standard_normal(d.D) * (0.3 + 0.01 * b)) for b in range(70)]
    hs[1] = sim.fp_quantize_vec(E[11].astype(np.float64) * 40.0)    # leads with rows 100/101
    hs[2] = sim.fp_quantize_vec(-E[11].astype(np.float64) * 40.0)
    hs[3] = np.zeros(d.D)                                            # all logits +0
    q = [sim.tile_quantize(h) for h in hs]
    hm = np.stack([x[0].reshape(-1) for x in q])
    he = np.stack([x[1] for x in q])
    am_full, lg = gm.head(hm, he, logits=True)      # logits asked for: the float64 matrix-core head
    am_b, _ = gm.head(hm, he)                       # argmax only: the bounded head
    for b in range(70):
        want = int(np.argmax(lg[b]))                # first index on ties
        assert am_full[b] == want, b
        assert am_b[b] == want, (b, am_b[b], want)
    assert am_b[3] == 0                             # every logit +0: the first row
    gm.close()


@pytest.mark.parametrize("graph", [True, False], ids=["graph", "direct"])
def test_decode_tiny(gpu, graph):
    d, om, gm = _setup(TINY, seed=5)
    from bfp import synth
    prompt = synth.make_prompt(d, 5, seed=5)
    want, whm, whe = _oracle_decode(om, prompt, 10)
    toks, (hm, he) = gm.decode(prompt[None, :], 10, hist=True, graph=graph)
    for s in range(whm.shape[0]):
        for li in range(d.NL):
            assert (he[0, s, li] == whe[s, li]).all() and (hm[0, s, li] == whm[s, li]).all(), \
                f"step {s} layer {li} differs"
    assert list(toks[0]) == list(want)
    gm.close()


def test_decode_batched(gpu):
    d, om, gm = _setup(TINY, seed=6, max_batch=3)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 4, seed=10 + b) for b in range(3)])
    toks, _ = gm.decode(prompts, 6)
    for b in range(3):
        want, _, _ = _oracle_decode(om, prompts[b], 6)
        assert list(toks[b]) == list(want), f"sequence {b}"
    gm.close()


def test_decode_single_token_prompt(gpu):
    """n_prompt = 1: the head runs from step 0 and step 1 re-feeds the prompt."""
    d, om, gm = _setup(TINY, seed=7)
    want, _, _ = _oracle_decode(om, [3], 4)
    toks, _ = gm.decode(np.array([[3]]), 4)
    assert list(toks[0]) == list(want)
    gm.close()


@pytest.mark.parametrize("graph", [True, False], ids=["graph", "direct"])
def test_decode_rtl_loop(gpu, graph):
    """The FPGA driver's loop policy (autoregress_bfp_top.sv:357-386): every
    step's prediction, the step after the prompt fed by the last prediction;
    batched sequences against the oracle's restatement."""
    d, om, gm = _setup(TINY, seed=13, max_batch=3)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 4, seed=40 + b) for b in range(3)])
    toks, _ = gm.decode(prompts, 7, graph=graph, rtl_loop=True)
    assert toks.shape == (3, 11)
    for b in range(3):
        assert list(toks[b]) == sim.decode_rtl_loop(om, prompts[b], 7), f"sequence {b}"
    gm.close()


def test_decode_errors(gpu):
    from bfp._lib import BfpError
    d, om, gm = _setup(TINY, seed=8)
    with pytest.raises(BfpError):
        gm.decode(np.array([[d.VOCAB]]), 2)           # token out of range
    with pytest.raises(BfpError):
        gm.decode(np.array([[1, 2]]), d.MAX_CTX)       # beyond the KV capacity
    gm.close()


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_non_finite_embedding_refused(gpu, bad):
    """The bounded head's logit bounds hold for finite embeddings only, so
    bfp_load_weights(BFP_EMBED) refuses a NaN or an infinity (naming its
    row and column); a finite embedding loaded afterwards decodes as the
    oracle does, on the batch-1 and the batched (bounded head) paths."""
    from bfp import Dims, synth
    from bfp._lib import BfpError
    from bfp.model import BfpModel
    d = Dims(**TINY)
    fm = synth.make_model(d, seed=21)
    om = sim.build_model(fm)
    gm = BfpModel(d, max_batch=32)
    gm.load_fp32(fm)
    e = fm.embed.copy()
    e[300, 77] = bad
    with pytest.raises(BfpError, match=r"\(300, 77\) is not finite"):
        gm.load_tensor("embed", fp32=e)
    gm.load_tensor("embed", fp32=fm.embed)
    prompts = np.stack([synth.make_prompt(d, 4, seed=60 + b) for b in range(32)])
    toks, _ = gm.decode(prompts, 5)
    for b in (0, 17, 31):
        assert list(toks[b]) == sim.decode(om, prompts[b], 5)[4:], f"sequence {b}"
    toks1, _ = gm.decode(prompts[:1], 5)
    assert list(toks1[0]) == list(toks[0])
    gm.close()


def test_decode_long_context(gpu):
    """BASELINE config 4's positions on a 2-layer model: a 48-token prompt,
    then greedy decode through position 2047 (KV cache of 2048 positions,
    softmax over up to 2048 scores), every layer output at every step
    against the oracle."""
    cfg = dict(TINY, MAX_CTX=2048)
    d, om, gm = _setup(cfg, seed=11)
    from bfp import synth
    prompt = synth.make_prompt(d, 48, seed=11)
    n_gen = 2048 - 48
    print("[decode] long context: oracle", flush=True)
    want, whm, whe = _oracle_decode(om, prompt, n_gen)
    print("[decode] long context: gpu", flush=True)
    toks, (hm, he) = gm.decode(prompt[None, :], n_gen, hist=True)
    bad = [s for s in range(2048) if not ((hm[0, s] == whm[s]).all() and (he[0, s] == whe[s]).all())]
    assert not bad, f"steps with differing layer outputs: {bad[:10]}"
    assert list(toks[0]) == list(want)
    gm.close()


def test_decode_long_context_full_width(gpu):
    """The long-context attention form (capacity above 512: four workgroups
    per head, one 16-dimension tile each) at SmolLM2's width -- 9 heads in 3
    KV groups -- for two sequences at once: every layer output at every step
    to position 519 against the oracle."""
    cfg = dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, NL=1, MAX_CTX=520, VOCAB=512)
    d, om, gm = _setup(cfg, seed=15, max_batch=2)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 10, seed=15 + b) for b in range(2)])
    n_gen = d.MAX_CTX - 10
    print("[decode] long context, full width: gpu", flush=True)
    toks, (hm, he) = gm.decode(prompts, n_gen, hist=True)
    for b in range(2):
        print(f"[decode] long context, full width: oracle seq {b}", flush=True)
        want, whm, whe = _oracle_decode(om, prompts[b], n_gen)
        bad = [s for s in range(d.MAX_CTX) if not ((hm[b, s] == whm[s]).all() and (he[b, s] == whe[s]).all())]
        assert not bad, f"seq {b}: steps with differing layer outputs: {bad[:10]}"
        assert list(toks[b]) == list(want)
    gm.close()


@pytest.mark.parametrize("max_ctx", [200, 300], ids=["lane-split-256", "per-thread-512"])
def test_decode_mid_context(gpu, max_ctx):
    """Context capacities of 129..256 (scores spread over 32-lane half-waves)
    and 257..512 (one score per thread), V staged in chunks of 128 rows:
    greedy decode to the capacity after a 10-token prompt, every layer output
    at every step against the oracle, for two sequences at once."""
    cfg = dict(TINY, MAX_CTX=max_ctx)
    d, om, gm = _setup(cfg, seed=14, max_batch=2)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 10, seed=14 + b) for b in range(2)])
    n_gen = max_ctx - 10
    toks, (hm, he) = gm.decode(prompts, n_gen, hist=True)
    for b in range(2):
        want, whm, whe = _oracle_decode(om, prompts[b], n_gen)
        bad = [s for s in range(max_ctx) if not ((hm[b, s] == whm[s]).all() and (he[b, s] == whe[s]).all())]
        assert not bad, f"seq {b}: steps with differing layer outputs: {bad[:10]}"
        assert list(toks[b]) == list(want)
    gm.close()


@pytest.mark.parametrize("grouped", [True, False], ids=["kv_group", "one_head"])
def test_decode_ragged_batch_joined_launches(gpu, grouped, monkeypatch):
    """40 sequences (groups of 16, 16 and 8) on a D=256 model, where the
    batched decode joins the Q|K|V matvec with the attention -- a KV group's
    query heads per workgroup (the default) or one head each
    (BFP_ATT_GROUP=0) -- and the RMSNorms with the residual matvecs (tagged
    hand-offs inside a launch): every sequence checked equals its
    single-sequence decode, and sequence 0 the oracle."""
    if not grouped:
        monkeypatch.setenv("BFP_ATT_GROUP", "0")
    cfg = dict(D=256, H_Q=4, H_KV=2, HD=64, FFN=512, NL=2, MAX_CTX=40, VOCAB=512)
    d, om, gm = _setup(cfg, seed=21, max_batch=40)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 6, seed=300 + b) for b in range(40)])
    toks, _ = gm.decode(prompts, 10, pipe=False)
    assert gm.decode_form() == ("mx+qkv_attn+attn_group+norm_fused" if grouped else "mx+qkv_attn+norm_fused")
    for b in (0, 15, 16, 33, 39):
        single, _ = gm.decode(prompts[b:b + 1], 10)
        assert list(single[0]) == list(toks[b]), b
    want, _, _ = _oracle_decode(om, prompts[0], 10)
    assert list(toks[0]) == list(want)
    gm.close()


def test_decode_batch64_matches_single(gpu):
    """64 independent sequences in one decode equal their single-sequence
    decodes (and sequence 0 the oracle)."""
    d, om, gm = _setup(TINY, seed=12, max_batch=64)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 8, seed=100 + b) for b in range(64)])
    toks, _ = gm.decode(prompts, 12)
    for b in (0, 1, 31, 63):
        single, _ = gm.decode(prompts[b:b + 1], 12)
        assert list(single[0]) == list(toks[b]), b
    want, _, _ = _oracle_decode(om, prompts[0], 12)
    assert list(toks[0]) == list(want)
    gm.close()


def test_batched_trace(gpu):
    """A traced batched decode on the matrix cores gives the untraced tokens,
    and every stamped block's phases are in order (entry, exponents staged,
    row maxima, tile sums, sums reduced, epilogue); the four kernels stamp
    their block counts (chunks x sequence groups), and the grouped attention
    workgroups of the joined Q|K|V launch (one per KV group and sequence,
    after the matvec blocks) theirs (entry, q|k|v in, RoPE and staged rows,
    scores, softmax, AV chains)."""
    cfg = dict(D=256, H_Q=4, H_KV=2, HD=64, FFN=512, NL=2, MAX_CTX=24, VOCAB=512)
    d, om, gm = _setup(cfg, seed=33, max_batch=24)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 6, seed=500 + b) for b in range(24)])
    want, _ = gm.decode(prompts, 8, pipe=False)
    got, _ = gm.decode(prompts, 8, trace=True, pipe=False)
    assert (got == want).all()
    tr = gm.decode_trace()
    assert tr is not None and tr.shape == (4, 1024, 6)
    groups = 2
    chunks = [(d.D + 2 * d.H_KV * d.HD) // 16, d.D // 16, d.FFN // 16, d.D // 16]
    assert "attn_group" in gm.decode_form()
    nblk = chunks[0] * groups
    att = tr[0][nblk:].astype(np.int64)
    att = att[att[:, 0] > 0]
    assert len(att) == d.H_KV * 24
    assert (np.diff(att, axis=1) >= 0).all()
    tr = tr.copy()
    tr[0][nblk:] = 0
    for k in range(4):
        st = tr[k][tr[k][:, 0] > 0].astype(np.int64)
        assert len(st) == chunks[k] * groups, (k, len(st))
        assert (np.diff(st, axis=1) >= 0).all(), k
    gm.close()
