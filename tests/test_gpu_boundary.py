"""GPU tests of the drop-in boundary beyond the matvec and the decode loop:
the float64 leaf ops (rmsnorm_fp, silu_fp, softmax_fp, rope_fp,
gen_smollm_blockfp_full.py:236-258), the exact BFP encoder, the context
matvec, and fwd_layer(h, lw, pos, kv, kv_pos) called exactly as the
reference calls it (caller-owned lw and kv, kv updated in place, pos and
kv_pos apart as gen_smollm_blockfp_bfp.py:42-43 drives them).

References: the single-layer baker's own stage dumps and the reference's
fwd_layer run on config 1 (tests/golden, written by the reference's code),
and the oracle (oracle/bfp_sim.py) where no reference vector covers a case.
"""
import numpy as np
import pytest

from oracle import bfp_sim as sim
from refcases import GOLDEN, baker_case

pytestmark = pytest.mark.gpu


def _ulp_dist(a, b):
    """|a - b| in units in the last place, elementwise, for finite float64
    values of one sign (the integer distance of their bit patterns)."""
    ia = np.asarray(a, np.float64).view(np.int64)
    ib = np.asarray(b, np.float64).view(np.int64)
    return np.abs(ia - ib)


# Floors of the softmax_fp comparison with numpy (test_softmax_fp).  Measured
# on MI355X against numpy 2.2.6 (AVX512F loops) on the GPU box's EPYC host:
# of 6,864 probabilities 5,991 bit-equal, 708 one ulp apart, 163 two, 2 three.
SOFTMAX_BIT_EQUAL_MIN = 0.85
SOFTMAX_FAR_MAX = 0.002


def _bfp_vec(rng, n, scale=1.0):
    """A decoded BFP vector (what every stage of the reference passes on)."""
    return sim.fp_quantize_vec(rng.standard_normal(n) * scale)


# --------------------------------------------------------------- leaf ops
def test_rmsnorm_fp(gpu):
    import bfp.api as api
    rng = np.random.default_rng(21)
    for n in (16, 64, 576, 1536, 4096):
        for scale in (1e-3, 1.0, 40.0):
            x = _bfp_vec(rng, n, scale)
            g = sim.fp_quantize_vec(1.0 + 0.05 * rng.standard_normal(n))
            got = api.rmsnorm_fp(x, g)
            want = sim.rmsnorm_fp(x, g)
            assert (got == want).all(), (n, scale)
    # raw float64 input and another eps, as the function allows
    x, g = rng.standard_normal(576), rng.standard_normal(576)
    assert (api.rmsnorm_fp(x, g, eps=1e-3) == sim.rmsnorm_fp(x, g, eps=1e-3)).all()


def test_silu_fp(gpu):
    import bfp.api as api
    rng = np.random.default_rng(22)
    x = np.concatenate([_bfp_vec(rng, 1536, s) for s in (0.01, 1.0, 8.0, 60.0)])
    assert (api.silu_fp(x) == sim.silu_fp(x)).all()


def test_softmax_fp(gpu):
    """Probabilities are float64 and not quantised, so numpy's SIMD exp and
    the device exp show through: each is within 1 ulp of exp, so two exps
    differ by at most 2 ulps, the pairwise sum (same order on both sides)
    by at most 2 ulps relative, and the quotient adds one rounding: the test
    bounds the difference at 6 ulps.  Where every exp is exact (equal
    scores: exp(0) = 1) the summation order alone decides, and the results
    must be identical."""
    import bfp.api as api
    rng = np.random.default_rng(23)
    hist = np.zeros(7, np.int64)   # probabilities by ulp distance 0..6
    for n in (1, 2, 7, 8, 9, 64, 129, 500, 2048, 4096):
        x = rng.standard_normal(n) * 3.0
        got, want = api.softmax_fp(x), sim.softmax_fp(x)
        np.testing.assert_array_max_ulp(got, want, maxulp=6)
        hist += np.bincount(_ulp_dist(got, want), minlength=7)[:7]
    total = int(hist.sum())
    print(f"softmax_fp vs numpy: probabilities by ulp distance 0..6: {hist.tolist()} of {total}")
    # measured on MI355X against numpy 2.2.6's AVX512F exp; a change in the
    # device exp or in the summation order moves this distribution
    assert hist[0] >= SOFTMAX_BIT_EQUAL_MIN * total, hist.tolist()
    assert hist[3:].sum() <= SOFTMAX_FAR_MAX * total, hist.tolist()
    # exp(0) == 1 exactly: equal scores give n ones summed in numpy's order
    for n in (3, 100, 1000, 4095):
        x = np.full(n, 0.625)
        assert (api.softmax_fp(x) == sim.softmax_fp(x)).all(), n


@pytest.mark.parametrize("name", ["small", "full"])
def test_softmax_fp_baker_probs(gpu, name):
    """softmax_fp on the last head's scores of the baker's case against the
    baker's own STAGE_PROBS dump (tile-quantised over 16 slots)."""
    import bfp.api as api
    from test_oracle_vs_reference import _last_head_scores, _pad16
    c = baker_case(name)
    f, MC = c["fixture"], c["cfg"]["MAX_CTX"]
    sc, _ = _last_head_scores(c)
    m, e = api.tile_quantize(_pad16(api.softmax_fp(sc), MC))
    assert (m.reshape(-1)[:MC] == f["PROBS_m"]).all() and (np.full(MC, e[0]) == f["PROBS_e"]).all()


def test_rope_fp(gpu):
    import bfp.api as api
    rng = np.random.default_rng(24)
    for pos in (0, 1, 5, 63, 2047, 100000):
        x = _bfp_vec(rng, 64, 2.0)
        assert (api.rope_fp(x, pos) == sim.rope_fp(x, pos)).all(), pos
    heads = _bfp_vec(rng, 9 * 64)
    want = np.concatenate([sim.rope_fp(heads[h * 64:(h + 1) * 64], 17) for h in range(9)])
    assert (api.rope_fp(heads, 17) == want).all()


# ------------------------------------------------------------ exact encode
def test_tile_encode_keeps_raw_tiles(gpu):
    """Decoded raw tiles whose largest magnitude is the mantissa -32768:
    tile_quantize re-rounds odd mantissas, tile_encode gives the values
    back; other tiles encode as tile_quantize does; non-BFP values raise."""
    import bfp.api as api
    rng = np.random.default_rng(25)
    m = rng.integers(-32768, 32768, size=(64, 16)).astype(np.int16)
    m[::2, 3] = -32768
    m[::4, 5] = 12345                                   # odd: re-rounded by tile_quantize
    e = rng.integers(-100, 100, size=64).astype(np.int8)
    v = sim.tile_decode(m, e)
    em, ee = api.tile_encode(v)
    assert (sim.tile_decode(em, ee) == v).all()
    qm, qe = sim.tile_quantize(v)
    exact_q = (sim.tile_decode(qm, qe).reshape(-1, 16) == v.reshape(-1, 16)).all(axis=1)
    assert (~exact_q).any()
    assert (em[exact_q] == qm[exact_q]).all() and (ee[exact_q] == qe[exact_q]).all()
    assert (em[~exact_q] == m[~exact_q]).all() and (ee[~exact_q] == e[~exact_q]).all()
    with pytest.raises(ValueError):
        api.tile_encode(rng.standard_normal(32))
    x = rng.standard_normal(32)
    wm, we = api.tile_encode(x, strict=False)           # non-BFP: tile_quantize's tiles
    qm, qe = sim.tile_quantize(x)
    assert (wm == qm).all() and (we == qe).all()
    zm, ze = api.tile_encode(np.zeros(16))
    assert (zm == 0).all() and (ze == -127).all()


# ---------------------------------------------------------- context matvec
def test_context_matvec_every_slot(gpu):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(NL=2, MAX_CTX=8, VOCAB=256)
    fm = synth.make_model(d, seed=26)
    om = sim.build_model(fm)
    gm = BfpModel(d)
    gm.load_fp32(fm)
    rng = np.random.default_rng(26)
    for layer in (0, 1):
        for name in ("Wq", "Wk", "Wv", "Wo", "Wg", "Wu", "Wd"):
            Wm, We = om.layers[layer][name]
            n_in = Wm.shape[1] * 16
            xs = [sim.tile_quantize(rng.standard_normal(n_in)) for _ in range(3)]
            ym, ye = gm.matvec(name, layer, np.stack([x[0].reshape(-1) for x in xs]),
                               np.stack([x[1] for x in xs]))
            for b, (xm, xe) in enumerate(xs):
                wm, we = sim.matvec_bfp(xm, xe, Wm, We)
                assert (ym[b] == wm.reshape(-1)).all() and (ye[b] == we).all(), (layer, name, b)
    gm.close()


# -------------------------------------------------- fwd_layer, drop-in form
@pytest.mark.parametrize("name", ["small", "full"])
def test_fwd_layer_baker_call_pattern(gpu, name):
    """The baker's sequence (gen_smollm_blockfp_bfp.py:304-344) with this
    package's functions in place of the reference's: quantize_W and
    fp_quantize_vec on the device, the preloaded cache as float64 rows,
    then fwd_layer(h_in_q, lw, POS, kv, KV_POS).  The output and the K/V
    row written at KV_POS must equal the baker's own dumps."""
    import bfp.api as api
    c = baker_case(name)
    cfg, f = c["cfg"], c["fixture"]
    lw = {n: api.quantize_W(W) for n, W in c["W"].items()}
    lw["g1"] = api.fp_quantize_vec(c["g1"])
    lw["g2"] = api.fp_quantize_vec(c["g2"])
    MC, H_KV, HD = cfg["MAX_CTX"], cfg["H_KV"], cfg["HD"]
    kv = {"k": np.zeros((MC, H_KV, HD)), "v": np.zeros((MC, H_KV, HD))}
    for t in range(MC):   # the baker's preloaded rows: tile_decode(tile_quantize(K_init[t]))
        kv["k"][t] = api.tile_decode(*c["kq"][t]).reshape(H_KV, HD)
        kv["v"][t] = api.tile_decode(*c["vq"][t]).reshape(H_KV, HD)
    h = api.tile_decode(f["HIN_m"], f["HIN_e"])
    out = api.fwd_layer(h, lw, cfg["POS"], kv, cfg["KV_POS"])
    om, oe = sim.tile_quantize(out)
    assert (om.reshape(-1) == f["HOUT_m"]).all() and (oe == f["HOUT_e"]).all()
    km, ke = sim.tile_quantize(kv["k"][cfg["KV_POS"]].reshape(-1))
    vm, ve = sim.tile_quantize(kv["v"][cfg["KV_POS"]].reshape(-1))
    assert (km.reshape(-1) == f["K_m"]).all() and (ke == f["K_e"]).all()
    assert (vm.reshape(-1) == f["V_m"]).all() and (ve == f["V_e"]).all()


def test_fwd_layer_config1_call_pattern(gpu):
    """BASELINE config 1 through the reference's own calls: lw from
    quantize_W / fp_quantize_vec, kv zeros of MAX_CTX 16, then
    fwd_layer(h, lw, pos=p, kv=kv, kv_pos=p) for p = 0..7 -- against the
    reference's fwd_layer run (ref_layer_cfg1.npz), outputs and cache."""
    import bfp.api as api
    from bfp import Dims, synth
    f = np.load(GOLDEN / "ref_layer_cfg1.npz")
    d = Dims(NL=1, MAX_CTX=16, VOCAB=256)
    fm = synth.make_model(d, seed=int(f["seed"]))
    xs = synth.make_layer_inputs(d, 8, seed=int(f["seed"]))
    lw0 = fm.layers[0]
    lw = {n: api.quantize_W(np.asarray(lw0[n]).astype(np.float64))
          for n in ("Wq", "Wk", "Wv", "Wo", "Wg", "Wu", "Wd")}
    lw["g1"] = api.fp_quantize_vec(np.asarray(lw0["g1"]).astype(np.float64))
    lw["g2"] = api.fp_quantize_vec(np.asarray(lw0["g2"]).astype(np.float64))
    kv = {"k": np.zeros((d.MAX_CTX, d.H_KV, d.HD)), "v": np.zeros((d.MAX_CTX, d.H_KV, d.HD))}
    for p in range(8):
        h = api.fp_quantize_vec(xs[p])
        out = api.fwd_layer(h, lw, pos=p, kv=kv, kv_pos=p)
        m, e = sim.tile_quantize(out)
        assert (m.reshape(-1) == f["hout_m"][p]).all() and (e == f["hout_e"][p]).all(), p
    km, ke = sim.tile_quantize(kv["k"][:8].reshape(-1))
    vm, ve = sim.tile_quantize(kv["v"][:8].reshape(-1))
    assert (km.reshape(8, -1) == f["k_m"]).all() and (ke.reshape(8, -1) == f["k_e"]).all()
    assert (vm.reshape(8, -1) == f["v_m"]).all() and (ve.reshape(8, -1) == f["v_e"]).all()
    assert not kv["k"][8:].any() and not kv["v"][8:].any()


@pytest.mark.parametrize("pos,kv_pos,max_ctx", [(2, 6, 8), (9, 3, 16), (100, 5, 8),
                                                 (3000, 40, 64), (700, 555, 600)])
def test_fwd_layer_pos_apart_from_kv_pos(gpu, pos, kv_pos, max_ctx):
    """RoPE position and cache slot apart (including positions past the
    RoPE table and the long-context attention form): every output and the
    cache against the oracle's fwd_layer on the same caller-owned kv."""
    import bfp.api as api
    from bfp import Dims, synth
    d = Dims(NL=1, MAX_CTX=max_ctx, VOCAB=256)
    fm = synth.make_model(d, seed=27)
    om = sim.build_model(fm)
    lw = om.layers[0]
    rng = np.random.default_rng(pos * 7 + kv_pos)
    kv_ref = sim.new_kv(om.dims, max_ctx)
    for t in range(kv_pos):   # a cache the reference could have written: decoded tiles
        kv_ref["k"][t] = _bfp_vec(rng, d.KV, 0.5).reshape(d.H_KV, d.HD)
        kv_ref["v"][t] = _bfp_vec(rng, d.KV, 0.5).reshape(d.H_KV, d.HD)
    kv_dev = {"k": kv_ref["k"].copy(), "v": kv_ref["v"].copy()}
    for step in range(2):
        h = _bfp_vec(rng, d.D)
        want = sim.fwd_layer(h, lw, pos=pos + step, kv=kv_ref, kv_pos=kv_pos + step, dims=om.dims)
        got = api.fwd_layer(h, lw, pos + step, kv_dev, kv_pos + step)
        assert (got == want).all(), step
        assert (kv_dev["k"] == kv_ref["k"]).all() and (kv_dev["v"] == kv_ref["v"]).all(), step


def test_fwd_layer_errors(gpu):
    import bfp.api as api
    from bfp import Dims, synth
    d = Dims(D=64, H_Q=1, H_KV=1, FFN=128, NL=1, MAX_CTX=4, VOCAB=256)
    om = sim.build_model(synth.make_model(d, seed=28))
    lw = om.layers[0]
    kv = sim.new_kv(om.dims, 4)
    h = sim.fp_quantize_vec(np.random.default_rng(0).standard_normal(64))
    with pytest.raises(IndexError):
        api.fwd_layer(h, lw, 0, kv, 4)
    with pytest.raises(ValueError):
        api.fwd_layer(h[:48], lw, 0, kv, 0)
    with pytest.raises(ValueError):                    # not a BFP vector
        api.fwd_layer(np.random.default_rng(1).standard_normal(64), lw, 0, kv, 0)


def test_fwd_layer_cache_rows_changed_by_caller(gpu):
    """fwd_layer sends only the cache rows that differ from what its device
    context already holds.  A caller that rewrites a middle row between calls,
    or a second caller with another cache on the same weights, must still get
    the oracle's outputs on its own rows."""
    import bfp.api as api
    from bfp import Dims, synth
    d = Dims(NL=1, MAX_CTX=24, VOCAB=256)
    om = sim.build_model(synth.make_model(d, seed=29))
    lw = om.layers[0]
    rng = np.random.default_rng(29)
    kv_ref = sim.new_kv(om.dims, d.MAX_CTX)
    kv_dev = {"k": kv_ref["k"].copy(), "v": kv_ref["v"].copy()}
    other_ref = sim.new_kv(om.dims, d.MAX_CTX)
    other_dev = {"k": other_ref["k"].copy(), "v": other_ref["v"].copy()}
    for p in range(12):
        if p == 7:   # the caller rewrites rows 3 (K) and 5 (V) of its own cache
            for kv in (kv_ref, kv_dev):
                kv["k"][3] = _bfp_vec(np.random.default_rng(3), d.KV).reshape(d.H_KV, d.HD)
                kv["v"][5] = _bfp_vec(np.random.default_rng(5), d.KV).reshape(d.H_KV, d.HD)
        h = _bfp_vec(rng, d.D)
        want = sim.fwd_layer(h, lw, pos=p, kv=kv_ref, kv_pos=p, dims=om.dims)
        got = api.fwd_layer(h, lw, p, kv_dev, p)
        assert (got == want).all(), p
        assert (kv_dev["k"] == kv_ref["k"]).all() and (kv_dev["v"] == kv_ref["v"]).all(), p
        if p % 4 == 3:   # another cache on the same weights, interleaved
            h2 = _bfp_vec(rng, d.D)
            q = p // 4
            want2 = sim.fwd_layer(h2, lw, pos=q, kv=other_ref, kv_pos=q, dims=om.dims)
            got2 = api.fwd_layer(h2, lw, q, other_dev, q)
            assert (got2 == want2).all(), ("other", q)
