"""The oracle against vectors written by the reference's own code
(tests/golden/gen_ref_vectors.py): the single-layer baker's 13 stage dumps
(+ pre-RoPE Q/K), the reference fwd_layer at BASELINE config 1, and a prefix
of BASELINE config 3's 30-layer decode."""
from pathlib import Path

import numpy as np
import pytest

from oracle import bfp_sim as sim
from refcases import GOLDEN, baker_case

STAGE_FIX = ["N1", "Q", "K", "V", "ATTN", "O", "H1", "N2", "G", "U", "MLP", "D"]


@pytest.mark.parametrize("name", ["small", "full"])
def test_baker_stage_dumps(name):
    c = baker_case(name)
    f, cfg = c["fixture"], c["cfg"]
    m, e = c["hq"]
    assert (m.reshape(-1) == f["HIN_m"]).all() and (e == f["HIN_e"]).all()
    dump = {}
    hout = sim.fwd_layer(c["h"], c["lw"], pos=cfg["POS"], kv=c["kv"], kv_pos=cfg["KV_POS"],
                         dims=c["dims"], dump=dump)
    for tag in STAGE_FIX:
        wm, we = sim.tile_quantize(dump[tag])
        assert (we == f[f"{tag}_e"]).all(), f"stage {tag} exponents"
        assert (wm.reshape(-1) == f[f"{tag}_m"]).all(), f"stage {tag} mantissas"
    hm, he = sim.tile_quantize(hout)
    assert (hm.reshape(-1) == f["HOUT_m"]).all() and (he == f["HOUT_e"]).all()
    # pre-RoPE projections (gen_smollm_blockfp_bfp.py:421-426)
    n1m, n1e = sim.tile_quantize(dump["N1"])
    for tag, w in (("QPRE", "Wq"), ("KPRE", "Wk")):
        pm, pe = sim.tile_quantize(sim.matvec_hw_golden(n1m, n1e, *c["lw"][w]))
        assert (pm.reshape(-1) == f[f"{tag}_m"]).all() and (pe == f[f"{tag}_e"]).all()


def _last_head_scores(c):
    """The scores and probabilities of the last query head at the baker's
    KV_POS, from the oracle's post-RoPE Q and its cache (what the baker
    saves, gen_smollm_blockfp_bfp.py:343-357)."""
    cfg, dims = c["cfg"], c["dims"]
    kv = {k: v.copy() for k, v in c["kv"].items()}
    dump = {}
    sim.fwd_layer(c["h"], c["lw"], pos=cfg["POS"], kv=kv, kv_pos=cfg["KV_POS"], dims=dims,
                  dump=dump)
    hq = cfg["H_Q"] - 1
    g = hq // (cfg["H_Q"] // cfg["H_KV"])
    q = dump["Q"][hq * 64:(hq + 1) * 64]
    sc = np.array([float(np.dot(q, kv["k"][t, g])) / 8.0 for t in range(cfg["KV_POS"] + 1)])
    return sc, sim.softmax_fp(sc)


def _pad16(x, max_ctx):
    p = np.zeros(16)
    p[:len(x)] = x
    return p[:16]


@pytest.mark.parametrize("name", ["small", "full"])
def test_baker_scores_and_probs(name):
    """STAGE_SCORES / STAGE_PROBS: the last head's float64 scores and softmax
    output, padded to 16 slots and tile-quantised as the baker writes them
    (gen_smollm_blockfp_bfp.py:362-372): pins the score and softmax order
    beyond the quantised ATTN stage."""
    c = baker_case(name)
    f, MC = c["fixture"], c["cfg"]["MAX_CTX"]
    sc, pr = _last_head_scores(c)
    for tag, v in (("SCORES", sc), ("PROBS", pr)):
        m, e = sim.tile_quantize(_pad16(v, MC))
        assert (m.reshape(-1)[:MC] == f[f"{tag}_m"]).all(), tag
        assert (np.full(MC, e[0]) == f[f"{tag}_e"]).all(), tag


def _cfg1_case():
    from bfp import Dims, synth
    f = np.load(GOLDEN / "ref_layer_cfg1.npz")
    d = Dims(NL=1, MAX_CTX=16, VOCAB=256)
    fm = synth.make_model(d, seed=int(f["seed"]))
    return f, d, fm, synth.make_layer_inputs(d, 8, seed=int(f["seed"]))


def test_config1_layer_vs_reference():
    f, d, fm, xs = _cfg1_case()
    om = sim.build_model(fm)
    kv = sim.new_kv(om.dims, d.MAX_CTX)
    for p in range(8):
        out = sim.fwd_layer(sim.fp_quantize_vec(xs[p]), om.layers[0], pos=p, kv=kv, kv_pos=p,
                            dims=om.dims)
        m, e = sim.tile_quantize(out)
        assert (m.reshape(-1) == f["hout_m"][p]).all() and (e == f["hout_e"][p]).all(), p
    km, ke = sim.tile_quantize(kv["k"][:8].reshape(-1))
    assert (km.reshape(8, -1) == f["k_m"]).all() and (ke.reshape(8, -1) == f["k_e"]).all()


def test_config3_prefix_vs_reference():
    """First 12 steps (8 prompt + 4 generated) of the 30-layer decode."""
    from bfp import Dims, synth
    path = GOLDEN / "ref_decode_cfg3.npz"
    if not path.exists():
        pytest.skip("ref_decode_cfg3.npz not generated")
    f = np.load(path)
    prompt = [int(t) for t in f["prompt"]]
    d = Dims(MAX_CTX=len(prompt) + len(f["tokens"]))
    fm = synth.make_model(d, seed=int(f["seed"]))
    assert list(synth.make_prompt(d, len(prompt), seed=int(f["seed"]))) == prompt
    om = sim.build_model(fm)
    digests, cur = [], {"ms": [], "es": []}

    def on_layer(step, li, h):
        m, e = sim.tile_quantize(h)
        cur["ms"].append(m.reshape(-1))
        cur["es"].append(e)
        if li == d.NL - 1:
            import hashlib
            hh = hashlib.sha256()
            for mm, ee in zip(cur["ms"], cur["es"]):
                hh.update(mm.astype(np.int16).tobytes())
                hh.update(ee.astype(np.int8).tobytes())
            digests.append(hh.hexdigest())
            cur["ms"].clear()
            cur["es"].clear()

    toks = sim.decode(om, prompt, 4, max_ctx=d.MAX_CTX, on_layer=on_layer)
    assert list(toks[len(prompt):]) == [int(t) for t in f["tokens"][:4]]
    assert digests == [str(x) for x in f["digests"][:12]]
