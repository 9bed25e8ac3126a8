"""GPU parity of the FPGA decode head and token loop (bfp_rtl_head,
bfp_rtl_decode: smollm_decode_head_bfp.sv:303-430 and
autoregress_bfp_top.sv:357-386 over the composed RTL layer) against
oracle/bfp_rtl.py:rtl_head / rtl_decode, bit for bit: every logit's (m, e),
the token, every step's last-layer output and every prediction."""
import numpy as np
import pytest

from oracle import bfp_rtl as rtl
from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

TINY = dict(D=128, H_Q=2, H_KV=1, HD=64, FFN=256, NL=2, MAX_CTX=40, VOCAB=256)
WIDE = dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, NL=1, MAX_CTX=8, VOCAB=512)


def _setup(cfg, seed):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=seed)
    gm = BfpModel(d)
    gm.load_fp32(fm)
    return d, sim.build_model(fm), gm


@pytest.mark.parametrize("cfg", [TINY, WIDE], ids=["tiny", "d576"])
def test_rtl_head_matches_oracle(gpu, cfg):
    d, om, gm = _setup(cfg, seed=5)
    print(f"[rtl head] dims {cfg}", flush=True)
    rng = np.random.default_rng(5)
    emb = rtl.embed_q(om.embed)
    for trial in range(4):
        hm, he = sim.tile_quantize(rng.standard_normal(d.D) * (1 + 3 * trial))
        wm, we, wt = rtl.rtl_head(hm.reshape(-1), he, om.norm_w_q, emb)
        tok, (lm, le) = gm.rtl_head(hm, he, logits=True)
        assert (le == we).all(), f"trial {trial}: logit exponents"
        assert (lm == wm).all(), f"trial {trial}: logit mantissas"
        assert tok == wt, f"trial {trial}: token"
    gm.close()


def test_rtl_decode_matches_oracle(gpu):
    """A 3-token prompt and 20 generated tokens on a 2-layer model: the
    positions cross the 16-position window of the RTL attention."""
    d, om, gm = _setup(TINY, seed=6)
    from bfp import synth
    prompt = [int(t) for t in synth.make_prompt(d, 3, seed=6)]
    n_gen = 20
    want_h = {}
    print("[rtl decode] oracle", flush=True)
    want = rtl.rtl_decode(om, prompt, n_gen, rtl.RtlTables(), d,
                          on_step=lambda s, m, e: want_h.__setitem__(s, (m.copy(), e.copy())))
    print("[rtl decode] gpu", flush=True)
    preds, (hm, he) = gm.rtl_decode(prompt, n_gen, hist=True)
    bad = [s for s in range(len(want)) if not ((hm[s] == want_h[s][0]).all() and (he[s] == want_h[s][1]).all())]
    assert not bad, f"steps with differing last-layer outputs: {bad[:10]}"
    assert list(preds) == list(want)
    # the loop runs on the device from a fresh state each call; no history
    assert list(gm.rtl_decode(prompt, n_gen)) == list(want)
    gm.close()


def test_rtl_decode_rejects_bad_arguments(gpu):
    from bfp._lib import BfpError
    d, om, gm = _setup(TINY, seed=7)
    with pytest.raises(BfpError):
        gm.rtl_decode([1, 2], d.MAX_CTX)          # beyond the KV capacity
    with pytest.raises(BfpError):
        gm.rtl_decode([d.VOCAB], 1)               # prompt id out of range
    with pytest.raises(BfpError):
        gm.rtl_decode([], 3)                      # empty prompt
    gm.close()
