"""CPU checks of the oracle's two token-loop policies (oracle/bfp_sim.py):
sim A's loop (rtl/vc707/host/gen_smollm_blockfp_full.py:432-443, with its
repeat of the last prompt token) and the FPGA driver's loop
(rtl/vc707/src/smollm/autoregress_bfp_top.sv:357-386).  The properties pin
the feed-back rule without restating it."""
import numpy as np

from oracle import bfp_sim as sim

TINY = dict(D=64, H_Q=1, H_KV=1, HD=64, FFN=128, NL=2, MAX_CTX=32, VOCAB=256)


def _model(seed):
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "tinyllm-fpga_amd"))
    from bfp import Dims, synth
    d = Dims(**TINY)
    return d, sim.build_model(synth.make_model(d, seed=seed))


def test_rtl_loop_is_teacher_forcing_on_its_own_predictions():
    """Step s >= n_prompt feeds prediction s-1: re-running with the chain as
    a longer prompt and no generation reproduces every prediction."""
    d, om = _model(3)
    prompt = [5, 17, 42]
    preds = sim.decode_rtl_loop(om, prompt, 6)
    assert len(preds) == len(prompt) + 6
    forced = prompt + preds[len(prompt) - 1:-1]
    assert sim.decode_rtl_loop(om, forced, 0) == preds


def test_rtl_loop_and_sim_loop_agree_until_the_prompt_ends():
    """Both loops see the same inputs for steps < n_prompt, so the first
    head result of sim A (step n_prompt - 1) is the RTL prediction there;
    sim A then repeats the last prompt token, the RTL feeds its prediction."""
    d, om = _model(4)
    prompt = [9, 3, 77, 1]
    heads = {}
    sim.decode(om, prompt, 3, on_step=lambda s, tid, nid: heads.__setitem__(s, (tid, nid)))
    preds = sim.decode_rtl_loop(om, prompt, 3)
    n = len(prompt)
    assert heads[n - 1][1] == preds[n - 1]
    assert heads[n][0] == prompt[-1]          # sim A's quirk: the last prompt token again


def test_rtl_loop_single_token_prompt():
    d, om = _model(5)
    preds = sim.decode_rtl_loop(om, [7], 4)
    assert len(preds) == 5
    assert sim.decode_rtl_loop(om, [7] + preds[:-1], 0) == preds
