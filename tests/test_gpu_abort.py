"""GPU: the give-up path of the decode's bounded waits.

The persistent batch-1 decode, the batched decode's joined launches and the
pipelined batched step hand data between workgroups through tagged words,
and every wait for them is bounded: one that gives up raises the decode's abort word, every other wait
then gives up too, all waves run to the end of their kernel, and the host
reports BFP_EIO.  BFP_DECODE_ABORT_TEST raises the abort word from the host
before the first launch, so each wait that does not find its words at once
gives up through its own loop.  The decode must fail with BFP_EIO, return
(no hang: the kernels finished), and the next decode on the same context
must give the oracle's tokens again (the word is cleared per decode)."""
import numpy as np
import pytest

from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

EIO = -5


def _setup(cfg, seed, max_batch):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=seed)
    gm = BfpModel(d, max_batch=max_batch)
    gm.load_fp32(fm)
    return d, sim.build_model(fm), gm


def _abort_then_recover(gm, om, prompts, n_gen, want_path, want_form, **kw):
    from bfp._lib import BfpError
    before, _ = gm.decode(prompts, n_gen, **kw)
    assert gm.decode_path() == want_path and gm.decode_form() == want_form
    print(f"[abort] {want_form}: decode with the abort word raised", flush=True)
    with pytest.raises(BfpError) as ei:
        gm.decode(prompts, n_gen, abort_test=True, **kw)
    assert ei.value.code == EIO, str(ei.value)
    assert "gave up" in str(ei.value) or "timed out" in str(ei.value), str(ei.value)
    print(f"[abort] {want_form}: decode after the abort", flush=True)
    after, _ = gm.decode(prompts, n_gen, **kw)
    assert gm.decode_path() == want_path and gm.decode_form() == want_form
    assert (after == before).all()
    want = sim.decode(om, prompts[0], n_gen)[len(prompts[0]):]
    assert list(after[0]) == list(want)


def test_persistent_decode_abort(gpu):
    """Batch 1 on the persistent kernel (two layers, D = 128)."""
    cfg = dict(D=128, H_Q=2, H_KV=1, HD=64, FFN=256, NL=2, MAX_CTX=32, VOCAB=512)
    d, om, gm = _setup(cfg, seed=31, max_batch=1)
    from bfp import synth
    prompt = synth.make_prompt(d, 6, seed=31)[None, :]
    _abort_then_recover(gm, om, prompt, 12, "persist", "persist")
    gm.close()


def test_batched_decode_abort(gpu):
    """24 sequences on the matrix-core path with both joined launch forms
    (Q|K|V with attention, the RMSNorms inside the O and D launches)."""
    cfg = dict(D=256, H_Q=4, H_KV=2, HD=64, FFN=512, NL=2, MAX_CTX=24, VOCAB=512)
    d, om, gm = _setup(cfg, seed=32, max_batch=24)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 6, seed=400 + b) for b in range(24)])
    _abort_then_recover(gm, om, prompts, 8, "graph", "mx+qkv_attn+attn_group+norm_fused", pipe=False)
    gm.close()


def test_pipelined_step_abort(gpu):
    """24 sequences (a group of 16 and one of 8) on the pipelined one-launch
    step: its flag waits give up, every workgroup finishes its jobs."""
    cfg = dict(D=256, H_Q=4, H_KV=2, HD=64, FFN=512, NL=2, MAX_CTX=24, VOCAB=512)
    d, om, gm = _setup(cfg, seed=34, max_batch=24)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 6, seed=450 + b) for b in range(24)])
    _abort_then_recover(gm, om, prompts, 8, "graph", "pipe", pipe=True)
    gm.close()
