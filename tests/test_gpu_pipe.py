"""GPU: the pipelined batched decode step (csrc/bfp_pipe.hip) -- every layer
of a decode step as one launch, the sequences passing the stages in groups
of 16 -- against the per-stage launches and the oracle (full.py:261-293,
426-443): token ids and every layer's output at every step, bit for bit."""
import numpy as np
import pytest

from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

TINY = dict(D=128, H_Q=2, H_KV=1, HD=64, FFN=256, NL=2, MAX_CTX=32, VOCAB=512)
MID = dict(D=256, H_Q=4, H_KV=2, HD=64, FFN=512, NL=3, MAX_CTX=40, VOCAB=512)


def _setup(cfg, seed, max_batch):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(**cfg)
    fm = synth.make_model(d, seed=seed)
    gm = BfpModel(d, max_batch=max_batch)
    gm.load_fp32(fm)
    return d, sim.build_model(fm), gm


def _oracle(om, prompt, n_gen):
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


@pytest.mark.parametrize("cfg,batch,n_prompt,n_gen", [(TINY, 16, 5, 10), (TINY, 20, 4, 12),
                                                      (MID, 40, 6, 12)])
def test_pipe_equals_launches(gpu, cfg, batch, n_prompt, n_gen):
    """Whole groups and a partial last group: tokens and every layer's
    output at every step equal the per-stage launches', and the first and
    last sequences equal the oracle."""
    d, om, gm = _setup(cfg, seed=40 + batch, max_batch=batch)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, n_prompt, seed=700 + b) for b in range(batch)])
    print(f"[pipe] D={d.D} batch={batch}: pipelined step", flush=True)
    toks, (hm, he) = gm.decode(prompts, n_gen, hist=True, pipe=True)
    assert gm.decode_form() == "pipe"
    print(f"[pipe] D={d.D} batch={batch}: per-stage launches", flush=True)
    ref, (rhm, rhe) = gm.decode(prompts, n_gen, hist=True, pipe=False)
    assert gm.decode_form().startswith("mx")
    assert (toks == ref).all()
    bad = [b for b in range(batch) if not ((hm[b] == rhm[b]).all() and (he[b] == rhe[b]).all())]
    assert not bad, f"sequences whose layer outputs differ: {bad[:8]}"
    for b in (0, batch - 1):
        want, whm, whe = _oracle(om, prompts[b], n_gen)
        assert list(toks[b]) == list(want), b
        assert (hm[b] == whm).all() and (he[b] == whe).all(), b
    gm.close()


def test_pipe_repeated_and_smaller_batch(gpu):
    """Two decodes in a row on one context (the flags are cleared per
    decode), then a smaller batch with its own schedule."""
    d, om, gm = _setup(TINY, seed=77, max_batch=32)
    from bfp import synth
    prompts = np.stack([synth.make_prompt(d, 6, seed=900 + b) for b in range(32)])
    a, _ = gm.decode(prompts, 8, pipe=True)
    b, _ = gm.decode(prompts, 8, pipe=True)
    assert gm.decode_form() == "pipe"
    assert (a == b).all()
    c, _ = gm.decode(prompts[:17], 8, pipe=True)
    assert gm.decode_form() == "pipe"
    assert (c == a[:17]).all()
    want, _, _ = _oracle(om, prompts[16], 8)
    assert list(c[16]) == list(want)
    gm.close()
