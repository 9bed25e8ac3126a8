"""GPU against vectors written by the reference's own code (no oracle in the
loop): the single-layer baker's stage dumps with its preloaded KV cache,
BASELINE config 1 (reference fwd_layer, 8 positions) and BASELINE config 3
(30 layers, 8-token prompt, 64 greedy tokens: token ids and a digest of every
layer's output at every step)."""
import hashlib

import numpy as np
import pytest

from refcases import GOLDEN, baker_case

pytestmark = pytest.mark.gpu

STAGES = ["N1", "Q", "K", "V", "ATTN", "O", "H1", "N2", "G", "U", "MLP", "D", "HOUT"]


@pytest.mark.parametrize("name", ["small", "full"])
def test_baker_stages_on_gpu(gpu, name):
    import bfp.api as api
    from bfp import Dims
    from bfp.model import BfpModel
    c = baker_case(name)
    cfg, f = c["cfg"], c["fixture"]
    print(f"[gpu-ref] baker {name} {cfg}", flush=True)
    d = Dims(D=cfg["D"], H_Q=cfg["H_Q"], H_KV=cfg["H_KV"], HD=cfg["HD"], FFN=cfg["FFN"], NL=1,
             MAX_CTX=cfg["MAX_CTX"], VOCAB=256)
    gm = BfpModel(d)
    for n, W in c["W"].items():                 # float64 weights quantised on the device
        m, e = api.quantize_W(W)
        gm.load_tensor(n, 0, m=m, e=e)
    for n in ("g1", "g2"):
        m, e = api.tile_quantize(c[n])
        gm.load_tensor(n, 0, m=m, e=e)
    MC = cfg["MAX_CTX"]
    kq = [api.tile_quantize(c["kv"]["k"][t].reshape(-1)) for t in range(MC)]
    vq = [api.tile_quantize(c["kv"]["v"][t].reshape(-1)) for t in range(MC)]
    gm.kv_io(0, 0, 0, MC, k=(np.stack([q[0].reshape(-1) for q in kq]), np.stack([q[1] for q in kq])),
             v=(np.stack([q[0].reshape(-1) for q in vq]), np.stack([q[1] for q in vq])))
    hm, he = f["HIN_m"], f["HIN_e"]
    out_m, out_e, st = gm.layer_step_bfp(0, cfg["POS"], hm[None, :], he[None, :], dump=True)
    for tag in STAGES:
        key = tag if tag != "HOUT" else "HOUT"
        gm_, ge_ = st[tag]
        assert (ge_[0] == f[f"{key}_e"]).all(), f"stage {tag} exponents"
        assert (gm_[0] == f[f"{key}_m"]).all(), f"stage {tag} mantissas"
    assert (out_m[0] == f["HOUT_m"]).all() and (out_e[0] == f["HOUT_e"]).all()
    gm.close()


def test_config1_on_gpu(gpu):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    import bfp.api as api
    f = np.load(GOLDEN / "ref_layer_cfg1.npz")
    d = Dims(NL=1, MAX_CTX=16, VOCAB=256)
    fm = synth.make_model(d, seed=int(f["seed"]))
    xs = synth.make_layer_inputs(d, 8, seed=int(f["seed"]))
    gm = BfpModel(d)
    gm.load_fp32(fm)
    for p in range(8):
        m, e = api.tile_quantize(xs[p])
        om_, oe_, _ = gm.layer_step_bfp(0, p, m.reshape(1, -1), e.reshape(1, -1))
        cm, ce = api.tile_quantize(api.tile_decode(om_[0], oe_[0]))    # canonical form
        assert (cm.reshape(-1) == f["hout_m"][p]).all() and (ce == f["hout_e"][p]).all(), p
    # the cache holds the raw tiles of k and v; the reference's values
    # re-quantised (tile_quantize) are the canonical form of those tiles
    from oracle import bfp_sim as sim
    (km, ke), (vm, ve) = gm.kv_io(0, 0, 0, 8)
    for (m, e), tag in (((km, ke), "k"), ((vm, ve), "v")):
        cm, ce = sim.tile_quantize(sim.tile_decode(m.reshape(-1, 16), e.reshape(-1)))
        assert (cm.reshape(8, -1) == f[f"{tag}_m"]).all() and (ce.reshape(8, -1) == f[f"{tag}_e"]).all()
    gm.close()


def test_config3_decode_on_gpu(gpu):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    path = GOLDEN / "ref_decode_cfg3.npz"
    f = np.load(path)
    prompt = f["prompt"]
    n_gen = len(f["tokens"])
    d = Dims(MAX_CTX=len(prompt) + n_gen)
    print("[gpu-ref] config 3: building the 30-layer model", flush=True)
    fm = synth.make_model(d, seed=int(f["seed"]))
    gm = BfpModel(d)
    gm.load_fp32(fm)
    print("[gpu-ref] config 3: decoding", flush=True)
    toks, (hm, he) = gm.decode(prompt[None, :], n_gen, hist=True)
    assert gm.decode_path() == "persist"
    for s in range(len(prompt) + n_gen):
        h = hashlib.sha256()
        for li in range(d.NL):
            h.update(hm[0, s, li].tobytes())
            h.update(he[0, s, li].tobytes())
        assert h.hexdigest() == str(f["digests"][s]), f"step {s}: layer outputs differ"
        assert (hm[0, s, d.NL - 1] == f["last_m"][s]).all()
    assert list(toks[0]) == [int(t) for t in f["tokens"]]
    gm.close()


def _digests(hm, he, b, steps, nl):
    out = []
    for s in range(steps):
        h = hashlib.sha256()
        for li in range(nl):
            h.update(hm[b, s, li].tobytes())
            h.update(he[b, s, li].tobytes())
        out.append(h.digest())
    return out


@pytest.mark.parametrize("path_env", ["persist", "graph"])
def test_config4_decode_on_gpu(gpu, path_env, monkeypatch):
    """BASELINE config 4 on the 30-layer model: 48-token prompt decoded
    through position 2047 (the long-context attention form, 9 heads over 3
    KV groups, up to 2048 positions), every step's 30 layer outputs (as a
    digest) and every token against the reference's own run -- on the
    persistent kernel (the default) and on the per-stage graph."""
    from bfp import Dims, synth
    from bfp.model import BfpModel
    path = GOLDEN / "ref_decode_cfg4.npz"
    if not path.exists():
        pytest.skip("ref_decode_cfg4.npz not generated")
    if path_env == "graph":
        monkeypatch.setenv("BFP_PERSIST", "0")
    f = np.load(path)
    prompt = f["prompt"]
    n_gen = len(f["tokens"])
    steps = len(prompt) + n_gen
    d = Dims(MAX_CTX=steps)
    print(f"[gpu-ref] config 4 ({path_env}): building the 30-layer model", flush=True)
    gm = BfpModel(d)
    gm.load_fp32(synth.make_model(d, seed=int(f["seed"])))
    print("[gpu-ref] config 4: decoding 2048 steps", flush=True)
    toks, (hm, he) = gm.decode(prompt[None, :], n_gen, hist=True)
    assert gm.decode_path() == ("persist" if path_env == "persist" else "graph")
    gm.close()
    got = _digests(hm, he, 0, steps, d.NL)
    bad = [s for s in range(steps) if got[s] != f["digests"][s].tobytes()]
    assert not bad, f"layer outputs differ from the reference at steps {bad[:8]} ({len(bad)} steps)"
    for k, s in enumerate(f["last_steps"]):
        assert (hm[0, s, d.NL - 1] == f["last_m"][k]).all() and (he[0, s, d.NL - 1] == f["last_e"][k]).all()
    assert list(toks[0]) == [int(t) for t in f["tokens"]]


@pytest.mark.parametrize("pipe", [False, True], ids=["launches", "pipelined"])
def test_config5_decode_on_gpu(gpu, pipe):
    """the 64 sequences decoded together -- on the
    per-stage matrix-core launches and on the pipelined one-launch step --
    every sequence's per-step layer-output digests and its 128 tokens
    against the reference's own single-sequence runs."""
    from bfp import Dims, synth
    from bfp.model import BfpModel
    path = GOLDEN / "ref_decode_cfg5.npz"
    if not path.exists():
        pytest.skip("ref_decode_cfg5.npz not generated")
    f = np.load(path)
    prompts = f["prompts"]
    B, n_prompt = prompts.shape
    n_gen = f["tokens"].shape[1]
    steps = n_prompt + n_gen
    d = Dims(MAX_CTX=steps)
    print("[gpu-ref] config 5: building the 30-layer model", flush=True)
    gm = BfpModel(d, max_batch=B)
    gm.load_fp32(synth.make_model(d, seed=int(f["seed"])))
    print(f"[gpu-ref] config 5: decoding {B} sequences x {steps} steps", flush=True)
    toks, (hm, he) = gm.decode(prompts, n_gen, hist=True, pipe=pipe)
    assert gm.decode_form() == ("pipe" if pipe else "mx+qkv_attn+attn_group+norm_fused")
    gm.close()
    for b in range(B):
        got = _digests(hm, he, b, steps, d.NL)
        bad = [s for s in range(steps) if got[s] != f["digests"][b, s].tobytes()]
        assert not bad, f"sequence {b}: layer outputs differ at steps {bad[:8]}"
    assert (toks == f["tokens"]).all()
