"""Golden vectors written by the REFERENCE's own simulator code.

Run in a container where /root/reference exists (it does not exist on the
GPU box); the outputs are committed next to this script:

  ref_stages_<cfg>.npz   the single-layer baker
                         rtl/vc707/host/gen_smollm_blockfp_bfp.py run as a
                         subprocess (its own np.random.seed(SEED) inputs, all
                         13 stage dumps + QPRE/KPRE + HIN/HOUT hex files, and
                         the last head's scores and softmax probabilities,
                         tile-quantised over 16 slots, that it writes for
                         MAX_CTX <= 16, gen_smollm_blockfp_bfp.py:362-372)
  ref_layer_cfg1.npz     BASELINE config 1: the reference's fwd_layer
                         (gen_smollm_blockfp_full.py:261-293) on this build's
                         seeded SmolLM2-shaped layer, positions 0..7
  ref_decode_cfg3.npz    BASELINE config 3: 30 layers, 8-token prompt, 64 new
                         tokens, driven by the reference's fwd_layer with the
                         token loop and head of gen_smollm_blockfp_full.py
                         :432-443; tokens + a digest of every layer output at
                         every step + the last layer's output per step
  ref_decode_cfg4.npz    BASELINE config 4: the same loop with a 48-token
                         prompt decoded through position 2047 (MAX_CTX 2048,
                         2000 new tokens); tokens + a raw SHA-256 digest of
                         all 30 layer outputs per step + the last layer's
                         output every 64 steps + the head's top-2 gaps
  ref_decode_cfg5.npz    BASELINE config 5: the 64 prompts of the batched
                         config (8 tokens each, 128 new), every sequence run
                         through the same loop (the reference decodes one
                         sequence at a time); tokens + per-step digests +
                         top-2 gaps for every sequence

The reference module reads its dimensions from environment variables at
import and creates its OUT directory; both are pointed at a temp dir here.
Usage:  python tests/golden/gen_ref_vectors.py [stages|cfg1|cfg3|cfg4|cfg5|all]
(cfg4 takes about half an hour on one core; cfg5 runs its 64 sequences in
parallel worker processes, GEN_WORKERS of them, default 6.)
"""
from __future__ import annotations

import hashlib
import importlib.util
import os
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "tinyllm-fpga_amd"))
HOST = Path("/root/reference/rtl/vc707/host")

BAKER_CFGS = {
    # the baker's defaults (vc707/Makefile's small self-test)
    "small": dict(D=64, H_Q=1, H_KV=1, HD=64, FFN=128, MAX_CTX=4, POS=3, KV_POS=3, SEED=0),
    # SmolLM2-135M shapes
    "full": dict(D=576, H_Q=9, H_KV=3, HD=64, FFN=1536, MAX_CTX=8, POS=5, KV_POS=5, SEED=0),
}
STAGE_TAGS = ["N1", "Q", "K", "V", "ATTN", "O", "H1", "N2", "G", "U", "MLP", "D", "QPRE", "KPRE",
              "HIN", "HOUT", "SCORES", "PROBS"]


def read_hex(path: Path, bits: int) -> np.ndarray:
    a = np.array([int(x, 16) for x in path.read_text().split()], dtype=np.int64)
    a = np.where(a >= 1 << (bits - 1), a - (1 << bits), a)
    return a.astype(np.int16 if bits == 16 else np.int8)


def gen_stages():
    for name, cfg in BAKER_CFGS.items():
        with tempfile.TemporaryDirectory() as td:
            env = dict(os.environ, OUT=td, PREFIX="lbfp_", **{k: str(v) for k, v in cfg.items()})
            subprocess.run([sys.executable, str(HOST / "gen_smollm_blockfp_bfp.py")], env=env,
                           check=True, cwd=td, capture_output=True)
            out = {k: np.array(v) for k, v in cfg.items()}
            for tag in STAGE_TAGS:
                pre = "STAGE_" if tag not in ("HIN", "HOUT") else ""
                out[f"{tag}_m"] = read_hex(Path(td) / f"lbfp_{pre}{tag}_m.hex", 16)
                out[f"{tag}_e"] = read_hex(Path(td) / f"lbfp_{pre}{tag}_e.hex", 8)
        np.savez_compressed(HERE / f"ref_stages_{name}.npz", **out)
        print("wrote", f"ref_stages_{name}.npz")


def load_reference(dims, tmp):
    """Import gen_smollm_blockfp_full.py with the given dims (module globals
    come from env vars)."""
    env = {"D": dims.D, "H_Q": dims.H_Q, "H_KV": dims.H_KV, "HD": dims.HD, "FFN": dims.FFN,
           "NL": dims.NL, "MAX_CTX": dims.MAX_CTX, "OUT": tmp}
    for k, v in env.items():
        os.environ[k] = str(v)
    spec = importlib.util.spec_from_file_location(f"ref_full_{dims.D}_{dims.NL}",
                                                  HOST / "gen_smollm_blockfp_full.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def ref_layers(ref, fm):
    layers = []
    for lw in fm.layers:
        q = {n: ref.quantize_W(np.asarray(lw[n]).astype(np.float64))
             for n in ("Wq", "Wk", "Wv", "Wo", "Wg", "Wu", "Wd")}
        q["g1"] = ref.fp_quantize_vec(np.asarray(lw["g1"]).astype(np.float64))
        q["g2"] = ref.fp_quantize_vec(np.asarray(lw["g2"]).astype(np.float64))
        layers.append(q)
    return layers


def gen_cfg1(seed=1):
    from bfp import Dims, synth
    d = Dims(NL=1, MAX_CTX=16, VOCAB=256)
    fm = synth.make_model(d, seed=seed)
    xs = synth.make_layer_inputs(d, 8, seed=seed)
    with tempfile.TemporaryDirectory() as td:
        ref = load_reference(d, td)
        lw = ref_layers(ref, fm)[0]
        kv = {"k": np.zeros((d.MAX_CTX, d.H_KV, d.HD)), "v": np.zeros((d.MAX_CTX, d.H_KV, d.HD))}
        hm, he = [], []
        for p in range(8):
            h = ref.fp_quantize_vec(xs[p])
            out = ref.fwd_layer(h, lw, pos=p, kv=kv, kv_pos=p)
            m, e = ref.tile_quantize(out)
            hm.append(m.reshape(-1))
            he.append(e)
        km, ke = ref.tile_quantize(kv["k"][:8].reshape(-1))
        vm, ve = ref.tile_quantize(kv["v"][:8].reshape(-1))
    np.savez_compressed(HERE / "ref_layer_cfg1.npz", seed=seed, hout_m=np.stack(hm),
                        hout_e=np.stack(he), k_m=km.reshape(8, -1), k_e=ke.reshape(8, -1),
                        v_m=vm.reshape(8, -1), v_e=ve.reshape(8, -1))
    print("wrote ref_layer_cfg1.npz")


def step_digest(ms, es):
    h = hashlib.sha256()
    for m, e in zip(ms, es):
        h.update(np.ascontiguousarray(m, dtype=np.int16).tobytes())
        h.update(np.ascontiguousarray(e, dtype=np.int8).tobytes())
    return h.hexdigest()


def gen_cfg3(seed=0, n_prompt=8, n_gen=64):
    from bfp import Dims, synth
    d = Dims(MAX_CTX=n_prompt + n_gen)
    fm = synth.make_model(d, seed=seed)
    ids = [int(t) for t in synth.make_prompt(d, n_prompt, seed=seed)]
    with tempfile.TemporaryDirectory() as td:
        ref = load_reference(d, td)
        layers = ref_layers(ref, fm)
        embed = fm.embed.astype(np.float64)
        norm_w_q = ref.fp_quantize_vec(fm.norm_w.astype(np.float64))
        kv = [{"k": np.zeros((d.MAX_CTX, d.H_KV, d.HD)), "v": np.zeros((d.MAX_CTX, d.H_KV, d.HD))}
              for _ in range(d.NL)]
        generated = list(ids)
        digests, last_m, last_e, heads = [], [], [], []
        for step in range(len(ids) + n_gen):
            tid = ids[step] if step < len(ids) else generated[-1]
            h = ref.fp_quantize_vec(embed[tid])           # embed_q[tid]
            ms, es = [], []
            for li in range(d.NL):
                h = ref.fwd_layer(h, layers[li], pos=step, kv=kv[li], kv_pos=step)
                m, e = ref.tile_quantize(h)
                ms.append(m.reshape(-1))
                es.append(e)
            digests.append(step_digest(ms, es))
            last_m.append(ms[-1])
            last_e.append(es[-1])
            if step >= len(ids) - 1:
                h_normed = (h / np.sqrt(np.mean(h * h) + 1e-5)) * norm_w_q
                logits = h_normed @ embed.T
                nid = int(np.argmax(logits))
                top2 = np.sort(logits)[-2:]
                heads.append((step, nid, float(top2[1] - top2[0])))
                if step >= len(ids):
                    generated.append(nid)
            print(f"  step {step} done", flush=True)
    np.savez_compressed(HERE / "ref_decode_cfg3.npz", seed=seed, prompt=np.array(ids, np.int32),
                        tokens=np.array(generated[len(ids):], np.int32),
                        digests=np.array(digests), last_m=np.stack(last_m),
                        last_e=np.stack(last_e), head_steps=np.array([h[0] for h in heads]),
                        head_ids=np.array([h[1] for h in heads]),
                        top2_gap=np.array([h[2] for h in heads]))
    print("wrote ref_decode_cfg3.npz; tokens", generated[len(ids):])


def _ref_decode(ref, layers, embed, norm_w_q, d, ids, n_gen, max_ctx, keep_last=None,
                log=None):
    """The golden-token loop of gen_smollm_blockfp_full.py:426-443 on the
    reference's own fwd_layer; returns (generated tokens, raw per-step
    digests (steps, 32) uint8, top-2 logit gaps per head step, last-layer
    outputs at the steps in keep_last)."""
    kv = [{"k": np.zeros((max_ctx, d.H_KV, d.HD)), "v": np.zeros((max_ctx, d.H_KV, d.HD))}
          for _ in range(d.NL)]
    generated = list(ids)
    digests, gaps, kept = [], [], {}
    for step in range(len(ids) + n_gen):
        tid = ids[step] if step < len(ids) else generated[-1]
        h = ref.fp_quantize_vec(embed[tid])           # embed_q[tid]
        hs = hashlib.sha256()
        for li in range(d.NL):
            h = ref.fwd_layer(h, layers[li], pos=step, kv=kv[li], kv_pos=step)
            m, e = ref.tile_quantize(h)
            hs.update(np.ascontiguousarray(m.reshape(-1), dtype=np.int16).tobytes())
            hs.update(np.ascontiguousarray(e, dtype=np.int8).tobytes())
        digests.append(np.frombuffer(hs.digest(), np.uint8))
        if keep_last is not None and step in keep_last:
            kept[step] = (m.reshape(-1).copy(), e.copy())
        if step >= len(ids) - 1:
            h_normed = (h / np.sqrt(np.mean(h * h) + 1e-5)) * norm_w_q
            logits = h_normed @ embed.T
            nid = int(np.argmax(logits))
            top2 = np.sort(logits)[-2:]
            gaps.append(float(top2[1] - top2[0]))
            if step >= len(ids):
                generated.append(nid)
        if log is not None:
            log(step)
    return generated[len(ids):], np.stack(digests), np.array(gaps), kept


def _setup_30(max_ctx, td):
    from bfp import Dims, synth
    d = Dims(MAX_CTX=max_ctx)
    fm = synth.make_model(d, seed=0)
    ref = load_reference(d, td)
    layers = ref_layers(ref, fm)
    embed = fm.embed.astype(np.float64)
    norm_w_q = ref.fp_quantize_vec(fm.norm_w.astype(np.float64))
    return d, ref, layers, embed, norm_w_q


def gen_cfg4(n_prompt=48, n_gen=2000, prompt_seed=4):
    """Config 4 as bench.py's long-context leg runs it: model seed 0,
    prompt synth.make_prompt(48, seed=4), steps 0..2047."""
    from bfp import synth
    import time
    steps = n_prompt + n_gen
    keep = set(range(0, steps, 64)) | {steps - 1}
    with tempfile.TemporaryDirectory() as td:
        d, ref, layers, embed, norm_w_q = _setup_30(steps, td)
        ids = [int(t) for t in synth.make_prompt(d, n_prompt, seed=prompt_seed)]
        t0 = time.time()

        def log(step):
            if step % 16 == 0 or step == steps - 1:
                print(f"  cfg4 step {step} ({time.time() - t0:.0f} s)", flush=True)
        toks, dig, gaps, kept = _ref_decode(ref, layers, embed, norm_w_q, d, ids, n_gen, steps,
                                            keep_last=keep, log=log)
    ks = sorted(kept)
    np.savez_compressed(HERE / "ref_decode_cfg4.npz", seed=0, prompt_seed=prompt_seed,
                        prompt=np.array(ids, np.int32), tokens=np.array(toks, np.int32),
                        digests=dig, top2_gap=gaps, last_steps=np.array(ks, np.int32),
                        last_m=np.stack([kept[k][0] for k in ks]),
                        last_e=np.stack([kept[k][1] for k in ks]))
    print("wrote ref_decode_cfg4.npz; first tokens", toks[:16])


_CFG5 = {}


def _cfg5_worker(seqs):
    c = _CFG5
    out = []
    for b in seqs:
        toks, dig, gaps, _ = _ref_decode(c["ref"], c["layers"], c["embed"], c["norm_w_q"],
                                         c["d"], c["prompts"][b], c["n_gen"], c["max_ctx"])
        out.append((b, toks, dig, gaps))
        print(f"  cfg5 sequence {b} done", flush=True)
    return out


def cfg5_prompts(d, B=64, n_prompt=8):
    """The prompts of bench.py's batch leg: sequence 0 is config 3's prompt,
    sequence b >= 1 is synth.make_prompt(8, seed=1000 + b)."""
    from bfp import synth
    return np.stack([synth.make_prompt(d, n_prompt, seed=0)] +
                    [synth.make_prompt(d, n_prompt, seed=1000 + b) for b in range(1, B)])


def gen_cfg5(B=64, n_prompt=8, n_gen=128):
    import multiprocessing as mp
    workers = int(os.environ.get("GEN_WORKERS", "6"))
    max_ctx = n_prompt + n_gen
    with tempfile.TemporaryDirectory() as td:
        d, ref, layers, embed, norm_w_q = _setup_30(max_ctx, td)
        prompts = cfg5_prompts(d, B, n_prompt)
        _CFG5.update(ref=ref, layers=layers, embed=embed, norm_w_q=norm_w_q, d=d,
                     prompts=[[int(t) for t in p] for p in prompts], n_gen=n_gen,
                     max_ctx=max_ctx)
        parts = [list(range(w, B, workers)) for w in range(workers)]
        with mp.get_context("fork").Pool(workers) as pool:
            res = [r for part in pool.map(_cfg5_worker, parts) for r in part]
    res.sort(key=lambda r: r[0])
    np.savez_compressed(HERE / "ref_decode_cfg5.npz", seed=0, prompts=prompts.astype(np.int32),
                        tokens=np.array([r[1] for r in res], np.int32),
                        digests=np.stack([r[2] for r in res]),
                        top2_gap=np.stack([r[3] for r in res]))
    print("wrote ref_decode_cfg5.npz")


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    if what in ("stages", "all"):
        gen_stages()
    if what in ("cfg1", "all"):
        gen_cfg1()
    if what in ("cfg3", "all"):
        gen_cfg3()
    if what in ("cfg4", "all"):
        gen_cfg4()
    if what in ("cfg5", "all"):
        gen_cfg5()
