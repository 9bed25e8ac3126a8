#!/usr/bin/env python3
"""Benchmark of the BFP decode datapath on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload: the standalone BFP matvec sweep at
batch 1 -- shapes 576x576, 192x576, 1536x576, 576x1536, 49152x576, 1000
reps each.  One "step" is the whole sweep: one launch per shape computing
1000 independent y = W x, each rep reading a weight copy from a ring of
>= 4 GiB (a distinct copy per rep for the four small shapes, 74 copies of
the 49152x576 one, read in rep order), so the bytes come from HBM, not from
the 256 MiB MALL.  Weights are N(0, 0.02) float32 quantised to BFP on the device,
inputs N(0, 1) quantised to BFP; everything is resident in HBM before the
timed region.  `value` is algorithmic bytes / second over the K timed steps
(out*in*2 + out*in/16 weight bytes + x and y BFP bytes per rep).

The JSON line also carries the roofline of the dominant matvec kernel
(HIP events on the launch stream), the parity check of sampled reps
against the CPU oracle, and the CPU baseline (the oracle timed on a bounded
sample on this host).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tinyllm-fpga_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
SHAPES = [(576, 576), (192, 576), (1536, 576), (576, 1536), (49152, 576)]
RING_BYTES = 4096 << 20   # 16x the MALL: a re-read copy has long left it


def alg_bytes(n_out, n_in):
    return n_out * n_in * 2 + n_out * n_in // 16 + n_in * 2 + n_in // 16 + n_out * 2 + n_out // 16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--reps", type=int, default=1000)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-workers", type=int, default=0,
                    help="processes for the all-cores CPU baseline (0: min(cpu count, 16))")
    ap.add_argument("--cpu-worker", type=float, default=None, help=argparse.SUPPRESS)
    ap.add_argument("--no-decode", action="store_true", help="skip the config-3 decode leg")
    ap.add_argument("--decode-only", action="store_true", help="run only the config-3 decode leg")
    ap.add_argument("--decode-reps", type=int, default=3)
    ap.add_argument("--long", dest="long", action="store_true", default=True,
                    help="run config 4 (long context; on by default)")
    ap.add_argument("--no-long", dest="long", action="store_false", help="skip config 4")
    ap.add_argument("--batch64", dest="batch64", action="store_true", default=True,
                    help="run config 5 (batch 64; on by default)")
    ap.add_argument("--no-batch64", dest="batch64", action="store_false", help="skip config 5")
    ap.add_argument("--no-layer", action="store_true", help="skip the config-1 layer-step leg")
    ap.add_argument("--no-config3", action="store_true",
                    help="with --decode-only: skip the config-3 decode (e.g. to profile config 5 alone)")
    ap.add_argument("--batch64-tokens", type=int, default=128,
                    help="tokens generated per sequence in the config-5 leg (128 = the config)")
    ap.add_argument("--probe", dest="probe", action="store_true", default=True,
                    help="time a 1 GiB device copy and a 2 GiB streaming read (practical HBM "
                         "ceiling; the copy calibrates rocprof counters; on by default)")
    ap.add_argument("--no-probe", dest="probe", action="store_false")
    return ap.parse_args()


class ShapeCase:
    """Device-resident ring of BFP weight copies + inputs for one shape."""

    def __init__(self, n_out, n_in, reps, seed):
        import torch
        from bfp import _dev
        from bfp._lib import call
        self.n_out, self.n_in, self.reps = n_out, n_in, reps
        self.bm = n_out * n_in * 2
        self.be = n_out * n_in // 16
        self.ring = min(reps, max(2, -(-RING_BYTES // (self.bm + self.be))))
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.Pm = torch.empty(self.ring * self.bm, dtype=torch.uint8, device="cuda")
        self.Pe = torch.empty(self.ring * self.be, dtype=torch.uint8, device="cuda")
        # generate and pack in slabs to bound the fp32 staging memory
        per = max(1, (256 << 20) // (n_out * n_in * 4))
        self.W0 = None
        for r0 in range(0, self.ring, per):
            k = min(per, self.ring - r0)
            W = torch.randn((k * n_out, n_in), generator=g, device="cuda", dtype=torch.float32)
            W.mul_(0.02)
            if r0 == 0:
                self.W0 = W[:n_out].cpu().numpy()
            call("bfp_quantize_pack_f32_d", W.data_ptr(), k * n_out, n_in,
                 self.Pm.data_ptr() + r0 * self.bm, self.Pe.data_ptr() + r0 * self.be,
                 _dev.stream())
            del W
        X = torch.randn((reps, n_in), generator=g, device="cuda", dtype=torch.float32)
        self.X_last = X[reps - 1].cpu().numpy()
        self.X0 = X[0].cpu().numpy()
        self.xm = torch.empty(reps * n_in, dtype=torch.int16, device="cuda")
        self.xe = torch.empty(reps * n_in // 16, dtype=torch.int8, device="cuda")
        call("bfp_tile_quantize_f32_d", X.data_ptr(), reps * n_in, self.xm.data_ptr(),
             self.xe.data_ptr(), _dev.stream())
        del X
        self.ym = torch.empty(reps * n_out, dtype=torch.int16, device="cuda")
        self.ye = torch.empty(reps * n_out // 16, dtype=torch.int8, device="cuda")
        self.waves = 0
        torch.cuda.synchronize()

    def launch(self):
        from bfp import _dev
        from bfp._lib import call
        call("bfp_matvec_ring_d", self.Pm.data_ptr(), self.Pe.data_ptr(), self.n_out, self.n_in,
             self.reps, self.ring, self.bm, self.be, self.xm.data_ptr(), self.xe.data_ptr(),
             self.n_in, self.ym.data_ptr(), self.ye.data_ptr(), self.n_out, self.waves,
             _dev.stream())

    def bytes_per_launch(self):
        return alg_bytes(self.n_out, self.n_in) * self.reps

    def check(self):
        """Reps 0 and reps-1 against the CPU oracle, bit for bit."""
        import numpy as np
        from oracle import bfp_sim as sim
        ym = self.ym.cpu().numpy().reshape(self.reps, -1)
        ye = self.ye.cpu().numpy().reshape(self.reps, -1)
        Wm, We = sim.tile_quantize(self.W0.astype(np.float64))
        nt = self.n_in // 16
        Wm, We = Wm.reshape(self.n_out, nt, 16), We.reshape(self.n_out, nt)
        ok = True
        for r, x in ((0, self.X0), (self.reps - 1, self.X_last)):
            if r % self.ring != 0:
                continue                      # only ring slot 0 is mirrored on the host
            xm, xe = sim.tile_quantize(x.astype(np.float64))
            wm, we = sim.tile_quantize(sim.matvec_hw_golden(xm, xe, Wm, We))
            ok &= bool((ym[r] == wm.reshape(-1)).all() and (ye[r] == we).all())
        return ok


def profiled_traffic(kernel, shape):
    """HBM bytes per launch of `kernel` on `shape` from the committed
    rocprofv3 counter summary (FETCH_SIZE x calibration + WRITE_SIZE), or
    None."""
    path = ROOT / "profiles" / "bfp_matvec_sweep.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if (len(parts) == 4 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel
                and parts[2] == shape):
            return int(parts[3])
    return None


def kernel_config(n_in):
    """(waves, tiles per lane) the library picks for this input width."""
    nT = n_in // 16
    nw = next(a for a in (1, 2, 3, 4, 6, 8, 9) if a >= (nT + 11) // 12) if nT <= 108 else 9
    tpt = -(-nT // (4 * nw))
    return nw, tpt


def kernel_name(n_out, n_in, reps):
    """The matvec kernel the library launches (one 16-row chunk of one
    problem per workgroup, csrc/bfp_core.hip:launch_matvec)."""
    nw, tpt = kernel_config(n_in)
    return "matvec_kernel<%d,%d>" % (nw, tpt)


def _cpu_matvec_sample(seconds):
    """The oracle's numpy matvec_hw_golden (restating full.py:217-233) on a
    bounded sample of the sweep: up to 1000 reps per shape, about
    seconds/5 per shape.  Returns (algorithmic bytes, seconds, reps)."""
    import numpy as np
    from oracle import bfp_sim as sim
    from bfp import synth
    total_b, total_t, done = 0, 0.0, []
    per_shape = seconds / len(SHAPES)
    for n_out, n_in in SHAPES:
        W, x = synth.make_matvec_case(n_out, n_in, seed=5)
        Wm, We = sim.tile_quantize(W[0].astype(np.float64))
        nt = n_in // 16
        Wm, We = Wm.reshape(n_out, nt, 16), We.reshape(n_out, nt)
        xm, xe = sim.tile_quantize(x[0])
        n, t0 = 0, time.perf_counter()
        while True:
            sim.matvec_hw_golden(xm, xe, Wm, We)
            n += 1
            dt = time.perf_counter() - t0
            if dt >= per_shape or n >= 1000:
                break
        total_b += alg_bytes(n_out, n_in) * n
        total_t += dt
        done.append(f"{n_out}x{n_in}:{n}")
    return total_b, total_t, done


def cpu_baseline(seconds):
    """The oracle's numpy matvec, single-threaded, on a bounded sample of
    the same sweep."""
    os.environ.setdefault("OPENBLAS_NUM_THREADS", "1")
    total_b, total_t, done = _cpu_matvec_sample(seconds)
    return {"value": round(total_b / total_t / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": "oracle/bfp_sim.matvec_hw_golden (numpy, 1 thread), reps per shape "
                      + ", ".join(done) + f" in {total_t:.1f} s"}


def cpu_baseline_all_cores(seconds, workers):
    """The same sample run concurrently by `workers` single-threaded child
    processes (this script with --cpu-worker; they import numpy and the
    oracle only, never the GPU runtime); aggregate bytes over the slowest
    worker's time."""
    import subprocess
    env = dict(os.environ, OPENBLAS_NUM_THREADS="1", OMP_NUM_THREADS="1")
    procs = [subprocess.Popen([sys.executable, str(Path(__file__).resolve()), "--cpu-worker",
                               str(seconds)], stdout=subprocess.PIPE, env=env, text=True)
             for _ in range(workers)]
    res = []
    for p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            raise RuntimeError(f"cpu worker exited with {p.returncode}")
        res.append(json.loads(out.strip().splitlines()[-1]))
    total_b = sum(r["bytes"] for r in res)
    t = max(r["seconds"] for r in res)
    return {"value": round(total_b / t / 1e9, 4), "unit": "GB/s", "cores": workers, "kind": "port",
            "sample": f"{workers} concurrent single-threaded processes, each the 1-thread sample "
                      f"({seconds:.0f} s budget), slowest {t:.1f} s"}


def decode_leg(reps):
    """30-layer SmolLM2-135M-shaped random-init model,
    8-token prompt, 64 greedy tokens.  Timed with HIP events inside
    bfp_decode (device time of the steps that emit the 64 tokens, and of all
    72 steps); tokens checked against the reference's own run
    (tests/golden/ref_decode_cfg3.npz)."""
    import numpy as np
    from bfp import Dims, synth
    from bfp.model import BfpModel
    n_prompt, n_gen = 8, 64
    d = Dims(MAX_CTX=n_prompt + n_gen)
    fm = synth.make_model(d, seed=0)
    prompt = synth.make_prompt(d, n_prompt, seed=0)
    gm = BfpModel(d)
    gm.load_fp32(fm)
    toks, _ = gm.decode(prompt[None, :], n_gen)          # warm-up + graph build
    gen_ms, tot_ms, walls = [], [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        toks, _ = gm.decode(prompt[None, :], n_gen)
        walls.append(time.perf_counter() - t0)
        t, g = gm.decode_time_ms()
        tot_ms.append(t)
        gen_ms.append(g)
    gm.close()
    ref = ROOT / "tests" / "golden" / "ref_decode_cfg3.npz"
    exact = None
    if ref.exists():
        f = np.load(ref)
        exact = bool(list(toks[0]) == [int(t) for t in f["tokens"]]
                     and list(prompt) == [int(t) for t in f["prompt"]])
    g = min(gen_ms)
    return {"workload": "config 3: 30 layers, prompt 8, 64 greedy tokens, batch 1",
            "tokens_per_s": round(n_gen / (g * 1e-3), 1),
            "ms_per_token": round(g / n_gen, 4),
            "steps_per_s_all": round((n_prompt + n_gen) / (min(tot_ms) * 1e-3), 1),
            "wall_s_per_decode": round(min(walls), 4),
            "tokens_match_reference": exact}


def long_context_leg():
    """30 layers, 48-token prompt, greedy decode through
    position 2047 (2000 new tokens); tokens/s overall and per position
    window from per-step HIP events."""
    import numpy as np
    from bfp import Dims, synth
    from bfp.model import BfpModel
    n_prompt, n_gen = 48, 2000
    d = Dims(MAX_CTX=2048)
    gm = BfpModel(d)
    gm.load_fp32(synth.make_model(d, seed=0))
    prompt = synth.make_prompt(d, n_prompt, seed=4)
    gm.decode(prompt[None, :], 16)                       # warm-up
    gm.decode(prompt[None, :], n_gen, step_times=True)
    st = gm.step_times_ms()
    t, g = gm.decode_time_ms()
    gm.close()
    win = {}
    for lo, hi in ((48, 112), (496, 560), (1008, 1072), (1984, 2048)):
        win[f"pos_{lo}_{hi - 1}"] = round((hi - lo) / (float(st[lo:hi].sum()) * 1e-3), 1)
    return {"workload": "config 4: 30 layers, prompt 48, decode to position 2047 (2000 tokens)",
            "tokens_per_s": round(n_gen / (g * 1e-3), 1), "ms_per_token_mean": round(g / n_gen, 4),
            "tokens_per_s_by_position": win}


def batch_leg(n_gen=128):
    """64 independent sequences, 8-token prompts, 128
    greedy tokens each; aggregate tokens/s.  Sequence 0 uses config 3's
    prompt: its first 64 tokens must equal the reference's config-3 tokens."""
    import numpy as np
    from bfp import Dims, synth
    from bfp.model import BfpModel
    B, n_prompt = 64, 8
    d = Dims(MAX_CTX=n_prompt + 128)
    gm = BfpModel(d, max_batch=B)
    gm.load_fp32(synth.make_model(d, seed=0))
    prompts = np.stack([synth.make_prompt(d, n_prompt, seed=0)] +
                       [synth.make_prompt(d, n_prompt, seed=1000 + b) for b in range(1, B)])
    gm.decode(prompts, 4)                                # warm-up
    toks, _ = gm.decode(prompts, n_gen)
    t, g = gm.decode_time_ms()
    gm.close()
    ref = ROOT / "tests" / "golden" / "ref_decode_cfg3.npz"
    exact = None
    if ref.exists():
        want = [int(x) for x in np.load(ref)["tokens"]][:n_gen]
        exact = bool(list(toks[0][:len(want)]) == want)
    return {"workload": f"config 5: 64 sequences, prompt 8, {n_gen} greedy tokens each",
            "tokens_per_s": round(B * n_gen / (g * 1e-3), 1),
            "ms_per_step": round(g / n_gen, 4), "seq0_matches_reference": exact}


def layer_leg():
    """the cost of one SmolLM2-135M-shaped decoder layer
    step at batch 1 inside the graph-replayed decode (positions 0..6 of an
    8-token prompt), as the marginal per-step time of a 10-layer over a
    2-layer model (HIP events per step; embedding and controller cancel).
    Parity of this layer against the reference's own fwd_layer is the GPU
    test test_config1_on_gpu."""
    import numpy as np
    from bfp import Dims, synth
    from bfp.model import BfpModel
    t = {}
    for nl in (2, 10):
        d = Dims(NL=nl, MAX_CTX=8)
        gm = BfpModel(d)
        gm.load_fp32(synth.make_model(d, seed=1))
        prompt = synth.make_prompt(d, 8, seed=1)
        gm.decode(prompt[None, :], 0)                       # warm-up + graph build
        best = None
        for _ in range(5):
            gm.decode(prompt[None, :], 0, step_times=True)
            st = gm.step_times_ms()[:7]                    # steps without the head
            best = st if best is None else np.minimum(best, st)
        t[nl] = float(best.mean())
        gm.close()
    us = (t[10] - t[2]) / 8 * 1e3
    return {"workload": "config 1: one SmolLM2-135M-shaped layer, batch 1, positions 0-6",
            "layer_step_us": round(us, 2), "steps_per_s": round(1e6 / us, 1)}


_ORACLE = {}


def _oracle_model():
    """The oracle's model of the bench's 30-layer synthetic weights (built once)."""
    if "m" not in _ORACLE:
        from oracle import bfp_sim as sim
        from bfp import Dims, synth
        _ORACLE["m"] = sim.build_model(synth.make_model(Dims(MAX_CTX=2048), seed=0))
    return _ORACLE["m"]


def cpu_decode_baseline():
    """Config 3 on the oracle: the step time at position 36, the mean
    position of its 72 steps (the per-position attention loops make the
    step time grow with the position)."""
    t36 = _cpu_step_seconds(36)
    return {"value": round(1.0 / t36, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"oracle/bfp_sim.fwd_layer x 30 + head_argmax, one step at position 36 "
                      f"({t36:.2f} s) over a synthetic KV cache"}


def _cpu_step_seconds(pos, reps=2):
    """One decode step of the oracle (30 fwd_layer calls + the head) at
    position pos over a synthetic KV cache of pos + 1 rows per layer (its
    values do not change the work: the per-position loops run pos + 1
    times whatever they hold); the best of reps, 1 thread."""
    import numpy as np
    from oracle import bfp_sim as sim
    om = _oracle_model()
    d = om.dims
    rng = np.random.default_rng(pos)
    kv = [{"k": rng.standard_normal((pos + 1, d.H_KV, d.HD)),
           "v": rng.standard_normal((pos + 1, d.H_KV, d.HD))} for _ in range(d.NL)]
    best = None
    for _ in range(reps):
        h = om.embed_row_q(1)
        t0 = time.perf_counter()
        for li in range(d.NL):
            h = sim.fwd_layer(h, om.layers[li], pos=pos, kv=kv[li], kv_pos=pos, dims=d)
        sim.head_argmax(h, om.norm_w_q, om.embed)
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    return best


def cpu_long_context_baseline():
    """Config 4 on the oracle: step time at positions 48 and 2000 (the
    per-position attention loops make it linear in the position), the mean
    over positions 48..2047 interpolated linearly from the two."""
    t48, t2000 = _cpu_step_seconds(48), _cpu_step_seconds(2000)
    mean = t48 + (t2000 - t48) * ((48 + 2047) / 2 - 48) / (2000 - 48)
    return {"value": round(1.0 / mean, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "by_position": {"pos_48": round(1.0 / t48, 4), "pos_2000": round(1.0 / t2000, 4)},
            "sample": f"oracle/bfp_sim.fwd_layer x 30 + head_argmax, one step at position 48 "
                      f"({t48:.2f} s) and at 2000 ({t2000:.2f} s) over a synthetic KV cache; "
                      f"mean over 48..2047 by linear interpolation"}


def cpu_batch_baseline():
    """Config 5 on the oracle, which decodes one sequence at a time: the
    step time at position 72 (the mean position of 8 + 128 steps) is the
    time per token."""
    t72 = _cpu_step_seconds(72)
    return {"value": round(1.0 / t72, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"oracle/bfp_sim.fwd_layer x 30 + head_argmax, one sequence's step at "
                      f"position 72 ({t72:.2f} s); the oracle has no batched form, so 64 "
                      f"sequences take 64 such steps"}


def stream_probe():
    """Practical HBM ceilings: a 1 GiB device-to-device copy (read + write
    bytes) and a plain 16-byte-load streaming read of 2 GiB (the library's
    bfp_probe_read_d, contiguous range per workgroup, 4 workgroups per CU)."""
    import torch
    from bfp import _dev
    from bfp._lib import call
    a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    f = torch.ones(1 << 29, dtype=torch.float32, device="cuda")
    n_wg = torch.cuda.get_device_properties(0).multi_processor_count * 4
    fold = torch.empty(n_wg, dtype=torch.int32, device="cuda")

    def read():
        call("bfp_probe_read_d", f.data_ptr(), 2 << 30, fold.data_ptr(), n_wg, _dev.stream())
    res = {}
    for name, fn, nbytes in (("copy_1GiB", lambda: b.copy_(a), 2 << 30),
                             ("read_2GiB", read, 2 << 30)):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name + "_GB_s"] = round(nbytes * 5 / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    del a, b, f
    return res


def main():
    args = parse()
    if args.cpu_worker is not None:   # child of cpu_baseline_all_cores: CPU only
        b, t, _ = _cpu_matvec_sample(args.cpu_worker)
        print(json.dumps({"bytes": b, "seconds": t}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py: only --gpus 1 is supported on this build (asked for {args.gpus}); "
              "the BFP datapath is measured on one GPU", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no HIP GPU visible", file=sys.stderr)
        sys.exit(1)
    from bfp import _lib
    _lib.lib()
    if args.decode_only:
        res = {} if args.no_config3 else {"decode": decode_leg(args.decode_reps)}
        if not args.no_layer:
            res["layer"] = layer_leg()
        if args.long:
            res["long_context"] = long_context_leg()
        if args.batch64:
            res["batch64"] = batch_leg(args.batch64_tokens)
        print(json.dumps(res), flush=True)
        return
    print(f"[bench] building device rings for {len(SHAPES)} shapes x {args.reps} reps",
          file=sys.stderr, flush=True)
    cases = [ShapeCase(o, i, args.reps, seed=17 + k) for k, (o, i) in enumerate(SHAPES)]
    for _ in range(args.warmup):
        for c in cases:
            c.launch()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in cases] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        for k, c in enumerate(cases):
            ev[s][k][0].record(stream)
            c.launch()
            ev[s][k][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    parity = all(c.check() for c in cases)
    print(f"[bench] parity of sampled reps vs oracle: {parity}", file=sys.stderr, flush=True)
    per_shape = []
    for k, c in enumerate(cases):
        ms = sum(ev[s][k][0].elapsed_time(ev[s][k][1]) for s in range(args.steps)) / args.steps
        gbs = c.bytes_per_launch() / (ms * 1e-3) / 1e9
        per_shape.append({"shape": f"{c.n_out}x{c.n_in}", "ms_per_launch": round(ms, 4),
                          "GB_s": round(gbs, 1), "ring": c.ring,
                          "kernel": kernel_name(c.n_out, c.n_in, c.reps)})
    total_bytes = sum(c.bytes_per_launch() for c in cases) * args.steps
    value = total_bytes / wall / 1e9
    # the dominant launch: the shape with the most time, and its kernel
    kd = max(range(len(cases)), key=lambda k: per_shape[k]["ms_per_launch"])
    kname, kshape = per_shape[kd]["kernel"], per_shape[kd]["shape"]
    kbytes = cases[kd].bytes_per_launch()
    achieved = kbytes / (per_shape[kd]["ms_per_launch"] * 1e-3) / 1e9
    out = {
        "metric": "decode tokens/s at 1 GPU + BFP matvec HBM GB/s (% of peak), bit-exact",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16",
        "data": "synthetic",
        "config": {"workload": "bfp_matvec_sweep (BASELINE configs[1])",
                   "shapes": [f"{o}x{i}" for o, i in SHAPES], "reps_per_shape": args.reps,
                   "batch": 1},
        "bit_exact": parity,
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "per_shape": per_shape,
        "roofline": {"bound": "hbm", "kernel": kname, "shape": kshape,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(kname, kshape),
                     "alg_bytes_per_launch": int(kbytes)},
    }
    if not args.no_decode:
        print("[bench] config 3 decode", file=sys.stderr, flush=True)
        out["decode"] = decode_leg(args.decode_reps)
        if not args.no_layer:
            print("[bench] config 1 layer step", file=sys.stderr, flush=True)
            out["layer"] = layer_leg()
        if args.long:
            print("[bench] config 4 long context", file=sys.stderr, flush=True)
            out["long_context"] = long_context_leg()
        if args.batch64:
            print("[bench] config 5 batch 64", file=sys.stderr, flush=True)
            out["batch64"] = batch_leg()
    if args.probe:
        out["stream_ceiling"] = stream_probe()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        workers = args.cpu_workers or min(os.cpu_count() or 1, 16)
        out["cpu_baseline_all_cores"] = cpu_baseline_all_cores(8.0, workers)
        if not args.no_decode:
            out["decode"]["cpu_baseline"] = cpu_decode_baseline()
            if args.long:
                out["long_context"]["cpu_baseline"] = cpu_long_context_baseline()
            if args.batch64:
                out["batch64"]["cpu_baseline"] = cpu_batch_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
