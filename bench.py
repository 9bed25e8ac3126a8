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


# ----------------------------------------------------------- decode bytes
def layer_weight_bytes(d):
    """BFP weights + exponents one layer step reads: Q|K|V, O, G|U, D."""
    elems = (d.D + 2 * d.KV) * d.D + d.D * d.D + 2 * d.FFN * d.D + d.D * d.FFN
    return elems * 2 + elems // 16


def kv_bytes_per_position(d):
    """K and V of one position of one layer: mantissas + tile exponents."""
    return 2 * (d.KV * 2 + d.KV // 16)


def head_bytes(d):
    """The sim-faithful head reads the raw float32 tied embedding once per
    step (full.py:439), whatever the batch."""
    return d.VOCAB * d.D * 4


def step_bytes(d, pos, batch=1, head=True):
    """Algorithmic HBM bytes of one decode step at position pos: every
    layer's weights once, each sequence's KV rows 0..pos (pos+1 rows: the
    cache read plus this step's row), and the head's embedding."""
    return (d.NL * (layer_weight_bytes(d) + batch * kv_bytes_per_position(d) * (pos + 1))
            + (head_bytes(d) if head else 0))


def hbm_roofline(nbytes, seconds, basis):
    gbs = nbytes / seconds / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "alg_bytes": int(nbytes), "basis": basis}


def cpu_info():
    """The host the CPU baselines ran on."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    return {"model": model, "nproc": nproc, "cpu_count": os.cpu_count()}


def numpy_runtime():
    """numpy's version, the BLAS core its OpenBLAS picked on this host (the
    ddot/dgemv kernels behind full.py:278,439) and whether its AVX512F
    loops (np.exp's SIMD form, full.py:242,246) are dispatched."""
    import numpy as np
    out = {"numpy": np.__version__}
    try:
        import threadpoolctl
        blas = [b for b in threadpoolctl.threadpool_info() if b.get("user_api") == "blas"]
        if blas:
            out["blas"] = "%s %s %s" % (blas[0].get("internal_api"), blas[0].get("version"),
                                        blas[0].get("architecture"))
    except Exception as e:   # noqa: BLE001 - informational only
        out["blas"] = f"unknown ({type(e).__name__})"
    try:
        from numpy._core import _multiarray_umath as mu
        out["avx512f"] = bool(mu.__cpu_features__.get("AVX512F"))
    except Exception:   # noqa: BLE001
        out["avx512f"] = None
    return out


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
    ap.add_argument("--cpu-decode-worker", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--no-decode", action="store_true", help="skip the config-3 decode leg")
    ap.add_argument("--decode-only", action="store_true", help="run only the config-3 decode leg")
    ap.add_argument("--decode-reps", type=int, default=3)
    ap.add_argument("--decode-tokens", type=int, default=64,
                    help="tokens generated in the config-3 leg (64 = the config; fewer for "
                         "counter profiles)")
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
    ap.add_argument("--decode-probe", action="store_true",
                    help="with --decode-only: also run the HBM ceiling probe (its fixed read "
                         "and copy sizes calibrate rocprof's FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--decode-trace", action="store_true",
                    help="with --decode-only: also run config 3 once with the persistent "
                         "kernel's stage stamps and report the per-stage times")
    ap.add_argument("--decode-trace-batch", action="store_true",
                    help="with --decode-only: config 5 once with the matrix-core blocks' phase "
                         "stamps (the last layer of the last step) and report their medians")
    ap.add_argument("--batch64-pipe", action="store_true",
                    help="with --decode-only: also run config 5 on the pipelined step (one "
                         "launch per step) and record it as batch64_pipelined")
    ap.add_argument("--decode-trace-pipe", action="store_true",
                    help="with --decode-only: config 5 once on the pipelined step with its job "
                         "stamps (the last step) and report per-stage medians")
    ap.add_argument("--decode-trace-long", action="store_true",
                    help="with --decode-only: the same stage stamps for config 4 (the long "
                         "attention form), medians over positions 1984-2047")
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
        # the reps checked against the oracle: first, last and three between
        # (their ring slots' float32 weights are kept on the host)
        self.check_reps = sorted({int(r) for r in
                                  (0, reps - 1, reps // 4, reps // 2, (3 * reps) // 4)})
        slots = {r % self.ring for r in self.check_reps}
        self.W_host = {}
        # generate and pack in slabs to bound the fp32 staging memory
        per = max(1, (256 << 20) // (n_out * n_in * 4))
        for r0 in range(0, self.ring, per):
            k = min(per, self.ring - r0)
            W = torch.randn((k * n_out, n_in), generator=g, device="cuda", dtype=torch.float32)
            W.mul_(0.02)
            for sl in slots:
                if r0 <= sl < r0 + k:
                    self.W_host[sl] = W[(sl - r0) * n_out:(sl - r0 + 1) * n_out].cpu().numpy()
            call("bfp_quantize_pack_f32_d", W.data_ptr(), k * n_out, n_in,
                 self.Pm.data_ptr() + r0 * self.bm, self.Pe.data_ptr() + r0 * self.be,
                 _dev.stream())
            del W
        X = torch.randn((reps, n_in), generator=g, device="cuda", dtype=torch.float32)
        self.X_host = {r: X[r].cpu().numpy() for r in self.check_reps}
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
        """The sampled reps (first, last and three between; each reads ring
        slot rep % ring) against the CPU oracle, bit for bit."""
        import numpy as np
        from oracle import bfp_sim as sim
        ym = self.ym.cpu().numpy().reshape(self.reps, -1)
        ye = self.ye.cpu().numpy().reshape(self.reps, -1)
        nt = self.n_in // 16
        packed = {}
        ok = True
        for r in self.check_reps:
            sl = r % self.ring
            if sl not in packed:
                Wm, We = sim.tile_quantize(self.W_host[sl].astype(np.float64))
                packed[sl] = (Wm.reshape(self.n_out, nt, 16), We.reshape(self.n_out, nt))
            xm, xe = sim.tile_quantize(self.X_host[r].astype(np.float64))
            wm, we = sim.matvec_bfp(xm, xe, *packed[sl])
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
    """The matvec kernel the library launches (csrc/bfp_core.hip:
    launch_matvec): two 16-row chunks of one problem per workgroup for
    576-input shapes with an even chunk count, the buffer-load form for
    1536-input ones, else one chunk per workgroup."""
    nw, tpt = kernel_config(n_in)
    if nw == 3 and tpt == 3 and (n_out // 16) % 2 == 0:
        return "matvec2_kernel<3,3>"
    if nw == 8 and tpt == 3:
        return "matvec_kernel<8,3,true>"
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


def _fixture(name):
    import numpy as np
    path = ROOT / "tests" / "golden" / name
    return np.load(path) if path.exists() else None


def decode_leg(reps, n_gen=64):
    """30-layer SmolLM2-135M-shaped random-init model,
    8-token prompt, 64 greedy tokens.  Timed with HIP events inside
    bfp_decode (device time of the steps that emit the 64 tokens, and of all
    72 steps); tokens checked against the reference's own run
    (tests/golden/ref_decode_cfg3.npz)."""
    from bfp import Dims, synth
    from bfp.model import BfpModel
    n_prompt = 8
    d = Dims(MAX_CTX=n_prompt + 64)
    fm = synth.make_model(d, seed=0)
    prompt = synth.make_prompt(d, n_prompt, seed=0)
    gm = BfpModel(d)
    gm.load_fp32(fm)
    toks, _ = gm.decode(prompt[None, :], n_gen)          # warm-up + graph build
    gen_ms, tot_ms, walls = [], [], []
    for _ in range(max(reps, 1)):
        t0 = time.perf_counter()
        toks, _ = gm.decode(prompt[None, :], n_gen)
        walls.append(time.perf_counter() - t0)
        t, g = gm.decode_time_ms()
        tot_ms.append(t)
        gen_ms.append(g)
    gm.close()
    f = _fixture("ref_decode_cfg3.npz")
    exact = None
    if f is not None:
        exact = bool(list(toks[0]) == [int(t) for t in f["tokens"]][:n_gen]
                     and list(prompt) == [int(t) for t in f["prompt"]])
    g = min(gen_ms)
    nbytes = sum(step_bytes(d, p) for p in range(n_prompt, n_prompt + n_gen))
    return {"workload": f"config 3: 30 layers, prompt 8, {n_gen} greedy tokens, batch 1",
            "tokens_per_s": round(n_gen / (g * 1e-3), 1),
            "ms_per_token": round(g / n_gen, 4),
            "steps_per_s_all": round((n_prompt + n_gen) / (min(tot_ms) * 1e-3), 1),
            "wall_s_per_decode": round(min(walls), 4),
            "tokens_match_reference": exact,
            "roofline": hbm_roofline(nbytes, g * 1e-3,
                                     "per generated step: 30 layers' BFP weights + the fp32 "
                                     "embedding the head reads + KV rows 0..pos")}


# Stage stamps of the persistent batch-1 decode (csrc/bfp_persist.hip:
# stamp k of (step, layer), taken by thread 0 of each role's first workgroup
# on the 100 MHz device clock): Q|K|V 0 (h in), 10 (RMSNorm done), 11
# (matvec done), 1 (q|k|v stored), 3 (attention job 0 done) with the job's
# phases 2 (its q|k|v input in), 16 (RoPE done), 17 (scores), 18 (softmax),
# 19 (AV chains); O 4 (attention output in), 15, 5; G/U 6 (h1 in), 12, 13, 7; D 8
# (mlp in), 14, 9 (h stored).  Head stamps per step: 0 (start), 1
# (vocabulary slices done), 2 (token chosen).
TRACE_INTERVALS = [
    ("h in -> Q|K|V start (hand-off)", (-1, 9), (0, 0)),
    ("Q|K|V RMSNorm", (0, 0), (0, 10)),
    ("Q|K|V matvec", (0, 10), (0, 11)),
    ("Q|K|V epilogue + store", (0, 11), (0, 1)),
    ("attention (incl. q|k|v hand-off)", (0, 1), (0, 3)),
    ("  attention: q|k|v hand-off", (0, 1), (0, 2)),
    ("  attention: RoPE + cache row", (0, 2), (0, 16)),
    ("  attention: scores", (0, 16), (0, 17)),
    ("  attention: softmax", (0, 17), (0, 18)),
    ("  attention: AV chains", (0, 18), (0, 19)),
    ("  attention: quantise + store", (0, 19), (0, 3)),
    ("attention -> O start (hand-off)", (0, 3), (0, 4)),
    ("O matvec", (0, 4), (0, 15)),
    ("O epilogue + store", (0, 15), (0, 5)),
    ("h1 -> G/U start (hand-off)", (0, 5), (0, 6)),
    ("G/U RMSNorm", (0, 6), (0, 12)),
    ("G/U matvec", (0, 12), (0, 13)),
    ("G/U epilogue + store", (0, 13), (0, 7)),
    ("mlp -> D start (hand-off)", (0, 7), (0, 8)),
    ("D matvec", (0, 8), (0, 14)),
    ("D epilogue + store", (0, 14), (0, 9)),
    ("layer (D store to D store)", (-1, 9), (0, 9)),
]


def decode_trace_leg(long=False):
    """Config 3 (or config 4 with long=True) once on the persistent path
    with stage stamps: the median over generated steps (config 4: positions
    1984-2047) and layers 1..NL-1 of each stage interval (us), and of the
    head's."""
    import numpy as np
    from bfp import Dims, synth
    from bfp.model import BfpModel
    n_prompt, n_gen, seed = (48, 2000, 4) if long else (8, 64, 0)
    d = Dims(MAX_CTX=n_prompt + n_gen)
    gm = BfpModel(d)
    gm.load_fp32(synth.make_model(d, seed=0))
    prompt = synth.make_prompt(d, n_prompt, seed=seed)
    gm.decode(prompt[None, :], 16 if long else n_gen)
    gm.decode(prompt[None, :], n_gen, trace=True)
    path = gm.decode_path()
    tr = gm.decode_trace()
    gm.close()
    if tr is None:
        return {"path": path, "stages_us": None}
    lay, head = tr
    lay = lay.astype(np.int64)
    head = head.astype(np.int64)
    steps = range(1984, 2048) if long else range(n_prompt, n_prompt + n_gen)
    out = {}
    for name, (dl0, k0), (dl1, k1) in TRACE_INTERVALS:
        v = [(lay[s, l + dl1, k1] - lay[s, l + dl0, k0]) / 100.0
             for s in steps for l in range(1, d.NL)]
        out[name] = round(float(np.median(v)), 2)
    out["last D store -> head start"] = round(float(np.median(
        [(head[s, 0] - lay[s, d.NL - 1, 9]) / 100.0 for s in steps])), 2)
    out["head: vocabulary slices"] = round(float(np.median(
        [(head[s, 1] - head[s, 0]) / 100.0 for s in steps])), 2)
    out["head: argmax gather"] = round(float(np.median(
        [(head[s, 2] - head[s, 1]) / 100.0 for s in steps])), 2)
    out["head end -> next step's Q|K|V start"] = round(float(np.median(
        [(lay[s + 1, 0, 0] - head[s, 2]) / 100.0 for s in list(steps)[:-1]])), 2)
    out["step"] = round(float(np.median(
        [(lay[s + 1, 0, 0] - lay[s, 0, 0]) / 100.0 for s in list(steps)[:-1]])), 2)
    return {"path": path, "steps": f"{steps[0]}..{steps[-1]}", "stages_us": out}


MX_PHASES = ("staging (exponents)", "pass 1 (row maxima)", "pass 2 (tile sums)",
             "A reduction", "epilogue (wave 0)")
ATT_PHASES = ("q|k|v in (wave 0)", "RoPE, rows staged", "scores", "softmax (wave 0)",
              "AV chains (wave 0)")


def batch_trace_leg():
    """Config 5 once with the matrix-core matvec blocks' phase stamps (the
    last launch of each kernel: the last layer of the last step): per kernel
    the blocks stamped, the spread of their start times, the span from the
    first start to the last epilogue, and the median of each phase (us);
    likewise the attention workgroups of the joined Q|K|V launch (entry to
    q|k|v in, RoPE and staging, scores, softmax, AV chains)."""
    import numpy as np
    from bfp import Dims, synth
    from bfp.model import BfpModel
    B, n_prompt, n_gen = 64, 8, 128
    d = Dims(MAX_CTX=n_prompt + n_gen)
    gm = BfpModel(d, max_batch=B)
    gm.load_fp32(synth.make_model(d, seed=0))
    prompts = np.stack([synth.make_prompt(d, n_prompt, seed=0)] +
                       [synth.make_prompt(d, n_prompt, seed=1000 + b) for b in range(1, B)])
    gm.decode(prompts, 4)
    gm.decode(prompts, n_gen, trace=True)
    form = gm.decode_form()
    tr = gm.decode_trace()
    gm.close()
    if tr is None:
        return {"form": form, "kernels": None}
    tr = tr.astype(np.int64)
    out = {}
    # the joined Q|K|V launch: its matvec blocks first, then the attention
    # workgroups (one per KV group and sequence), whose rows hold their own
    # phases
    nblk = (d.D + 2 * d.H_KV * d.HD) // 16 * ((B + 15) // 16)
    att = tr[0][nblk:]
    att = att[att[:, 0] > 0]
    if "attn_group" in form and len(att):
        t0 = att[:, 0].min()
        r = {"workgroups": int(len(att)), "start_spread_us": round(float((att[:, 0].max() - t0) / 100), 2),
             "span_us": round(float((att[:, 5].max() - t0) / 100), 2)}
        for j, ph in enumerate(ATT_PHASES):
            r[ph] = round(float(np.median((att[:, j + 1] - att[:, j]) / 100)), 2)
        out["attention"] = r
        tr = tr.copy()
        tr[0][nblk:] = 0
    for k, name in enumerate(("Q|K|V", "O", "G/U", "D")):
        st = tr[k][tr[k][:, 0] > 0]
        if not len(st):
            continue
        t0 = st[:, 0].min()
        r = {"blocks": int(len(st)), "start_spread_us": round(float((st[:, 0].max() - t0) / 100), 2),
             "span_us": round(float((st[:, 5].max() - t0) / 100), 2)}
        for j, ph in enumerate(MX_PHASES):
            r[ph] = round(float(np.median((st[:, j + 1] - st[:, j]) / 100)), 2)
        out[name] = r
    return {"form": form, "step": f"{n_prompt + n_gen - 1} (last layer)", "kernels_us": out}


PIPE_STAGES = ("N1", "QKV", "ATT", "O", "N2", "GU", "D")


def pipe_trace_leg(n_gen=128):
    """Config 5 once on the pipelined step with its job stamps (the last
    step's launch: every job's start, inputs in LDS, end, and per kind its
    phases), summarised per stage in us: jobs, median and 90th percentile of
    the wait (start to inputs in) and of the work (inputs in to end); the
    matrix-core jobs' phases (inputs to row maxima, to tile sums, to the
    epilogue's stores, to the end) and the attention jobs' (start to q|k|v
    in, RoPE, scores, softmax, AV chains, outputs); the launch's span and
    the workgroups' busy fraction (work over span)."""
    import numpy as np
    from bfp import Dims, synth
    from bfp.model import BfpModel
    B, n_prompt = 64, 8
    d = Dims(MAX_CTX=n_prompt + 128)
    gm = BfpModel(d, max_batch=B)
    gm.load_fp32(synth.make_model(d, seed=0))
    prompts = np.stack([synth.make_prompt(d, n_prompt, seed=0)] +
                       [synth.make_prompt(d, n_prompt, seed=1000 + b) for b in range(1, B)])
    gm.decode(prompts, 4, pipe=True)
    gm.decode(prompts, n_gen, trace=True, pipe=True)
    form = gm.decode_form()
    _, g = gm.decode_time_ms()
    tr = gm.decode_trace()
    gm.close()
    if form != "pipe" or tr is None:
        return {"form": form, "stages": None}
    tr = tr.astype(np.int64)
    used = tr[:, :, 0] > 0
    code = tr[:, :, 0] - 1
    stage = (code >> 23) & 7
    t0 = tr[:, :, 1][used].min()
    span = (tr[:, :, 3][used].max() - t0) / 100

    def q(v):
        return {"med": round(float(np.median(v)), 2), "p90": round(float(np.percentile(v, 90)), 2)}
    out = {}
    for k, name in enumerate(PIPE_STAGES):
        m = used & (stage == k)
        if not m.any():
            continue
        j = tr[m]
        r = {"jobs": int(m.sum()), "wait": q((j[:, 2] - j[:, 1]) / 100),
             "work": q((j[:, 3] - j[:, 2]) / 100)}
        if name in ("QKV", "O", "GU", "D"):
            ph = np.stack([j[:, 5] - j[:, 2], j[:, 6] - j[:, 5], j[:, 7] - j[:, 6],
                           j[:, 3] - j[:, 7]], 1) / 100
            r["phases_med"] = dict(zip(("row maxima", "tile sums", "epilogue stored", "end"),
                                       [round(float(v), 2) for v in np.median(ph, 0)]))
        if name == "ATT":
            ph = np.stack([j[:, 2] - j[:, 1], j[:, 4] - j[:, 2], j[:, 5] - j[:, 4],
                           j[:, 6] - j[:, 5], j[:, 7] - j[:, 6], j[:, 3] - j[:, 7]], 1) / 100
            r["phases_med"] = dict(zip(("q|k|v in", "RoPE", "scores", "softmax", "AV", "outputs"),
                                       [round(float(v), 2) for v in np.median(ph, 0)]))
        out[name] = r
    busy = ((tr[:, :, 3] - tr[:, :, 2]) * used).sum(1) / 100 / span
    return {"form": form, "step": f"{n_prompt + n_gen - 1}", "ms_per_step": round(g / n_gen, 4),
            "launch_span_us": round(float(span), 1), "workgroups": int(tr.shape[0]),
            "busy_frac_med": round(float(np.median(busy)), 3), "stages_us": out}


def long_context_leg():
    """30 layers, 48-token prompt, greedy decode through
    position 2047 (2000 new tokens); tokens/s overall and per position
    window from per-step HIP events; tokens checked against the reference's
    own run (tests/golden/ref_decode_cfg4.npz) when it is present."""
    from bfp import Dims, synth
    from bfp.model import BfpModel
    n_prompt, n_gen = 48, 2000
    d = Dims(MAX_CTX=2048)
    gm = BfpModel(d)
    gm.load_fp32(synth.make_model(d, seed=0))
    prompt = synth.make_prompt(d, n_prompt, seed=4)
    gm.decode(prompt[None, :], 16)                       # warm-up
    toks, _ = gm.decode(prompt[None, :], n_gen, step_times=True)
    st = gm.step_times_ms()
    t, g = gm.decode_time_ms()
    gm.close()
    win = {}
    for lo, hi in ((48, 112), (496, 560), (1008, 1072), (1984, 2048)):
        win[f"pos_{lo}_{hi - 1}"] = round((hi - lo) / (float(st[lo:hi].sum()) * 1e-3), 1)
    f = _fixture("ref_decode_cfg4.npz")
    exact = None
    if f is not None:
        exact = bool(list(toks[0]) == [int(x) for x in f["tokens"]]
                     and list(prompt) == [int(x) for x in f["prompt"]])
    nbytes = sum(step_bytes(d, p) for p in range(n_prompt, n_prompt + n_gen))
    lo, hi = 1984, 2048
    tail_bytes = sum(step_bytes(d, p) for p in range(lo, hi))
    return {"workload": "config 4: 30 layers, prompt 48, decode to position 2047 (2000 tokens)",
            "tokens_per_s": round(n_gen / (g * 1e-3), 1), "ms_per_token_mean": round(g / n_gen, 4),
            "tokens_per_s_by_position": win, "tokens_match_reference": exact,
            "roofline": hbm_roofline(nbytes, g * 1e-3,
                                     "per generated step: 30 layers' BFP weights + the fp32 "
                                     "embedding the head reads + KV rows 0..pos"),
            "roofline_pos_1984_2047": hbm_roofline(tail_bytes, float(st[lo:hi].sum()) * 1e-3,
                                                   "the same over positions 1984..2047")}


def batch_leg(n_gen=128, pipe=None):
    """64 independent sequences, 8-token prompts, 128
    greedy tokens each; aggregate tokens/s.  Every sequence's tokens are
    checked against the reference's own runs (tests/golden/ref_decode_cfg5.npz).
    pipe=True runs the pipelined step (one launch per step) instead of the
    per-stage launches."""
    import numpy as np
    from bfp import Dims, synth
    from bfp.model import BfpModel
    B, n_prompt = 64, 8
    d = Dims(MAX_CTX=n_prompt + 128)
    gm = BfpModel(d, max_batch=B)
    gm.load_fp32(synth.make_model(d, seed=0))
    prompts = np.stack([synth.make_prompt(d, n_prompt, seed=0)] +
                       [synth.make_prompt(d, n_prompt, seed=1000 + b) for b in range(1, B)])
    gm.decode(prompts, 4, pipe=pipe)                     # warm-up
    toks, _ = gm.decode(prompts, n_gen, pipe=pipe)
    t, g = gm.decode_time_ms()
    form = gm.decode_form()
    gm.close()
    f = _fixture("ref_decode_cfg5.npz")
    exact = None
    if f is not None:
        exact = bool((f["prompts"] == prompts).all() and
                     (toks[:, :n_gen] == f["tokens"][:, :n_gen]).all())
    nbytes = sum(step_bytes(d, p, batch=B) for p in range(n_prompt, n_prompt + n_gen))
    return {"workload": f"config 5: 64 sequences, prompt 8, {n_gen} greedy tokens each",
            "tokens_per_s": round(B * n_gen / (g * 1e-3), 1),
            "ms_per_step": round(g / n_gen, 4), "all_tokens_match_reference": exact,
            "form": form,
            "roofline": hbm_roofline(nbytes, g * 1e-3,
                                     "per generated step: 30 layers' BFP weights once + the "
                                     "fp32 embedding once + each sequence's KV rows 0..pos")}


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
    d = Dims(NL=1, MAX_CTX=8)
    nbytes = sum(layer_weight_bytes(d) + kv_bytes_per_position(d) * (p + 1) for p in range(7)) / 7
    return {"workload": "config 1: one SmolLM2-135M-shaped layer, batch 1, positions 0-6",
            "layer_step_us": round(us, 2), "steps_per_s": round(1e6 / us, 1),
            "roofline": hbm_roofline(nbytes, us * 1e-6,
                                     "one layer's BFP weights + KV rows 0..pos, mean over "
                                     "positions 0-6"),
            "dropin": layer_dropin_leg()}


def layer_dropin_leg(reps=5):
    """BASELINE config 1 as written: one layer, 8 positions decoded one at a
    time from N(0,1) activations (synth.make_layer_inputs, the generator of
    tests/golden/ref_layer_cfg1.npz), each position one bfp_layer_step_kv
    call with host buffers -- the drop-in fwd_layer's cost, PCIe copies and
    the call's synchronisation included.  Wall clock per call, the best of
    `reps` passes per position; every pass's outputs are compared with the
    reference's own run of the same layer (the fixture)."""
    import numpy as np
    import bfp.api as api
    from bfp import Dims, synth
    from bfp.model import BfpModel
    f = _fixture("ref_layer_cfg1.npz")
    seed = int(f["seed"]) if f is not None else 1
    d = Dims(NL=1, MAX_CTX=16, VOCAB=256)
    gm = BfpModel(d)
    gm.load_fp32(synth.make_model(d, seed=seed))
    xs = synth.make_layer_inputs(d, 8, seed=seed)
    qin = [tuple(a.reshape(1, -1) for a in api.tile_quantize(xs[p])) for p in range(8)]
    best = np.full(8, np.inf)
    exact = True if f is not None else None
    for _ in range(reps + 1):                      # the first pass warms up
        gm.reset_kv()
        for p in range(8):
            t0 = time.perf_counter()
            om_, oe_, _ = gm.layer_step_bfp(0, p, *qin[p])
            best[p] = min(best[p], time.perf_counter() - t0)
            if f is not None:
                cm, ce = api.tile_quantize(api.tile_decode(om_[0], oe_[0]))   # canonical form
                exact = exact and bool((cm.reshape(-1) == f["hout_m"][p]).all() and
                                       (ce == f["hout_e"][p]).all())
    gm.close()
    us = float(best.mean()) * 1e6
    return {"workload": "config 1 as written: 1 layer, positions 0-7, N(0,1) activations, "
                        "one host-buffer call per position",
            "call_us": round(us, 2), "positions_per_s": round(1e6 / us, 1),
            "outputs_match_reference": exact}


# ------------------------------------------------------------ CPU baselines
# The oracle (oracle/bfp_sim.py, line-faithful to full.py) and its
# numpy-vectorised restatement (oracle/bfp_vec.py), timed in child
# processes so that each run sets its own BLAS thread count before numpy
# loads.  A child builds the bench's synthetic model once and times one
# decode step (NL fwd_layer calls, and the head for the 30-layer model) at
# each asked position over a synthetic KV cache of pos + 1 rows per layer
# (the per-position loops run pos + 1 times whatever the rows hold).
def _cpu_decode_worker(spec):
    import numpy as np
    from bfp import Dims, synth
    from oracle import bfp_sim as sim
    from oracle import bfp_vec as vec
    mod = vec if spec["kind"] == "vec" else sim
    nl = spec.get("nl", 30)
    d = Dims(NL=nl, MAX_CTX=2048, VOCAB=49152 if nl == 30 else 256)
    t0 = time.perf_counter()
    om = mod.build_model(synth.make_model(d, seed=0 if nl == 30 else 1))
    build_s = time.perf_counter() - t0
    out = {"build_s": round(build_s, 2), "steps": {}}
    for pos in spec["positions"]:
        rng = np.random.default_rng(pos)
        kv = [{"k": sim.fp_quantize_vec(rng.standard_normal((pos + 1) * d.KV)).reshape(
                   pos + 1, d.H_KV, d.HD),
               "v": sim.fp_quantize_vec(rng.standard_normal((pos + 1) * d.KV)).reshape(
                   pos + 1, d.H_KV, d.HD)} for _ in range(nl)]
        best = None
        for _ in range(spec.get("reps", 2) if pos < 1000 else 1):
            h = om.embed_row_q(1) if nl == 30 else sim.fp_quantize_vec(rng.standard_normal(d.D))
            t0 = time.perf_counter()
            for li in range(nl):
                h = mod.fwd_layer(h, om.layers[li], pos=pos, kv=kv[li], kv_pos=pos, dims=om.dims)
            if nl == 30:
                sim.head_argmax(h, om.norm_w_q, om.embed)
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        out["steps"][str(pos)] = best
    print(json.dumps(out), flush=True)


def _run_cpu_workers(spec, threads, n=1):
    """n concurrent children running spec with `threads` BLAS threads each;
    returns their results."""
    import subprocess
    env = dict(os.environ, OPENBLAS_NUM_THREADS=str(threads), OMP_NUM_THREADS=str(threads))
    cmd = [sys.executable, str(Path(__file__).resolve()), "--cpu-decode-worker", json.dumps(spec)]
    procs = [subprocess.Popen(cmd, stdout=subprocess.PIPE, env=env, text=True) for _ in range(n)]
    res = []
    for p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            raise RuntimeError(f"cpu decode worker exited with {p.returncode}")
        res.append(json.loads(out.strip().splitlines()[-1]))
    return res


def cpu_decode_baselines():
    """The decode configs on the CPU: line-faithful and vectorised, 1 BLAS
    thread and all cores.  Returns {leg: {name: cpu_baseline dict}}."""
    info = cpu_info()
    nproc = info["nproc"]
    P = [36, 48, 72, 2000]
    runs = {("port", 1): _run_cpu_workers({"kind": "faithful", "positions": P}, 1)[0],
            ("vec", 1): _run_cpu_workers({"kind": "vec", "positions": P}, 1)[0],
            ("vec", nproc): _run_cpu_workers({"kind": "vec", "positions": P}, nproc)[0]}
    par = min(nproc, 16)
    batch_par = _run_cpu_workers({"kind": "vec", "positions": [72]}, 1, n=par)
    layer = {k: _run_cpu_workers({"kind": k, "positions": list(range(7)), "nl": 1}, 1)[0]
             for k in ("faithful", "vec")}
    name = {"port": "oracle/bfp_sim (line-faithful numpy restatement of full.py)",
            "vec": "oracle/bfp_vec (numpy-vectorised restatement, bit-identical)"}

    def entry(kind, threads, value, sample, blas=None):
        blas = threads if blas is None else blas
        return {"value": round(value, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
                "variant": "line-faithful" if kind == "port" else "vectorised",
                "sample": f"{name[kind]}, OPENBLAS_NUM_THREADS={blas}: {sample}"}

    out = {"decode": {}, "long_context": {}, "batch64": {}, "layer": {}}
    for (kind, thr), r in runs.items():
        st = r["steps"]
        key = f"{'faithful' if kind == 'port' else 'vectorised'}_{thr}t"
        out["decode"][key] = entry(kind, thr, 1.0 / st["36"],
                                   f"one 30-layer step at position 36 (the mean of config 3's "
                                   f"72 steps), {st['36']:.3f} s")
        t48, t2000 = st["48"], st["2000"]
        mean = t48 + (t2000 - t48) * ((48 + 2047) / 2 - 48) / (2000 - 48)
        out["long_context"][key] = entry(kind, thr, 1.0 / mean,
                                         f"steps at positions 48 ({t48:.3f} s) and 2000 "
                                         f"({t2000:.3f} s), mean over 48..2047 by linear "
                                         f"interpolation (the step time is linear in the "
                                         f"position)")
        out["batch64"][key] = entry(kind, thr, 1.0 / st["72"],
                                    f"one sequence's step at position 72 ({st['72']:.3f} s); "
                                    f"the simulator decodes one sequence at a time")
    t72 = max(r["steps"]["72"] for r in batch_par)
    out["batch64"][f"vectorised_{par}proc"] = entry(
        "vec", par, par / t72, f"{par} concurrent single-threaded processes, one sequence's step "
        f"at position 72 each (independent sequences), slowest {t72:.3f} s", blas=1)
    for k, r in layer.items():
        ts = [r["steps"][str(p)] for p in range(7)]
        kk = "port" if k == "faithful" else "vec"
        e = entry(kk, 1, 7.0 / sum(ts), f"one D=576 layer (fwd_layer) at positions 0-6, "
                  f"{sum(ts) / 7 * 1e3:.2f} ms per step")
        e["unit"] = "layer steps/s"
        out["layer"][f"{'faithful' if k == 'faithful' else 'vectorised'}_1t"] = e
    return out


def stream_probe():
    """Practical HBM ceilings: a 1 GiB device-to-device copy (read + write
    bytes) and a 4 GiB streaming read with the library's bfp_probe_read_d
    (16-byte loads, 16 KB per workgroup, 262144 workgroups), with ordinary
    and with non-temporal loads (the matvec's weight-stream policy).  The
    best read is the ceiling the matvec is compared with."""
    import torch
    from bfp import _dev
    from bfp._lib import call
    a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    f = torch.ones(1 << 30, dtype=torch.float32, device="cuda")       # 4 GiB
    n_wg = (4 << 30) // 16384
    fold = torch.empty(n_wg, dtype=torch.int32, device="cuda")

    def read(nt):
        return lambda: call("bfp_probe_read_d", f.data_ptr(), 4 << 30, fold.data_ptr(), n_wg,
                            nt, _dev.stream())
    res = {}
    for name, fn, nbytes in (("copy_1GiB", lambda: b.copy_(a), 2 << 30),
                             ("read_4GiB", read(0), 4 << 30),
                             ("read_nt_4GiB", read(1), 4 << 30)):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name + "_GB_s"] = round(nbytes * 5 / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    res["read_ceiling_GB_s"] = max(res["read_4GiB_GB_s"], res["read_nt_4GiB_GB_s"])
    del a, b, f
    return res


def main():
    args = parse()
    if args.cpu_worker is not None:   # child of cpu_baseline_all_cores: CPU only
        b, t, _ = _cpu_matvec_sample(args.cpu_worker)
        print(json.dumps({"bytes": b, "seconds": t}), flush=True)
        return
    if args.cpu_decode_worker is not None:   # child of cpu_decode_baselines: CPU only
        _cpu_decode_worker(json.loads(args.cpu_decode_worker))
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
        def note(msg):
            print(f"[bench] {msg}", file=sys.stderr, flush=True)
        res = {}
        if not args.no_config3:
            note("config 3 decode")
            res["decode"] = decode_leg(args.decode_reps, args.decode_tokens)
        if not args.no_layer:
            note("config 1 layer step")
            res["layer"] = layer_leg()
        if args.long:
            note("config 4 long context")
            res["long_context"] = long_context_leg()
        if args.batch64:
            note("config 5 batch 64")
            res["batch64"] = batch_leg(args.batch64_tokens)
        if args.batch64_pipe:
            note("config 5 batch 64, pipelined step")
            res["batch64_pipelined"] = batch_leg(args.batch64_tokens, pipe=True)
        if args.decode_probe:
            note("HBM ceiling probe")
            res["stream_ceiling"] = stream_probe()
        if args.decode_trace:
            note("config 3 persistent-decode stage trace")
            res["decode_trace"] = decode_trace_leg()
        if args.decode_trace_batch:
            note("config 5 matrix-core block phase trace")
            res["decode_trace_batch"] = batch_trace_leg()
        if args.decode_trace_pipe:
            note("config 5 pipelined-step job trace")
            res["decode_trace_pipe"] = pipe_trace_leg(args.batch64_tokens)
        if args.decode_trace_long:
            note("config 4 persistent-decode stage trace (positions 1984-2047)")
            res["decode_trace_long"] = decode_trace_leg(long=True)
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
        print("[bench] HBM read ceiling probe", file=sys.stderr, flush=True)
        out["stream_ceiling"] = stream_probe()
        out["roofline"]["frac_of_read_ceiling"] = round(
            achieved / out["stream_ceiling"]["read_ceiling_GB_s"], 4)
    if not args.no_cpu:
        print("[bench] CPU baselines", file=sys.stderr, flush=True)
        out["cpu"] = dict(cpu_info(), **numpy_runtime())
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        workers = args.cpu_workers or min(cpu_info()["nproc"], 16)
        out["cpu_baseline_all_cores"] = cpu_baseline_all_cores(8.0, workers)
        if not args.no_decode:
            cb = cpu_decode_baselines()
            for leg, key in (("decode", "decode"), ("layer", "layer"),
                             ("long_context", "long_context"), ("batch64", "batch64")):
                if leg in out:
                    out[leg]["cpu_baseline"] = cb[key]["faithful_1t"]
                    out[leg]["cpu_baselines"] = cb[key]
    # the full record (every baseline's sample text) goes to stderr; the
    # JSON line on stdout keeps every figure in a few KB
    print("[bench] detail " + json.dumps(out), file=sys.stderr, flush=True)
    print(json.dumps(compact(out)), flush=True)


def compact(out):
    """The stdout record: the same figures without the long texts --
    rooflines without their basis text, each leg's alternative CPU
    baselines as bare values."""
    def roof(r):
        return {k: v for k, v in r.items() if k != "basis"}

    res = {}
    for k, v in out.items():
        if not isinstance(v, dict) or k in ("config", "roofline", "cpu_baseline", "cpu"):
            res[k] = v
            continue
        leg = {}
        for kk, vv in v.items():
            if kk.startswith("roofline"):
                leg[kk] = roof(vv)
            elif kk == "cpu_baselines":
                leg[kk] = {n: b["value"] for n, b in vv.items()}
            else:
                leg[kk] = vv
        res[k] = leg
    return res


if __name__ == "__main__":
    main()
