"""Golden vectors for the RTL-exact leaf ops, written by the reference's own
generators (run in a container where /root/reference exists; the npz is
committed next to this script).

Each per-op generator in rtl/vc707/host/ draws its inputs with
np.random.seed(0), computes its bit-exact golden, and writes both as hex
into ./generated.  They read their LUTs from ./generated too: exp_lut.hex
and silu_lut.hex come from rtl/vc707/sim/gen_exp_lut.py and
gen_swiglu_lut.py (OUT= points them at the temp dir); rope_freq_turns.svh is
the reference's committed table (rtl/vc707/src/smollm/rope_freq_turns.svh),
because its generator can only write inside the reference tree.

Output: ref_rtl_ops.npz with, per case, the inputs and outputs as int arrays,
plus the exp LUT and a digest of the SiLU LUT.
Usage: python tests/golden/gen_rtl_vectors.py
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
VC = Path("/root/reference/rtl/vc707")


def rd(path, bits, signed=True):
    vals = [int(x.split("//")[0], 16) for x in Path(path).read_text().split("\n")
            if x.split("//")[0].strip()]
    a = np.array(vals, dtype=np.int64)
    if signed:
        a = np.where(a >= 1 << (bits - 1), a - (1 << bits), a)
    return a


def run(script, td, **env):
    e = dict(os.environ, **{k: str(v) for k, v in env.items()})
    subprocess.run([sys.executable, str(VC / "host" / script)], cwd=td, env=e, check=True,
                   capture_output=True)


def main():
    out = {}
    with tempfile.TemporaryDirectory() as td:
        gen = Path(td) / "generated"
        gen.mkdir()
        for s in ("gen_exp_lut.py", "gen_swiglu_lut.py"):
            subprocess.run([sys.executable, str(VC / "sim" / s)], env=dict(os.environ, OUT=str(gen)),
                           check=True, capture_output=True)
        shutil.copy(VC / "src" / "smollm" / "rope_freq_turns.svh", gen / "rope_freq_turns.svh")
        out["exp_lut"] = rd(gen / "exp_lut.hex", 16, signed=False).astype(np.int32)
        silu = rd(gen / "silu_lut.hex", 16).astype(np.int16)
        out["silu_lut_sha256"] = np.array(hashlib.sha256(silu.tobytes()).hexdigest())
        out["silu_lut_head"] = silu[:64]
        out["silu_lut_tail"] = silu[-64:]

        for D in (64, 576):
            run("gen_matvec_bfp_golden.py", td, D=D)
            k = f"matvec_D{D}"
            out[k + "_xm"] = rd(gen / "matvec_bfp_xm.hex", 16)
            out[k + "_xe"] = rd(gen / "matvec_bfp_xe.hex", 8)
            out[k + "_wm"] = rd(gen / "matvec_bfp_wm.hex", 16)   # (t, k, lane) order
            out[k + "_we"] = rd(gen / "matvec_bfp_we.hex", 8)    # (t, lane) order
            out[k + "_ym"] = rd(gen / "matvec_bfp_ym.hex", 16)
            out[k + "_ye"] = rd(gen / "matvec_bfp_ye.hex", 8)
        for D in (64, 576):
            run("gen_rmsnorm_bfp_golden.py", td, D=D)
            k = f"rmsnorm_D{D}"
            for n, b in (("xm", 16), ("xe", 8), ("gm", 16), ("ge", 8), ("ym", 16), ("ye", 8)):
                out[f"{k}_{n}"] = rd(gen / f"rmsnorm_bfp_{n}.hex", b)
        for pos in (0, 3, 100, 2047):
            run("gen_rope_bfp_golden.py", td, POS=pos)
            k = f"rope_P{pos}"
            for n, b in (("xm", 16), ("xe", 8), ("ym", 16), ("ye", 8)):
                out[f"{k}_{n}"] = rd(gen / f"rope_bfp_{n}.hex", b)
        for N in (1, 8, 64):
            run("gen_softmax_bfp_golden.py", td, N=N)
            k = f"softmax_N{N}"
            out[k + "_xm"] = rd(gen / "softmax_bfp_xm.hex", 16)
            cfg = (gen / "softmax_bfp_cfg.svh").read_text().split()
            xe = int(cfg[cfg.index("SMBFP_XE") + 1])
            out[k + "_xe"] = np.array(xe - 256 if xe >= 128 else xe)
            out[k + "_ym"] = rd(gen / "softmax_bfp_ym.hex", 16)
            out[k + "_ye"] = rd(gen / "softmax_bfp_ye.hex", 8)
        for D in (64, 1536):
            run("gen_swiglu_bfp_golden.py", td, D=D)
            k = f"swiglu_D{D}"
            for n, b in (("gatem", 16), ("gatee", 8), ("upm", 16), ("upe", 8), ("ym", 16),
                         ("ye", 8)):
                out[f"{k}_{n}"] = rd(gen / f"swiglu_bfp_{n}.hex", b)
        for D in (64, 576):
            run("gen_residual_bfp_golden.py", td, D=D)
            k = f"residual_D{D}"
            for n, b in (("am", 16), ("ae", 8), ("bm", 16), ("be", 8), ("ym", 16), ("ye", 8)):
                out[f"{k}_{n}"] = rd(gen / f"res_bfp_{n}.hex", b)
        freq = [int(x.split("32'd")[1].split(",")[0].split()[0])
                for x in (gen / "rope_freq_turns.svh").read_text().splitlines() if "32'd" in x]
        out["rope_freq_turns"] = np.array(freq, np.int64)
    np.savez_compressed(HERE / "ref_rtl_ops.npz", **out)
    print("wrote ref_rtl_ops.npz:", len(out), "arrays")


if __name__ == "__main__":
    main()
