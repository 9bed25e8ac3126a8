"""The RTL-exact leaf-op oracle (oracle/bfp_rtl.py) against vectors written
by the reference's own per-op generators (tests/golden/gen_rtl_vectors.py),
plus independent checks: the LUTs and the frequency table against the
reference's committed/generated tables, the CORDIC against libm within the
reference testbench's +-2 LSB (rtl/vc707/sim/tb_cordic.cpp:113-119), the
Newton-Raphson RMSNorm against float math, and the argmax against numpy."""
import hashlib
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import bfp_rtl as rtl
from oracle import bfp_sim as sim

F = np.load(Path(__file__).resolve().parent / "golden" / "ref_rtl_ops.npz")


def test_luts_and_freq_table():
    assert rtl.exp_lut() == [int(v) for v in F["exp_lut"]]
    lut = rtl.silu_lut()
    assert hashlib.sha256(lut.tobytes()).hexdigest() == str(F["silu_lut_sha256"])
    assert rtl.rope_freq_turns() == [int(v) for v in F["rope_freq_turns"]]


@pytest.mark.parametrize("D", [64, 576])
def test_matvec(D):
    nt = D // 16
    Wm = F[f"matvec_D{D}_wm"].reshape(nt, 16, 16).transpose(2, 0, 1)   # (t,k,lane)->(lane,t,k)
    We = F[f"matvec_D{D}_we"].reshape(nt, 16).T
    m, e = rtl.rtl_matvec(F[f"matvec_D{D}_xm"].reshape(nt, 16), F[f"matvec_D{D}_xe"], Wm, We)
    assert (m == F[f"matvec_D{D}_ym"]).all() and (e == F[f"matvec_D{D}_ye"]).all()


@pytest.mark.parametrize("D", [64, 576])
def test_rmsnorm(D):
    k = f"rmsnorm_D{D}"
    m, e = rtl.rtl_rmsnorm(F[k + "_xm"], F[k + "_xe"], F[k + "_gm"], F[k + "_ge"])
    assert (m == F[k + "_ym"]).all() and (e == F[k + "_ye"]).all()


@pytest.mark.parametrize("pos", [0, 3, 100, 2047])
def test_rope(pos):
    k = f"rope_P{pos}"
    m, e = rtl.rtl_rope(F[k + "_xm"], F[k + "_xe"], pos, rtl.rope_freq_turns())
    assert (m == F[k + "_ym"]).all() and (e == F[k + "_ye"]).all()


@pytest.mark.parametrize("n", [1, 8, 64])
def test_softmax(n):
    k = f"softmax_N{n}"
    m, e = rtl.rtl_softmax(F[k + "_xm"], int(F[k + "_xe"]), n, rtl.exp_lut())
    assert (m == F[k + "_ym"]).all() and e == int(F[k + "_ye"][0])


@pytest.mark.parametrize("D", [64, 1536])
def test_swiglu(D):
    k = f"swiglu_D{D}"
    m, e = rtl.rtl_swiglu(F[k + "_gatem"], F[k + "_gatee"], F[k + "_upm"], F[k + "_upe"],
                          rtl.silu_lut())
    assert (m == F[k + "_ym"]).all() and (e == F[k + "_ye"]).all()


@pytest.mark.parametrize("D", [64, 576])
def test_residual(D):
    k = f"residual_D{D}"
    m, e = rtl.rtl_residual(F[k + "_am"], F[k + "_ae"], F[k + "_bm"], F[k + "_be"])
    assert (m == F[k + "_ym"]).all() and (e == F[k + "_ye"]).all()


def test_cordic_vs_libm():
    """CORDIC cos/sin within +-2 LSB of the Q1.15-quantised libm values."""
    worst = 0
    for i in range(2001):
        th = -math.pi + 2 * math.pi * i / 2000
        a = int(round(th * (1 << 27)))
        c, s = rtl.cordic_sincos(a)
        worst = max(worst, abs(c - round(math.cos(th) * 32768)), abs(s - round(math.sin(th) * 32768)))
    assert worst <= 2


def test_rope_angle_wraps_turns():
    """pos*freq in turns wraps modulo one turn: angle(pos) == angle of the
    fractional turn, in Q3.27 radians."""
    f = rtl.rope_freq_turns()
    for pos in (1, 7, 1000, 2047):
        for j in (0, 5, 31):
            turns = (pos * f[j]) / (1 << 31)
            frac = turns - math.floor(turns)
            frac = frac - 1 if frac >= 0.5 else frac
            got = rtl.rope_angle_q27(pos, f[j]) / (1 << 27)
            assert abs(got - 2 * math.pi * frac) < 1e-6


def test_rmsnorm_nr_vs_float():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(576) * 3
    g = 1 + 0.05 * rng.standard_normal(576)
    xm, xe = sim.tile_quantize(x)
    gm, ge = sim.tile_quantize(g)
    m, e = rtl.rtl_rmsnorm(xm, xe, gm, ge)
    got = sim.tile_decode(m.reshape(-1, 16), e)
    xv, gv = sim.tile_decode(xm, xe), sim.tile_decode(gm, ge)
    want = xv * gv / math.sqrt(np.mean(xv * xv) + 1e-5)
    lsb = np.repeat(2.0 ** (e.astype(np.float64) - 15), 16)
    err = np.abs(got - want) / lsb            # error in output LSBs of each tile
    assert err.max() < 16 and np.median(err) < 8


def test_requant_and_argmax():
    rng = np.random.default_rng(4)
    m = rng.integers(-32768, 32768, 64).astype(np.int16)
    e = rng.integers(-20, 20, 64).astype(np.int8)
    qm, qe = rtl.rtl_requant(m, e)
    for c in range(4):
        em = int(e[16 * c:16 * c + 16].max())
        assert qe[c] == em
        for k in range(16):
            i = 16 * c + k
            sh = em - int(e[i])
            assert qm[i] == (0 if sh >= 16 else int(m[i]) >> sh)
    # argmax over well-separated values equals the float argmax
    vals = rng.permutation(4096)[:256].astype(np.float64) * 0.37 - 500
    tm, te = sim.tile_quantize(vals)
    assert rtl.rtl_argmax(tm.reshape(-1), np.repeat(te, 16)) == int(np.argmax(vals))
    # strict '>' keeps the first of equal values
    assert rtl.rtl_argmax([5] * 32, [0] * 32) == 0
    assert rtl.bfp_gt(16384, 1, 32767, 0) and not rtl.bfp_gt(16383, 1, 32767, 0)
