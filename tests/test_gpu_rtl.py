"""GPU parity of the RTL-exact leaf ops: against the reference's own per-op
goldens (tests/golden/ref_rtl_ops.npz) and against the oracle
(oracle/bfp_rtl.py) on random batches with wide exponent ranges and edge
values.  Integer work: bit-exact."""
from pathlib import Path

import numpy as np
import pytest

from oracle import bfp_rtl as ort

pytestmark = pytest.mark.gpu
F = np.load(Path(__file__).resolve().parent / "golden" / "ref_rtl_ops.npz")


def _rand(rng, n, elo=-8, ehi=8):
    m = rng.integers(-32768, 32768, n).astype(np.int16)
    e = rng.integers(elo, ehi + 1, n // 16).astype(np.int8)
    return m, e


@pytest.mark.parametrize("D", [64, 576])
def test_matvec_fixture_and_random(gpu, D):
    from bfp import rtl
    nt = D // 16
    Wm = F[f"matvec_D{D}_wm"].reshape(nt, 16, 16).transpose(2, 0, 1)
    We = F[f"matvec_D{D}_we"].reshape(nt, 16).T
    m, e = rtl.golden_matvec(F[f"matvec_D{D}_xm"], F[f"matvec_D{D}_xe"], Wm, We)
    assert (m == F[f"matvec_D{D}_ym"]).all() and (e == F[f"matvec_D{D}_ye"]).all()
    rng = np.random.default_rng(D)
    xm, xe = _rand(rng, D, -60, 60)
    Wm = rng.integers(-32768, 32768, (48, nt, 16)).astype(np.int16)
    We = rng.integers(-60, 60, (48, nt)).astype(np.int8)
    Wm[0] = -32768
    Wm[1] = 0
    m, e = rtl.golden_matvec(xm, xe, Wm, We)
    wm, we = ort.rtl_matvec(xm.reshape(nt, 16), xe, Wm, We)
    assert (m == wm).all() and (e == we).all()


def test_requant(gpu):
    from bfp import rtl
    rng = np.random.default_rng(1)
    m = rng.integers(-32768, 32768, 256).astype(np.int16)
    e = rng.integers(-40, 40, 256).astype(np.int8)
    gm, ge = rtl.requant(m, e)
    wm, we = ort.rtl_requant(m, e)
    assert (gm == wm).all() and (ge == we).all()


@pytest.mark.parametrize("D", [64, 576])
def test_rmsnorm(gpu, D):
    from bfp import rtl
    k = f"rmsnorm_D{D}"
    m, e = rtl.golden_rmsnorm(F[k + "_xm"], F[k + "_xe"], F[k + "_gm"], F[k + "_ge"])
    assert (m[0] == F[k + "_ym"]).all() and (e[0] == F[k + "_ye"]).all()
    rng = np.random.default_rng(D + 1)
    xs = [_rand(rng, D, -10, 10) for _ in range(5)]
    gm_, ge_ = _rand(rng, D, -2, 2)
    xs[1] = (np.zeros(D, np.int16), xs[1][1])                  # all-zero input
    m, e = rtl.golden_rmsnorm(np.stack([x[0] for x in xs]), np.stack([x[1] for x in xs]), gm_, ge_)
    for b, (xm, xe) in enumerate(xs):
        wm, we = ort.rtl_rmsnorm(xm, xe, gm_, ge_)
        assert (m[b] == wm).all() and (e[b] == we).all(), b


@pytest.mark.parametrize("pos", [0, 3, 100, 2047])
def test_rope(gpu, pos):
    from bfp import rtl
    k = f"rope_P{pos}"
    m, e = rtl.golden_rope(F[k + "_xm"], F[k + "_xe"], pos)
    assert (m == F[k + "_ym"]).all() and (e == F[k + "_ye"]).all()
    rng = np.random.default_rng(pos)
    xm, xe = _rand(rng, 9 * 64, -20, 20)
    m, e = rtl.golden_rope(xm, xe, pos)
    f = ort.rope_freq_turns()
    for h in range(9):
        wm, we = ort.rtl_rope(xm[h * 64:(h + 1) * 64], xe[h * 4:(h + 1) * 4], pos, f)
        assert (m[h * 64:(h + 1) * 64] == wm).all() and (e[h * 64:(h + 1) * 64] == we).all()


@pytest.mark.parametrize("n", [1, 8, 64])
def test_softmax_fixture(gpu, n):
    from bfp import rtl
    k = f"softmax_N{n}"
    m, e = rtl.golden_softmax(F[k + "_xm"], int(F[k + "_xe"]), n)
    assert (m[0] == F[k + "_ym"]).all() and e[0] == int(F[k + "_ye"][0])


def test_softmax_random(gpu):
    from bfp import rtl
    rng = np.random.default_rng(7)
    lut = ort.exp_lut()
    for n in (2, 17, 200, 2048):
        xm = rng.integers(-32768, 32768, (4, n)).astype(np.int16)
        xe = np.array([-5, 0, 8, 20], np.int8)
        m, e = rtl.golden_softmax(xm, xe, n)
        for b in range(4):
            wm, we = ort.rtl_softmax(xm[b], int(xe[b]), n, lut)
            assert (m[b] == wm).all() and e[b] == we, (n, b)


@pytest.mark.parametrize("D", [64, 1536])
def test_swiglu(gpu, D):
    from bfp import rtl
    k = f"swiglu_D{D}"
    m, e = rtl.golden_swiglu(F[k + "_gatem"], F[k + "_gatee"], F[k + "_upm"], F[k + "_upe"])
    assert (m == F[k + "_ym"]).all() and (e == F[k + "_ye"]).all()
    rng = np.random.default_rng(D + 2)
    gm, ge = _rand(rng, D, -30, 30)
    um, ue = _rand(rng, D, -30, 30)
    m, e = rtl.golden_swiglu(gm, ge, um, ue)
    wm, we = ort.rtl_swiglu(gm, ge, um, ue, ort.silu_lut())
    assert (m == wm).all() and (e == we).all()


@pytest.mark.parametrize("D", [64, 576])
def test_residual(gpu, D):
    from bfp import rtl
    k = f"residual_D{D}"
    m, e = rtl.golden_residual(F[k + "_am"], F[k + "_ae"], F[k + "_bm"], F[k + "_be"])
    assert (m == F[k + "_ym"]).all() and (e == F[k + "_ye"]).all()
    rng = np.random.default_rng(D + 3)
    am, ae = _rand(rng, D, -20, 20)
    bm, be = _rand(rng, D, -20, 20)
    m, e = rtl.golden_residual(am, ae, bm, be)
    wm, we = ort.rtl_residual(am, ae, bm, be)
    assert (m == wm).all() and (e == we).all()


def test_argmax(gpu):
    from bfp import rtl
    rng = np.random.default_rng(9)
    n = 49152
    m = rng.integers(-32768, 32768, (2, n)).astype(np.int16)
    e = rng.integers(-3, 3, (2, n)).astype(np.int8)
    got = rtl.argmax(m, e)
    for b in range(2):
        assert got[b] == ort.rtl_argmax(m[b], e[b])
    assert rtl.argmax(np.full(64, 7, np.int16), np.zeros(64, np.int8))[0] == 0
