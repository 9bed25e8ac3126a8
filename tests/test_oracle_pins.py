"""Pins of the CPU oracle (oracle/bfp_sim.py) that do not need the reference.

Each check is one a plausible mistake in the restatement would fail: closed
forms of the quantiser, a float-free brute force of the quantiser and the
matvec, idempotence, invariants on the reference's own committed BFP data
(rtl/vc707/release/*.hex, copied as tests/golden/release_*.npz), and the
restated numpy/BLAS reduction orders against the library calls.
"""
import math
import random
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import bfp_bigint as bi
from oracle import bfp_sim as sim

GOLDEN = Path(__file__).resolve().parent / "golden"


# ------------------------------------------------------------ tile_quantize
def test_power_of_two_closed_form():
    for k in range(-20, 20):
        v = np.zeros(16)
        v[3] = 2.0 ** k
        v[7] = -(2.0 ** (k - 3))
        m, e = sim.tile_quantize(v)
        assert e[0] == k + 1
        assert m[0, 3] == 16384 and m[0, 7] == -2048


def test_zero_tile_and_clip():
    m, e = sim.tile_quantize(np.zeros(32))
    assert (e == -127).all() and (m == 0).all()
    v = np.zeros(16)
    v[0] = 1.0 - 2.0 ** -17          # rounds to 32768 -> clipped
    v[1] = -(1.0 - 2.0 ** -17)       # rounds to -32768 -> kept
    m, e = sim.tile_quantize(v)
    assert e[0] == 0 and m[0, 0] == 32767 and m[0, 1] == -32768


def test_round_half_even():
    v = np.zeros(16)
    v[0] = 0.75                      # sets e = 0: unit = 2**-15
    for i, (num, want) in enumerate([(2.5, 2), (3.5, 4), (-2.5, -2), (-3.5, -4), (0.5, 0),
                                     (1.5, 2)], start=1):
        v[i] = num / 32768.0
    m, e = sim.tile_quantize(v)
    assert e[0] == 0
    assert list(m[0, 1:7]) == [2, 4, -2, -4, 0, 2]


def test_tile_quantize_vs_bigint():
    rng = np.random.default_rng(11)
    for scale in (1e-30, 1e-3, 0.02, 1.0, 37.0, 1e20):
        v = rng.standard_normal(16 * 40) * scale
        v[:16] = 0.0
        v[16] = scale * 2.0 ** -300 if scale > 1e-10 else v[16]
        m, e = sim.tile_quantize(v)
        bm, be = bi.quantize_vec([float(x) for x in v])
        assert list(e) == be
        assert m.tolist() == bm


def _below_pow2(k, n):
    """The double n spacings below 2^k (in the binade [2^(k-1), 2^k))."""
    return float(np.ldexp(1.0, k) - n * np.ldexp(1.0, k - 53))


def test_np_log2_roundup_closed_form():
    """np.log2 rounds to the integer k for doubles up to n_up(k) spacings
    below 2^k; the closed form the kernels use (log2_up_ulps) must give that
    count for every exponent a tile can have."""
    for k in range(-130, 131):
        n = 0
        while np.floor(np.log2(_below_pow2(k, n + 1))) >= k:
            n += 1
        assert n == bi.log2_up_ulps(k), k


def test_near_power_of_two_tiles_vs_bigint():
    """Tiles whose max sits 0..100 doubles below a power of two: numpy's
    quantiser (floor(np.log2) + 1) against the decimal-logarithm model.  A
    quantiser using the exact floor(log2) (frexp) fails at n <= n_up(k)."""
    rng = np.random.default_rng(13)
    hit = 0
    for k in list(range(-127, -100)) + list(range(-70, 70)) + list(range(100, 128)):
        for n in (1, 2, 5, 11, 22, 44, 45, 88, 100):
            v = rng.standard_normal(16) * np.ldexp(1.0, k - 3)
            v[rng.integers(16)] = _below_pow2(k, n) * (1 if rng.random() < .5 else -1)
            m, e = sim.tile_quantize(v)
            bm, be = bi.quantize_vec([float(x) for x in v])
            assert list(e) == be and m.tolist() == bm, (k, n)
            hit += n <= bi.log2_up_ulps(k)
    assert hit > 100


def test_epilogue_int_near_power_of_two():
    """The float-free matvec epilogue's round-up rule (row key 2L + u)
    against quantize_tile of the exact row values, on rows whose |y| lies
    just below 2^k with |k| >= 65 (n_up = 44 or 88, so |A| >= 2^47 - 44*32
    reaches the rule)."""
    rng = random.Random(14)
    for M in (64 + 30 - 48, 65 + 30 - 48, 96, -300 + 30 + 48 + 100, -48):
        for gap in (1, 2, 3, 4, 31, 32, 33, 64):
            rows = []
            for r in range(16):
                A = rng.randrange(-(1 << 46), 1 << 46)
                rows.append((A, M + rng.randrange(-3, 1)))
            sign = 1 if rng.random() < .5 else -1
            rows[5] = (sign * ((1 << 48) - gap), M)
            vals = [Fraction(A) * Fraction(2) ** (m - 30) for A, m in rows]
            assert bi.epilogue_int(rows) == bi.quantize_tile(vals), (M, gap)


def test_idempotence():
    rng = np.random.default_rng(12)
    v = rng.standard_normal(576) * np.exp(rng.standard_normal(576))
    m, e = sim.tile_quantize(v)
    m2, e2 = sim.tile_quantize(sim.tile_decode(m, e))
    assert (m == m2).all() and (e == e2).all()


@pytest.mark.parametrize("name", ["G1", "G2", "NORM_W"])
def test_release_fixtures(name):
    """The reference's committed real-model BFP gammas: normalised tiles
    (max|m| in [2^14, 2^15]) and quantise(decode(.)) is the identity."""
    f = np.load(GOLDEN / "release_bfp.npz")
    m, e = f[f"{name}_m"], f[f"{name}_e"]
    m = m.reshape(-1, 16)
    amax = np.abs(m.astype(np.int32)).max(axis=1)
    assert ((amax >= 2 ** 14) & (amax <= 2 ** 15)).all()
    m2, e2 = sim.tile_quantize(sim.tile_decode(m, e))
    assert (m2 == m).all() and (e2 == e).all()


# ------------------------------------------------------------------ matvec
def _rand_bfp(rng, n, e_lo, e_hi, neg_edge=True):
    m = rng.integers(-32768, 32768, size=(n // 16, 16)).astype(np.int16)
    if neg_edge:
        m[0, 0] = -32768
    e = rng.integers(e_lo, e_hi + 1, size=n // 16).astype(np.int8)
    return m, e


@pytest.mark.parametrize("n_out,n_in,espread", [(16, 16, 3), (32, 64, 10), (48, 96, 60),
                                                (16, 160, 127)])
def test_matvec_vs_bigint(n_out, n_in, espread):
    rng = np.random.default_rng(n_out * 1000 + n_in + espread)
    x_m, x_e = _rand_bfp(rng, n_in, -espread // 2, espread // 2)
    W_m = rng.integers(-32768, 32768, size=(n_out, n_in // 16, 16)).astype(np.int16)
    W_m[0, :, :] = -32768          # S = 16 * 2^30 at the -32768 x -32768 corner
    W_e = rng.integers(-espread // 2, espread // 2 + 1, size=(n_out, n_in // 16)).astype(np.int8)
    A, M = sim.matvec_acc(x_m, x_e, W_m, W_e)
    rows = bi.matvec_rows(x_m.tolist(), x_e.tolist(), W_m.tolist(), W_e.tolist())
    assert [int(a) for a in A] == [a for a, _ in rows]
    assert [int(m) for m in M] == [m for _, m in rows]
    y = sim.matvec_hw_golden(x_m, x_e, W_m, W_e)
    m, e = sim.tile_quantize(y)
    bm, be = bi.matvec(x_m.tolist(), x_e.tolist(), W_m.tolist(), W_e.tolist())
    assert m.tolist() == bm and list(e) == be
    # the float-free epilogue of the HIP kernel equals the float path
    for g in range(n_out // 16):
        em, ee = bi.epilogue_int(rows[16 * g:16 * g + 16])
        assert em == bm[g] and ee == be[g]


def test_matvec_shift_drop_boundary():
    """A tile 47 below the row max is floor-shifted, 48 below is dropped."""
    x_m = np.zeros((3, 16), np.int16)
    x_e = np.array([0, 0, 0], np.int8)
    W_m = np.zeros((16, 3, 16), np.int16)
    W_e = np.zeros((16, 3), np.int8)
    x_m[:, 0] = 1
    W_m[0, 0, 0] = 1          # S=1 at E=100
    W_m[0, 1, 0] = -32768     # S=-32768 at E=53 -> shift 47 -> floor -> -1
    W_m[0, 2, 0] = 32767      # S=32767 at E=52 -> shift 48 -> dropped
    W_e[0] = [100, 53, 52]
    A, M = sim.matvec_acc(x_m, x_e, W_m, W_e)
    assert M[0] == 100 and A[0] == 1 - 1


def test_requantise_neg_full_scale():
    """Re-quantising a decoded tile whose max magnitude is the mantissa
    -32768 gives (round_half_even(m/2), e+1): the form fwd_layer's next
    matvec sees (full.py:264,283,287,291 quantise decoded values)."""
    m = np.zeros((1, 16), np.int16)
    m[0, :5] = [-32768, 3, -3, 5, 16383]
    e = np.array([4], np.int8)
    m2, e2 = sim.tile_quantize(sim.tile_decode(m, e))
    assert e2[0] == 5
    assert list(m2[0, :5]) == [-16384, 2, -2, 2, 8192]
    bm, be = bi.quantize_vec(bi.decode_vec(m.tolist(), e.tolist()))
    assert be == [5] and bm[0][:5] == [-16384, 2, -2, 2, 8192]


def test_epilogue_int_random():
    rng = random.Random(5)
    for _ in range(300):
        rows = [(rng.randint(-(1 << rng.randint(0, 46)), 1 << rng.randint(0, 46)),
                 rng.randint(-60, 60)) for _ in range(16)]
        if rng.random() < 0.1:
            rows = [(0, M) for _, M in rows]
        vals = [Fraction(A) * Fraction(2) ** (M - 30) for A, M in rows]
        assert bi.epilogue_int(rows) == bi.quantize_tile(vals)


# ------------------------------------------------- numpy / BLAS reductions
def test_pairwise_sum_matches_numpy():
    rng = np.random.default_rng(3)
    for n in list(range(1, 140)) + [255, 256, 576, 1536, 2047, 2048]:
        a = rng.standard_normal(n) * np.exp(rng.standard_normal(n) * 4)
        assert sim.pairwise_sum(a) == float(np.sum(a))
        assert sim.pairwise_sum(a * a) / n == float(np.mean(a * a))


def test_ddot_order_matches_blas():
    """np.dot of two 64-vectors (attention scores, full.py:278) is OpenBLAS
    ddot; the restated SkylakeX order must match it on this machine."""
    rng = np.random.default_rng(4)
    a, b = rng.standard_normal(64), rng.standard_normal(64)
    if sim.ddot_skx_order(a, b) != float(np.dot(a, b)):
        pytest.skip("this CPU's OpenBLAS ddot kernel is not the SkylakeX one")
    for _ in range(200):
        a, b = rng.standard_normal(64), rng.standard_normal(64) * 3
        assert sim.ddot_skx_order(a, b) == float(np.dot(a, b))


def test_rope_matches_complex_rotation():
    """rope_fp (full.py:250-258) rotates pair (j, j+32) by theta_j =
    pos / 10000**(2j/64): compare with numpy's complex exponential (an
    independent formulation) before quantisation, and check pos = 0 is the
    identity after it."""
    rng = np.random.default_rng(9)
    x = sim.fp_quantize_vec(rng.standard_normal(64))
    assert (sim.rope_fp(x, 0) == x).all()
    for pos in (1, 7, 100, 2047):
        z = (x[:32] + 1j * x[32:]) * np.exp(1j * pos * 10000.0 ** (-np.arange(32) / 32.0))
        want = np.concatenate([z.real, z.imag])
        got = sim.rope_fp(x, pos)
        # quantisation step of each 16-tile bounds the difference
        m, e = sim.tile_quantize(want)
        step = np.repeat(2.0 ** (e.astype(float) - 15), 16)
        assert (np.abs(got - want) <= step).all()
