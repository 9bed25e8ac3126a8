"""CPU pins of the bounded decode head's arithmetic (k_embq_build,
k_head_norm's quantised hidden, k_headq_mx, k_headq_pick in
csrc/bfp_layer.hip), restated here in numpy and checked against exact
rational arithmetic:

- the split-byte identity that forms an int16 dot product from four int8
  matrix-core products;
- the interval [A - B, A + B] around each logit holds both the exact real
  dot product h.e_r and the float64 logit the head forms (the FMA chains
  of k_head_logits over k = 64i + 4l + c, then the 16-lane butterfly,
  full.py:438-440), each FMA rounded once;
- the block selection (largest lower bound T; blocks whose upper bound
  reaches T) keeps the first-index argmax of those logits."""
from fractions import Fraction

import numpy as np
import pytest


def _split(v):
    v = v.astype(np.int64)
    hi = v >> 8
    lo = (v & 255) - 128
    return hi, lo


def _scale_exp(mx):
    """The power-of-two exponent that puts mx in (16383, 32767]."""
    if mx == 0.0:
        return 0
    e = int(np.frexp(mx)[1]) - 1 - 14
    if np.ldexp(mx, -e) > 32767.0:
        e += 1
    return e


def _quant(v):
    e = _scale_exp(float(np.abs(v).max()))
    q = np.rint(np.ldexp(v.astype(np.float64), -e)).astype(np.int64)
    assert np.abs(q).max() <= 32767
    return e, q


def _bounds(h, E):
    """Lower and upper bound of every row's logit, as k_headq_mx forms them."""
    eh, qh = _quant(h)
    h1 = float(np.abs(h).sum()) * (1.0 + 2.0 ** -40)
    lo = np.empty(len(E))
    hi = np.empty(len(E))
    for r, e in enumerate(E):
        emax = float(np.abs(e).max())
        if emax == 0.0:
            lo[r] = hi[r] = 0.0
            continue
        er, qe = _quant(e)
        S = int(qh @ qe)
        A = np.ldexp(float(S), er + eh)
        B = np.ldexp(h1, er - 1) + np.ldexp(float(np.abs(qe).sum()), er + eh - 1) + 2.0 ** -45 * h1 * emax
        B = B * (1.0 + 2.0 ** -20) + 2.0 ** -50 * abs(A)
        lo[r] = A - B
        hi[r] = A + B
    return lo, hi


def _fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))   # one rounding


def _head_logit(h, e):
    """k_head_logits' order: lane l sums k = 64i + 4l + c (i, then c, ascending)
    with FMA; the 16 partials are added q and q + 8, then 4, 2, 1 apart."""
    D = len(h)
    p = []
    for l in range(16):
        acc = 0.0
        for i in range(D // 64):
            for c in range(4):
                k = 64 * i + 4 * l + c
                acc = _fma(float(e[k]), float(h[k]), acc)
        p.append(acc)
    for m in (8, 4, 2, 1):
        p = [p[q] + p[q ^ m] for q in range(16)]
    return p[0]


def test_split_identity():
    rng = np.random.default_rng(5)
    for D in (32, 576, 1728):
        for kind in ("random", "extreme"):
            if kind == "random":
                W = rng.integers(-32768, 32768, D)
                x = rng.integers(-32768, 32768, D)
            else:
                W = rng.choice([-32768, -32767, -1, 0, 1, 255, 256, 32767], D)
                x = rng.choice([-32768, -32767, -1, 0, 1, 255, 256, 32767], D)
            wh, wl = _split(W)
            xh, xl = _split(x)
            for v in (wh, wl, xh, xl):
                assert v.min() >= -128 and v.max() <= 127
            P = lambda a, b: int(a @ b)   # noqa: E731  (each < 2^24 in magnitude)
            for a, b in ((wh, xh), (wh, xl), (wl, xh), (wl, xl)):
                assert abs(P(a, b)) < 2 ** 24 * (D // 576 + 1)
            S = (65536 * P(wh, xh) + 256 * (P(wh, xl) + P(wl, xh)) + P(wl, xl)
                 + 128 * (int(W.sum()) + int(x.sum())) - 16384 * D)
            assert S == int(W.astype(np.int64) @ x.astype(np.int64))


@pytest.mark.parametrize("D", [64, 192, 576])
def test_bounds_hold_exact_and_float64_logits(D):
    rng = np.random.default_rng(D)
    rows = []
    for kind in range(6):
        e = (rng.standard_normal(D) * 0.02).astype(np.float32)
        if kind == 1:
            e *= np.float32(1e-30)
        elif kind == 2:
            e *= np.float32(3e4)
        elif kind == 3:
            e[rng.integers(0, D, D // 2)] = 0.0
        elif kind == 4:
            e = np.nextafter(e, np.float32(np.inf))
        elif kind == 5:
            e[:] = np.float32(0.0)
            e[3] = np.float32(-7.5e-3)
        rows.append(e)
    E = np.stack(rows)
    for trial in range(4):
        h = rng.standard_normal(D) * (1.0 + 0.05 * rng.standard_normal(D))
        if trial == 1:
            h *= 1e-3
        elif trial == 2:
            h[: D // 2] = 0.0
        elif trial == 3:
            h = E[0].astype(np.float64) * 50.0
        lo, hi = _bounds(h, E)
        for r in range(len(E)):
            exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(h, E[r]))
            L = _head_logit(h, E[r])
            assert Fraction(lo[r]) <= exact <= Fraction(hi[r]), (trial, r)
            assert lo[r] <= L <= hi[r], (trial, r)


def test_block_selection_keeps_first_argmax():
    D, V = 64, 256
    rng = np.random.default_rng(9)
    E = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    E[21] = E[50] = E[7] * np.float32(40.0)          # a tie across blocks
    E[130] = np.nextafter(E[129], np.float32(np.inf))  # 1 ulp apart, one block
    E[129] *= np.float32(1.0)
    E[64:80] = 0.0                                   # a zero block
    for trial in range(12):
        h = rng.standard_normal(D)
        if trial % 3 == 1:
            h = E[7].astype(np.float64) * (1.0 + 0.01 * trial)
        elif trial % 3 == 2:
            h = E[129].astype(np.float64) * 30.0 + 1e-6 * rng.standard_normal(D)
        lo, hi = _bounds(h, E)
        blo = lo.reshape(-1, 16).max(1)
        bhi = hi.reshape(-1, 16).max(1)
        T = blo.max()
        cand = [c for c in range(V // 16) if bhi[c] >= T]
        L = np.array([_head_logit(h, E[r]) for r in range(V)])
        best, besti = -np.inf, None
        for c in cand:
            for r in range(16 * c, 16 * c + 16):
                if L[r] > best:
                    best, besti = L[r], r
        assert besti == int(np.argmax(L)), trial
        assert len(cand) <= 3, (trial, len(cand))
