"""Float-free brute-force model of the BFP integer semantics -- TEST
INFRASTRUCTURE ONLY (same import rule as ``oracle/bfp_sim.py``).

Everything here uses Python integers, ``fractions.Fraction`` and
``decimal`` logarithms at 80 digits; nothing goes through numpy or libm.  It is the independent check
that pins ``bfp_sim.tile_quantize`` and ``bfp_sim.matvec_hw_golden``
(reference ``rtl/vc707/host/gen_smollm_blockfp_full.py:90-97,217-233``) on
small inputs, and it is the statement of the exact-integer output epilogue
that the HIP matvec kernel implements.
"""
from __future__ import annotations

import math
from fractions import Fraction

TILE = 16
ALIGN_MAX = 47


def floor_log2(q: Fraction) -> int:
    """floor(log2(q)) for q > 0, exactly."""
    assert q > 0
    n, d = q.numerator, q.denominator
    k = n.bit_length() - d.bit_length()
    # 2**k <= n/d < 2**(k+1) after the adjustment below
    if (n << max(0, -k)) < (d << max(0, k)):
        k -= 1
    return k


def cr_log2(q: Fraction) -> float:
    """log2(q) rounded to the nearest double, as a correctly rounded log2
    (numpy's np.log2) returns it: ln via ``decimal`` at 80 digits, then
    Python's correctly rounded Fraction -> float conversion.  An exact log2
    is never within 1e-60 of a rounding midpoint for these inputs."""
    from decimal import Decimal, localcontext
    assert q > 0
    with localcontext() as ctx:
        ctx.prec = 80
        v = (Decimal(q.numerator).ln() - Decimal(q.denominator).ln()) / Decimal(2).ln()
    return float(Fraction(v))


def np_floor_log2(q: Fraction) -> int:
    """floor(np.log2(q)): the exact floor_log2, plus one where the rounded
    logarithm reaches the next integer (q a few doubles below a power of
    two; gen_smollm_blockfp_full.py:92 takes floor(np.log2(max|v|)))."""
    return math.floor(cr_log2(q))


def log2_up_ulps(k: int) -> int:
    """n_up(k): for a double a in [2^(k-1), 2^k), np.log2(a) rounds to k
    exactly when a >= 2^k (1 - n_up(k) 2^-53).  Closed form floor(2^p ln 2),
    p = floor(log2|k|) (less one for a power of two k > 0); 0 for k = 0 and
    p <= 0.  The kernels use the same form (bfp_device.h: log2_up_ulps); the
    tests check it against np.log2 and against np_floor_log2."""
    if k == 0:
        return 0
    a = abs(k)
    p = a.bit_length() - 1
    if k > 0 and a & (a - 1) == 0:
        p -= 1
    if p <= 0:
        return 0
    return int(0xB17217F7D1CF79AB >> (64 - min(p, 10)))


def rne(q: Fraction) -> int:
    """Round a rational to the nearest integer, ties to even."""
    f = math.floor(q)
    r = q - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1):
        return f + 1
    return f


def quantize_tile(vals):
    """Exact BFP quantisation of 16 values (floats or Fractions).

    e = clip(floor(np.log2(max|v|)) + 1, -127, 127) with a correctly
    rounded log2 (``np_floor_log2``), or -127 for an all-zero tile (the
    reference floors max|v| at 1e-300, whose log2 is < -127);
    m = clip(rne(v * 2**(15-e)), -32768, 32767).
    """
    fr = [Fraction(v) for v in vals]
    amax = max(abs(v) for v in fr)
    if amax == 0:
        e = -127
    else:
        k = floor_log2(amax)
        # the decimal logarithm is only needed where rounding can reach k+1
        if amax >= Fraction(2) ** (k + 1) * (1 - Fraction(1024, 2 ** 53)):
            k = np_floor_log2(amax)
        e = min(127, max(-127, k + 1))
    m = [min(32767, max(-32768, rne(v * Fraction(2) ** (15 - e)))) for v in fr]
    return m, e


def quantize_vec(vals):
    assert len(vals) % TILE == 0
    ms, es = [], []
    for i in range(0, len(vals), TILE):
        m, e = quantize_tile(vals[i:i + TILE])
        ms.append(m)
        es.append(e)
    return ms, es


def decode_vec(ms, es):
    out = []
    for m, e in zip(ms, es):
        out.extend(Fraction(mi) * Fraction(2) ** (e - 15) for mi in m)
    return out


def matvec_rows(x_m, x_e, W_m, W_e):
    """Per-row (A, M) of the reference matvec with Python ints.

    x_m: list of nt lists of 16 ints; x_e: nt ints; W_m[o][t][k]; W_e[o][t].
    """
    rows = []
    for o in range(len(W_m)):
        S = [sum(int(x_m[t][k]) * int(W_m[o][t][k]) for k in range(TILE)) for t in range(len(x_e))]
        E = [int(x_e[t]) + int(W_e[o][t]) for t in range(len(x_e))]
        M = max(E)
        A = 0
        for s, ee in zip(S, E):
            sh = M - ee
            if sh <= ALIGN_MAX:
                A += s >> sh          # Python >> on ints is floor division
        A = max(-(1 << 47), min((1 << 47) - 1, A))
        rows.append((A, M))
    return rows


def matvec(x_m, x_e, W_m, W_e):
    """Reference matvec output as exact rationals, re-quantised over 16-row
    tiles, returned as (m tiles, e list)."""
    rows = matvec_rows(x_m, x_e, W_m, W_e)
    vals = [Fraction(A) * Fraction(2) ** (M - 30) for A, M in rows]
    return quantize_vec(vals)


def epilogue_int(rows):
    """The float-free output epilogue the HIP kernel uses, for one 16-row
    group given per-row (A, M): identical to quantize_tile of A*2**(M-30).

    Per row with A != 0: L = msb|A| + M - 30 = floor(log2|y|), and u = 1 when
    np.log2(|y|) rounds up to L + 1, i.e. (2^(b+1) - |A|) 2^(52-b) <= n_up(L+1)
    with b = msb|A| (|y| within n_up doubles below 2^(L+1)).
    e = clip(max of (L + u) over the rows + 1, -127, 127), where the max takes
    u from a row of the largest L; -127 if all rows are zero;
    m = clip(rne(A * 2**(M - 15 - e))) computed with a floor shift plus a
    round-half-even correction.
    """
    assert len(rows) == TILE
    keys = []
    for A, M in rows:
        if A == 0:
            continue
        b = abs(A).bit_length() - 1
        L = b + M - 30
        gap = (2 << b) - abs(A)
        u = 1 if b <= 52 and (gap << (52 - b)) <= log2_up_ulps(L + 1) else 0
        keys.append(2 * L + u)
    if not keys:
        e = -127
    else:
        k = max(keys)
        e = min(127, max(-127, (k >> 1) + (k & 1) + 1))
    m = []
    for A, M in rows:
        s = e + 15 - M            # right-shift amount
        if s <= 0:
            v = A << (-s)
        else:
            q = A >> s
            r = A - (q << s)
            h = 1 << (s - 1)
            v = q + (1 if (r > h or (r == h and (q & 1))) else 0)
        m.append(min(32767, max(-32768, v)))
    return m, e
