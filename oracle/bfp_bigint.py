"""Float-free brute-force model of the BFP integer semantics -- TEST
INFRASTRUCTURE ONLY (same import rule as ``oracle/bfp_sim.py``).

Everything here uses Python integers and ``fractions.Fraction``; nothing
goes through numpy, log2 or float rounding.  It is the independent check
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


def rne(q: Fraction) -> int:
    """Round a rational to the nearest integer, ties to even."""
    f = math.floor(q)
    r = q - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1):
        return f + 1
    return f


def quantize_tile(vals):
    """Exact BFP quantisation of 16 values (floats or Fractions).

    e = clip(floor(log2(max|v|)) + 1, -127, 127), or -127 for an all-zero
    tile (the reference floors max|v| at 1e-300, whose log2 is < -127);
    m = clip(rne(v * 2**(15-e)), -32768, 32767).
    """
    fr = [Fraction(v) for v in vals]
    amax = max(abs(v) for v in fr)
    if amax == 0:
        e = -127
    else:
        e = min(127, max(-127, floor_log2(amax) + 1))
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

    e = clip(max over A != 0 of (msb|A| + M - 30) + 1, -127, 127), -127 if all
    rows are zero; m = clip(rne(A * 2**(M - 15 - e))) computed with a floor
    shift plus a round-half-even correction.
    """
    assert len(rows) == TILE
    L = [abs(A).bit_length() - 1 + M - 30 for A, M in rows if A != 0]
    e = -127 if not L else min(127, max(-127, max(L) + 1))
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
