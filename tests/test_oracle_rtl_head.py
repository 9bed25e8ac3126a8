"""The RTL decode head's composition in the oracle (oracle/bfp_rtl.py:rtl_head,
smollm_decode_head_bfp.sv:303-430) pinned independently of its restatement:

* every logit (m, e) equals the exact dot product of the RMSNorm engine's
  output with that embedding row -- computed here with Python integers from
  the decoded BFP operands -- within the matvec engine's truncation bound:
  one unit at the largest tile scale per tile fold (each alignment shift
  floors) plus one unit of the 16-bit result (the final normalise floors);
* the token is the exact argmax wherever the top two exact logits are
  further apart than twice that bound plus bfp_gt's alignment floor;
* the token is the first of equal maxima (strict > in the running argmax).
"""
import numpy as np
import pytest

from oracle import bfp_rtl as rtl
from oracle import bfp_sim as sim

TILE = 16


def _exact_logits(xm, xe, Wm, We):
    """Exact sum_k x_k W_k per row as (numerator, shift): value = num * 2^-S."""
    nt = We.shape[1]
    xm = np.asarray(xm, np.int64).reshape(nt, TILE)
    S = 60 + 2 * 128   # common fixed-point shift, deep enough for every tile scale
    out = []
    for r in range(Wm.shape[0]):
        num = 0
        for t in range(nt):
            s = int(np.dot(xm[t], Wm[r, t].astype(np.int64)))
            sh = int(xe[t]) + int(We[r, t]) - 30 + S      # value of one unit of s: 2^(E - 30)
            num += s << sh
        out.append(num)
    return out, S


@pytest.mark.parametrize("D,V,seed", [(128, 256, 1), (576, 160, 2), (64, 512, 3)])
def test_rtl_head_logits_and_token_against_exact_arithmetic(D, V, seed):
    rng = np.random.default_rng(seed)
    embed = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    emb = rtl.embed_q(embed)
    norm_w = sim.fp_quantize_vec(1.0 + 0.05 * rng.standard_normal(D))
    checked_tokens = 0
    for trial in range(6):
        h_m, h_e = sim.tile_quantize(rng.standard_normal(D) * (0.5 + trial))
        lm, le, tok = rtl.rtl_head(h_m.reshape(-1), h_e, norm_w, emb)
        g_m, g_e = sim.tile_quantize(np.asarray(norm_w, np.float64))
        xm, xe = rtl.rtl_rmsnorm(h_m.reshape(-1), h_e, g_m.reshape(-1), g_e)
        Wm, We = emb
        nt = D // TILE
        num, S = _exact_logits(xm, xe, Wm, We)
        bounds = []
        for r in range(V):
            emaxr = max(int(xe[t]) + int(We[r, t]) for t in range(nt))
            # |logit - exact| <= nt * 2^(emaxr - 30) + 2^(le - 15), in units of 2^-S
            b = nt * (1 << (emaxr - 30 + S)) + (1 << (int(le[r]) - 15 + S))
            got = int(lm[r]) << (int(le[r]) - 15 + S)
            assert abs(got - num[r]) <= b, (trial, r)
            bounds.append(b)
        order = np.argsort(np.array([float(v) for v in num]))[::-1]
        top, second = int(order[0]), int(order[1])
        cmp_floor = 1 << (max(int(le[top]), int(le[second])) - 15 + S)
        if num[top] - num[second] > 2 * max(bounds) + 2 * cmp_floor:
            assert tok == top, trial
            checked_tokens += 1
    assert checked_tokens >= 3


def test_rtl_argmax_first_of_equal_maxima():
    m = np.array([3, 7, 7, 1] * 8, np.int16)
    e = np.zeros(32, np.int8)
    assert rtl.rtl_argmax(m, e) == 1
    m2 = m.copy()
    m2[17] = 7                       # the same maximum again in the second chunk
    assert rtl.rtl_argmax(m2, e) == 1
    m2[20] = 8
    assert rtl.rtl_argmax(m2, e) == 20
