"""CPU check of the int8 split behind the matrix-core batched matvec
(tinyllm-fpga_amd/csrc/bfp_mx.h): for int16 tiles W, x with
v = 256*vh + vl' + 128 (vh = v >> 8, vl' = (v & 255) - 128, both int8),
  sum_k W_k x_k = 65536*Phh + 256*(Phl + Plh + 128*sum Wh)
                  + (Pll + 128*sum Wl') + 128*sum x,
every int8 product sum fits the MFMA's int32 accumulator, and the part
below 65536*Phh fits int32, so the kernel can form the exact tile sum of
the engine (rtl/vc707/host/gen_smollm_blockfp_full.py:223-229).  The
check is the identity itself on random, extreme and alternating tiles,
computed in Python integers."""
import numpy as np


def _split(v):
    v = np.asarray(v, np.int64)
    return v >> 8, (v & 255) - 128


def _parts(W, x):
    Wh, Wl = _split(W)
    xh, xl = _split(x)
    assert Wh.min() >= -128 and Wh.max() <= 127 and Wl.min() >= -128 and Wl.max() <= 127
    phh = int((Wh * xh).sum())
    pc = int((Wh * xl).sum() + (Wl * xh).sum() + 128 * Wh.sum())
    pll = int((Wl * xl).sum() + 128 * Wl.sum())
    cx = 128 * int(np.asarray(x, np.int64).sum())
    return phh, pc, pll, cx


def test_split_identity_and_bounds():
    rng = np.random.default_rng(0)
    ext = [-32768, -32767, -256, -129, -128, -1, 0, 1, 127, 128, 255, 256, 32767]
    cases = [(rng.integers(-32768, 32768, 16), rng.integers(-32768, 32768, 16)) for _ in range(3000)]
    for a in (-32768, 32767):
        for b in (-32768, 32767):
            cases.append((np.full(16, a), np.full(16, b)))
    cases.append((np.array([-32768, 32767] * 8), np.array([32767, -32768] * 8)))
    cases += [(rng.choice(ext, 16), rng.choice(ext, 16)) for _ in range(2000)]
    worst = 0
    for W, x in cases:
        phh, pc, pll, cx = _parts(W, x)
        lo = (pc << 8) + pll + cx
        assert 65536 * phh + lo == int((np.asarray(W, np.int64) * np.asarray(x, np.int64)).sum())
        assert abs(phh) <= 2 ** 18 and abs(pc) < 2 ** 20 and abs(pll) <= 2 ** 19
        assert abs(lo) < 2 ** 31   # the 32-bit low part of the kernel
        worst = max(worst, abs(lo))
    assert worst < 2 ** 29


def _mfma32(a, b):
    """One 32-deep int8 product sum as v_mfma_i32_16x16x32_i8 forms it for a
    (row, sequence) pair: k-groups 0-1 and 2-3 hold the 16-element tile
    twice; a and b are (32,) int8 operands."""
    a, b = np.asarray(a, np.int64), np.asarray(b, np.int64)
    assert a.min() >= -128 and a.max() <= 127 and b.min() >= -128 and b.max() <= 127
    return int((a * b).sum())


def test_select_free_doubled_form():
    """The select-free form of the kernels: every operand holds both copies
    of the tile except the constant k1 (ones in the first copy, zeros in the
    second), so each 32-deep product is twice the tile's, and with
    sum x = 256 sum xh + sum xl' + 2048
      2 S = 65536 (P(Wh, xh) + P(Wh, k1) + P(k1, xh) + 8)
            + 256 (P(Wh, xl') + P(Wl', xh) + P(Wl', k1) + P(k1, xl'))
            + P(Wl', xl')
    with P the MFMA's 32-deep sum; floor(S / 2^d) = floor(2S / 2^(d+1)).
    Each accumulator and the 32-bit low part fit int32."""
    rng = np.random.default_rng(1)
    ext = [-32768, -32767, -256, -129, -128, -1, 0, 1, 127, 128, 255, 256, 32767]
    cases = [(rng.integers(-32768, 32768, 16), rng.integers(-32768, 32768, 16)) for _ in range(2000)]
    for a in (-32768, 32767):
        for b in (-32768, 32767):
            cases.append((np.full(16, a), np.full(16, b)))
    cases += [(rng.choice(ext, 16), rng.choice(ext, 16)) for _ in range(2000)]
    k1 = np.array([1] * 16 + [0] * 16)
    for W, x in cases:
        Wh, Wl = _split(W)
        xh, xl = _split(x)
        dup = lambda v: np.concatenate([v, v])   # noqa: E731
        hh = _mfma32(dup(xh), k1) + 8 + _mfma32(dup(Wh), dup(xh)) + _mfma32(dup(Wh), k1)
        cr = _mfma32(dup(xl), k1) + _mfma32(dup(Wh), dup(xl)) + _mfma32(dup(Wl), dup(xh)) + _mfma32(dup(Wl), k1)
        ll = _mfma32(dup(Wl), dup(xl))
        S = int((np.asarray(W, np.int64) * np.asarray(x, np.int64)).sum())
        lo = (cr << 8) + ll
        assert 65536 * hh + lo == 2 * S
        assert abs(hh) < 2 ** 20 and abs(cr) < 2 ** 22 and abs(ll) < 2 ** 20 and abs(lo) < 2 ** 31
        for d in (0, 1, 5, 16, 17, 33, 47):
            assert (2 * S) >> (d + 1) == S >> d
