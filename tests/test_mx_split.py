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
