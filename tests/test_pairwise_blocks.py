"""CPU check of the leaf decomposition behind the device's float64
pairwise sum (tinyllm-fpga_amd/csrc/bfp_f64.h pairwise_sum_block): numpy
splits a range longer than 128 at n/2 rounded down to a multiple of 8, so
each 64-element block [64g, 64g+64) holds at most one leaf start; the group
owning block g sums the leaf with numpy's 8 accumulators and the leaves are
combined by the same splits.  The scheme, run in Python float64, must equal
numpy's own np.add.reduce bit for bit for every n the kernels use
(1..4096): RMSNorm over D, the softmax denominator over pos+1 scores, the
final norm."""
import numpy as np


def _leaf(a, lo, n):
    if n < 8:
        r = 0.0
        for i in range(n):
            r += a[lo + i]
        return r
    acc = [a[lo + j] for j in range(8)]
    top = n - n % 8
    for i in range(8, top, 8):
        for j in range(8):
            acc[j] += a[lo + i + j]
    res = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]))
    for i in range(top, n):
        res += a[lo + i]
    return res


def _block_scheme(a):
    n = len(a)
    ng = (n + 63) // 64
    leafbuf = {}
    for g in range(ng):
        e = min(g * 64 + 63, n - 1)
        flo, fn = 0, n
        while fn > 128:
            n2 = fn // 2
            n2 -= n2 % 8
            if e < flo + n2:
                fn = n2
            else:
                flo, fn = flo + n2, fn - n2
        if flo >= g * 64:
            assert g not in leafbuf
            leafbuf[g] = _leaf(a, flo, fn)

    def comb(lo, m):
        if m > 128:
            n2 = m // 2
            n2 -= n2 % 8
            return comb(lo, n2) + comb(lo + n2, m - n2)
        return leafbuf[lo >> 6]
    return 0.0 + comb(0, n)


def test_block_scheme_equals_numpy():
    rng = np.random.default_rng(3)
    sizes = list(range(1, 300)) + [576, 1536, 1728] + list(range(300, 4097, 37)) + [4095, 4096]
    for n in sizes:
        a = rng.standard_normal(n) * np.exp(rng.uniform(-20, 20, n))
        a = [float(v) for v in a]
        want = float(np.add.reduce(np.array(a)))
        assert _block_scheme(a) == want, n
