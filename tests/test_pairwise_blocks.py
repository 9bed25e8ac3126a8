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


def _equal_leaves(n):
    """(nl, L) when numpy's splits of n give nl <= 8 equal leaves of L
    elements, L % 8 == 0 (csrc/bfp_f64.h pw_equal_leaves), else None."""
    nl, L = 1, n
    while L > 128:
        n2 = L // 2
        n2 -= n2 % 8
        if 2 * n2 != L:
            return None
        L, nl = n2, nl * 2
    return (nl, L) if nl <= 8 and L % 8 == 0 and L >= 8 else None


def _wave_scheme(a, nl, L):
    """csrc/bfp_f64.h sum_sq_wave on 64 lanes: lane 8f + j runs accumulator
    j of leaf f; quad swaps i^1, i^2, the 8-lane half-mirror (i <-> 7-i),
    then the 16-lane mirror (i <-> 15-i) and the 16- and 32-lane swaps;
    lane 0's value, plus numpy's initial 0.0."""
    lanes = []
    for lane in range(64):
        f, j = lane >> 3, lane & 7
        base = (f if f < nl else 0) * L + j
        r = a[base]
        for k in range(1, L // 8):
            r = r + a[base + 8 * k]
        lanes.append(r)

    def step(partner):
        return [lanes[i] + lanes[partner(i)] for i in range(64)]
    lanes = step(lambda i: i ^ 1)
    lanes = step(lambda i: i ^ 2)
    lanes = step(lambda i: (i & ~7) | (7 - (i & 7)))
    if nl >= 2:
        lanes = step(lambda i: (i & ~15) | (15 - (i & 15)))
    if nl >= 4:
        lanes = step(lambda i: i ^ 16)
    if nl >= 8:
        lanes = step(lambda i: i ^ 32)
    return 0.0 + lanes[0]


def test_wave_scheme_equals_numpy():
    """Every D % 64 == 0 up to 1024 has numpy leaves of the wave form, and the
    wave's accumulators and butterfly give np.add.reduce's bits; 1536 (FFN)
    does not (it keeps the block-wide sum).  Squares of BFP values like the
    RMSNorm's, plus wide-range and cancelling inputs."""
    rng = np.random.default_rng(11)
    for D in range(64, 1025, 64):
        nl_L = _equal_leaves(D)
        assert nl_L is not None, D
        nl, L = nl_L
        assert nl * L == D
        for trial in range(20):
            if trial % 3 == 0:
                x = rng.integers(-32768, 32768, D) * 2.0 ** rng.integers(-40, 10, D // 16).repeat(16)
                a = x * x
            elif trial % 3 == 1:
                a = rng.standard_normal(D) * 10.0 ** rng.integers(-8, 8, D)
            else:
                a = rng.standard_normal(D)
            want = np.add.reduce(a)
            got = _wave_scheme(a, nl, L)
            assert np.float64(got).view(np.int64) == np.float64(want).view(np.int64), (D, trial)
    assert _equal_leaves(576) == (8, 72)
    assert _equal_leaves(1536) is None


def _wave256_scheme(a):
    """csrc/bfp_f64.h pairwise_sum_wave256 on 64 lanes: up to three leaves
    (numpy's split of n > 128, and of a right part longer than 128), lane
    group k = lane / 8 on leaf k: accumulator j = lane % 8 over the leaf's
    elements below its last multiple of 8, quad swaps i^1, i^2 and the
    8-lane half-mirror, then the leftover elements in order (a leaf of
    fewer than 8: 0.0 plus its elements); lanes 0, 8, 16 combined as
    L0, L0 + L1 or L0 + (L1 + L2), plus numpy's initial 0.0."""
    n = len(a)
    n2, nr, m2 = n, 0, 0
    if n > 128:
        n2 = n // 2 - (n // 2) % 8
        nr = n - n2
        m2 = nr
        if nr > 128:
            m2 = nr // 2 - (nr // 2) % 8
    lanes, fns, flos = [], [], []
    for lane in range(64):
        k, j = lane >> 3, lane & 7
        flo = 0 if k == 0 else (n2 if k == 1 else n2 + m2)
        fn = n2 if k == 0 else (m2 if k == 1 else (nr - m2 if k == 2 else 0))
        top = fn - fn % 8
        r = a[flo + j] if j < top else 0.0
        t = flo + 8 + j
        while t < flo + top:
            r = r + a[t]
            t += 8
        lanes.append(r)
        fns.append(fn)
        flos.append(flo)

    def step(partner):
        return [lanes[i] + lanes[partner(i)] for i in range(64)]
    lanes = step(lambda i: i ^ 1)
    lanes = step(lambda i: i ^ 2)
    lanes = step(lambda i: (i & ~7) | (7 - (i & 7)))
    res = []
    for lane in range(64):
        fn, flo = fns[lane], flos[lane]
        top = fn - fn % 8
        if fn < 8:
            r = 0.0
            for t in range(fn):
                r += a[flo + t]
        else:
            r = lanes[lane]
            for t in range(flo + top, flo + fn):
                r += a[t]
        res.append(r)
    root = res[0]
    if n > 128:
        root = root + (res[8] + res[16]) if nr > 128 else root + res[8]
    return 0.0 + root


def test_wave256_scheme_equals_numpy():
    """The one-wave softmax denominator of the grouped attention
    (tinyllm-fpga_amd/csrc/bfp_attn_grp.h) equals np.add.reduce bit for bit
    for every n of 1..256 (softmax terms in (0, 1], wide-range and
    cancelling inputs); n = 255 has three leaves (120, 64, 71)."""
    rng = np.random.default_rng(12)
    for n in range(1, 257):
        for trial in range(6):
            if trial % 3 == 0:
                a = np.exp(-np.abs(rng.standard_normal(n)) * 3.0)
            elif trial % 3 == 1:
                a = rng.standard_normal(n) * 10.0 ** rng.integers(-8, 8, n)
            else:
                a = rng.standard_normal(n)
            want = np.add.reduce(a)
            got = _wave256_scheme([float(v) for v in a])
            assert np.float64(got).view(np.int64) == np.float64(want).view(np.int64), (n, trial)
