"""The float64 identities the long-context attention kernel (k_attn, AV
phase) relies on to form numpy's `p[t] * V[t]` (full.py:280-281) with one
multiply per product.  V[t] holds BFP values m * 2^(e-15) (exact in
float64), so the reference product is one rounding of the real
p * m * 2^(e-15).

* ps = p * 2^(e-15) is exact whenever it is a normal number (or p = 0), so
  ps * m is the same single rounding: bit-identical on every input of that
  kind;
* when ps falls below the normal range the two can differ: the kernel's
  slow path (p * (m * 2^(e-15))) exists for that case, and this test shows
  the fast form would be wrong there;
* positions past the sum are fed as products of +-0: adding +-0 leaves a
  float64 sum that started at +0.0 unchanged.
"""
import numpy as np


def _cases(rng, n):
    p = rng.random(n) ** rng.integers(1, 40, n)            # (0, 1], many tiny
    p[rng.random(n) < 0.05] = 0.0
    k = 20_000                                             # straddle the ps underflow edge
    p[:k] = np.ldexp(1.0 + rng.random(k), -rng.integers(860, 1000, k))
    e = rng.integers(-127, 128, n)
    e[:k] = rng.integers(-127, -100, k)
    m = rng.integers(-32768, 32768, n)
    return p, e, m


def test_one_multiply_product_equals_reference_when_ps_normal():
    rng = np.random.default_rng(3)
    p, e, m = _cases(rng, 400_000)
    ref = p * (m.astype(np.float64) * np.ldexp(1.0, e - 15))
    ps = p * np.ldexp(1.0, e - 15)
    fast = ps * m.astype(np.float64)
    normal = (ps >= np.finfo(np.float64).tiny) | (p == 0.0)
    assert normal.sum() > 300_000
    assert np.array_equal(fast[normal].view(np.int64), ref[normal].view(np.int64))
    # outside that range the fast form is not the reference: the guard matters
    sub = ~normal
    assert sub.sum() > 1000
    assert not np.array_equal(fast[sub].view(np.int64), ref[sub].view(np.int64))


def test_adding_signed_zero_is_the_identity_on_the_running_sum():
    rng = np.random.default_rng(4)
    terms = rng.normal(size=(200, 64)) * np.ldexp(1.0, rng.integers(-60, 60, (200, 64)))
    terms[rng.random(terms.shape) < 0.1] = -0.0
    acc = np.zeros(64)                                     # +0.0, as in the kernel
    for t in range(terms.shape[0]):
        acc = acc + terms[t]
        assert not np.any((acc == 0) & np.signbit(acc))    # the sum is never -0
        for z in (0.0, -0.0):
            assert np.array_equal((acc + z).view(np.int64), acc.view(np.int64))
