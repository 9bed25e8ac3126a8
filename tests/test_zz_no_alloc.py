"""The allocation-free entry point bfp_rtl_argmax_static_d against the
workspace form bfp_rtl_argmax_d (the same kernel over caller-allocated
scratch), through the C ABI: two calls in a row, the second smaller, so the
static scratch holds the first call's entries when the second runs; and
the size limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(rng, batch, n):
    m = rng.integers(-32768, 32768, size=batch * n).astype(np.int16)
    e = rng.integers(-12, 13, size=batch * n).astype(np.int8)
    # candidates that tie or nearly tie after the bfp_gt alignment
    for b in range(batch):
        i, j = rng.integers(n, size=2)
        m[b * n + i], e[b * n + i] = 30000, 14
        m[b * n + j], e[b * n + j] = 15000, 15
    return m, e


def test_argmax_static_matches_workspace_form(gpu):
    from bfp import _dev
    from bfp._lib import BfpError, call
    rng = np.random.default_rng(61)
    for batch, n in ((64, 49152), (3, 4096)):
        print(f"[no-alloc] rtl argmax batch {batch} n {n}", flush=True)
        m, e = _case(rng, batch, n)
        dm, de = _dev.to_dev(m), _dev.to_dev(e)
        work = _dev.empty(3 * batch * (n // 16), "int32")
        want, got = _dev.zeros(batch, "int32"), _dev.zeros(batch, "int32")
        call("bfp_rtl_argmax_d", _dev.ptr(dm), _dev.ptr(de), n, batch, _dev.ptr(work),
             _dev.ptr(want), _dev.stream())
        call("bfp_rtl_argmax_static_d", _dev.ptr(dm), _dev.ptr(de), n, batch, _dev.ptr(got),
             _dev.stream())
        assert (_dev.to_host(got) == _dev.to_host(want)).all()
    # beyond the static scratch: refused before any launch
    with pytest.raises(BfpError):
        call("bfp_rtl_argmax_static_d", _dev.ptr(dm), _dev.ptr(de), 16 * 262145, 1,
             _dev.ptr(got), _dev.stream())
