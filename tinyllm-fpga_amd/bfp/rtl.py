"""The FPGA engines' RTL-exact leaf ops on the GPU (libbfp.so bfp_rtl_*).

Names follow the reference's per-op golden generators
(rtl/vc707/host/gen_{matvec,rmsnorm,rope,softmax,swiglu,residual}_bfp_golden.py)
and the decode head's argmax (rtl/vc707/src/smollm/smollm_decode_head_bfp.sv).
numpy in, numpy out.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _dev
from ._lib import call, lib

TILE = 16
_TABLES = {}


def tables(head_dim=64, base=10000.0):
    """(exp_lut uint16[1024], silu_lut int16[65536], freq_q31 uint32[hd/2]),
    built by the library on the host."""
    key = (head_dim, base)
    if key not in _TABLES:
        el = np.zeros(1024, np.uint16)
        sl = np.zeros(65536, np.int16)
        fq = np.zeros(head_dim // 2, np.uint32)
        call("bfp_rtl_tables", el.ctypes.data, sl.ctypes.data, fq.ctypes.data, head_dim,
             C.c_double(base))
        _TABLES[key] = (el, sl, fq)
    return _TABLES[key]


def _d(a, dt):
    return _dev.to_dev(np.ascontiguousarray(np.asarray(a, dtype=dt).reshape(-1)))


def golden_matvec(x_m, x_e, W_m, W_e):
    """matvec_bfp_engine.sv: W_m (rows, in/16, 16), W_e (rows, in/16) ->
    per-row (m, e)."""
    W_m = np.asarray(W_m)
    n_out, nt = W_m.shape[0], W_m.shape[1]
    ym, ye = _dev.empty(n_out, "int16"), _dev.empty(n_out, "int8")
    xm, xe, wm, we = _d(x_m, np.int16), _d(x_e, np.int8), _d(W_m, np.int16), _d(W_e, np.int8)
    call("bfp_rtl_matvec_d", xm.data_ptr(), xe.data_ptr(), wm.data_ptr(), we.data_ptr(), n_out,
         nt * TILE, ym.data_ptr(), ye.data_ptr(), _dev.stream())
    return _dev.to_host(ym), _dev.to_host(ye)


def requant(m, e):
    m = np.asarray(m).reshape(-1)
    n = m.size
    om, oe = _dev.empty(n, "int16"), _dev.empty(n // TILE, "int8")
    dm, de = _d(m, np.int16), _d(e, np.int8)
    call("bfp_rtl_requant_d", dm.data_ptr(), de.data_ptr(), n, om.data_ptr(), oe.data_ptr(),
         _dev.stream())
    return _dev.to_host(om), _dev.to_host(oe)


def golden_rmsnorm(x_m, x_e, g_m, g_e):
    """rmsnorm_bfp.sv; x may hold a batch (batch, D)."""
    x_m = np.asarray(x_m)
    D = np.asarray(g_m).size
    batch = x_m.size // D
    ym, ye = _dev.empty(batch * D, "int16"), _dev.empty(batch * D // TILE, "int8")
    a = [_d(x_m, np.int16), _d(x_e, np.int8), _d(g_m, np.int16), _d(g_e, np.int8)]
    call("bfp_rtl_rmsnorm_d", *[t.data_ptr() for t in a], D, batch, ym.data_ptr(), ye.data_ptr(),
         _dev.stream())
    return _dev.to_host(ym).reshape(batch, D), _dev.to_host(ye).reshape(batch, D // TILE)


def golden_rope(x_m, x_e, pos):
    """rope_bfp.sv on heads of 64: (heads*64,) mantissas, (heads*4,) tile
    exponents -> (m, e) with one exponent per element."""
    x_m = np.asarray(x_m).reshape(-1)
    heads = x_m.size // 64
    fq = _dev.to_dev(tables()[2].astype(np.uint32).view(np.int32))
    ym, ye = _dev.empty(heads * 64, "int16"), _dev.empty(heads * 64, "int8")
    dm, de = _d(x_m, np.int16), _d(x_e, np.int8)
    call("bfp_rtl_rope_d", dm.data_ptr(), de.data_ptr(), int(pos), heads, fq.data_ptr(),
         ym.data_ptr(), ye.data_ptr(), _dev.stream())
    return _dev.to_host(ym), _dev.to_host(ye)


def golden_softmax(x_m, e_shared, n):
    """softmax_bfp.sv: one problem (n mantissas, one shared exponent) or a
    batch (x_m (batch, n), e_shared (batch,))."""
    x_m = np.atleast_2d(np.asarray(x_m))
    batch, stride = x_m.shape
    e = np.atleast_1d(np.asarray(e_shared))
    lut = _dev.to_dev(tables()[0].view(np.int16))
    ym, ye = _dev.empty(batch * stride, "int16"), _dev.empty(batch, "int8")
    dm, de = _d(x_m, np.int16), _d(e, np.int8)
    call("bfp_rtl_softmax_d", dm.data_ptr(), de.data_ptr(), int(n), batch, stride, lut.data_ptr(),
         ym.data_ptr(), ye.data_ptr(), _dev.stream())
    return _dev.to_host(ym).reshape(batch, stride)[:, :n], _dev.to_host(ye)


def golden_swiglu(gate_m, gate_e, up_m, up_e):
    n = np.asarray(gate_m).size
    lut = _dev.to_dev(tables()[1])
    ym, ye = _dev.empty(n, "int16"), _dev.empty(n // TILE, "int8")
    a = [_d(gate_m, np.int16), _d(gate_e, np.int8), _d(up_m, np.int16), _d(up_e, np.int8)]
    call("bfp_rtl_swiglu_d", *[t.data_ptr() for t in a], n, lut.data_ptr(), ym.data_ptr(),
         ye.data_ptr(), _dev.stream())
    return _dev.to_host(ym), _dev.to_host(ye)


def golden_residual(a_m, a_e, b_m, b_e):
    n = np.asarray(a_m).size
    ym, ye = _dev.empty(n, "int16"), _dev.empty(n // TILE, "int8")
    a = [_d(a_m, np.int16), _d(a_e, np.int8), _d(b_m, np.int16), _d(b_e, np.int8)]
    call("bfp_rtl_residual_d", *[t.data_ptr() for t in a], n, ym.data_ptr(), ye.data_ptr(),
         _dev.stream())
    return _dev.to_host(ym), _dev.to_host(ye)


def argmax(m, e):
    """bfp_gt running argmax over rows of (m, e) pairs: m, e (batch, n) or (n,)."""
    m = np.atleast_2d(np.asarray(m))
    batch, n = m.shape
    work = _dev.empty(3 * batch * n // TILE, "int32")
    out = _dev.empty(batch, "int32")
    dm, de = _d(m, np.int16), _d(e, np.int8)
    call("bfp_rtl_argmax_d", dm.data_ptr(), de.data_ptr(), n, batch, work.data_ptr(),
         out.data_ptr(), _dev.stream())
    return _dev.to_host(out)
