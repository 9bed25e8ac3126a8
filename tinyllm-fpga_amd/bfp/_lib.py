"""ctypes binding of libbfp.so (the C ABI declared in include/bfp.h).

The library is built in-tree by ``tinyllm-fpga_amd/build.py`` (or
``__graft_entry__.build()``).  There is no fallback: if the library is
missing, or was built for another architecture, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libbfp.so"

BFP_OK = 0
ERRNAMES = {-22: "EINVAL", -12: "ENOMEM", -5: "EIO", -34: "ERANGE"}


class BfpError(RuntimeError):
    """A libbfp entry point returned a negative status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed: {ERRNAMES.get(code, code)}: {msg}")
        self.code = code


vp, i32, i64, sz = C.c_void_p, C.c_int, C.c_longlong, C.c_size_t
N_STAGES = 13


class DimsC(C.Structure):
    """struct bfp_dims."""
    _fields_ = [(n, C.c_int) for n in ("D", "H_Q", "H_KV", "HD", "FFN", "NL", "MAX_CTX", "VOCAB")]


class StageDumpC(C.Structure):
    """struct bfp_stage_dump."""
    _fields_ = [("m", C.c_void_p * N_STAGES), ("e", C.c_void_p * N_STAGES)]


# name -> (restype, argtypes); the list of exported symbols is checked by the
# CPU test suite against include/bfp.h.
SIGNATURES = {
    "bfp_last_error": (C.c_char_p, []),
    "bfp_version": (C.c_char_p, []),
    "bfp_packed_bytes_m": (sz, [i32, i32]),
    "bfp_packed_bytes_e": (sz, [i32, i32]),
    "bfp_pack_d": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "bfp_unpack_d": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "bfp_tile_quantize_f64_d": (i32, [vp, sz, vp, vp, vp]),
    "bfp_tile_quantize_f32_d": (i32, [vp, sz, vp, vp, vp]),
    "bfp_quantize_pack_f32_d": (i32, [vp, i32, i32, vp, vp, vp]),
    "bfp_tile_decode_d": (i32, [vp, vp, sz, vp, vp]),
    "bfp_tile_encode_f64_d": (i32, [vp, sz, vp, vp, vp, vp]),
    "bfp_rmsnorm_fp_d": (i32, [vp, vp, i32, i32, C.c_double, vp, vp]),
    "bfp_silu_fp_d": (i32, [vp, sz, vp, vp]),
    "bfp_softmax_fp_d": (i32, [vp, i32, i32, vp, vp]),
    "bfp_rope_cos_sin": (i32, [i32, i32, C.c_double, vp]),
    "bfp_rope_fp_d": (i32, [vp, i32, vp, vp, vp]),
    "bfp_matvec_d": (i32, [vp, vp, i32, i32, i32, i64, i64, vp, vp, i64, vp, vp, i64, i32, vp]),
    "bfp_matvec_ring_d": (i32, [vp, vp, i32, i32, i32, i32, i64, i64, vp, vp, i64, vp, vp, i64,
                                i32, vp]),
    "bfp_matvec_h": (i32, [vp, vp, i32, i32, vp, vp, vp, vp]),
    "bfp_probe_read_d": (i32, [vp, sz, vp, i32, i32, vp]),
    "bfp_pack_wide_d": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "bfp_load_weights_wide": (i32, [vp, i32, i32, vp, vp]),
    "bfp_rtl_tables": (i32, [vp, vp, vp, i32, C.c_double]),
    "bfp_rtl_matvec_d": (i32, [vp, vp, vp, vp, i32, i32, vp, vp, vp]),
    "bfp_rtl_requant_d": (i32, [vp, vp, i32, vp, vp, vp]),
    "bfp_rtl_rmsnorm_d": (i32, [vp, vp, vp, vp, i32, i32, vp, vp, vp]),
    "bfp_rtl_rope_d": (i32, [vp, vp, i32, i32, vp, vp, vp, vp]),
    "bfp_rtl_softmax_d": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp]),
    "bfp_rtl_swiglu_d": (i32, [vp, vp, vp, vp, i32, vp, vp, vp, vp]),
    "bfp_rtl_residual_d": (i32, [vp, vp, vp, vp, i32, vp, vp, vp]),
    "bfp_rtl_argmax_d": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "bfp_rtl_argmax_static_d": (i32, [vp, vp, i32, i32, vp, vp]),
    "bfp_create": (vp, [C.POINTER(DimsC), i32, i32]),
    "bfp_destroy": (None, [vp]),
    "bfp_get_dims": (i32, [vp, C.POINTER(DimsC)]),
    "bfp_load_weights": (i32, [vp, i32, i32, vp, vp, vp]),
    "bfp_reset_kv": (i32, [vp]),
    "bfp_kv_io": (i32, [vp, i32, i32, i32, i32, vp, vp, vp, vp, i32]),
    "bfp_layer_step": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, C.POINTER(StageDumpC)]),
    "bfp_layer_step_kv": (i32, [vp, i32, i32, i32, i32, vp, vp, vp, vp, C.POINTER(StageDumpC)]),
    "bfp_kv_io_f64": (i32, [vp, i32, i32, i32, i32, vp, vp, i32]),
    "bfp_matvec": (i32, [vp, vp, vp, i32, i32, i32, vp, vp]),
    "bfp_rtl_layer_step": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, C.POINTER(StageDumpC)]),
    "bfp_head": (i32, [vp, i32, vp, vp, vp, vp]),
    "bfp_rtl_head": (i32, [vp, vp, vp, vp, vp, vp]),
    "bfp_rtl_decode": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "bfp_decode": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, i32]),
    "bfp_decode_time": (i32, [vp, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    "bfp_decode_step_times": (i32, [vp, vp, i32]),
    "bfp_decode_path": (i32, [vp]),
    "bfp_decode_form": (i32, [vp]),
    "bfp_decode_trace": (i32, [vp, vp, sz]),
    "bfp_vocab_open": (i32, [C.c_char_p, C.POINTER(vp)]),
    "bfp_vocab_parse": (i32, [vp, sz, C.POINTER(vp)]),
    "bfp_vocab_close": (None, [vp]),
    "bfp_vocab_size": (i32, [vp]),
    "bfp_vocab_token": (i32, [vp, i32, C.POINTER(C.c_char_p), C.POINTER(sz)]),
    "bfp_vocab_decode": (i64, [vp, vp, i32, vp, sz]),
    "bfp_embed_gather_d": (i32, [vp, vp, i32, i32, i32, vp, i32, vp, vp, vp]),
}

_LIB = None


def lib():
    """Load (once) and return the configured ctypes library."""
    global _LIB
    if _LIB is None:
        # One HIP runtime per process: torch ships its own libamdhip64 (same
        # SONAME as /opt/rocm's) and loads it by file name, so it must be in
        # the process before libbfp.so resolves its libamdhip64.so.7 -- the
        # other order maps two runtimes and torch then sees no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              "`python tinyllm-fpga_amd/build.py` (no CPU fallback exists)")
        L = C.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
    return _LIB


def check(fn: str, rc: int):
    if rc != BFP_OK:
        msg = lib().bfp_last_error()
        raise BfpError(fn, rc, msg.decode() if msg else "")
    return rc


def call(fn: str, *args):
    """Call an int-returning entry point and raise BfpError on failure."""
    return check(fn, getattr(lib(), fn)(*args))
