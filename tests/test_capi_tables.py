"""The library's host-side RTL tables (bfp_rtl_tables) against the
reference's own LUT generators' output and committed frequency table
(tests/golden/ref_rtl_ops.npz) -- a CPU call, no GPU needed."""
import ctypes as C
import hashlib
from pathlib import Path

import numpy as np

F = np.load(Path(__file__).resolve().parent / "golden" / "ref_rtl_ops.npz")


def test_rtl_tables_match_reference():
    from bfp import _lib
    L = _lib.lib()
    el = np.zeros(1024, np.uint16)
    sl = np.zeros(65536, np.int16)
    fq = np.zeros(32, np.uint32)
    assert L.bfp_rtl_tables(el.ctypes.data, sl.ctypes.data, fq.ctypes.data, 64, C.c_double(1e4)) == 0
    assert (el.astype(np.int64) == F["exp_lut"]).all()
    assert hashlib.sha256(sl.tobytes()).hexdigest() == str(F["silu_lut_sha256"])
    assert (fq.astype(np.int64) == F["rope_freq_turns"]).all()
