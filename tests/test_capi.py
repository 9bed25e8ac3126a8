"""CPU checks of the C ABI: libbfp.so loads and exports exactly the
functions include/bfp.h declares, and the ctypes signature table covers them.
No compute call is made (there is no GPU here)."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(bfp_\w+)\s*\(", text))
    return names


def test_library_exports_header():
    import ctypes
    from bfp import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail("libbfp.so is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(str(_lib.LIB_PATH))
    declared = _declared()
    assert declared, "no declarations found"
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"
    untyped = sorted(declared - set(_lib.SIGNATURES))
    assert not untyped, f"declared but not bound in _lib.SIGNATURES: {untyped}"
    assert set(_lib.SIGNATURES) <= declared


def test_version_string():
    from bfp import _lib
    assert b"gfx950" in _lib.lib().bfp_version()


def test_size_helpers():
    from bfp import _lib
    L = _lib.lib()
    assert L.bfp_packed_bytes_m(576, 576) == 576 * 576 * 2
    assert L.bfp_packed_bytes_e(576, 1536) == 576 * 96
    assert L.bfp_packed_bytes_m(15, 16) == 0
