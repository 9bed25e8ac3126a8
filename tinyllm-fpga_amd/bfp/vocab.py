"""Token ids -> readable text, and the vocabulary file that maps them.

* ``Vocab``: the "BFPV" table read and decoded by libbfp (``bfp_vocab_*``),
  the counterpart of the reference's native client
  (rtl/vc707/host/bfp_client.cpp:866-1027: ``Vocab::load``, ``bytes_for``,
  ``decode_tokens`` with its Windows-1252 mojibake repair).
* ``vocab_bin_bytes`` / ``write_vocab_bin``: the table from a byte-level BPE
  ``vocab.json`` ({token string: id}), as rtl/vc707/host/gen_bfp_vocab_bin.py
  bakes it: each token string mapped back through the GPT-2 byte<->unicode
  table to the raw bytes it stands for.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import struct
from pathlib import Path

from ._lib import BfpError, lib

MAGIC = b"BFPV"
VERSION = 1


def gpt2_bytes_to_unicode() -> dict[int, str]:
    """The byte-level BPE alphabet (gen_bfp_vocab_bin.py:22-34): printable
    Latin-1 bytes stand for themselves, the other 68 bytes take the code
    points from U+0100 on, in byte order."""
    keep = [*range(0x21, 0x7F), *range(0xA1, 0xAD), *range(0xAE, 0x100)]
    table = {b: chr(b) for b in keep}
    nxt = 0x100
    for b in range(256):
        if b not in table:
            table[b] = chr(nxt)
            nxt += 1
    return table


def vocab_bin_bytes(vocab: dict[str, int]) -> bytes:
    """The BFPV v1 file for a {token string: id} map (gen_bfp_vocab_bin.py:
    44-74): n_tokens = max id + 1, blob in the map's iteration order, ids
    absent from the map get (0, 0).  Raises ValueError for a character
    outside the byte alphabet."""
    inv = {u: b for b, u in gpt2_bytes_to_unicode().items()}
    n = max(vocab.values()) + 1
    entries = [(0, 0)] * n
    blob = bytearray()
    for s, tid in vocab.items():
        try:
            data = bytes(inv[ch] for ch in s)
        except KeyError as err:
            raise ValueError(f"unmapped char in token id={tid}: {err}") from None
        entries[tid] = (len(blob), len(data))
        blob += data
    head = MAGIC + struct.pack("<III", VERSION, n, len(blob))
    return head + b"".join(struct.pack("<II", o, ln) for o, ln in entries) + bytes(blob)


def write_vocab_bin(vocab_json, out) -> Path:
    """Bake a vocab.json into a BFPV file (gen_bfp_vocab_bin.py:37-78)."""
    raw = json.loads(Path(vocab_json).read_text(encoding="utf-8"))
    if not isinstance(raw, dict):
        raise ValueError("vocab.json must be a {token: id} dict")
    out = Path(out)
    out.write_bytes(vocab_bin_bytes(raw))
    return out


class Vocab:
    """A BFPV table held by libbfp."""

    def __init__(self, handle: int):
        self._h = handle

    @classmethod
    def open(cls, path) -> "Vocab":
        h = C.c_void_p()
        rc = lib().bfp_vocab_open(os.fsencode(os.fspath(path)), C.byref(h))
        if rc:
            raise BfpError("bfp_vocab_open", rc, lib().bfp_last_error().decode())
        return cls(h.value)

    @classmethod
    def from_bytes(cls, buf: bytes) -> "Vocab":
        h = C.c_void_p()
        b = C.create_string_buffer(bytes(buf), len(buf))
        rc = lib().bfp_vocab_parse(C.cast(b, C.c_void_p), len(buf), C.byref(h))
        if rc:
            raise BfpError("bfp_vocab_parse", rc, lib().bfp_last_error().decode())
        return cls(h.value)

    def close(self):
        if self._h:
            lib().bfp_vocab_close(self._h)
            self._h = None

    __del__ = close

    def __len__(self) -> int:
        return lib().bfp_vocab_size(self._h)

    def bytes_for(self, tid: int) -> bytes:
        p, n = C.c_char_p(), C.c_size_t()
        rc = lib().bfp_vocab_token(self._h, int(tid), C.byref(p), C.byref(n))
        if rc:
            raise BfpError("bfp_vocab_token", rc, lib().bfp_last_error().decode())
        return C.string_at(p, n.value) if n.value else b""

    def decode_bytes(self, ids) -> bytes:
        """decode_tokens: the repaired UTF-8 bytes of an id sequence."""
        a = (C.c_int32 * len(ids))(*[int(t) for t in ids])
        n = lib().bfp_vocab_decode(self._h, C.cast(a, C.c_void_p), len(ids), None, 0)
        if n < 0:
            raise BfpError("bfp_vocab_decode", n, lib().bfp_last_error().decode())
        buf = C.create_string_buffer(n + 1)
        lib().bfp_vocab_decode(self._h, C.cast(a, C.c_void_p), len(ids), C.cast(buf, C.c_void_p),
                               n + 1)
        return buf.raw[:n]

    def decode_tokens(self, ids) -> str:
        """decode_tokens as text (undecodable sequences replaced)."""
        return self.decode_bytes(ids).decode("utf-8", errors="replace")
