"""Token-id -> text, restated in Python -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module.  It restates, one step at a time,
the reference's vocabulary file format and decoder so the C-ABI versions in
libbfp (``bfp_vocab_*``) can be checked against it:

* ``parse``: the "BFPV" v1 reader of rtl/vc707/host/bfp_client.cpp:876-903
  (format written by rtl/vc707/host/gen_bfp_vocab_bin.py:10-17,69-74);
* ``bytes_for``: bfp_client.cpp:906-911;
* ``utf8_next_cp`` / ``cp_to_utf8`` / ``cp_to_win1252_byte`` /
  ``fix_mojibake`` / ``decode_tokens``: bfp_client.cpp:913-1027.

Independent pins (tests/test_vocab.py): the Windows-1252 table against
Python's ``cp1252`` codec, the repair against ``str.encode('cp1252')`` /
``bytes.decode('utf-8')`` on mojibake built from real text, identity on
valid UTF-8 that has no Windows-1252 high characters, and the reference
README's decoded sample (README.md:63-68).
"""
from __future__ import annotations

import struct

_W1252_HIGH = {
    0x20AC: 0x80, 0x201A: 0x82, 0x0192: 0x83, 0x201E: 0x84, 0x2026: 0x85, 0x2020: 0x86,
    0x2021: 0x87, 0x02C6: 0x88, 0x2030: 0x89, 0x0160: 0x8A, 0x2039: 0x8B, 0x0152: 0x8C,
    0x017D: 0x8E, 0x2018: 0x91, 0x2019: 0x92, 0x201C: 0x93, 0x201D: 0x94, 0x2022: 0x95,
    0x2013: 0x96, 0x2014: 0x97, 0x02DC: 0x98, 0x2122: 0x99, 0x0161: 0x9A, 0x203A: 0x9B,
    0x0153: 0x9C, 0x017E: 0x9E, 0x0178: 0x9F,
}


def parse(buf: bytes):
    """-> (entries [(offset, length)], blob); raises ValueError as Vocab::load throws."""
    if len(buf) < 16 or buf[:4] != b"BFPV":
        raise ValueError("bad vocab magic")
    version, n, blob_size = struct.unpack_from("<III", buf, 4)
    if version != 1:
        raise ValueError(f"unsupported vocab version {version}")
    if len(buf) < 16 + 8 * n + blob_size:
        raise ValueError("vocab truncated")
    entries = [struct.unpack_from("<II", buf, 16 + 8 * i) for i in range(n)]
    blob = buf[16 + 8 * n:16 + 8 * n + blob_size]
    return entries, blob


def bytes_for(entries, blob, tid: int) -> bytes:
    if tid < 0 or tid >= len(entries):
        return b""
    off, ln = entries[tid]
    if off + ln > len(blob):
        return b""
    return blob[off:off + ln]


def utf8_next_cp(s: bytes, i: int):
    """-> (code point, next index)."""
    b = s[i]
    if b < 0x80:
        return b, i + 1
    if b & 0xE0 == 0xC0:
        n, cp = 2, b & 0x1F
    elif b & 0xF0 == 0xE0:
        n, cp = 3, b & 0x0F
    elif b & 0xF8 == 0xF0:
        n, cp = 4, b & 0x07
    else:
        return b, i + 1
    if i + n > len(s):
        return b, i + 1
    for k in range(1, n):
        c = s[i + k]
        if c & 0xC0 != 0x80:
            return b, i + 1
        cp = (cp << 6) | (c & 0x3F)
    return cp, i + n


def cp_to_utf8(cp: int) -> bytes:
    if cp < 0x80:
        return bytes([cp])
    if cp < 0x800:
        return bytes([0xC0 | (cp >> 6), 0x80 | (cp & 0x3F)])
    if cp < 0x10000:
        return bytes([0xE0 | (cp >> 12), 0x80 | ((cp >> 6) & 0x3F), 0x80 | (cp & 0x3F)])
    return bytes([(0xF0 | (cp >> 18)) & 0xFF, 0x80 | ((cp >> 12) & 0x3F),
                  0x80 | ((cp >> 6) & 0x3F), 0x80 | (cp & 0x3F)])


def cp_to_win1252_byte(cp: int) -> int:
    if cp < 0x80 or 0xA0 <= cp <= 0xFF:
        return cp
    return _W1252_HIGH.get(cp, -1)


def fix_mojibake(s: bytes) -> bytes:
    cps, i = [], 0
    while i < len(s):
        cp, i = utf8_next_cp(s, i)
        cps.append(cp)
    out = bytearray()
    i = 0
    while i < len(cps):
        if cp_to_win1252_byte(cps[i]) < 0x80:
            out += cp_to_utf8(cps[i])
            i += 1
            continue
        j, run = i, bytearray()
        while j < len(cps):
            b = cp_to_win1252_byte(cps[j])
            if b < 0x80:
                break
            run.append(b)
            j += 1
        decoded, bi, ok, gained = bytearray(), 0, len(run) > 0, False
        while bi < len(run):
            prev = bi
            cp2, bi = utf8_next_cp(bytes(run), bi)
            if bi == prev + 1 and run[prev] >= 0x80:
                ok = False
                break
            if cp2 > 0xFF:
                gained = True
            decoded += cp_to_utf8(cp2)
        if ok and gained:
            out += decoded
        else:
            for k in range(i, j):
                out += cp_to_utf8(cps[k])
        i = j
    return bytes(out)


def decode_tokens(entries, blob, ids) -> bytes:
    return fix_mojibake(b"".join(bytes_for(entries, blob, int(t)) for t in ids))
