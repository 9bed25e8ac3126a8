"""Token-id -> text (libbfp's bfp_vocab_*, host code, so these run on the
CPU): the reference's BFPV vocabulary table (rtl/vc707/host/
gen_bfp_vocab_bin.py) and its native client's decoder
(rtl/vc707/host/bfp_client.cpp:866-1027).

Pins, independent of the restatement in oracle/bfp_vocab.py:
* the reference README's sample run (README.md:63-68): its 19 token ids,
  looked up in the reference's own table (fixture tests/golden/
  vocab_subset.json, made by tests/golden/gen_vocab_subset.py), decode to
  the text the README prints;
* the Windows-1252 table against Python's cp1252 codec;
* mojibake built from real text with str.encode('utf-8').decode('cp1252')
  is repaired back to that text, and valid UTF-8 without Windows-1252 high
  characters is returned unchanged;
* the byte-level BPE alphabet against transformers' GPT-2 tokenizer table.
Then the C ABI equals the restatement on seeded random byte streams."""
import json
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import bfp_vocab as ov

ROOT = Path(__file__).resolve().parent.parent
FIX = json.loads((ROOT / "tests" / "golden" / "vocab_subset.json").read_text())
REF_BIN = Path("/root/reference/rtl/vc707/host/bfp_vocab.bin")
README_TEXT = "##â town when the world was not yet in its\n\n\"The world was not only"


def _subset_bin():
    """A BFPV file with the fixture's entries at their ids, (0, 0) elsewhere."""
    n = FIX["n_tokens"]
    entries, blob = [(0, 0)] * n, bytearray()
    for k, hx in FIX["entries"].items():
        b = bytes.fromhex(hx)
        entries[int(k)] = (len(blob), len(b))
        blob += b
    head = b"BFPV" + struct.pack("<III", 1, n, len(blob))
    return head + b"".join(struct.pack("<II", o, ln) for o, ln in entries) + bytes(blob)


@pytest.fixture(scope="module")
def vocab():
    from bfp.vocab import Vocab
    v = Vocab.from_bytes(_subset_bin())
    yield v
    v.close()


def test_readme_sample_decodes_to_readme_text(vocab):
    ids = FIX["readme_ids"]
    assert len(vocab) == 49152
    assert vocab.decode_tokens(ids) == README_TEXT
    entries, blob = ov.parse(_subset_bin())
    assert ov.decode_tokens(entries, blob, ids).decode("utf-8") == README_TEXT


@pytest.mark.skipif(not REF_BIN.exists(), reason="the reference tree is not mounted")
def test_reference_table_file(tmp_path):
    """The reference's committed table, opened from its path, agrees with
    the fixture entry for entry and decodes the README sample."""
    from bfp.vocab import Vocab
    v = Vocab.open(REF_BIN)
    assert len(v) == FIX["n_tokens"]
    for k, hx in FIX["entries"].items():
        assert v.bytes_for(int(k)) == bytes.fromhex(hx), k
    assert v.decode_tokens(FIX["readme_ids"]) == README_TEXT
    v.close()


def test_token_lookup_edges(vocab):
    assert vocab.bytes_for(0) == b"<|endoftext|>"
    assert vocab.bytes_for(-1) == b"" and vocab.bytes_for(49152) == b""
    assert vocab.bytes_for(301) == b""          # a gap of the subset: (0, 0)
    assert vocab.decode_bytes([]) == b""
    assert vocab.decode_bytes([-5, 10 ** 6]) == b""


def test_w1252_table_matches_codec():
    for b in range(256):
        try:
            ch = bytes([b]).decode("cp1252")
        except UnicodeDecodeError:            # 0x81 0x8D 0x8F 0x90 0x9D: undefined
            assert b in (0x81, 0x8D, 0x8F, 0x90, 0x9D)
            assert ov.cp_to_win1252_byte(b) == -1
            continue
        assert ov.cp_to_win1252_byte(ord(ch)) == b, hex(b)
    high = [cp for cp in range(0x100, 0x10000) if ov.cp_to_win1252_byte(cp) >= 0]
    assert len(high) == 27


# (no character whose UTF-8 holds 0x81 0x8D 0x8F 0x90 0x9D, bytes cp1252 leaves
# undefined: such mojibake cannot be written in the first place)
MOJIBAKE_TEXTS = ["—", "café — naïve ‘quotes’ “x“", "€5 ™", "Ã©té ’s é—", "中文 … end"]


@pytest.mark.parametrize("text", MOJIBAKE_TEXTS)
def test_mojibake_is_repaired(vocab, text):
    """text -> UTF-8 bytes -> read as cp1252 -> UTF-8 again: the web
    mojibake the repair targets; it must come back as text wherever a run
    holds a character above U+00FF."""
    moj = text.encode("utf-8").decode("cp1252", errors="strict")
    got = ov.fix_mojibake(moj.encode("utf-8")).decode("utf-8")
    # runs whose decoding gains no code point above U+00FF stay as they were
    want = []
    for word in text.split(" "):
        w_moj = word.encode("utf-8").decode("cp1252")
        want.append(word if any(ord(c) > 0xFF for c in word) else w_moj)
    assert got == " ".join(want)
    v = _vocab_of([moj.encode("utf-8")])
    assert v.decode_tokens([0]) == got
    v.close()


def _vocab_of(tokens):
    from bfp.vocab import Vocab
    blob, ent = b"".join(tokens), []
    off = 0
    for t in tokens:
        ent.append((off, len(t)))
        off += len(t)
    head = b"BFPV" + struct.pack("<III", 1, len(tokens), len(blob))
    return Vocab.from_bytes(head + b"".join(struct.pack("<II", *e) for e in ent) + blob)


def test_clean_utf8_is_unchanged():
    text = "plain ASCII, café, über, 中文, \U0001F600, tab\tnew\nline"
    b = text.encode("utf-8")
    assert ov.fix_mojibake(b) == b
    v = _vocab_of([b])
    assert v.decode_bytes([0]) == b
    v.close()


def test_capi_equals_restatement_on_random_bytes():
    """Seeded streams biased toward UTF-8 lead/continuation bytes, cut into
    random tokens: C ABI == restatement, byte for byte."""
    rng = np.random.default_rng(7)
    pool = np.array([*range(0x20, 0x7F), *range(0x80, 0xC0), *range(0xC0, 0x100)] + [0xE2] * 40
                    + [0x80] * 20 + [0xC3] * 20, dtype=np.uint8)
    for trial in range(40):
        n_tok = int(rng.integers(1, 40))
        toks = [rng.choice(pool, size=int(rng.integers(0, 6))).tobytes() for _ in range(n_tok)]
        v = _vocab_of(toks)
        ids = list(rng.integers(-2, n_tok + 2, size=int(rng.integers(0, 60))))
        ent, blob = ov.parse(bytes(_bin_of(toks)))
        assert v.decode_bytes(ids) == ov.decode_tokens(ent, blob, ids), trial
        v.close()


def _bin_of(tokens):
    blob = b"".join(tokens)
    ent, off = [], 0
    for t in tokens:
        ent.append((off, len(t)))
        off += len(t)
    return b"BFPV" + struct.pack("<III", 1, len(tokens), len(blob)) + b"".join(
        struct.pack("<II", *e) for e in ent) + blob


def test_parse_errors(tmp_path):
    from bfp._lib import BfpError
    from bfp.vocab import Vocab
    good = _bin_of([b"a", b"bc"])
    for bad in (b"XFPV" + good[4:], good[:4] + struct.pack("<I", 2) + good[8:], good[:-1],
                good[:12]):
        with pytest.raises(BfpError):
            Vocab.from_bytes(bad)
        with pytest.raises(ValueError):
            ov.parse(bad)
    with pytest.raises(BfpError):
        Vocab.open(tmp_path / "missing.bin")
    # an entry reaching past the blob reads as empty (bytes_for's bounds check)
    broken = b"BFPV" + struct.pack("<III", 1, 2, 3) + struct.pack("<II", 0, 2) + \
        struct.pack("<II", 2, 5) + b"xyz"
    v = Vocab.from_bytes(broken)
    assert v.bytes_for(0) == b"xy" and v.bytes_for(1) == b""
    v.close()


def test_gpt2_alphabet_matches_tokenizer_libraries():
    """The byte alphabet against transformers' table and the tokenizers
    library's ByteLevel alphabet (two independent implementations)."""
    from bfp.vocab import gpt2_bytes_to_unicode
    mine = gpt2_bytes_to_unicode()
    tr = pytest.importorskip("transformers.convert_slow_tokenizer")
    assert mine == tr.bytes_to_unicode()
    tk = pytest.importorskip("tokenizers.pre_tokenizers")
    assert set(mine.values()) == set(tk.ByteLevel.alphabet())
    assert mine[0x20] == "\u0120" and mine[0x0A] == "\u010a"   # "Ġ", "Ċ"


def test_writer_round_trip(tmp_path):
    """vocab.json (byte-level BPE strings) -> BFPV -> bytes: every fixture
    token survives, gaps read as empty, and the README sample still decodes."""
    from bfp.vocab import Vocab, gpt2_bytes_to_unicode, write_vocab_bin
    enc = gpt2_bytes_to_unicode()
    vj = {"".join(enc[b] for b in bytes.fromhex(hx)): int(k) for k, hx in FIX["entries"].items()}
    (tmp_path / "vocab.json").write_text(json.dumps(vj), encoding="utf-8")
    out = write_vocab_bin(tmp_path / "vocab.json", tmp_path / "v.bin")
    v = Vocab.open(out)
    assert len(v) == max(vj.values()) + 1
    for k, hx in FIX["entries"].items():
        assert v.bytes_for(int(k)) == bytes.fromhex(hx)
    assert v.bytes_for(301) == b""
    assert v.decode_tokens(FIX["readme_ids"]) == README_TEXT
    v.close()
    with pytest.raises(ValueError):
        from bfp.vocab import vocab_bin_bytes
        vocab_bin_bytes({"中": 0})
