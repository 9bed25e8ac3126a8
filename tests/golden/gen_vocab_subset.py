"""Write tests/golden/vocab_subset.json from the reference's committed
vocabulary table rtl/vc707/host/bfp_vocab.bin (a data file: "BFPV" v1,
49152 SmolLM2 tokens, written by rtl/vc707/host/gen_bfp_vocab_bin.py).

The fixture keeps the entries the tests decode: the token ids of the
reference README's sample run (README.md:63), ids 0-299 (special tokens,
ASCII and the single raw-byte tokens), the tokens whose bytes are the UTF-8
of the Windows-1252 high characters (the pieces of web mojibake), and every
97th id.  Each entry is stored as hex of its raw bytes.

    python tests/golden/gen_vocab_subset.py [/root/reference]
"""
import json
import struct
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
README_IDS = [712, 9612, 3102, 645, 260, 905, 436, 441, 2408, 281, 624, 198, 198, 18, 504, 905,
              436, 441, 805]


def main(ref_root="/root/reference"):
    buf = (Path(ref_root) / "rtl/vc707/host/bfp_vocab.bin").read_bytes()
    assert buf[:4] == b"BFPV"
    version, n, blob_size = struct.unpack_from("<III", buf, 4)
    blob = buf[16 + 8 * n:16 + 8 * n + blob_size]
    tok = [blob[o:o + ln] for o, ln in (struct.unpack_from("<II", buf, 16 + 8 * i)
                                        for i in range(n))]
    high = {bytes([b]).decode("cp1252").encode("utf-8")
            for b in range(0x80, 0x100) if b not in (0x81, 0x8D, 0x8F, 0x90, 0x9D)}
    keep = set(README_IDS) | set(range(300)) | set(range(0, n, 97))
    keep |= {i for i, t in enumerate(tok) if t in high}
    out = {"source": "rtl/vc707/host/bfp_vocab.bin", "version": version, "n_tokens": n,
           "blob_size": blob_size, "readme_ids": README_IDS,
           "entries": {str(i): tok[i].hex() for i in sorted(keep)}}
    (HERE / "vocab_subset.json").write_text(json.dumps(out, indent=0) + "\n")
    print(f"{len(keep)} entries")


if __name__ == "__main__":
    main(*sys.argv[1:])
