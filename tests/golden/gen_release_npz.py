"""Convert the reference's committed BFP release data (real SmolLM2-135M
gammas, rtl/vc707/release/lbfp_full_{G1,G2,NORM_W}_{m,e}.hex, one hex value
per line) into tests/golden/release_bfp.npz.  Run in a container where
/root/reference exists; the npz is committed."""
from pathlib import Path

import numpy as np

REL = Path("/root/reference/rtl/vc707/release")
OUT = Path(__file__).resolve().parent / "release_bfp.npz"


def read_hex(path, bits):
    vals = [int(l, 16) for l in path.read_text().split()]
    a = np.array(vals, dtype=np.int64)
    a = np.where(a >= 1 << (bits - 1), a - (1 << bits), a)
    return a.astype(np.int16 if bits == 16 else np.int8)


def main():
    out = {}
    for name in ("G1", "G2", "NORM_W"):
        out[f"{name}_m"] = read_hex(REL / f"lbfp_full_{name}_m.hex", 16)
        out[f"{name}_e"] = read_hex(REL / f"lbfp_full_{name}_e.hex", 8)
    np.savez_compressed(OUT, **out)
    print({k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
