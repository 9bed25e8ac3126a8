"""The reference's weight-image formats, read into a BfpModel.

Two on-disk forms carry the same BFP model:

* the FPGA's DDR3 image ``<PREFIX>DDR3.bin`` written by
  rtl/vc707/host/gen_smollm_blockfp_ddr.py:155-221 and read by the weight
  streamer at the offsets of rtl/vc707/src/smollm/lbfp_ddr3.svh:45-86;
* the per-tensor hex sets ``<PREFIX><TAG>_m.hex`` / ``_e.hex`` written by
  rtl/vc707/host/gen_smollm_blockfp_full.py:131-207,333-404 for $readmemh.

Matrices are in the reference's "wide" layout: one 32-byte mantissa entry
per (16-row chunk, input column) holding the 16 rows' int16 little-endian,
and one 16-byte exponent entry per (chunk, tile); NL layers concatenated
per matrix.  Gammas, the final norm weight and the embedding lookup table
are "narrow": one int16 per element and one int8 per 16-element tile.

The matrices go to the device as they are and are repacked there
(bfp_load_weights_wide).  The image holds only the BFP embedding; its
decoded values (exact in float32) stand in for the float embedding that
the model-level simulator's head reads (full.py:439).
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .dims import Dims

ALIGN = 4096                # gen_smollm_blockfp_ddr.py:38 (LBFP_DDR3_ALIGN)
LANES = 16
EMBED_LU_E_ROW = 64         # exponent bytes per row of EMBED_LU_e (ddr.py:203-214)

# (image tag, bfp_which slot) in image order (ddr.py:170-185)
MATRICES = (("WQ", 0), ("WK", 1), ("WV", 2), ("WO", 3), ("WG", 4), ("WU", 5), ("WDN", 6))


def matrix_shape(d: Dims, tag: str) -> tuple[int, int]:
    """(n_out, n_in) of a matrix tag (full.py:333-339)."""
    kv = d.H_KV * d.HD
    return {"WQ": (d.D, d.D), "WK": (kv, d.D), "WV": (kv, d.D), "WO": (d.D, d.D),
            "WG": (d.FFN, d.D), "WU": (d.FFN, d.D), "WDN": (d.D, d.FFN)}[tag]


def vocab_padded(d: Dims) -> int:
    """Rows of the embedding tables: VOCAB rounded up to LANES (ddr.py:199-200)."""
    return -(-d.VOCAB // LANES) * LANES


def _align(n: int) -> int:
    return (n + ALIGN - 1) & ~(ALIGN - 1)


def image_layout(d: Dims) -> dict[str, tuple[int, int]]:
    """Region name -> (byte offset, byte length) in a DDR3 image: regions in
    the order gen_smollm_blockfp_ddr.py:168-221 appends them, each starting
    on a 4 KiB boundary.  (lbfp_ddr3.svh places NORM_W_e 64 KiB after
    NORM_W_m; the baker, which writes the file, aligns to 4 KiB and is
    followed here.)"""
    vp = vocab_padded(d)
    sizes = []
    for tag, _ in MATRICES:
        n_out, n_in = matrix_shape(d, tag)
        sizes += [(tag + "_m", d.NL * n_out * n_in * 2), (tag + "_e", d.NL * n_out * n_in // 16)]
    for g in ("G1", "G2"):
        sizes += [(g + "_m", d.NL * d.D * 2), (g + "_e", d.NL * d.D // 16)]
    sizes += [("EMBED_m", vp * d.D * 2), ("EMBED_e", vp * d.D // 16),
              ("EMBED_LU_m", vp * d.D * 2), ("EMBED_LU_e", vp * EMBED_LU_E_ROW),
              ("NORM_W_m", d.D * 2), ("NORM_W_e", d.D // 16)]
    out, off = {}, 0
    for name, n in sizes:
        out[name] = (off, n)
        off += _align(n)
    return out


def image_bytes(d: Dims) -> int:
    """Total size of a DDR3 image for these dims."""
    off, n = list(image_layout(d).values())[-1]
    return off + _align(n)


# ------------------------------------------------------------------ hex
def _hex_words(path: Path, nbytes: int) -> np.ndarray:
    """$readmemh file of one nbytes-wide little-endian word per line ->
    bytes (n, nbytes): hex digits are most-significant first, the word's
    byte 0 (lane 0) is its least-significant byte."""
    text = "".join(ln.strip() for ln in path.read_text().splitlines() if ln.strip())
    raw = np.frombuffer(bytes.fromhex(text), dtype=np.uint8)
    if raw.size % nbytes:
        raise ValueError(f"{path}: {raw.size} bytes is not a whole number of {nbytes}-byte words")
    return raw.reshape(-1, nbytes)[:, ::-1]


def read_hex_narrow(path, bits: int) -> np.ndarray:
    """One value per line, `bits` (16 or 8) wide, two's complement ->
    int16 / int8 (emit_gamma_concat, NORM_W, EMBED_LOOKUP, PROMPT)."""
    w = _hex_words(Path(path), bits // 8)
    return np.ascontiguousarray(w).view(np.int16 if bits == 16 else np.int8).reshape(-1)


def read_hex_wide(path, nbytes: int) -> np.ndarray:
    """Wide entries (32-byte mantissa or 16-byte exponent words, emit_W_concat
    / emit_table_wide) -> the image's byte stream (entries in file order)."""
    return np.ascontiguousarray(_hex_words(Path(path), nbytes)).reshape(-1)


# ---------------------------------------------------------------- image
@dataclass
class WeightImage:
    """The regions of one BFP model as byte arrays (uint8), named as in the
    DDR3 image."""
    dims: Dims
    regions: dict

    @classmethod
    def from_ddr(cls, path, dims: Dims) -> "WeightImage":
        """Memory-map a DDR3 image; raises ValueError if it is shorter than
        the layout of `dims` needs."""
        buf = np.memmap(os.fspath(path), dtype=np.uint8, mode="r")
        lay = image_layout(dims)
        need = max(off + n for off, n in lay.values())
        if buf.size < need:
            raise ValueError(f"{path}: {buf.size} bytes, the layout for {dims} needs {need}")
        return cls(dims, {k: buf[off:off + n] for k, (off, n) in lay.items()})

    @classmethod
    def from_hex_dir(cls, directory, dims: Dims, prefix: str = "lbfp_full_") -> "WeightImage":
        """Read a hex set (full.py's emitters); the regions become the same
        byte streams the DDR3 image holds."""
        d, root = dims, Path(directory)
        f = lambda tag: root / f"{prefix}{tag}.hex"   # noqa: E731
        reg = {}
        for tag, _ in MATRICES:
            reg[tag + "_m"] = read_hex_wide(f(tag + "_m"), 32)
            reg[tag + "_e"] = read_hex_wide(f(tag + "_e"), 16)
        for g in ("G1", "G2", "NORM_W"):
            reg[g + "_m"] = read_hex_narrow(f(g + "_m"), 16).view(np.uint8)
            reg[g + "_e"] = read_hex_narrow(f(g + "_e"), 8).view(np.uint8)
        reg["EMBED_m"] = read_hex_wide(f("EMBED_m"), 32)
        reg["EMBED_e"] = read_hex_wide(f("EMBED_e"), 16)
        lu_m = read_hex_narrow(f("EMBED_LOOKUP_m"), 16)
        lu_e = read_hex_narrow(f("EMBED_LOOKUP_e"), 8).reshape(-1, d.D // 16)
        pad = np.zeros((lu_e.shape[0], EMBED_LU_E_ROW), np.int8)
        pad[:, :d.D // 16] = lu_e
        reg["EMBED_LU_m"] = lu_m.view(np.uint8)
        reg["EMBED_LU_e"] = pad.reshape(-1).view(np.uint8)
        img = cls(d, reg)
        img.check()
        return img

    def check(self):
        """Every region has the length the layout gives."""
        for k, (_, n) in image_layout(self.dims).items():
            if self.regions[k].size != n:
                raise ValueError(f"region {k}: {self.regions[k].size} bytes, expected {n}")

    # views ---------------------------------------------------------------
    def matrix_wide(self, tag: str, layer: int) -> tuple[np.ndarray, np.ndarray]:
        """One layer's wide mantissa and exponent bytes of a matrix."""
        n_out, n_in = matrix_shape(self.dims, tag)
        bm, be = n_out * n_in * 2, n_out * n_in // 16
        m = self.regions[tag + "_m"][layer * bm:(layer + 1) * bm]
        e = self.regions[tag + "_e"][layer * be:(layer + 1) * be]
        return np.ascontiguousarray(m), np.ascontiguousarray(e)

    def matrix(self, tag: str, layer: int) -> tuple[np.ndarray, np.ndarray]:
        """One layer's matrix in the reference layout quantize_W returns:
        m (n_out, n_in/16, 16) int16, e (n_out, n_in/16) int8."""
        n_out, n_in = matrix_shape(self.dims, tag)
        wm, we = self.matrix_wide(tag, layer)
        m = wm.view(np.int16).reshape(n_out // LANES, n_in, LANES).transpose(0, 2, 1)
        e = we.view(np.int8).reshape(n_out // LANES, n_in // 16, LANES).transpose(0, 2, 1)
        return (np.ascontiguousarray(m).reshape(n_out, n_in // 16, 16),
                np.ascontiguousarray(e).reshape(n_out, n_in // 16))

    def narrow(self, tag: str, layer: int = 0) -> tuple[np.ndarray, np.ndarray]:
        """(m (D,) int16, e (D/16,) int8) of a gamma (G1/G2, per layer) or NORM_W."""
        D = self.dims.D
        m = self.regions[tag + "_m"].view(np.int16)[layer * D:(layer + 1) * D]
        e = self.regions[tag + "_e"].view(np.int8)[layer * (D // 16):(layer + 1) * (D // 16)]
        return np.ascontiguousarray(m), np.ascontiguousarray(e)

    def embed_rows(self) -> tuple[np.ndarray, np.ndarray]:
        """The narrow embedding lookup table: m (VOCAB, D) int16, e (VOCAB, D/16) int8."""
        d = self.dims
        m = self.regions["EMBED_LU_m"].view(np.int16).reshape(-1, d.D)[:d.VOCAB]
        e = self.regions["EMBED_LU_e"].view(np.int8).reshape(-1, EMBED_LU_E_ROW)[:d.VOCAB, :d.D // 16]
        return np.ascontiguousarray(m), np.ascontiguousarray(e)

    def embed_lookup(self, ids) -> tuple[np.ndarray, np.ndarray]:
        """Rows (m (n, D), e (n, D/16)) of token ids from the narrow table,
        gathered on the device as the FPGA's embedding lookup reads them."""
        from .api import embed_lookup
        d = self.dims
        lu_m = self.regions["EMBED_LU_m"].view(np.int16).reshape(-1, d.D)
        lu_e = self.regions["EMBED_LU_e"].view(np.int8).reshape(-1, EMBED_LU_E_ROW)
        return embed_lookup(lu_m, lu_e, ids, vocab=d.VOCAB)

    def embed_f32(self) -> np.ndarray:
        """The embedding's BFP values, m * 2^(e-15), exact in float32."""
        m, e = self.embed_rows()
        d = self.dims
        v = m.reshape(d.VOCAB, d.D // 16, 16).astype(np.float64) * np.ldexp(
            1.0, e.astype(np.int32) - 15)[:, :, None]
        return v.reshape(d.VOCAB, d.D).astype(np.float32)


def load_image(model, img: WeightImage):
    """Push every tensor of an image into a BfpModel context: matrices in
    the wide layout (repacked on the device), gammas and the final norm
    weight as (m, e), the embedding as its decoded BFP values."""
    from ._lib import call
    d = model.dims
    shape = lambda x: (x.D, x.H_Q, x.H_KV, x.HD, x.FFN, x.NL, x.VOCAB)   # noqa: E731
    if shape(img.dims) != shape(d):
        raise ValueError(f"image dims {img.dims} do not match the context's {d}")
    for tag, which in MATRICES:
        for li in range(d.NL):
            wm, we = img.matrix_wide(tag, li)
            call("bfp_load_weights_wide", model._h, which, li, wm.ctypes.data, we.ctypes.data)
    for li in range(d.NL):
        for tag, name in (("G1", "g1"), ("G2", "g2")):
            m, e = img.narrow(tag, li)
            model.load_tensor(name, li, m=m, e=e)
    m, e = img.narrow("NORM_W")
    model.load_tensor("norm_w", m=m, e=e)
    model.load_tensor("embed", fp32=img.embed_f32())


def read_prompt_hex(path) -> np.ndarray:
    """<PREFIX>PROMPT.hex (full.py:387-392): token ids, one 16-bit word per line."""
    return read_hex_narrow(path, 16).astype(np.uint16).astype(np.int32)
