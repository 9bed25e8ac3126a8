"""Writers of the reference's weight-image formats -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module: it produces DDR3 images and hex sets
from a quantised model so that the product's readers
(``tinyllm-fpga_amd/bfp/image.py``) and device repack
(``bfp_load_weights_wide``) can be checked against the oracle's own model.

Restated from the reference (no code copied):

* ``pack_layer_mantissas`` / ``pack_layer_exponents``:
  rtl/vc707/host/gen_smollm_blockfp_ddr.py:88-117 -- mantissa entry
  (chunk, col) = the 16 rows' int16 little-endian (lane 0 first), exponent
  entry (chunk, tile) = the 16 rows' int8;
* the image: regions in the order of gen_smollm_blockfp_ddr.py:168-221
  (7 matrices with NL layers concatenated, G1, G2, wide EMBED, narrow
  EMBED_LU with exponent rows padded to 64 bytes, NORM_W), each padded to a
  4 KiB multiple;
* the hex set: gen_smollm_blockfp_full.py:131-207,333-404 -- one
  $readmemh word per line, most-significant hex digit first, a wide word's
  lane 0 in its least-significant bits.

``pack_layer_mantissas_literal`` / ``pack_layer_exponents_literal`` follow
the reference's per-entry loops one value at a time (struct.pack_into) and
pin the vectorised versions on small shapes.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

from . import bfp_sim as sim

LANES = 16
ALIGN = 4096
EMBED_LU_E_ROW = 64
MATRIX_TAGS = (("WQ", "Wq"), ("WK", "Wk"), ("WV", "Wv"), ("WO", "Wo"), ("WG", "Wg"),
               ("WU", "Wu"), ("WDN", "Wd"))


def pack_layer_mantissas(m):
    """m (D_out, NT_in, 16) int16 -> bytes of (D_out/16, D_in, 16) int16 LE."""
    D_out, NT_in, _ = m.shape
    a = np.asarray(m, np.int16).reshape(D_out // LANES, LANES, NT_in * 16).transpose(0, 2, 1)
    return np.ascontiguousarray(a).astype("<i2").tobytes()


def pack_layer_exponents(e):
    """e (D_out, NT_in) int8 -> bytes of (D_out/16, NT_in, 16) int8."""
    D_out, NT_in = e.shape
    a = np.asarray(e, np.int8).reshape(D_out // LANES, LANES, NT_in).transpose(0, 2, 1)
    return np.ascontiguousarray(a).tobytes()


def pack_layer_mantissas_literal(m):
    """Entry by entry, as gen_smollm_blockfp_ddr.py:88-104 loops."""
    D_out, NT_in, _ = m.shape
    D_in = NT_in * 16
    buf = bytearray((D_out // LANES) * D_in * 32)
    for chunk in range(D_out // LANES):
        for col in range(D_in):
            for lane in range(LANES):
                v = int(m[chunk * LANES + lane, col // 16, col % 16]) & 0xFFFF
                struct.pack_into("<H", buf, (chunk * D_in + col) * 32 + lane * 2, v)
    return bytes(buf)


def pack_layer_exponents_literal(e):
    """Entry by entry, as gen_smollm_blockfp_ddr.py:107-117 loops."""
    D_out, NT_in = e.shape
    buf = bytearray((D_out // LANES) * NT_in * 16)
    for chunk in range(D_out // LANES):
        for tile in range(NT_in):
            for lane in range(LANES):
                buf[(chunk * NT_in + tile) * 16 + lane] = int(e[chunk * LANES + lane, tile]) & 0xFF
    return bytes(buf)


def _pad4k(b: bytes) -> bytes:
    return b + b"\0" * ((-len(b)) % ALIGN)


def _embed_tables(model: sim.Model):
    """Wide and narrow BFP embedding of the model's float embedding,
    VOCAB padded to 16 rows with zeros (ddr.py:197-216)."""
    emb = np.asarray(model.embed, np.float64)
    pad = (-emb.shape[0]) % LANES
    if pad:
        emb = np.vstack([emb, np.zeros((pad, emb.shape[1]))])
    wm, we = sim.quantize_W(emb)
    m, e = sim.tile_quantize(emb.reshape(-1))
    return wm, we, m.reshape(emb.shape[0], -1), e.reshape(emb.shape[0], -1)


def ddr_image_bytes(model: sim.Model) -> bytes:
    """The DDR3 image of an oracle model (gen_smollm_blockfp_ddr.py:168-221)."""
    d = model.dims
    out = []
    for tag, key in MATRIX_TAGS:
        mb = b"".join(pack_layer_mantissas(model.layers[li][key][0]) for li in range(d.NL))
        eb = b"".join(pack_layer_exponents(model.layers[li][key][1]) for li in range(d.NL))
        out += [_pad4k(mb), _pad4k(eb)]
    for g in ("g1", "g2"):
        q = [sim.tile_quantize(model.layers[li][g]) for li in range(d.NL)]
        out += [_pad4k(b"".join(x[0].astype("<i2").tobytes() for x in q)),
                _pad4k(b"".join(x[1].tobytes() for x in q))]
    wm, we, lm, le = _embed_tables(model)
    out += [_pad4k(pack_layer_mantissas(wm)), _pad4k(pack_layer_exponents(we)),
            _pad4k(lm.astype("<i2").tobytes())]
    lep = np.zeros((le.shape[0], EMBED_LU_E_ROW), np.int8)
    lep[:, :le.shape[1]] = le
    out.append(_pad4k(lep.tobytes()))
    nm, ne = sim.tile_quantize(model.norm_w_q)
    out += [_pad4k(nm.astype("<i2").tobytes()), _pad4k(ne.tobytes())]
    return b"".join(out)


def _write(path: Path, lines):
    path.write_text("".join(ln + "\n" for ln in lines))


def _wide_lines(buf: bytes, nbytes: int):
    a = np.frombuffer(buf, np.uint8).reshape(-1, nbytes)[:, ::-1]
    return [row.tobytes().hex() for row in a]


def write_hex_set(model: sim.Model, directory, prefix="lbfp_full_"):
    """The hex set of full.py's baker: per-matrix wide _m/_e (NL layers
    concatenated), narrow G1/G2/NORM_W, wide EMBED and narrow EMBED_LOOKUP."""
    d = model.dims
    root = Path(directory)
    for tag, key in MATRIX_TAGS:
        mb = b"".join(pack_layer_mantissas(model.layers[li][key][0]) for li in range(d.NL))
        eb = b"".join(pack_layer_exponents(model.layers[li][key][1]) for li in range(d.NL))
        _write(root / f"{prefix}{tag}_m.hex", _wide_lines(mb, 32))
        _write(root / f"{prefix}{tag}_e.hex", _wide_lines(eb, 16))
    for tag, g in (("G1", "g1"), ("G2", "g2")):
        q = [sim.tile_quantize(model.layers[li][g]) for li in range(d.NL)]
        _write(root / f"{prefix}{tag}_m.hex",
               [f"{int(v) & 0xFFFF:04x}" for x in q for v in x[0].reshape(-1)])
        _write(root / f"{prefix}{tag}_e.hex", [f"{int(v) & 0xFF:02x}" for x in q for v in x[1]])
    wm, we, lm, le = _embed_tables(model)
    _write(root / f"{prefix}EMBED_m.hex", _wide_lines(pack_layer_mantissas(wm), 32))
    _write(root / f"{prefix}EMBED_e.hex", _wide_lines(pack_layer_exponents(we), 16))
    _write(root / f"{prefix}EMBED_LOOKUP_m.hex", [f"{int(v) & 0xFFFF:04x}" for v in lm.reshape(-1)])
    _write(root / f"{prefix}EMBED_LOOKUP_e.hex", [f"{int(v) & 0xFF:02x}" for v in le.reshape(-1)])
    nm, ne = sim.tile_quantize(model.norm_w_q)
    _write(root / f"{prefix}NORM_W_m.hex", [f"{int(v) & 0xFFFF:04x}" for v in nm.reshape(-1)])
    _write(root / f"{prefix}NORM_W_e.hex", [f"{int(v) & 0xFF:02x}" for v in ne])


def bfp_exact_model(model: sim.Model) -> sim.Model:
    """The model an image of `model` describes: the same quantised layers,
    and the float embedding replaced by its BFP values (the image has no
    other), so the oracle's head reads what a context loaded from the image
    reads."""
    emb = np.asarray(model.embed, np.float64)
    m, e = sim.tile_quantize(emb.reshape(-1))
    return sim.Model(model.dims, model.layers, sim.tile_decode(m, e).reshape(emb.shape),
                     model.norm_w_q)
