"""CPU checks of the reference weight-image formats (tinyllm-fpga_amd/bfp/
image.py, restating rtl/vc707/host/gen_smollm_blockfp_ddr.py:88-221 and
gen_smollm_blockfp_full.py:131-207): region sizes against the reference's
own offset macros (rtl/vc707/src/smollm/lbfp_ddr3.svh:24-86), the
vectorised packers against the reference's per-entry loops, image and hex
round trips, and the hex reader against the reference's committed release
files."""
from pathlib import Path

import numpy as np
import pytest

from oracle import bfp_image as oimg
from oracle import bfp_sim as sim

ROOT = Path(__file__).resolve().parent.parent
RELEASE = Path("/root/reference/rtl/vc707/release")
SMALL = dict(D=64, H_Q=1, H_KV=1, HD=64, FFN=128, NL=2, MAX_CTX=16, VOCAB=256)


def _dims(**kw):
    from bfp import Dims
    return Dims(**kw)


def test_layout_matches_reference_offset_macros():
    """SmolLM2-135M: the region sizes lbfp_ddr3.svh states (WQ 19,906,560 /
    622,080 B, WK 6,635,520 B), its fixed G1/G2 spacing (0x9000 / 0x1000),
    and its EMBED_* / NORM_W_M offset arithmetic."""
    from bfp import image
    d = _dims(NL=30)
    L = image.image_layout(d)
    assert L["WQ_m"] == (0, 19_906_560)
    assert L["WQ_e"][1] == 622_080
    assert L["WK_m"][1] == 6_635_520
    assert L["G1_e"][0] - L["G1_m"][0] == 0x9000
    assert L["G2_m"][0] - L["G1_e"][0] == 0x1000
    assert L["G2_e"][0] - L["G2_m"][0] == 0x9000
    assert L["EMBED_m"][0] - L["G2_e"][0] == 0x1000
    V, D = d.VOCAB, d.D
    assert L["EMBED_e"][0] - L["EMBED_m"][0] == V // 16 * D * 32
    assert L["EMBED_LU_m"][0] - L["EMBED_e"][0] == V // 16 * (D // 16) * 16
    assert L["EMBED_LU_e"][0] - L["EMBED_LU_m"][0] == V * D * 2
    assert L["NORM_W_m"][0] - L["EMBED_LU_e"][0] == V * 64
    # every region starts on a 4 KiB boundary, in image order, without overlap
    offs = sorted(L.values())
    assert all(o % 4096 == 0 for o, _ in offs)
    assert all(o0 + n0 <= o1 for (o0, n0), (o1, _) in zip(offs, offs[1:]))


@pytest.mark.parametrize("shape", [(16, 1), (32, 4), (48, 36)])
def test_vectorised_packers_match_reference_loops(shape):
    rng = np.random.default_rng(sum(shape))
    d_out, nt = shape
    m = rng.integers(-32768, 32768, size=(d_out, nt, 16)).astype(np.int16)
    e = rng.integers(-128, 128, size=(d_out, nt)).astype(np.int8)
    assert oimg.pack_layer_mantissas(m) == oimg.pack_layer_mantissas_literal(m)
    assert oimg.pack_layer_exponents(e) == oimg.pack_layer_exponents_literal(e)


def _oracle_model(seed, **cfg):
    from bfp import synth
    d = _dims(**{**SMALL, **cfg})
    return d, sim.build_model(synth.make_model(d, seed=seed))


def test_ddr_image_round_trip(tmp_path):
    from bfp import image
    d, om = _oracle_model(3)
    raw = oimg.ddr_image_bytes(om)
    assert len(raw) == image.image_bytes(d)
    path = tmp_path / "img_DDR3.bin"
    path.write_bytes(raw)
    img = image.WeightImage.from_ddr(path, d)
    for tag, key in oimg.MATRIX_TAGS:
        for li in range(d.NL):
            m, e = img.matrix(tag, li)
            wm, we = om.layers[li][key]
            assert (m == wm).all() and (e == we).all(), (tag, li)
    for li in range(d.NL):
        for tag, key in (("G1", "g1"), ("G2", "g2")):
            m, e = img.narrow(tag, li)
            wm, we = sim.tile_quantize(om.layers[li][key])
            assert (m == wm.reshape(-1)).all() and (e == we).all()
    m, e = img.embed_rows()
    wm, we = sim.tile_quantize(om.embed.reshape(-1))
    assert (m.reshape(-1) == wm.reshape(-1)).all() and (e.reshape(-1) == we).all()
    assert (img.embed_f32().astype(np.float64) == oimg.bfp_exact_model(om).embed).all()
    with pytest.raises(ValueError):
        short = tmp_path / "short.bin"
        short.write_bytes(raw[:-8192])
        image.WeightImage.from_ddr(short, d)


def test_hex_set_matches_ddr_image(tmp_path):
    from bfp import image
    d, om = _oracle_model(4)
    oimg.write_hex_set(om, tmp_path, prefix="t_")
    hx = image.WeightImage.from_hex_dir(tmp_path, d, prefix="t_")
    raw = np.frombuffer(oimg.ddr_image_bytes(om), np.uint8)
    for name, (off, n) in image.image_layout(d).items():
        assert (hx.regions[name] == raw[off:off + n]).all(), name


@pytest.mark.skipif(not RELEASE.exists(), reason="the reference tree is not mounted")
def test_hex_reader_on_reference_release_files():
    """The reference's committed release hex (real SmolLM2-135M BFP gammas)
    read by bfp.image equals the fixture tests/golden/release_bfp.npz, which
    an independent line-by-line parser made from the same files."""
    from bfp import image
    f = np.load(ROOT / "tests" / "golden" / "release_bfp.npz")
    for name in ("G1", "G2", "NORM_W"):
        assert (image.read_hex_narrow(RELEASE / f"lbfp_full_{name}_m.hex", 16) == f[name + "_m"]).all()
        assert (image.read_hex_narrow(RELEASE / f"lbfp_full_{name}_e.hex", 8) == f[name + "_e"]).all()
    prompt = image.read_prompt_hex(RELEASE / "lbfp_full_PROMPT.hex")
    assert prompt.dtype == np.int32 and len(prompt) == 8 and (prompt >= 0).all()
