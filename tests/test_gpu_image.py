"""GPU parity of the reference weight-image path: the device repack of the
wide layout (bfp_pack_wide_d) against the reference-layout pack, and whole
decodes of models loaded from a DDR3 image / hex set (written by
oracle/bfp_image.py, restating rtl/vc707/host/gen_smollm_blockfp_ddr.py and
gen_smollm_blockfp_full.py) against the oracle's decode of the same model."""
from pathlib import Path

import numpy as np
import pytest

from oracle import bfp_image as oimg
from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
TINY = dict(D=128, H_Q=2, H_KV=1, HD=64, FFN=256, NL=2, MAX_CTX=32, VOCAB=512)


@pytest.mark.parametrize("n_out,n_in", [(576, 576), (192, 576), (1536, 576), (576, 1536), (16, 16)])
def test_pack_wide_equals_pack(gpu, n_out, n_in):
    import torch
    from bfp import _dev
    from bfp._lib import call
    rng = np.random.default_rng(n_out + n_in)
    m = rng.integers(-32768, 32768, size=(n_out, n_in // 16, 16)).astype(np.int16)
    e = rng.integers(-128, 128, size=(n_out, n_in // 16)).astype(np.int8)
    wm = np.frombuffer(oimg.pack_layer_mantissas(m), np.uint8).copy()
    we = np.frombuffer(oimg.pack_layer_exponents(e), np.uint8).copy()
    bm, be = n_out * n_in * 2, n_out * n_in // 16
    out = [torch.zeros(b, dtype=torch.uint8, device="cuda") for b in (bm, be, bm, be)]
    dm, de, dwm, dwe = (_dev.to_dev(x) for x in (m, e, wm, we))
    call("bfp_pack_d", dm.data_ptr(), de.data_ptr(), n_out, n_in, out[0].data_ptr(),
         out[1].data_ptr(), _dev.stream())
    call("bfp_pack_wide_d", dwm.data_ptr(), dwe.data_ptr(), n_out, n_in, out[2].data_ptr(),
         out[3].data_ptr(), _dev.stream())
    assert torch.equal(out[0], out[2]) and torch.equal(out[1], out[3])


def _decode_pair(om, d, gm, prompt, n_gen):
    want = oimg.bfp_exact_model(om)
    hm = np.zeros((len(prompt) + n_gen, d.NL, d.D), np.int16)
    he = np.zeros((len(prompt) + n_gen, d.NL, d.D // 16), np.int8)

    def on_layer(step, li, h):
        m, e = sim.tile_quantize(h)
        hm[step, li] = m.reshape(-1)
        he[step, li] = e

    toks = sim.decode(want, prompt, n_gen, on_layer=on_layer)[len(prompt):]
    got, (ghm, ghe) = gm.decode(np.asarray(prompt)[None, :], n_gen, hist=True)
    assert (ghm[0] == hm).all() and (ghe[0] == he).all()
    assert list(got[0]) == list(toks)


@pytest.mark.parametrize("fmt", ["ddr", "hex"])
def test_decode_from_reference_image(gpu, tmp_path, fmt):
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(**TINY)
    om = sim.build_model(synth.make_model(d, seed=21))
    gm = BfpModel(d)
    if fmt == "ddr":
        path = tmp_path / "m_DDR3.bin"
        path.write_bytes(oimg.ddr_image_bytes(om))
        gm.load_ddr_image(path)
    else:
        oimg.write_hex_set(om, tmp_path, prefix="m_")
        gm.load_hex_dir(tmp_path, prefix="m_")
    _decode_pair(om, d, gm, [3, 100, 7, 42, 5], 8)
    gm.close()


def test_decode_with_release_gammas(gpu, tmp_path):
    """SmolLM2-shaped layers (D 576, 9/3 heads, FFN 1536; 4 layers, small
    vocabulary) whose RMSNorm gammas and final norm weight are the
    reference's released real-model BFP values (tests/golden/
    release_bfp.npz), matrices random: image -> context -> decode equals
    the oracle."""
    from bfp import Dims, synth
    from bfp.model import BfpModel
    d = Dims(NL=4, VOCAB=512, MAX_CTX=16)
    f = np.load(ROOT / "tests" / "golden" / "release_bfp.npz")
    om = sim.build_model(synth.make_model(d, seed=22))
    g1 = sim.tile_decode(f["G1_m"].reshape(-1, 16), f["G1_e"]).reshape(30, d.D)
    g2 = sim.tile_decode(f["G2_m"].reshape(-1, 16), f["G2_e"]).reshape(30, d.D)
    for li in range(d.NL):
        om.layers[li]["g1"], om.layers[li]["g2"] = g1[li], g2[li]
    om.norm_w_q = sim.tile_decode(f["NORM_W_m"].reshape(-1, 16), f["NORM_W_e"])
    path = tmp_path / "rel_DDR3.bin"
    path.write_bytes(oimg.ddr_image_bytes(om))
    gm = BfpModel(d)
    gm.load_ddr_image(path)
    _decode_pair(om, d, gm, [11, 400, 2, 99], 6)
    gm.close()


def test_embed_lookup_from_image(gpu, tmp_path):
    """Narrow rows gathered from a DDR3 image's EMBED_LU table equal the
    oracle's tile_quantize of the embedding rows; ids outside the
    vocabulary give the zero tile."""
    from bfp import Dims, image, synth
    d = Dims(**TINY)
    om = sim.build_model(synth.make_model(d, seed=23))
    path = tmp_path / "e_DDR3.bin"
    path.write_bytes(oimg.ddr_image_bytes(om))
    img = image.WeightImage.from_ddr(path, d)
    ids = [0, 5, d.VOCAB - 1, 3, 3, -1, d.VOCAB, 10 ** 6]
    m, e = img.embed_lookup(ids)
    assert m.shape == (len(ids), d.D) and e.shape == (len(ids), d.D // 16)
    for r, t in enumerate(ids):
        if 0 <= t < d.VOCAB:
            wm, we = sim.tile_quantize(om.embed[t])
            assert (m[r] == wm.reshape(-1)).all() and (e[r] == we).all(), t
        else:
            assert (m[r] == 0).all() and (e[r] == -127).all(), t


def test_embed_lookup_full_table(gpu):
    """SmolLM2 size (49152 x 576, exponent rows of 64 bytes): 4096 random
    ids and the table's first and last rows against numpy indexing."""
    from bfp.api import embed_lookup
    rng = np.random.default_rng(5)
    V, D = 49152, 576
    lu_m = rng.integers(-32768, 32768, size=(V, D), dtype=np.int16)
    lu_e = rng.integers(-128, 128, size=(V, 64), dtype=np.int8)
    ids = np.concatenate([[0, V - 1], rng.integers(0, V, 4096)]).astype(np.int32)
    m, e = embed_lookup(lu_m, lu_e, ids)
    assert (m == lu_m[ids]).all() and (e == lu_e[ids, :D // 16]).all()
    m0, e0 = embed_lookup(lu_m, lu_e, [])
    assert m0.shape == (0, D) and e0.shape == (0, D // 16)
