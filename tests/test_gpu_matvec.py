"""GPU parity: device quantisation, layout and the BFP matvec against the
oracle (oracle/bfp_sim.py, restating rtl/vc707/host/gen_smollm_blockfp_full.py
:90-119,217-233).  Integer/byte work: the bar is bit-exact."""
import numpy as np
import pytest

from oracle import bfp_sim as sim

pytestmark = pytest.mark.gpu

SHAPES = [(576, 576), (192, 576), (1536, 576), (576, 1536), (49152, 576)]


def _synth(n_out, n_in, seed):
    from bfp import synth
    W, x = synth.make_matvec_case(n_out, n_in, seed=seed)
    return W[0], x[0]


def _oracle_quantize_W(W):
    # whole-matrix tile_quantize == the reference's per-row loop (tiles never
    # straddle rows); test_oracle_vec.py pins that equivalence
    n_out, n_in = W.shape
    m, e = sim.tile_quantize(W.astype(np.float64))
    return m.reshape(n_out, n_in // 16, 16), e.reshape(n_out, n_in // 16)


@pytest.mark.parametrize("n_out,n_in", SHAPES)
def test_matvec_baseline_shapes(gpu, n_out, n_in):
    import bfp.api as api
    print(f"[matvec] shape {n_out}x{n_in}", flush=True)
    W, x = _synth(n_out, n_in, seed=n_out + n_in)
    Wm, We = _oracle_quantize_W(W)
    xm, xe = sim.tile_quantize(x)
    want = sim.matvec_bfp(xm, xe, Wm, We)
    P = api.PackedMatrix.from_float(W)                 # device quantize_W
    gm, ge = P.unpack()
    assert (gm == Wm).all() and (ge == We).all()
    ym, ye = P.matvec_bfp(xm, xe)
    assert (ye == want[1]).all()
    assert (ym == want[0].reshape(-1)).all()


@pytest.mark.parametrize("waves", [1, 2, 3, 4, 6, 8, 9])
def test_matvec_wave_shapes(gpu, waves):
    """Every workgroup shape gives identical bits (in = 576 and 1536)."""
    import bfp.api as api
    for n_out, n_in in ((64, 576), (48, 1536)):
        W, x = _synth(n_out, n_in, seed=7 * waves)
        Wm, We = _oracle_quantize_W(W)
        xm, xe = sim.tile_quantize(x)
        want_m, want_e = sim.matvec_bfp(xm, xe, Wm, We)
        ym, ye = api.PackedMatrix(Wm, We).matvec_bfp(xm, xe, waves=waves)
        assert (ye == want_e).all() and (ym == want_m.reshape(-1)).all()


@pytest.mark.parametrize("n_out,n_in,espread", [(16, 16, 4), (32, 48, 40), (64, 576, 120),
                                                (48, 1536, 100), (16, 4096, 30)])
def test_matvec_integer_edges(gpu, n_out, n_in, espread):
    """Full-range mantissas incl. -32768 x -32768 tiles (S = 2^34), exponent
    spreads beyond the 47-bit alignment window, zero rows and tiles."""
    import bfp.api as api
    rng = np.random.default_rng(n_out + n_in + espread)
    xm = rng.integers(-32768, 32768, size=(n_in // 16, 16)).astype(np.int16)
    xe = rng.integers(-espread // 2, espread // 2 + 1, size=n_in // 16).astype(np.int8)
    Wm = rng.integers(-32768, 32768, size=(n_out, n_in // 16, 16)).astype(np.int16)
    We = rng.integers(-espread // 2, espread // 2 + 1, size=(n_out, n_in // 16)).astype(np.int8)
    xm[0, :] = -32768
    Wm[0, 0, :] = -32768
    Wm[1] = 0                      # an all-zero row
    Wm[min(17, n_out - 1)] = 0
    if n_out >= 32:
        Wm[16:32] = 0              # an all-zero output chunk -> e = -127
    want_m, want_e = sim.matvec_bfp(xm, xe, Wm, We)
    ym, ye = api.matvec_bfp(xm, xe, Wm, We)
    assert (ye == want_e).all() and (ym == want_m.reshape(-1)).all()


def _ring_case(n_out, n_in, ring, n_mats, seed):
    """n_mats problems over a ring of `ring` weight copies in one launch;
    returns (W ring, X, ym, ye) with device results on the host."""
    import torch
    from bfp import _dev
    from bfp._lib import call
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((ring, n_out, n_in)).astype(np.float32) * np.float32(0.02)
    X = rng.standard_normal((n_mats, n_in))
    bm = n_out * n_in * 2
    be = n_out * n_in // 16
    Pm = torch.empty(ring * bm, dtype=torch.uint8, device="cuda")
    Pe = torch.empty(ring * be, dtype=torch.uint8, device="cuda")
    dW = _dev.to_dev(W)
    for r in range(ring):
        call("bfp_quantize_pack_f32_d", dW.data_ptr() + r * W[0].nbytes, n_out, n_in,
             Pm.data_ptr() + r * bm, Pe.data_ptr() + r * be, _dev.stream())
    xm, xe = sim.tile_quantize(X.reshape(-1))
    dxm = _dev.to_dev(xm.reshape(n_mats, -1))
    dxe = _dev.to_dev(xe.reshape(n_mats, -1))
    ym = torch.empty(n_mats * n_out, dtype=torch.int16, device="cuda")
    ye = torch.empty(n_mats * n_out // 16, dtype=torch.int8, device="cuda")
    call("bfp_matvec_ring_d", Pm.data_ptr(), Pe.data_ptr(), n_out, n_in, n_mats, ring, bm, be,
         dxm.data_ptr(), dxe.data_ptr(), n_in, ym.data_ptr(), ye.data_ptr(), n_out, 0,
         _dev.stream())
    return (W, xm.reshape(n_mats, -1, 16), xe.reshape(n_mats, -1),
            ym.cpu().numpy().reshape(n_mats, -1), ye.cpu().numpy().reshape(n_mats, -1))


@pytest.mark.parametrize("n_out,n_in,ring,n_mats", [(192, 576, 5, 401), (576, 1536, 3, 121),
                                                    (16, 576, 7, 5003)],
                         ids=["12chunk", "ffn-in", "1chunk"])
def test_matvec_long_batches(gpu, n_out, n_in, ring, n_mats):
    """Long batches over a ring of weight copies (up to 5003 problems in one
    launch, one chunk of one problem per workgroup): every problem
    bit-exact against the oracle."""
    print(f"[matvec] long batch {n_out}x{n_in} ring {ring} x {n_mats}", flush=True)
    W, xm, xe, ym, ye = _ring_case(n_out, n_in, ring, n_mats, seed=n_mats)
    Wq = [_oracle_quantize_W(W[r]) for r in range(ring)]
    for i in range(n_mats):
        want_m, want_e = sim.matvec_bfp(xm[i], xe[i], *Wq[i % ring])
        assert (ye[i] == want_e).all() and (ym[i] == want_m.reshape(-1)).all(), f"problem {i}"


def test_matvec_batched_ring(gpu):
    """n_mats problems in one launch over a ring of distinct weight copies."""
    import torch
    from bfp import _dev
    from bfp._lib import call
    n_out, n_in, ring, n_mats = 192, 576, 3, 7
    rng = np.random.default_rng(1)
    W = rng.standard_normal((ring, n_out, n_in)).astype(np.float32) * np.float32(0.02)
    X = rng.standard_normal((n_mats, n_in))
    bm = n_out * n_in * 2
    be = n_out * n_in // 16
    Pm = torch.empty(ring * bm, dtype=torch.uint8, device="cuda")
    Pe = torch.empty(ring * be, dtype=torch.uint8, device="cuda")
    dW = _dev.to_dev(W)
    for r in range(ring):
        call("bfp_quantize_pack_f32_d", dW.data_ptr() + r * W[0].nbytes, n_out, n_in,
             Pm.data_ptr() + r * bm, Pe.data_ptr() + r * be, _dev.stream())
    xq = [sim.tile_quantize(X[i]) for i in range(n_mats)]
    dxm = _dev.to_dev(np.stack([q[0].reshape(-1) for q in xq]))
    dxe = _dev.to_dev(np.stack([q[1] for q in xq]))
    ym = torch.empty(n_mats * n_out, dtype=torch.int16, device="cuda")
    ye = torch.empty(n_mats * n_out // 16, dtype=torch.int8, device="cuda")
    call("bfp_matvec_ring_d", Pm.data_ptr(), Pe.data_ptr(), n_out, n_in, n_mats, ring, bm, be,
         dxm.data_ptr(), dxe.data_ptr(), n_in, ym.data_ptr(), ye.data_ptr(), n_out, 0,
         _dev.stream())
    ym, ye = ym.cpu().numpy().reshape(n_mats, -1), ye.cpu().numpy().reshape(n_mats, -1)
    for i in range(n_mats):
        Wm, We = _oracle_quantize_W(W[i % ring])
        want_m, want_e = sim.matvec_bfp(xq[i][0], xq[i][1], Wm, We)
        assert (ye[i] == want_e).all() and (ym[i] == want_m.reshape(-1)).all()


@pytest.mark.parametrize("n_out,n_in", [(192, 576), (48, 1536), (16, 576)],
                         ids=["chunk-pairs", "buffer-load", "one-chunk"])
def test_matvec_output_alignment(gpu, n_out, n_in):
    """Outputs at a 2-byte-aligned address (the dword store form needs 4)
    give the same bits as at an aligned one, for each kernel form; the
    bytes on both sides of the output are left alone."""
    import torch
    from bfp import _dev
    from bfp._lib import call
    rng = np.random.default_rng(n_out + n_in)
    W = rng.standard_normal((n_out, n_in)).astype(np.float32) * np.float32(0.02)
    n_mats = 3
    X = rng.standard_normal((n_mats, n_in))
    bm, be = n_out * n_in * 2, n_out * n_in // 16
    Pm = torch.empty(bm, dtype=torch.uint8, device="cuda")
    Pe = torch.empty(be, dtype=torch.uint8, device="cuda")
    dW = _dev.to_dev(W)
    call("bfp_quantize_pack_f32_d", dW.data_ptr(), n_out, n_in, Pm.data_ptr(), Pe.data_ptr(),
         _dev.stream())
    xq = [sim.tile_quantize(X[i]) for i in range(n_mats)]
    dxm = _dev.to_dev(np.stack([q[0].reshape(-1) for q in xq]))
    dxe = _dev.to_dev(np.stack([q[1] for q in xq]))
    outs = []
    for off in (0, 1):
        ym = torch.full((n_mats * n_out + 2,), 0x5A5A, dtype=torch.int16, device="cuda")
        ye = torch.empty(n_mats * n_out // 16, dtype=torch.int8, device="cuda")
        call("bfp_matvec_ring_d", Pm.data_ptr(), Pe.data_ptr(), n_out, n_in, n_mats, 1, bm, be,
             dxm.data_ptr(), dxe.data_ptr(), n_in, ym.data_ptr() + 2 * off, ye.data_ptr(), n_out,
             0, _dev.stream())
        h = ym.cpu().numpy()
        assert h[0] == 0x5A5A or off == 0
        assert h[off + n_mats * n_out] == 0x5A5A
        outs.append((h[off:off + n_mats * n_out].reshape(n_mats, -1), ye.cpu().numpy()))
    assert (outs[0][0] == outs[1][0]).all() and (outs[0][1] == outs[1][1]).all()
    Wm, We = _oracle_quantize_W(W)
    for i in range(n_mats):
        want_m, _ = sim.matvec_bfp(xq[i][0], xq[i][1], Wm, We)
        assert (outs[1][0][i] == want_m.reshape(-1)).all()


def _neg_full_scale_case():
    """One output row with A = -(2^20 - 1) at M = 30: y = -1048575 rounds to
    mantissa -32768 at e = 20 (raw); re-quantised it is (-16384, 21)."""
    xm = np.zeros((2, 16), np.int16)
    xe = np.array([15, 0], np.int8)
    Wm = np.zeros((16, 2, 16), np.int16)
    We = np.zeros((16, 2), np.int8)
    xm[0, 0], xm[0, 1] = 32, 31
    Wm[0, 0, 0], Wm[0, 0, 1] = -32767, -1
    We[0, 0] = 15
    Wm[3, 0, 0] = 3                # an odd mantissa elsewhere in the chunk
    We[3, 0] = 15
    return xm, xe, Wm, We


def test_matvec_neg_full_scale_raw(gpu):
    import bfp.api as api
    xm, xe, Wm, We = _neg_full_scale_case()
    m, e = sim.matvec_bfp(xm, xe, Wm, We)
    assert m[0, 0] == -32768 and e[0] == 20
    ym, ye = api.matvec_bfp(xm, xe, Wm, We)
    assert (ym == m.reshape(-1)).all() and (ye == e).all()
    # the decoded values are the reference's float64 output
    assert (api.matvec_hw_golden(xm, xe, Wm, We) == sim.matvec_hw_golden(xm, xe, Wm, We)).all()


def test_tile_quantize_and_decode(gpu):
    import bfp.api as api
    rng = np.random.default_rng(2)
    parts = [rng.standard_normal(16 * 50) * s for s in (1e-300, 1e-40, 1e-5, 0.02, 1.0, 3e4, 1e30)]
    v = np.concatenate(parts + [np.zeros(32)])
    v[100] = 1.0 - 2.0 ** -17
    v[116] = -(1.0 - 2.0 ** -17)
    v[132] = 2.0 ** -3                       # exact power of two
    m, e = api.tile_quantize(v)
    wm, we = sim.tile_quantize(v)
    assert (m == wm).all() and (e == we).all()
    assert (api.tile_decode(m, e) == sim.tile_decode(wm, we)).all()
    assert (api.fp_quantize_vec(v) == sim.fp_quantize_vec(v)).all()


def test_tile_quantize_near_power_of_two(gpu):
    """Tile maxima 1..100 doubles below 2^k: the device exponent follows
    floor(np.log2(.)) + 1, which rounds up to k + 1 within n_up(k) doubles
    (e.g. nextafter(256, 0) -> e 9, m 16384), for every k a tile exponent
    can take, both signs."""
    import bfp.api as api
    rng = np.random.default_rng(3)
    tiles = []
    for k in range(-128, 129):
        for n in (1, 2, 5, 6, 11, 12, 22, 23, 44, 45, 88, 89):
            t = rng.standard_normal(16) * np.ldexp(1.0, k - 4)
            b = float(np.ldexp(1.0, k) - n * np.ldexp(1.0, k - 53))
            t[rng.integers(16)] = b if rng.random() < 0.5 else -b
            tiles.append(t)
    v = np.concatenate(tiles)
    m, e = api.tile_quantize(v)
    wm, we = sim.tile_quantize(v)
    assert (e == we).all() and (m == wm).all()
    m, e = api.tile_quantize(np.r_[np.nextafter(256.0, 0.0), np.zeros(15)])
    assert e[0] == 9 and m[0, 0] == 16384


def test_bad_shapes_raise(gpu):
    import bfp.api as api
    from bfp._lib import BfpError
    with pytest.raises(ValueError):
        api.tile_quantize(np.zeros(17))
    with pytest.raises(BfpError):
        from bfp import _dev
        from bfp._lib import call
        call("bfp_matvec_d", 0, 0, 15, 16, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, _dev.stream())
