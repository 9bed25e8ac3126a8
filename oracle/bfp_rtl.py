"""CPU oracle for the RTL-exact BFP leaf ops -- TEST INFRASTRUCTURE ONLY
(same import rule as oracle/bfp_sim.py).

The reference's hardware leaf ops are specified bit-for-bit by their Python
golden generators under rtl/vc707/host/ and the LUT generators under
rtl/vc707/sim/.  Each function below restates one of them with Python
integers (the goldens are Python-int arithmetic) and cites the lines it
follows.  Unlike the model-level simulator, these ops keep per-lane or
per-element exponents and truncating shifts.
"""
from __future__ import annotations

import math

import numpy as np

TILE = 16
ACC_W = 48


def _low16(v: int) -> int:
    """Two's-complement low 16 bits as a signed int (`sh & 0xFFFF`, sign fix)."""
    m = v & 0xFFFF
    return m - 0x10000 if m & 0x8000 else m


def _clamp8(e: int) -> int:
    return max(-128, min(127, e))


def _lead(v: int) -> int:
    return abs(v).bit_length() - 1 if v else 0


def _norm16(v: int, lead: int):
    """Leading-bit normalise: shift = lead - 14, mantissa = low 16 bits of
    the shifted value.  Returns (m, shift)."""
    sh = lead - 14
    return _low16(v >> sh if sh >= 0 else v << (-sh)), sh


# ------------------------------------------------------------------ matvec
def rtl_matvec(x_m, x_e, W_m, W_e):
    """matvec_bfp_engine.sv golden (gen_matvec_bfp_golden.py:53-108): per
    row, tiles folded in order -- the side with the smaller exponent is
    arithmetic-shifted right (zeroed past 47), added, and saturated to 48
    bits; then a leading-bit normalise gives a per-row (m, e)."""
    hi, lo = (1 << (ACC_W - 1)) - 1, -(1 << (ACC_W - 1))
    n_out, nt = W_e.shape
    out_m = np.zeros(n_out, np.int16)
    out_e = np.zeros(n_out, np.int8)
    for i in range(n_out):
        acc = acc_e = 0
        for t in range(nt):
            s = int(np.dot(x_m[t].astype(np.int64), W_m[i, t].astype(np.int64)))
            te = int(x_e[t]) + int(W_e[i, t])
            if t == 0:
                acc, acc_e = s, te
                continue
            d = te - acc_e
            if d > 0:
                acc = 0 if d > ACC_W - 1 else acc >> d
                acc_e = te
            elif d < 0:
                s = 0 if -d > ACC_W - 1 else s >> (-d)
            acc = max(lo, min(hi, acc + s))
        m, sh = _norm16(acc, _lead(acc))
        out_m[i] = m
        out_e[i] = _clamp8(acc_e + sh - 15)
    return out_m, out_e


def _wrap8(v):
    """An integer reduced to the 8-bit two's-complement range."""
    return ((int(v) + 128) & 0xFF) - 128


def shr8(m: int, e_to: int, e_from: int) -> int:
    """requant_mant (smollm_layer_bfp.sv:1387-1396): the shift e_to - e_from
    is held in `logic signed [7:0]`, so it wraps; >= 16 gives 0, a negative
    (wrapped) shift leaves m unchanged.  The AV pre-shift of V
    (:2149-2166) has the same form."""
    sh = _wrap8(e_to - e_from)
    if sh >= 16:
        return 0
    return int(m) >> sh if sh >= 0 else int(m)


def rtl_requant(m, e):
    """Per-lane exponents of a 16-lane chunk -> one tile exponent
    (smollm_layer_bfp.sv:1387-1396 requant_mant, :1672-1693 emax):
    emax = max(e); each m through shr8(m, emax, e)."""
    m = np.asarray(m, np.int64).reshape(-1, TILE)
    e = np.asarray(e, np.int64).reshape(-1, TILE)
    emax = e.max(axis=1)
    out = np.array([[shr8(m[c, k], emax[c], e[c, k]) for k in range(TILE)]
                    for c in range(m.shape[0])], np.int64)
    return out.astype(np.int16).reshape(-1), emax.astype(np.int8)


# ----------------------------------------------------------------- rmsnorm
RMS_SEED_Q12_12 = {31: 2365, 30: 3344, 29: 4730, 28: 6689, 27: 9459, 26: 13377,
                   25: 18919, 24: 26755, 23: 37837, 22: 53510, 21: 75674, 20: 107020,
                   19: 151349, 18: 214040, 17: 302698, 16: 428079, 15: 605396,
                   14: 856159, 13: 1210791, 12: 1712317, 11: 2421583, 10: 3424635,
                   9: 4843165, 8: 6849270, 7: 9686330, 6: 13698540}
"""rsqrt seed LUT of rmsnorm_bfp.sv, by msb of v (gen_rmsnorm_bfp_golden.py:34-38);
other msbs seed with 2^24 - 1."""
EPS_Q30 = 10737


def rtl_rmsnorm(x_m, x_e, g_m, g_e):
    """rmsnorm_bfp.sv golden (gen_rmsnorm_bfp_golden.py:42-142)."""
    x_m = np.asarray(x_m, np.int64).reshape(-1, TILE)
    g_m = np.asarray(g_m, np.int64).reshape(-1, TILE)
    nt = x_m.shape[0]
    D = nt * TILE
    inv_d = (1 << 32) // D
    sums = [int((x_m[t] * x_m[t]).sum()) for t in range(nt)]
    exps = [2 * int(x_e[t]) for t in range(nt)]
    acc, acc_e = sums[0], exps[0]
    for t in range(1, nt):
        d = exps[t] - acc_e
        if d > 0:
            acc = 0 if d > ACC_W - 1 else acc >> d
            acc_e = exps[t]
            acc += sums[t]
        elif d < 0:
            acc += (sums[t] >> -d) if -d <= ACC_W - 1 else 0
        else:
            acc += sums[t]
    mean = (acc * inv_d) >> 32
    lead = _lead(mean)
    if (acc_e + lead) & 1:
        lead -= 1
    v = (mean >> (lead - 30) if lead >= 30 else mean << (30 - lead)) + EPS_Q30
    inv = RMS_SEED_Q12_12.get(_lead(v), (1 << 24) - 1)
    C = (3 * (1 << 30)) // 2
    for _ in range(3):
        vy2 = (v * inv * inv) >> 24
        corr = 0 if vy2 >= (1 << 32) else max(0, C - (vy2 >> 1))
        inv = min((inv * corr + (1 << 29)) >> 30, (1 << 24) - 1)
    e_inv = (30 - acc_e - lead) >> 1
    out_m = np.zeros(D, np.int16)
    out_e = np.zeros(nt, np.int8)
    for t in range(nt):
        prods = [int(x_m[t, k]) * int(g_m[t, k]) * inv for k in range(TILE)]
        ml = max([_lead(p) for p in prods if p] or [0])
        for k in range(TILE):
            out_m[t * TILE + k], sh = _norm16(prods[k], ml)
        out_e[t] = _clamp8(int(x_e[t]) + int(g_e[t]) + e_inv + (ml - 14) - 27)
    return out_m, out_e


# -------------------------------------------------------------------- rope
PI_HALF_Q27 = 210828714
PI_Q27 = 421657428
PI_OVER_8_Q29 = 210828714
K_Q3_27 = 81504109
ATAN_Q3_27 = [105414357, 62229729, 32880480, 16690645, 8377711, 4192939, 2096981, 1048555,
              524285, 262144, 131072, 65536, 32768, 16384, 8192, 4096]
"""CORDIC constants of cordic_sincos.sv (gen_rope_bfp_golden.py:28-34)."""


def rope_freq_turns(base=10000.0, head_dim=64):
    """FREQ_TURNS_Q31 (sim/gen_rope_freq_table.py:31-37): round(freq/(2 pi)
    * 2^31) with freq = 1/base^(2j/head_dim)."""
    out = []
    for j in range(head_dim // 2):
        f = 1.0 / (base ** (2.0 * j / head_dim))
        out.append(round(f / (2.0 * math.pi) * (1 << 31)))
    return out


def cordic_sincos(a):
    """16-iteration Q3.27 CORDIC (gen_rope_bfp_golden.py:37-60) -> Q1.15
    (cos, sin)."""
    if a > PI_HALF_Q27:
        z, neg = PI_Q27 - a, True
    elif a < -PI_HALF_Q27:
        z, neg = -PI_Q27 - a, True
    else:
        z, neg = a, False
    x, y = K_Q3_27, 0
    for i in range(16):
        xs, ys = x >> i, y >> i
        if z >= 0:
            x, y, z = x - ys, y + xs, z - ATAN_Q3_27[i]
        else:
            x, y, z = x + ys, y - xs, z + ATAN_Q3_27[i]
    xr, yr = (x + 2048) >> 12, (y + 2048) >> 12
    if xr > 32767:
        c = -32767 if neg else 32767
    elif xr < -32768:
        c = 32767 if neg else -32768
    else:
        c = -xr if neg else xr
    s = max(-32768, min(32767, yr))
    return c, s


def _wrap31(v):
    v &= (1 << 31) - 1
    return v - (1 << 31) if v & (1 << 30) else v


def rope_angle_q27(pos, freq_q31):
    """Angle of pair j at pos in Q3.27 (gen_rope_bfp_golden.py:77-83)."""
    turns = _wrap31(pos * freq_q31)
    return _wrap31((turns * PI_OVER_8_Q29) >> 29)


def rtl_rope(x_m, x_e, pos, freq):
    """rope_bfp.sv golden (gen_rope_bfp_golden.py:72-121) for one 64-wide
    head: pair (j, j+32) aligned to its larger exponent (>>, 0 when >= 16),
    rotated by the CORDIC (cos, sin), re-normalised per element.  Returns
    (m (64,), e (64,)) -- one exponent per element."""
    x_m = np.asarray(x_m, np.int64).reshape(-1)
    x_e = np.asarray(x_e, np.int64).reshape(-1)
    hd = x_m.size
    h2 = hd // 2
    prod = [0] * hd
    ee = [0] * hd
    for j in range(h2):
        c, s = cordic_sincos(rope_angle_q27(pos, freq[j]))
        a, b = int(x_m[j]), int(x_m[j + h2])
        ea, eb = int(x_e[j // TILE]), int(x_e[(j + h2) // TILE])
        em = max(ea, eb)
        aa = a >> (em - ea) if em - ea < 16 else 0
        ba = b >> (em - eb) if em - eb < 16 else 0
        prod[j] = aa * c - ba * s
        prod[j + h2] = ba * c + aa * s
        ee[j] = ee[j + h2] = em
    out_m = np.zeros(hd, np.int16)
    out_e = np.zeros(hd, np.int8)
    for k in range(hd):
        out_m[k], sh = _norm16(prod[k], _lead(prod[k]))
        out_e[k] = _clamp8(ee[k] + sh - 15)
    return out_m, out_e


# ----------------------------------------------------------------- softmax
def exp_lut():
    """EXP_LUT[i] = round(exp((i - 1023)/128) * 32768), clamped to uint16
    (sim/gen_exp_lut.py:36-42)."""
    return [min(65535, max(0, round(math.exp((i - 1023) / 128.0) * 32768))) for i in range(1024)]


def rtl_softmax(x_m, e_shared, n, lut):
    """softmax_bfp.sv golden (gen_softmax_bfp_golden.py:33-78): LUT exp of
    the shifted difference to the max, 4-step Newton-Raphson reciprocal,
    one shared output exponent.  Returns (m (n,), e)."""
    xs = [int(v) for v in np.asarray(x_m).reshape(-1)[:n]]
    mx = max(xs)
    sh = e_shared - 8
    vals = []
    for v in xs:
        d = v - mx
        ds = d << sh if sh >= 0 else d >> (-sh)
        idx = 1023 if ds >= 0 else (0 if ds <= -1023 else ds + 1023)
        vals.append(int(lut[idx]))
    tot = sum(vals)
    y = 1 << (31 - _lead(tot))
    for _ in range(4):
        y = (y * ((1 << 33) - tot * y)) >> 32
    prods = [v * y for v in vals]
    ml = max([_lead(p) for p in prods if p] or [0])
    out = np.array([_norm16(p, ml)[0] for p in prods], np.int16)
    return out, _clamp8(ml - 14 - 17)


def rtl_score_prealign(s_m, s_e, n):
    """The layer's pre-align of QK scores before the softmax
    (smollm_layer_bfp.sv:2038-2053): each score (per-timestep exponent)
    shifted to the shared max exponent (0 when >= 16); the shared exponent
    drops by 3 for 1/sqrt(64)."""
    s_m = [int(v) for v in np.asarray(s_m).reshape(-1)[:n]]
    s_e = [int(v) for v in np.asarray(s_e).reshape(-1)[:n]]
    es = max(s_e)
    m = [0 if es - e >= 16 else v >> (es - e) for v, e in zip(s_m, s_e)]
    return np.array(m, np.int16), es - 3


# ------------------------------------------------------------------ swiglu
SILU_LUT_SCALE_LOG2 = 5


def silu_lut():
    """SILU_LUT over all 65536 int16 codes (sim/gen_swiglu_lut.py:27-44):
    x = code/32768 * 32, silu(x) = x * (1/(1 + exp(-x))), back to Q at
    scale 32 with round-half-even, clipped.  Indexed by code & 0xFFFF."""
    code = np.arange(65536, dtype=np.uint16).view(np.int16).astype(np.float64)
    g = code / 32768.0 * 32.0
    s = g * (1.0 / (1.0 + np.exp(-g)))
    return np.clip(np.round(s * 32768.0 / 32.0).astype(np.int64), -32768, 32767).astype(np.int16)


def rtl_swiglu(g_m, g_e, u_m, u_e, lut):
    """swiglu_bfp.sv golden (gen_swiglu_bfp_golden.py:43-78)."""
    g_m = np.asarray(g_m, np.int64).reshape(-1, TILE)
    u_m = np.asarray(u_m, np.int64).reshape(-1, TILE)
    nt = g_m.shape[0]
    out_m = np.zeros(nt * TILE, np.int16)
    out_e = np.zeros(nt, np.int8)
    for t in range(nt):
        sh = int(g_e[t]) - SILU_LUT_SCALE_LOG2
        prods = []
        for k in range(TILE):
            mg = int(g_m[t, k])
            idx = mg << sh if sh >= 0 else mg >> (-sh)
            idx = max(-32768, min(32767, idx))
            prods.append(int(lut[idx & 0xFFFF]) * int(u_m[t, k]))
        ml = max([_lead(p) for p in prods if p] or [0])
        for k in range(TILE):
            out_m[t * TILE + k], s = _norm16(prods[k], ml)
        out_e[t] = _clamp8(int(u_e[t]) + (ml - 14) - 10)
    return out_m, out_e


# ---------------------------------------------------------------- residual
def rtl_residual(a_m, a_e, b_m, b_e):
    """residual_bfp.sv golden (gen_residual_bfp_golden.py:23-48)."""
    a_m = np.asarray(a_m, np.int64).reshape(-1, TILE)
    b_m = np.asarray(b_m, np.int64).reshape(-1, TILE)
    nt = a_m.shape[0]
    out_m = np.zeros(nt * TILE, np.int16)
    out_e = np.zeros(nt, np.int8)
    for t in range(nt):
        ea, eb = int(a_e[t]), int(b_e[t])
        em = max(ea, eb)
        sums = []
        for k in range(TILE):
            av = int(a_m[t, k]) >> (em - ea) if em - ea < 16 else 0
            bv = int(b_m[t, k]) >> (em - eb) if em - eb < 16 else 0
            sums.append(av + bv)
        ml = max([_lead(s) for s in sums if s] or [0])
        for k in range(TILE):
            out_m[t * TILE + k], sh = _norm16(sums[k], ml)
        out_e[t] = _clamp8(em + ml - 14)
    return out_m, out_e


# ------------------------------------------------------------------ argmax
def bfp_gt(ma, ea, mb, eb):
    """(ma, ea) > (mb, eb) after aligning to the larger exponent
    (smollm_decode_head_bfp.sv:253-274)."""
    de = ea - eb
    if de == 0:
        return ma > mb
    if de > 0:
        return ma > (0 if de >= 16 else mb >> de)
    return (0 if -de >= 16 else ma >> -de) > mb


def rtl_argmax(m, e):
    """The decode head's running argmax (smollm_decode_head_bfp.sv:322-324,
    399-430): per 16-lane chunk, a local best starting at lane 0 replaced on
    strict bfp_gt; chunks folded into a global best that starts at
    (-32768, -128), also on strict bfp_gt.  m, e: one per row."""
    m = [int(v) for v in np.asarray(m).reshape(-1)]
    e = [int(v) for v in np.asarray(e).reshape(-1)]
    best_m, best_e, best_i = -32768, -128, 0
    for c in range(len(m) // TILE):
        lm, le, li = m[c * TILE], e[c * TILE], 0
        for k in range(1, TILE):
            if bfp_gt(m[c * TILE + k], e[c * TILE + k], lm, le):
                lm, le, li = m[c * TILE + k], e[c * TILE + k], k
        if bfp_gt(lm, le, best_m, best_e):
            best_m, best_e, best_i = lm, le, c * TILE + li
    return best_i


# ------------------------------------------------------- composed RTL layer
class RtlTables:
    """The engines' lookup tables: EXP_LUT, SILU_LUT, FREQ_TURNS_Q31."""

    def __init__(self, head_dim=64, base=10000.0):
        self.exp = exp_lut()
        self.silu = silu_lut()
        self.freq = rope_freq_turns(base, head_dim)


def rtl_kv_cache(max_ctx, kv):
    """One layer's RTL KV cache: per position the post-RoPE K and the V as
    BFP (m per element, e per 16-element tile)."""
    return {"k_m": np.zeros((max_ctx, kv), np.int16), "k_e": np.zeros((max_ctx, kv // TILE), np.int8),
            "v_m": np.zeros((max_ctx, kv), np.int16), "v_e": np.zeros((max_ctx, kv // TILE), np.int8)}


def _mv_tile(x_m, x_e, W):
    """A matvec on the engine, then the chunk re-tile (S_xMV_DRAIN/REQ):
    per-lane (m, e) -> requant per 16 output rows."""
    Wm, We = W
    nt = We.shape[1]
    m, e = rtl_matvec(np.asarray(x_m).reshape(nt, TILE), np.asarray(x_e).reshape(-1), Wm, We)
    return rtl_requant(m, e)


def rtl_fwd_layer(h_m, h_e, lw, pos, kv_pos, kv, tabs, dims, stages=None):
    """One decoder layer as smollm_layer_bfp.sv:1603-2600 wires its engines.

    h (D BFP) -> out (D BFP); kv (rtl_kv_cache) gets slot kv_pos.  lw holds
    the layer's (m, e) matrices and float gammas (BFP-exact; the ROM holds
    their tile_quantize).  Order of the FSM:
      NORM1 -> Q/K/V matvec + re-tile (:1616-1829) -> RoPE per head and
      re-tile (:1831-1954) -> KV write (:1956-1974) -> per head: QK on the
      engine's lane 0 for t = 0..kv_pos (:1976-2036), pre-align to the
      shared max exponent and softmax with exponent - 3 (:2038-2072), AV per
      16-dim chunk with V pre-shifted to its max exponent over t <= kv_pos
      and one 16-input tile of probabilities (t <= 15 only, :2074-2226) ->
      O matvec (:2228-2294) -> residual 1 (:2296-2327) -> NORM2
      (:2329-2349) -> G, U matvecs -> SwiGLU (:2470-2494) -> D matvec ->
      residual 2 (:2496-2580).
    ``stages`` (optional dict) receives each stage's (m, e) under the
    names N1 Q K V ATTN O H1 N2 G U MLP D HOUT (Q, K after RoPE)."""
    from . import bfp_sim as sim
    D, H_Q, H_KV, HD = dims.D, dims.H_Q, dims.H_KV, dims.HD
    KV = H_KV * HD
    st = stages if stages is not None else {}

    def gamma(g):
        m, e = sim.tile_quantize(np.asarray(g, np.float64))
        return m.reshape(-1), e

    n1 = rtl_rmsnorm(h_m, h_e, *gamma(lw["g1"]))
    st["N1"] = n1
    q = _mv_tile(*n1, lw["Wq"])
    k = _mv_tile(*n1, lw["Wk"])
    v = _mv_tile(*n1, lw["Wv"])
    st["V"] = v

    def rope_all(x, n_heads):
        xm, xe = x
        om, oe = np.zeros(n_heads * HD, np.int16), np.zeros(n_heads * HD // TILE, np.int8)
        for hh in range(n_heads):
            rm, re = rtl_rope(xm[hh * HD:(hh + 1) * HD], xe[hh * HD // TILE:(hh + 1) * HD // TILE],
                              pos, tabs.freq)
            tm, te = rtl_requant(rm, re)
            om[hh * HD:(hh + 1) * HD], oe[hh * HD // TILE:(hh + 1) * HD // TILE] = tm, te
        return om, oe

    q = rope_all(q, H_Q)
    k = rope_all(k, H_KV)
    st["Q"], st["K"] = q, k
    kv["k_m"][kv_pos], kv["k_e"][kv_pos] = k
    kv["v_m"][kv_pos], kv["v_e"][kv_pos] = v

    att_m, att_e = np.zeros(D, np.int16), np.zeros(D // TILE, np.int8)
    ntq = HD // TILE
    n = kv_pos + 1
    for hh in range(H_Q):
        g = (hh * H_KV) // H_Q
        qm = q[0][hh * HD:(hh + 1) * HD].reshape(ntq, TILE)
        qe = q[1][hh * ntq:(hh + 1) * ntq]
        sm, se = np.zeros(n, np.int64), np.zeros(n, np.int64)
        for t in range(n):
            km = kv["k_m"][t, g * HD:(g + 1) * HD].reshape(1, ntq, TILE)
            ke = kv["k_e"][t, g * ntq:(g + 1) * ntq].reshape(1, ntq)
            m1, e1 = rtl_matvec(qm, qe, km, ke)
            sm[t], se[t] = int(m1[0]), int(e1[0])
        es = max(-128, int(se.max()))
        xm = [0 if es - int(se[t]) >= 16 else int(sm[t]) >> (es - int(se[t])) for t in range(n)]
        pm, pe = rtl_softmax(xm, _wrap8(es - 3), n, tabs.exp)
        x_av = np.zeros((1, TILE), np.int64)
        x_av[0, :min(n, TILE)] = pm[:min(n, TILE)]
        for c in range(ntq):
            tile = g * ntq + c
            emax = int(kv["v_e"][:n, tile].max())
            W = np.zeros((TILE, 1, TILE), np.int64)
            for t in range(min(n, TILE)):
                for lane in range(TILE):
                    W[lane, 0, t] = shr8(kv["v_m"][t, tile * TILE + lane], emax,
                                         kv["v_e"][t, tile])
            m16, e16 = rtl_matvec(x_av, np.array([int(pe)]), W, np.full((TILE, 1), emax))
            tm, te = rtl_requant(m16, e16)
            att_m[(hh * ntq + c) * TILE:(hh * ntq + c + 1) * TILE] = tm
            att_e[hh * ntq + c] = te[0]
    st["ATTN"] = (att_m, att_e)
    o = _mv_tile(att_m, att_e, lw["Wo"])
    st["O"] = o
    h1 = rtl_residual(h_m, h_e, *o)
    st["H1"] = h1
    n2 = rtl_rmsnorm(*h1, *gamma(lw["g2"]))
    st["N2"] = n2
    gg = _mv_tile(*n2, lw["Wg"])
    uu = _mv_tile(*n2, lw["Wu"])
    st["G"], st["U"] = gg, uu
    mlp = rtl_swiglu(*gg, *uu, tabs.silu)
    st["MLP"] = mlp
    dd = _mv_tile(*mlp, lw["Wd"])
    st["D"] = dd
    out = rtl_residual(*h1, *dd)
    st["HOUT"] = out
    return out


# ------------------------------------------------------------- decode head
def embed_q(embed):
    """The tied embedding as the FPGA image holds it: every row
    tile_quantize'd (gen_smollm_blockfp_ddr.py:203-216); (m (V, nt, 16),
    e (V, nt))."""
    from . import bfp_sim as sim
    V, D = embed.shape
    m, e = sim.tile_quantize(np.asarray(embed, np.float64).reshape(-1))
    return m.reshape(V, D // TILE, TILE), e.reshape(V, D // TILE)


def rtl_head(h_m, h_e, norm_w, emb):
    """smollm_decode_head_bfp.sv:303-430: S_NORM (the RMSNorm engine with the
    final norm gamma from its ROM, i.e. tile_quantize'd), the lm_head as one
    matvec-engine pass per 16 embedding rows (S_MV_*, per-row (m, e)), and
    the bfp_gt running argmax (S_MV_LANE_CMP / S_MV_MERGE).  emb: embed_q's
    (m, e).  Returns (logit_m, logit_e, token).

    Parity of the composition: the three ops are the per-op restatements
    above (each pinned by the reference's golden recipes); the wiring is
    pinned by tests/test_oracle_rtl_head.py, which checks the logits against
    the exact float64 dot products within the engine's truncation bound and
    the token against the exact argmax where the top two are apart."""
    from . import bfp_sim as sim
    g_m, g_e = sim.tile_quantize(np.asarray(norm_w, np.float64))
    xm, xe = rtl_rmsnorm(h_m, h_e, g_m.reshape(-1), g_e)
    Wm, We = emb
    nt = We.shape[1]
    lm, le = rtl_matvec(np.asarray(xm).reshape(nt, TILE), np.asarray(xe).reshape(-1), Wm, We)
    return lm, le, rtl_argmax(lm, le)


def rtl_decode(model, prompt, n_gen, tabs, dims, max_ctx=None, on_step=None):
    """The FPGA's token loop (autoregress_bfp_top.sv:357-386) over the
    composed RTL layer and head: step s embeds prompt[s] while s <
    len(prompt), else the prediction of step s-1 (the tile-quantised
    embedding row), runs every layer at position and KV slot s, and records
    the head's prediction (the loop policy of bfp_sim.decode_rtl_loop).
    model: a bfp_sim.Model.  on_step(step, h_m, h_e) sees the last layer's
    output.  Returns the len(prompt) + n_gen predictions."""
    from . import bfp_sim as sim
    ids = [int(t) for t in prompt]
    steps = len(ids) + int(n_gen)
    n_ctx = max_ctx if max_ctx is not None else steps
    KV = dims.H_KV * dims.HD
    kv = [rtl_kv_cache(n_ctx, KV) for _ in range(dims.NL)]
    emb = embed_q(model.embed)
    preds = []
    for step in range(steps):
        tid = ids[step] if step < len(ids) else preds[-1]
        h_m, h_e = sim.tile_quantize(np.asarray(model.embed[tid], np.float64))
        h_m = h_m.reshape(-1)
        for li in range(dims.NL):
            h_m, h_e = rtl_fwd_layer(h_m, h_e, model.layers[li], step, step, kv[li], tabs, dims)
        if on_step is not None:
            on_step(step, h_m, h_e)
        preds.append(rtl_head(h_m, h_e, model.norm_w_q, emb)[2])
    return preds
