// The attention of one KV group of one sequence -- all its query heads in
// one workgroup -- for contexts of at most 256 positions
// (rtl/vc707/host/gen_smollm_blockfp_full.py:268-283; the lane-split short
// forms of attn_body, bfp_layer_dev.h).
//
// Every query head of a group reads the same K and V rows, so a workgroup
// that takes the whole group loads each K row and stages each V row once
// for all of them: wave h < G rotates q head h, wave G the group's k and
// wave G + 1 its v; every 32-lane half-wave scores one position against all
// G heads; wave h runs head h's softmax and AV add chain.  The
// arithmetic of each head -- the SkylakeX ddot order of the scores, numpy's
// softmax and pairwise sum, the ascending-t AV chain -- is attn_body's, so
// the outputs are bit-identical to the one-head-per-workgroup form (whose
// softmax past 128 positions is block-wide: here each head's stays in its
// wave, up to 256).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bfp_layer_dev.h"

namespace bfp {

constexpr int AG_MAXG = 4;   // query heads per KV group

// LDS bytes of attn_group_body for G heads per group and PB rows of AV
// products per head.
inline size_t attn_grp_lds_bytes(int max_ctx, int G, int PB) {
  const size_t scl = (size_t)((max_ctx + 1) & ~1);
  return ((size_t)64 * G + 128) * 8 + (size_t)G * scl * 8 + (size_t)2 * ATT_AVC * (64 * 2 + 4) +
         (size_t)G * PB * 64 * 8;
}

// KV group g of sequence b: its G = H_Q / H_KV query heads g*G .. g*G+G-1,
// over KV slots 0..pos with RoPE position rpos (posf); io as for attn_body
// (its k_put / v_put store the cache row, out the outputs).  PPW 2: at most
// 128 positions; 3: at most 256.  PB: rows of AV products per head held in
// LDS at once (a multiple of 16, at most ATT_AVC).  a.dump must be null.
template <int PPW, int PB, class IO, class PosF>
__device__ __forceinline__ void attn_group_body(const LayerArgs &a, IO &io, int g, int b, PosF posf,
                                                double *dsm) {
  static_assert(PPW == 2 || PPW == 3, "the lane-split short forms");
  constexpr int NT = 64 * ATT_WAVES;
  constexpr int AVC = ATT_AVC;
  constexpr int VL = AVC * 8 / NT;
  constexpr int LS_PASS = (PPW == 2 ? 128 : 256) / (2 * ATT_WAVES);
  constexpr int LS_PRE = LS_PASS < 8 ? LS_PASS : 8;
  static_assert(PB % 16 == 0 && PB <= ATT_AVC, "AV product block");
  const int G = a.H_Q / a.H_KV;
  const int HD = 64;
  const int scl = (a.max_ctx + 1) & ~1;
  double *q = dsm;                   // G x 64
  double *kc = dsm + 64 * G;         // 64 (current position, post-rope)
  double *vc = kc + 64;              // 64
  double *sc = vc + 64;              // G x scl: scores, then probabilities
  int16_t *vsm = reinterpret_cast<int16_t *>(sc + G * scl);   // 2 x AVC x 64
  int8_t *vse = reinterpret_cast<int8_t *>(vsm + 2 * AVC * 64);  // 2 x AVC x 4
  double *prod = reinterpret_cast<double *>(vse + 2 * AVC * 4);  // G x PB x 64
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const long long kv_tok = (long long)a.H_KV * HD;   // elements per position
  int16_t *Km = a.k_m + (long long)b * a.max_ctx * kv_tok;
  int8_t *Ke = a.k_e + (long long)b * a.max_ctx * (kv_tok / 16);
  int16_t *Vm = a.v_m + (long long)b * a.max_ctx * kv_tok;
  int8_t *Ve = a.v_e + (long long)b * a.max_ctx * (kv_tok / 16);

  // the K elements of LS_PRE passes of 2 * ATT_WAVES positions: half-wave
  // (w, l / 32) scores position 2 * ATT_WAVES * pass + 2w + l / 32, lane
  // j = l % 32 holding elements j and 32 + j (rows clamped to `last`)
  int lsm[LS_PRE][2], lse[LS_PRE][2];
  auto ls_load = [&](int g0, int last) {
#pragma unroll
    for (int ps_ = 0; ps_ < LS_PRE; ++ps_) {
      int t = 2 * ATT_WAVES * (g0 + ps_) + 2 * w + (l >> 5);
      t = t < last ? t : last;
      const long long o = ((long long)t * a.H_KV + g) * HD + (l & 31);
      lsm[ps_][0] = io.km1(Km + o);
      lsm[ps_][1] = io.km1(Km + o + 32);
      lse[ps_][0] = io.ke1(Ke + (o >> 4));
      lse[ps_][1] = io.ke1(Ke + ((o + 32) >> 4));
    }
  };
  ls_load(0, a.max_ctx - 1);
  // V staging: chunk c holds rows c*AVC .. c*AVC+AVC-1 (clamped to `last`,
  // so no load sits in a branch); thread tid loads 16-byte part tid%8 of
  // rows tid/8 + 64j and, for tid < AVC, the 4 exponent bytes of row tid
  uint4 vr[VL];
  int ver = 0;
  const int16_t *Vg = Vm + (long long)g * HD + 8 * (tid & 7);
  const int8_t *Veg = Ve + (long long)g * (HD / 16);
  const long long vstride = kv_tok;
  auto load_v = [&](int c, int last) {
#pragma unroll
    for (int j = 0; j < VL; ++j) {
      int t_ = c * AVC + (tid >> 3) + j * (NT / 8);
      t_ = t_ < last ? t_ : last;
      vr[j] = io.v16(Vg + t_ * vstride);
    }
    int t_ = c * AVC + (tid < AVC ? tid : 0);
    t_ = t_ < last ? t_ : last;
    ver = io.ve4(Veg + t_ * (vstride / 16));
  };
  auto store_v = [&](int c) {
    int16_t *dst = vsm + (c & 1) * AVC * 64;
#pragma unroll
    for (int j = 0; j < VL; ++j)
      *reinterpret_cast<uint4 *>(dst + ((tid >> 3) + j * (NT / 8)) * 64 + 8 * (tid & 7)) = vr[j];
    if (tid < AVC) *reinterpret_cast<int *>(vse + (c & 1) * AVC * 4 + tid * 4) = ver;
  };
  // the first V chunk is loaded with the K elements, before the q|k|v input
  // and the position (rows past the position are never used)
  load_v(0, a.max_ctx - 1);
  // this wave's q|k|v input: q head g*G + w (waves below G), k (wave G),
  // v (the rest, which only wave G + 1 uses)
  int in_m, in_e;
  io.qkv(w < G ? (g * G + w) * HD + l : (w == G ? a.D + g * HD + l : a.D + a.KV + g * HD + l), in_m, in_e);
  io.mark(ATT_MARK_QKV);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const int2 pp = posf();   // (KV slot, RoPE position)
  const int pos = pp.x, rpos = pp.y;
  const int n = pos + 1;
  const double *cs = a.rope + (long long)rpos * HD;
  double rcos = 0.0, rsin = 0.0;
  if (w <= G) io.rope_cs(cs, l & 31, rcos, rsin);

  // RoPE of the G q heads and of k; k and v of slot pos into the cache
  if (w < G) {
    int e;
    const int m = rope_lane(bfp_val(in_m, in_e), rcos, rsin, e);
    q[w * 64 + l] = bfp_val(m, e);
  } else if (w == G) {
    int e;
    const int m = rope_lane(bfp_val(in_m, in_e), rcos, rsin, e);
    kc[l] = bfp_val(m, e);
    const long long o = ((long long)pos * a.H_KV + g) * HD + l;
    io.k_put(Km + o, Ke + (o >> 4), m, e, (l & 15) == 0);
  } else if (w == G + 1) {
    vc[l] = bfp_val(in_m, in_e);
    const long long o = ((long long)pos * a.H_KV + g) * HD + l;
    io.v_put(Vm + o, Ve + (o >> 4), in_m, in_e, (l & 15) == 0);
  }
  lds_barrier();
  io.mark(ATT_MARK_ROPE);

  // scores[h][t] = float(np.dot(q_h, K[t])) / sqrt(HD)   (full.py:277-278):
  // attn_body's lane-split SkylakeX ddot order, every head against the
  // half-wave's row; row pos from LDS (its writer may not have stored it)
  {
    const int j = l & 31;
    double q0[AG_MAXG], q1[AG_MAXG];
#pragma unroll
    for (int h = 0; h < AG_MAXG; ++h) {
      q0[h] = h < G ? q[h * 64 + j] : 0.0;
      q1[h] = h < G ? q[h * 64 + 32 + j] : 0.0;
    }
    const double k0 = kc[j], k1 = kc[32 + j];
    for (int g0 = 0; g0 < LS_PASS && 2 * ATT_WAVES * g0 < n; g0 += LS_PRE) {   // uniform
      if (g0 > 0) ls_load(g0, n - 1);
#pragma unroll
      for (int ps_ = 0; ps_ < LS_PRE; ++ps_) {
        if (2 * ATT_WAVES * (g0 + ps_) >= n) break;   // uniform
        const int t = 2 * ATT_WAVES * (g0 + ps_) + 2 * w + (l >> 5);
        const double y0 = t == pos ? k0 : bfp_val(lsm[ps_][0], lse[ps_][0]);
        const double y1 = t == pos ? k1 : bfp_val(lsm[ps_][1], lse[ps_][1]);
#pragma unroll
        for (int h = 0; h < AG_MAXG; ++h) {
          if (h < G) {   // uniform
            const double acc = fma(q1[h], y1, fma(q0[h], y0, 0.0));
            const double f = acc + peer<4>(acc);
            const double t01 = peer<16>(f + peer<8>(f));
            const double sl = (t01 + peer<8>(f)) + f;
            const double s2 = sl + peer<2>(sl);
            const double tot = s2 + peer<1>(s2);
            if (j == 31 && t < n) sc[h * scl + t] = tot * a.score_mul;
          }
        }
      }
    }
  }
  store_v(0);
  lds_barrier();
  io.mark(ATT_MARK_SCORES);
  // softmax_fp (full.py:245-247) of each head, wave h on head h: lane l
  // holds positions l + 64i; numpy's pairwise sum in one wave (at most
  // three leaves, pairwise_sum_wave256), so the G heads run side by side
  {
    constexpr int NV = PPW == 2 ? 2 : 4;   // positions per lane
    if (w < G) {
      double *sh = sc + w * scl;
      double s[NV], e[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) s[i] = l + 64 * i < n ? sh[l + 64 * i] : -INFINITY;
      double mx = s[0];
#pragma unroll
      for (int i = 1; i < NV; ++i) mx = fmax(mx, s[i]);
      mx = fmax(mx, peer<32>(mx));
      mx = fmax(mx, peer<16>(mx));
      mx = fmax(mx, peer<8>(mx));
      mx = fmax(mx, peer<4>(mx));
      mx = fmax(mx, peer<2>(mx));
      mx = fmax(mx, peer<1>(mx));
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (64 * i < n) {   // uniform
          e[i] = exp_f64(s[i] - mx);
          if (l + 64 * i < n) sh[l + 64 * i] = e[i];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      const double sum = pairwise_sum_wave256(sh, n);
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (l + 64 * i < n) sh[l + 64 * i] = e[i] / sum;
    }
    lds_barrier();
  }
  io.mark(ATT_MARK_SOFTMAX);

  // attn_h = sum_t p_h[t] * V[t], ascending t from 0.0 (full.py:280-281):
  // every thread forms a block of PB rows' products of every head into LDS,
  // wave h adds head h's, one dimension per lane; row pos (this launch's V)
  // last
  double acc = 0.0;
  const int nch = (n + AVC - 1) / AVC;
  for (int c = 0; c < nch; ++c) {
    load_v(c + 1 < nch ? c + 1 : c, n - 1);
    const int t0 = c * AVC, t1 = min(pos, t0 + AVC);   // rows t0 .. t1-1
    const int16_t *vmc = vsm + (c & 1) * AVC * 64;
    const int8_t *vec = vse + (c & 1) * AVC * 4;
    for (int r0 = 0; r0 < t1 - t0; r0 += PB) {   // uniform
      const int nr = min(PB, t1 - t0 - r0);
      // each V element decoded once, its product with every head's p
      for (int qq = tid; qq < nr * 64; qq += NT) {
        const int r = r0 + (qq >> 6), dd = qq & 63;
        const double v = ldexp((double)vmc[r * 64 + dd], (int)vec[r * 4 + (dd >> 4)] - 15);
        for (int h = 0; h < G; ++h) prod[h * PB * 64 + qq] = sc[h * scl + t0 + r] * v;
      }
      lds_barrier();
      if (w < G) {
        const double *pl = prod + w * PB * 64 + l;
        int r = 0;
        for (; r + 16 <= nr; r += 16) {
          double pv[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) pv[i] = pl[(r + i) * 64];
#pragma unroll
          for (int i = 0; i < 16; ++i) acc = acc + pv[i];
        }
        for (; r < nr; ++r) acc = acc + pl[r * 64];
      }
      lds_barrier();   // the block's LDS is refilled
    }
    if (w < G && c == nch - 1) acc = acc + sc[w * scl + pos] * vc[l];
    if (c + 1 < nch) store_v(c + 1);
    lds_barrier();
  }
  io.mark(ATT_MARK_AV);
  io.before_out();
  if (w < G) {
    int e;
    const int m = quantize16_lanes(acc, e, true);   // tile_quantize(fp_quantize_vec(attn))
    io.out((g * G + w) * HD + l, m, e, (l & 15) == 0);
  }
}

}  // namespace bfp
