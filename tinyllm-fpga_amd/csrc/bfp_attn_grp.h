// The attention of one KV group of one sequence -- all its query heads in
// one workgroup -- for contexts of at most 256 positions
// (rtl/vc707/host/gen_smollm_blockfp_full.py:268-283; the lane-split short
// forms of attn_body, bfp_layer_dev.h).
//
// Every query head of a group reads the same K and V rows, so a workgroup
// that takes the whole group stages each K and V row in LDS once for all
// of them: wave h < G rotates q head h, wave G the group's k and wave G + 1
// its v; each lane scores one (head, position) pair on its own
// (ddot64_skx_bfp, no cross-lane steps); wave h runs head h's softmax and
// its AV add chains, one dimension per lane, straight from the staged V
// rows.  The arithmetic of each head -- the SkylakeX ddot order of the
// scores, numpy's softmax and pairwise sum, the ascending-t AV chain -- is
// attn_body's, so the outputs are bit-identical to the one-head-per-
// workgroup form.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bfp_layer_dev.h"

namespace bfp {

constexpr int AG_MAXG = 4;   // query heads per KV group
constexpr int AG_KS = 72;    // K row stride in LDS (int16): 144 bytes, so the 16-byte
                             // reads of 8 consecutive rows hit 8 distinct bank groups

// LDS bytes of attn_group_body for G heads per group: q, the scores, the
// staged V rows (64 mantissas a row) and K rows (AG_KS) with their
// exponents (4 a row).
inline size_t attn_grp_lds_bytes(int max_ctx, int G) {
  const size_t scl = (size_t)((max_ctx + 1) & ~1);
  const size_t ex = (scl * 4 + 15) & ~(size_t)15;
  return (size_t)64 * G * 8 + (size_t)G * scl * 8 + scl * 64 * 2 + ex + scl * AG_KS * 2 + ex;
}

// KV group g of sequence b: its G = H_Q / H_KV query heads g*G .. g*G+G-1,
// over KV slots 0..pos with RoPE position rpos (posf); io as for attn_body
// (its k_put / v_put store the cache row, out the outputs).  PPW 2: at most
// 128 positions; 3: at most 256.  a.dump must be null.
//
// The K and V rows 0 .. pos-1 of the cache (the group's 64 mantissas and 4
// exponents a row) are loaded at entry, before the q|k|v input is in, in
// 16-byte parts (thread t: part t % 8 of rows t / 8 + 64j), and written to
// LDS once the input is in; row pos is this launch's k (after RoPE) and v,
// written by waves G and G + 1 instead.
template <int PPW, class IO, class PosF>
__device__ __forceinline__ void attn_group_body(const LayerArgs &a, IO &io, int g, int b, PosF posf,
                                                double *dsm) {
  static_assert(PPW == 2 || PPW == 3, "the lane-split short forms");
  constexpr int NT = 64 * ATT_WAVES;
  constexpr int RT = PPW == 2 ? 2 : 4;           // staged rows per thread: 64 * RT >= max_ctx
  constexpr int ER = PPW == 2 ? 128 : 256;       // rows whose exponents a thread may load
  static_assert(NT == 512, "staging geometry");
  const int G = a.H_Q / a.H_KV;
  const int HD = 64;
  const int scl = (a.max_ctx + 1) & ~1;
  const int exb = (scl * 4 + 15) & ~15;
  double *q = dsm;                                                // G x 64
  double *sc = q + 64 * G;                                        // G x scl: scores, then probabilities
  int16_t *vst = reinterpret_cast<int16_t *>(sc + G * scl);       // scl x 64 V mantissas
  int8_t *vex = reinterpret_cast<int8_t *>(vst + scl * 64);       // scl x 4 V exponents
  int16_t *kst = reinterpret_cast<int16_t *>(vex + exb);          // scl x AG_KS K mantissas
  int8_t *kex = reinterpret_cast<int8_t *>(kst + scl * AG_KS);    // scl x 4 K exponents
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const long long kv_tok = (long long)a.H_KV * HD;   // elements per position
  int16_t *Km = a.k_m + (long long)b * a.max_ctx * kv_tok;
  int8_t *Ke = a.k_e + (long long)b * a.max_ctx * (kv_tok / 16);
  int16_t *Vm = a.v_m + (long long)b * a.max_ctx * kv_tok;
  int8_t *Ve = a.v_e + (long long)b * a.max_ctx * (kv_tok / 16);

  // the position first (the q|k|v input, polled below, arrives well after
  // it), then the staging loads of rows 0 .. pos-1 only (rows from pos on
  // read row 0, a cache hit, and are never used; no load sits in a branch)
  const int2 pp = posf();   // (KV slot, RoPE position)
  const int pos = pp.x, rpos = pp.y;
  uint4 kr[RT], vr[RT];
  {
    const int16_t *Kg = Km + (long long)g * HD + 8 * (tid & 7);
    const int16_t *Vg = Vm + (long long)g * HD + 8 * (tid & 7);
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      int t = (tid >> 3) + 64 * j;
      t = t < pos ? t : 0;
      kr[j] = io.k16(Kg + t * kv_tok);
      vr[j] = io.v16(Vg + t * kv_tok);
    }
  }
  const int te = (tid & (ER - 1)) < pos ? (tid & (ER - 1)) : 0;
  const int ker = io.ke4(Ke + (te * kv_tok + (long long)g * HD) / 16);
  const int ver = io.ve4(Ve + (te * kv_tok + (long long)g * HD) / 16);
  // this wave's q|k|v input: q head g*G + w (waves below G), k (wave G),
  // v (the rest, which only wave G + 1 uses)
  int in_m, in_e;
  io.qkv(w < G ? (g * G + w) * HD + l : (w == G ? a.D + g * HD + l : a.D + a.KV + g * HD + l), in_m, in_e);
  io.mark(ATT_MARK_QKV);
  const int n = pos + 1;
  const double *cs = a.rope + (long long)rpos * HD;
  double rcos = 0.0, rsin = 0.0;
  if (w <= G) io.rope_cs(cs, l & 31, rcos, rsin);

  // RoPE of the G q heads and of k; k and v of slot pos into row pos of the
  // staged rows
  if (w < G) {
    int e;
    const int m = rope_lane(bfp_val(in_m, in_e), rcos, rsin, e);
    q[w * 64 + l] = bfp_val(m, e);
  } else if (w == G) {
    int e;
    const int m = rope_lane(bfp_val(in_m, in_e), rcos, rsin, e);
    kst[pos * AG_KS + l] = (int16_t)m;
    if ((l & 15) == 0) kex[pos * 4 + (l >> 4)] = (int8_t)e;
    in_m = m;   // the cache row, stored after the scores
    in_e = e;
  } else if (w == G + 1) {
    vst[pos * 64 + l] = (int16_t)in_m;
    if ((l & 15) == 0) vex[pos * 4 + (l >> 4)] = (int8_t)in_e;
  }
  // the staged rows 0 .. pos-1 into LDS
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    const int t = (tid >> 3) + 64 * j;
    if (t < pos) {
      *reinterpret_cast<uint4 *>(kst + t * AG_KS + 8 * (tid & 7)) = kr[j];
      *reinterpret_cast<uint4 *>(vst + t * 64 + 8 * (tid & 7)) = vr[j];
    }
  }
  if (tid < ER && tid < pos) {
    *reinterpret_cast<int *>(kex + tid * 4) = ker;
    *reinterpret_cast<int *>(vex + tid * 4) = ver;
  }
  lds_barrier();
  io.mark(ATT_MARK_ROPE);

  // scores[h][t] = float(np.dot(q_h, K[t])) / sqrt(HD)   (full.py:277-278):
  // one (head, position) pair per lane, the SkylakeX ddot order
  for (int i = tid; i < G * n; i += NT) {
    int h = 0, t = i;
    while (t >= n) {
      t -= n;
      ++h;
    }
    const uint4 *km = reinterpret_cast<const uint4 *>(kst + t * AG_KS);
    const int ke = *reinterpret_cast<const int *>(kex + t * 4);
    sc[h * scl + t] = ddot64_skx_bfp(q + h * 64, km, ke) * a.score_mul;
  }
  lds_barrier();
  io.mark(ATT_MARK_SCORES);
  // k and v of slot pos into the cache, by waves G and G + 1 (no work left
  // for them), once the staged rows are in LDS: stored before, the wait for
  // the staged loads would also wait for these stores to complete
  if (w == G || w == G + 1) {
    const long long o = ((long long)pos * a.H_KV + g) * HD + l;
    if (w == G) io.k_put(Km + o, Ke + (o >> 4), in_m, in_e, (l & 15) == 0);
    else io.v_put(Vm + o, Ve + (o >> 4), in_m, in_e, (l & 15) == 0);
  }
  // softmax_fp (full.py:245-247) of each head, wave h on head h: lane l
  // holds positions l + 64i; numpy's pairwise sum in one wave (at most
  // three leaves, pairwise_sum_wave256), so the G heads run side by side
  double acc = 0.0;
  if (w < G) {
    constexpr int NV = PPW == 2 ? 2 : 4;   // positions per lane
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
      e[i] = 0.0;
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
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    io.mark(ATT_MARK_SOFTMAX);

    // attn_h = sum_t p_h[t] * V[t], ascending t from 0.0 (full.py:280-281):
    // lane l adds dimension l's products in order, each V element decoded
    // exactly, the products of 8 rows formed ahead of their adds
    const int16_t *vcol = vst + l;
    const int8_t *vecol = vex + (l >> 4);
    int t = 0;
    for (; t + 8 <= n; t += 8) {
      double pr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        pr[i] = sh[t + i] * ldexp((double)vcol[(t + i) * 64], (int)vecol[(t + i) * 4] - 15);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = acc + pr[i];
    }
    for (; t < n; ++t) acc = acc + sh[t] * ldexp((double)vcol[t * 64], (int)vecol[t * 4] - 15);
    io.mark(ATT_MARK_AV);
  }
  io.before_out();
  if (w < G) {
    int e;
    const int m = quantize16_lanes(acc, e, true);   // tile_quantize(fp_quantize_vec(attn))
    io.out((g * G + w) * HD + l, m, e, (l & 15) == 0);
  }
}

}  // namespace bfp
