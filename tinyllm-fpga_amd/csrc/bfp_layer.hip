// Fused decoder-layer, head and driver kernels of the BFP decode datapath.
//
// One decode step of one layer is five launches (rtl/vc707/host/
// gen_smollm_blockfp_full.py:261-293 is the sequence they implement):
//   qkv   : n1 = rmsnorm(h, g1) (recomputed per workgroup) -> q|k|v matvec
//   attn  : RoPE q,k (per head), KV-cache write, scores/softmax/AV in float64,
//           attn re-quantised                    (one workgroup per q head)
//   o_res : o = Wo attn, h1 = q(h + o)          (residual in the epilogue)
//   gu    : n2 = rmsnorm(h1, g2) -> g, u (same 16 rows per workgroup) ->
//           mlp = q(q(silu(g)) * u)              (SwiGLU in the epilogue)
//   d_res : d = Wd mlp, h_out = q(h1 + d)
// Every launch handles `batch` independent sequences (grid.y).
#include <stdint.h>

#include <map>
#include <mutex>
#include <utility>

#include "bfp.h"
#include "bfp_device.h"
#include "bfp_f64.h"
#include "bfp_internal.h"
#include "bfp_layer.h"
#include "bfp_mv.h"
#include "bfp_mx.h"

namespace bfp {

// Canonical copy (m, e) of a raw tile held one mantissa per lane.
__device__ __forceinline__ void canon_copy(int m, int e, int &cm, int &ce) {
  cm = m;
  ce = e;
  canon16_lanes(cm, ce);
}

__device__ __forceinline__ int cur_pos(const LayerArgs &a) {
  return a.pos_ptr ? *a.pos_ptr : a.pos_const;
}

// The KV slot of this step: the position itself in the decode loop
// (full.py:436), or the caller's kv_pos (fwd_layer's separate argument,
// full.py:261, which the single-layer harness sets apart from pos,
// gen_smollm_blockfp_bfp.py:42-43).
__device__ __forceinline__ int cur_kv_pos(const LayerArgs &a) {
  return a.pos_ptr ? *a.pos_ptr : (a.kv_pos_const >= 0 ? a.kv_pos_const : a.pos_const);
}

// rmsnorm_fp (full.py:236-238) of a BFP vector, re-quantised, into the
// matvec's LDS input form.  v = pairwise_sum(x*x)/D + 1e-5, y = (x*g)/sqrt(v).
// dbuf: D shorts of LDS, leaf: PW_MAX_LEAVES doubles.  Thread tid keeps
// elements tid + k*bs (k < 4) and their gammas in registers from one batch
// of loads; the owners of numpy's pairwise leaves load their x elements
// themselves (pairwise_sum_block_g), so nothing is staged in LDS before the
// sum, and the up-to-four divisions and tile quantisations of a thread are
// independent chains.  All threads call.
__device__ __forceinline__ void rmsnorm_to_x(const int16_t *__restrict__ hm, const int8_t *__restrict__ he,
                             const double *__restrict__ g, int D, int *xs, int *xes, double *dbuf,
                             double *leaf, int16_t *dm, int8_t *de) {
  constexpr int KE = 4;
  const int bs = blockDim.x, tid = threadIdx.x;
  int m[KE], e[KE];
  double gg[KE];
  auto load = [&](int base) {
#pragma unroll
    for (int k = 0; k < KE; ++k) {
      int i = base + tid + k * bs;
      i = i < D ? i : D - 1;
      m[k] = hm[i];
      e[k] = he[i >> 4];
      gg[k] = g[i];
    }
  };
  load(0);
  const double s = pairwise_sum_block_g(
      [&](int i) {
        const double x = bfp_val(hm[i], he[i >> 4]);
        return x * x;
      },
      D, leaf);
  const double rt = sqrt(s / (double)D + 1e-5);
  short *mq = reinterpret_cast<short *>(dbuf);
  for (int base = 0; base < D; base += KE * bs) {   // one pass when D <= 4*bs
    if (base > 0) load(base);
    int mm[KE], ee[KE];
#pragma unroll
    for (int k = 0; k < KE; ++k) {
      const int i = base + tid + k * bs;
      const double y = i < D ? (bfp_val(m[k], e[k]) * gg[k]) / rt : 0.0;
      mm[k] = quantize16_lanes(y, ee[k], true);   // tile_quantize(rmsnorm_fp(.)): canonical
    }
#pragma unroll
    for (int k = 0; k < KE; ++k) {
      const int i = base + tid + k * bs;
      if (i < D) {
        mq[i] = (short)mm[k];
        if ((i & 15) == 0) xes[i >> 4] = ee[k];
        if (dm) {
          dm[i] = (int16_t)mm[k];
          if ((i & 15) == 0) de[i >> 4] = (int8_t)ee[k];
        }
      }
    }
  }
  __syncthreads();
  for (int p = tid; p < D / 2; p += bs) put_x_pair(xs, p >> 3, p & 7, mq[2 * p], mq[2 * p + 1]);
}

// ------------------------------------------------------------- epilogues
// Run by wave 0 (threads < 64) of a chunk's workgroup after chunk_AM: lane
// r + 16k holds row r of chunk c of sequence b (b may differ between the
// four 16-lane groups); only groups with wr set store.

// q|k|v rows: raw BFP out (V dumped here; Q and K post-RoPE by k_attn).
__device__ __forceinline__ void epi_qkv(const LayerArgs &a, int b, int c, long long A, int M,
                                        bool wr) {
  const int nq = a.D + 2 * a.KV;
  int m, e;
  chunk_quant(A, M, m, e);
  const int lane = threadIdx.x & 15;
  if (wr) a.qkv_m[b * nq + c * 16 + lane] = (int16_t)m;
  if (wr && lane == 0) a.qkv_e[b * (nq / 16) + c] = (int8_t)e;
  if (a.dump) {
    // V is not rotated: dump it here (Q and K are dumped post-RoPE by k_attn)
    int cm, ce;
    canon_copy(m, e, cm, ce);
    int row = c * 16 + lane;
    if (wr && row >= a.D + a.KV) {
      int r = row - a.D - a.KV;
      a.dump->m[ST_V][b * a.dump->mstride[ST_V] + r] = (int16_t)cm;
      if (lane == 0) a.dump->e[ST_V][b * (a.dump->mstride[ST_V] / 16) + r / 16] = (int8_t)ce;
    }
  }
}

// Residual epilogue: y = q(res + o) over the chunk (wave 0, lane r holds row r).
__device__ __forceinline__ int residual_lane(int om, int oe, int rm, int re, int &e) {
  double s = bfp_val(rm, re) + bfp_val(om, oe);
  return quantize16_lanes(s, e);
}

// o = Wo attn; h1 = q(h + o)   (full.py:284-285)
// rm, re: this lane's row of h (the residual), loaded by the caller.
__device__ __forceinline__ void epi_ores(const LayerArgs &a, int b, int c, long long A, int M,
                                         bool wr, int rm, int re) {
  const int r = threadIdx.x & 15;
  int om, oe;
  chunk_quant(A, M, om, oe);
  const int row = b * a.D + c * 16 + r;
  const int tile = b * (a.D / 16) + c;
  int e;
  int m = residual_lane(om, oe, rm, re, e);
  int com = om, coe = oe, chm = m, che = e;
  if (a.dump) {
    canon16_lanes(com, coe);
    canon16_lanes(chm, che);
  }
  if (wr) {
    a.h1_m[row] = (int16_t)m;
    if (r == 0) a.h1_e[tile] = (int8_t)e;
    if (a.dump) {
      const StageDump *d = a.dump;
      d->m[ST_O][b * d->mstride[ST_O] + c * 16 + r] = (int16_t)com;
      d->m[ST_H1][b * d->mstride[ST_H1] + c * 16 + r] = (int16_t)chm;
      if (r == 0) {
        d->e[ST_O][b * (d->mstride[ST_O] / 16) + c] = (int8_t)coe;
        d->e[ST_H1][b * (d->mstride[ST_H1] / 16) + c] = (int8_t)che;
      }
    }
  }
}

// g, u -> mlp = q(q(silu(g)) * u)   (full.py:241-242,288-290)
__device__ __forceinline__ void epi_gu(const LayerArgs &a, int b, int c, long long Ag, int Mg,
                                       long long Au, int Mu, bool wr) {
  const int r = threadIdx.x & 15;
  int gm, ge, um, ue;
  chunk_quant(Ag, Mg, gm, ge);
  chunk_quant(Au, Mu, um, ue);
  // silu_fp: fp_quantize_vec(g / (1 + exp(-g)))   (full.py:241-242)
  const double gv = bfp_val(gm, ge);
  int se;
  int sm = quantize16_lanes(gv / (1.0 + exp_f64(-gv)), se);
  // mlp = fp_quantize_vec(silu * u)                (full.py:290)
  int me;
  int mm = quantize16_lanes(bfp_val(sm, se) * bfp_val(um, ue), me, true);   // D's input
  if (a.dump) {
    canon16_lanes(gm, ge);      // values of g and u are no longer needed
    canon16_lanes(um, ue);
  }
  if (wr) {
    const int row = b * a.FFN + c * 16 + r;
    const int tile = b * (a.FFN / 16) + c;
    a.mlp_m[row] = (int16_t)mm;
    if (r == 0) a.mlp_e[tile] = (int8_t)me;
    if (a.dump) {
      const StageDump *d = a.dump;
      d->m[ST_G][b * d->mstride[ST_G] + c * 16 + r] = (int16_t)gm;
      d->m[ST_U][b * d->mstride[ST_U] + c * 16 + r] = (int16_t)um;
      d->m[ST_MLP][b * d->mstride[ST_MLP] + c * 16 + r] = (int16_t)mm;
      if (r == 0) {
        d->e[ST_G][b * (d->mstride[ST_G] / 16) + c] = (int8_t)ge;
        d->e[ST_U][b * (d->mstride[ST_U] / 16) + c] = (int8_t)ue;
        d->e[ST_MLP][b * (d->mstride[ST_MLP] / 16) + c] = (int8_t)me;
      }
    }
  }
}

// d = Wd mlp; h_out = q(h1 + d)   (full.py:291-293)
// rm, re: this lane's row of h1 (the residual), loaded by the caller.
__device__ __forceinline__ void epi_dres(const LayerArgs &a, int b, int c, long long A, int M,
                                         bool wr, int rm, int re) {
  const int r = threadIdx.x & 15;
  int dmv, dev;
  chunk_quant(A, M, dmv, dev);
  const int row = b * a.D + c * 16 + r;
  const int tile = b * (a.D / 16) + c;
  int e;
  int m = residual_lane(dmv, dev, rm, re, e);
  int cdm = dmv, cde = dev, chm = m, che = e;
  if (a.dump || a.hist_m) {
    canon16_lanes(cdm, cde);
    canon16_lanes(chm, che);
  }
  if (wr) {
    a.h_m[row] = (int16_t)m;
    if (r == 0) a.h_e[tile] = (int8_t)e;
    if (a.dump) {
      const StageDump *d = a.dump;
      d->m[ST_D][b * d->mstride[ST_D] + c * 16 + r] = (int16_t)cdm;
      d->m[ST_HOUT][b * d->mstride[ST_HOUT] + c * 16 + r] = (int16_t)chm;
      if (r == 0) {
        d->e[ST_D][b * (d->mstride[ST_D] / 16) + c] = (int8_t)cde;
        d->e[ST_HOUT][b * (d->mstride[ST_HOUT] / 16) + c] = (int8_t)che;
      }
    }
    if (a.hist_m) {
      const int pos = cur_pos(a);
      if (pos < a.hist_steps) {
        long long o = (((long long)b * a.hist_steps + pos) * a.NL + a.layer) * a.D;
        a.hist_m[o + c * 16 + r] = (int16_t)chm;
        if (r == 0) a.hist_e[(o >> 4) + c] = (int8_t)che;
      }
    }
  }
}

// ------------------------------------------------------------------- qkv
template <int NW, int TPT>
__global__ __launch_bounds__(64 * NW) void k_qkv(LayerArgs a) {
  extern __shared__ double dsm[];
  const int nT = a.D / 16;
  double *dbuf = dsm;                                   // 3*D
  double *leaf = dsm + 3 * a.D;                         // PW_MAX_LEAVES
  int *xs = reinterpret_cast<int *>(leaf + PW_MAX_LEAVES);   // nT*16
  int *xes = xs + nT * 16;                              // nT
  __shared__ int redM[NW * 16];
  __shared__ long long redA[NW * 16];
  const int c = blockIdx.x, b = blockIdx.y;

  ChunkRegs<TPT> R;
  load_chunk<NW, TPT>(R, a.w_qkv_m + (long long)c * nT * 32, a.w_qkv_e + (long long)c * nT * 16, nT);
  int16_t *dm = nullptr;
  int8_t *de = nullptr;
  if (a.dump && c == 0) {
    dm = a.dump->m[ST_N1] + b * a.dump->mstride[ST_N1];
    de = a.dump->e[ST_N1] + b * (a.dump->mstride[ST_N1] / 16);
  }
  rmsnorm_to_x(a.h_m + b * a.D, a.h_e + b * (a.D / 16), a.g1, a.D, xs, xes, dbuf, leaf, dm, de);
  __syncthreads();
  long long A;
  int M;
  chunk_AM<NW, TPT>(R, xs, xes, nT, redM, redA, A, M);
  if (threadIdx.x < 64) epi_qkv(a, b, c, A, M, threadIdx.x < 16);
}

// ------------------------------------------------------------------ attn

// Attention of one q head (full.py:268-283) in workgroups of ATT_WAVES
// waves:
//  1. waves 0-2: RoPE of q (head hq) and k (group g), v of group g; one
//     workgroup of the group stores k, v at slot pos of the KV cache;
//  2. all threads: scores[t] = np.dot(q, K[t]) / sqrt(HD), in OpenBLAS's
//     SkylakeX ddot order;
//  3. softmax: exp(s - max) / pairwise_sum (numpy's order);
//  4. attn = sum_t p[t] * V[t] in ascending t from 0.0 (numpy's
//     `attn[h] += p[t] * V[t]` loop, full.py:280-281), one add chain per
//     dimension.
// Short contexts (at most 64 * ATT_WAVES positions): one workgroup per
// head.  V rows are staged through LDS in chunks of AVC rows by every
// thread (16-byte loads, the next chunk's loads in flight while the current
// one is used); wave 0 forms each product and runs the chains, one
// dimension per lane, straight from LDS.
// Long contexts: ATT_DSPLIT workgroups per head, workgroup dg owning the
// 16 dimensions (one output tile) 16dg .. 16dg+15.  Each computes the whole
// score vector and softmax (the chip has far more CUs than heads) and the
// AV chains of its own tile only, so the LDS traffic of the products is a
// quarter of a whole head's.
constexpr int ATT_WAVES = 8;

// V rows per staged chunk of the AV phase (short contexts).
constexpr int ATT_AVC = 128;

// Long contexts: workgroups per head, and the AV phase's geometry.  Waves
// 1 .. AVL_PW form the products of blocks of AVL_TB positions into an LDS
// double buffer while lanes 0-15 of wave 0 add the previous block, V
// prefetched AVL_DEPTH blocks ahead.  Producer lane l holds dimensions
// 8(l/32) .. +7 of the tile for rows 2(l%32) and 2(l%32)+1 of its wave's
// 64 (one 16-byte load per row); products are stored dimension-major,
// AVL_TBP doubles per dimension, so each write is a 16-byte pair of rows
// and the 32 lanes of a half-wave write 512 contiguous bytes, and the
// chain lane of dimension d reads two positions per 16-byte load at
// d*AVL_TBP: the padding of 2 puts the 16 lanes in 16 distinct bank
// groups.
constexpr int ATT_DSPLIT = 4;
constexpr int AVL_PW = 3;
constexpr int AVL_TB = AVL_PW * 64;
constexpr int AVL_TBP = AVL_TB + 2;
constexpr int AVL_DEPTH = 4;
constexpr int AVL_G = 8;        // chain: positions per group of LDS reads
constexpr int AVL_AHEAD = 3;    // chain: groups of reads in flight ahead of the adds
size_t attn_lds_bytes(int max_ctx, int ppw) {
  const size_t sc_len = (size_t)((max_ctx + 1) & ~1);
  const size_t av = ppw <= 4 ? (size_t)2 * ATT_AVC * (64 * 2 + 4) : (size_t)2 * 16 * AVL_TBP * 8;
  return (256 + sc_len) * 8 + av;
}

// One K row of the cache (64 mantissas, 4 tile exponents) in registers.
struct KRow {
  uint4 m[8];
  int e4;
};
__device__ __forceinline__ void load_krow(KRow &r, const int16_t *Km, const int8_t *Ke, long long o) {
  const uint4 *p = reinterpret_cast<const uint4 *>(Km + o);
#pragma unroll
  for (int i = 0; i < 8; ++i) r.m[i] = p[i];
  r.e4 = *reinterpret_cast<const int *>(Ke + (o >> 4));
}

// SHORT: max_ctx <= 64 * ATT_WAVES, at most one score per thread (PPW 4) or
// one per 32-lane half-wave (PPW 2: max_ctx <= 128, PPW 3: <= 256); fewer
// registers -- at most 80 for PPW 3, so three workgroups fit a CU (many
// sequences at short context), two for PPW 2 and 4 (PPW 2 at 80 registers
// measured 1.6% slower at batch 1).
template <int PPW, bool SHORT>
__global__ __launch_bounds__(64 * ATT_WAVES, (SHORT ? (PPW == 3 ? 6 : 4) : 2)) void k_attn(LayerArgs a) {
  constexpr int NT = 64 * ATT_WAVES;
  constexpr int AVC = ATT_AVC;                 // V rows per staged chunk (short)
  constexpr int VL = AVC * 8 / NT;             // 16-byte V loads per thread and chunk
  constexpr int TB = AVL_TB;                   // positions per AV block (long)
  static_assert(SHORT || PPW == 8, "the long form is instantiated as PPW 8");
  static_assert(AVL_PW + 1 <= ATT_WAVES && AVL_TB % 8 == 0 && AVL_TBP % 2 == 0, "long AV geometry");
  extern __shared__ double dsm[];
  double *q = dsm;                  // 64
  double *kc = dsm + 64;            // 64 (current position, post-rope)
  double *vc = dsm + 128;           // 64
  double *leaf = dsm + 192;         // PW_MAX_LEAVES (= 64)
  double *sc = dsm + 256;           // max_ctx, rounded up to even
  // short: staged V, 2 x AVC x 64 mantissas and 2 x AVC x 4 exponents;
  // long: product double buffer, 2 x 16 dimensions x AVL_TBP doubles
  int16_t *vsm = reinterpret_cast<int16_t *>(sc + ((a.max_ctx + 1) & ~1));
  int8_t *vse = reinterpret_cast<int8_t *>(vsm + 2 * AVC * 64);
  double *buf = sc + ((a.max_ctx + 1) & ~1);
  __shared__ double red[ATT_WAVES];
  const int hq = SHORT ? blockIdx.x : blockIdx.x / ATT_DSPLIT, b = blockIdx.y;
  const int dg = SHORT ? 0 : blockIdx.x % ATT_DSPLIT;   // long: the tile of dimensions 16dg ..
  const bool lead = dg == 0;                             // stores the cache row and the dumps
  const int grp = a.H_Q / a.H_KV, g = hq / grp;
  const int HD = 64;
  const int pos = cur_kv_pos(a);                       // KV slot: attention over 0..pos
  const int n = pos + 1;
  const int nq = a.D + 2 * a.KV;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int16_t *qm = a.qkv_m + b * nq;
  const int8_t *qe = a.qkv_e + b * (nq / 16);
  const double *cs = a.rope_row ? a.rope_row                 // (HD/2) x (cos, sin)
                                : a.rope + (long long)cur_pos(a) * HD;
  const long long kv_tok = (long long)a.H_KV * HD;     // elements per position
  int16_t *Km = a.k_m + (long long)b * a.max_ctx * kv_tok;
  int8_t *Ke = a.k_e + (long long)b * a.max_ctx * (kv_tok / 16);
  int16_t *Vm = a.v_m + (long long)b * a.max_ctx * kv_tok;
  int8_t *Ve = a.v_e + (long long)b * a.max_ctx * (kv_tok / 16);
  const bool writer = (hq % grp) == 0 && lead;

  // AV staging: chunk c holds rows c*AVC .. c*AVC+AVC-1 (clamped to n-1, so
  // no load sits in a branch); thread tid loads 16-byte part tid%8 of rows
  // tid/8 + 64j and, for tid < AVC, the 4 exponent bytes of row tid.
  uint4 vr[VL];
  int ver = 0;
  const int16_t *Vg = Vm + (long long)g * HD + 8 * (tid & 7);
  const int8_t *Veg = Ve + (long long)g * (HD / 16);
  const long long vstride = (long long)a.H_KV * HD;    // elements per position
#define BFP_ATT_LOAD_V(c)                                                        \
  {                                                                              \
    _Pragma("unroll") for (int j = 0; j < VL; ++j) {                             \
      int t_ = (c) * AVC + (tid >> 3) + j * (NT / 8);                            \
      t_ = t_ < n ? t_ : n - 1;                                                  \
      vr[j] = *reinterpret_cast<const uint4 *>(Vg + t_ * vstride);               \
    }                                                                            \
    int t_ = (c) * AVC + (tid < AVC ? tid : 0);                                  \
    t_ = t_ < n ? t_ : n - 1;                                                    \
    ver = *reinterpret_cast<const int *>(Veg + t_ * (vstride / 16));             \
  }
#define BFP_ATT_STORE_V(c)                                                       \
  {                                                                              \
    int16_t *dst_ = vsm + ((c) & 1) * AVC * 64;                                  \
    _Pragma("unroll") for (int j = 0; j < VL; ++j)                               \
        *reinterpret_cast<uint4 *>(dst_ + ((tid >> 3) + j * (NT / 8)) * 64 +     \
                                   8 * (tid & 7)) = vr[j];                       \
    if (tid < AVC) *reinterpret_cast<int *>(vse + ((c) & 1) * AVC * 4 + tid * 4) = ver; \
  }

  // Long contexts: V prefetch ring of the AV phase (filled after the
  // scores).  Producer wave pw + 1 owns rows tt0 = 64pw + 2(l%32) and
  // tt0 + 1 of block k (positions k*TB + row); lane l holds dimensions
  // 16dg + 8(l/32) .. +7 of both rows: one 16-byte mantissa load and one
  // exponent byte per row and block.  Every wave issues the same loads on
  // every path (positions past the end are clamped to a valid row and their
  // products zeroed; the other waves load a copy they do not use), so the
  // compiler can count AVL_DEPTH blocks of loads in flight instead of
  // draining them.
  const bool producer = w >= 1 && w <= AVL_PW;
  const int pw = producer ? w - 1 : 0, hh = l >> 5;
  const int tt0 = 64 * pw + 2 * (l & 31);
  uint4 rm[SHORT ? 1 : AVL_DEPTH][2];
  int re[SHORT ? 1 : AVL_DEPTH][2];
  auto load_blk = [&](int k, uint4 (&m)[2], int (&e)[2]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      int t = k * TB + tt0 + r;
      t = t < n ? t : n - 1;
      const long long o = ((long long)t * a.H_KV + g) * HD + 16 * dg + 8 * hh;
      m[r] = *reinterpret_cast<const uint4 *>(Vm + o);
      e[r] = Ve[o >> 4];
    }
  };

  // the first K row of this thread's scores, in flight during the RoPE phase
  // (long contexts: KR rows per thread in flight, the first since the RoPE
  // phase, so a pass over 64 * ATT_WAVES * KR positions waits for memory once)
  constexpr int KR = SHORT ? 1 : 2;
  KRow kr[KR];
  // contexts of at most 128 (PPW 2) or 256 (PPW 3) positions: each 32-lane
  // half-wave scores one position, lane j (of 32) holding elements j and
  // 32 + j of its K row, in passes of 2*ATT_WAVES positions.  The elements
  // of LS_PRE passes (128 positions) are in registers at once: the first
  // group's are in flight during the RoPE phase, a second group's (PPW 3,
  // more than 128 positions) are loaded after the first is scored.  (Eight
  // passes keep the PPW 3 form within 80 registers: three workgroups per CU.)
  constexpr bool LANE_SPLIT = SHORT && (PPW == 2 || PPW == 3);
  constexpr int LS_PASS = LANE_SPLIT ? (PPW == 2 ? 128 : 256) / (2 * ATT_WAVES) : 1;
  constexpr int LS_PRE = LS_PASS < 8 ? LS_PASS : 8;
  int lsm[LS_PRE][2], lse[LS_PRE][2];
  auto ls_load = [&](int g0) {   // passes g0 .. g0 + LS_PRE - 1
#pragma unroll
    for (int ps_ = 0; ps_ < LS_PRE; ++ps_) {
      int t = 2 * ATT_WAVES * (g0 + ps_) + 2 * w + (l >> 5);
      t = t < n ? t : n - 1;
      const long long o = ((long long)t * a.H_KV + g) * HD + (l & 31);
      lsm[ps_][0] = Km[o];
      lsm[ps_][1] = Km[o + 32];
      lse[ps_][0] = Ke[o >> 4];
      lse[ps_][1] = Ke[(o + 32) >> 4];
    }
  };
  if constexpr (LANE_SPLIT) {
    ls_load(0);
  } else {
    load_krow(kr[0], Km, Ke, ((long long)(tid < n ? tid : n - 1) * a.H_KV + g) * HD);
  }

  if (w == 0) {            // q head hq
    int idx = hq * HD + l;
    int e;
    int m = rope_lane(bfp_val(qm[idx], qe[idx >> 4]), cs, e);
    q[l] = bfp_val(m, e);
    if (a.dump && lead) {
      int cm, ce;
      canon_copy(m, e, cm, ce);
      a.dump->m[ST_Q][b * a.dump->mstride[ST_Q] + idx] = (int16_t)cm;
      if ((l & 15) == 0) a.dump->e[ST_Q][b * (a.dump->mstride[ST_Q] / 16) + (idx >> 4)] = (int8_t)ce;
    }
  } else if (w == 1) {     // k head g
    int idx = a.D + g * HD + l;
    int e;
    int m = rope_lane(bfp_val(qm[idx], qe[idx >> 4]), cs, e);
    kc[l] = bfp_val(m, e);
    long long o = ((long long)pos * a.H_KV + g) * HD + l;
    if (writer) {
      Km[o] = (int16_t)m;
      if ((l & 15) == 0) Ke[o >> 4] = (int8_t)e;
    }
    if (a.dump && writer) {
      int cm, ce;
      canon_copy(m, e, cm, ce);
      int r = g * HD + l;
      a.dump->m[ST_K][b * a.dump->mstride[ST_K] + r] = (int16_t)cm;
      if ((l & 15) == 0) a.dump->e[ST_K][b * (a.dump->mstride[ST_K] / 16) + (r >> 4)] = (int8_t)ce;
    }
  } else if (w == 2) {     // v head g (not rotated)
    int idx = a.D + a.KV + g * HD + l;
    int m = qm[idx], e = qe[idx >> 4];
    vc[l] = bfp_val(m, e);
    long long o = ((long long)pos * a.H_KV + g) * HD + l;
    if (writer) {
      Vm[o] = (int16_t)m;
      if ((l & 15) == 0) Ve[o >> 4] = (int8_t)e;
    }
  }
  __syncthreads();

  if constexpr (SHORT) BFP_ATT_LOAD_V(0)   // in flight during the scores
  // scores[t] = float(np.dot(q, K[t])) / sqrt(HD)   (full.py:277-278), one
  // position per thread, two rows in flight.  Row pos is read from global
  // memory like the others (the writer may not have stored it yet) and its
  // score is recomputed from LDS afterwards by the same thread.
  if constexpr (LANE_SPLIT) {
    // ddot64_skx's order spread over 32 lanes: lane j = 8r + c forms
    // accumulator (r, c) = fma(x[32+j], y[32+j], fma(x[j], y[j], 0)); then
    // f_r(c) = acc(r, c) + acc(r, c+4) lands in lane 8r + c + 4,
    // s_c = ((f_0 + f_1) + f_2) + f_3 in lane 28 + c, and
    // (s_0 + s_2) + (s_1 + s_3) in lane 31 (each single addition commutes).
    // Row pos comes from LDS (its writer may not have stored it yet).
    const int j = l & 31;
    const double q0 = q[j], q1 = q[32 + j];
    const double k0 = kc[j], k1 = kc[32 + j];
    for (int g0 = 0; g0 < LS_PASS && 2 * ATT_WAVES * g0 < n; g0 += LS_PRE) {   // uniform
      if (g0 > 0) ls_load(g0);
#pragma unroll
      for (int ps_ = 0; ps_ < LS_PRE; ++ps_) {
        if (2 * ATT_WAVES * (g0 + ps_) >= n) break;   // uniform
        const int t = 2 * ATT_WAVES * (g0 + ps_) + 2 * w + (l >> 5);
        const double y0 = t == pos ? k0 : bfp_val(lsm[ps_][0], lse[ps_][0]);
        const double y1 = t == pos ? k1 : bfp_val(lsm[ps_][1], lse[ps_][1]);
        const double acc = fma(q1, y1, fma(q0, y0, 0.0));
        const double f = acc + peer<4>(acc);
        const double t01 = peer<16>(f + peer<8>(f));
        const double sl = (t01 + peer<8>(f)) + f;
        const double s2 = sl + peer<2>(sl);
        const double tot = s2 + peer<1>(s2);
        if (j == 31 && t < n) sc[t] = tot / a.inv_sqrt_hd_div;
      }
    }
  } else if constexpr (SHORT) {
    // contexts of at most NT positions: one row per thread, the one in
    // flight since the RoPE phase
    if (tid < n) sc[tid] = ddot64_skx_bfp(q, kr[0].m, kr[0].e4) / a.inv_sqrt_hd_div;
    if (tid == pos) sc[pos] = ddot64_skx(q, kc) / a.inv_sqrt_hd_div;
  } else {
    // passes of KR rows per thread: rows t0 + tid + j*NT; kr[0] of the next
    // pass is loaded as soon as this pass's kr[0] is consumed
    const int last = n - 1;
    for (int t0 = 0; t0 < n; t0 += KR * NT) {
#pragma unroll
      for (int j = 1; j < KR; ++j) {
        const int t = t0 + tid + j * NT;
        load_krow(kr[j], Km, Ke, ((long long)(t < n ? t : last) * a.H_KV + g) * HD);
      }
#pragma unroll
      for (int j = 0; j < KR; ++j) {
        const int t = t0 + tid + j * NT;
        const double sj = ddot64_skx_bfp(q, kr[j].m, kr[j].e4) / a.inv_sqrt_hd_div;
        if (j == 0) {
          const int tn = t + KR * NT;
          load_krow(kr[0], Km, Ke, ((long long)(tn < n ? tn : last) * a.H_KV + g) * HD);
        }
        if (t < n) sc[t] = sj;
      }
    }
    if (tid == pos % NT) sc[pos] = ddot64_skx(q, kc) / a.inv_sqrt_hd_div;
  }
  if constexpr (SHORT) {
    BFP_ATT_STORE_V(0)
  } else {
#pragma unroll
    for (int d = 0; d < AVL_DEPTH; ++d) load_blk(d, rm[d], re[d]);   // overlaps the softmax
  }
  __syncthreads();
  // softmax_fp (full.py:245-247): e = exp(s - max); p = e / pairwise_sum(e)
  double mx = -INFINITY;
  for (int t = tid; t < n; t += NT) mx = fmax(mx, sc[t]);
  mx = fmax(mx, peer<32>(mx));
  mx = fmax(mx, peer<16>(mx));
  mx = fmax(mx, peer<8>(mx));
  mx = fmax(mx, peer<4>(mx));
  mx = fmax(mx, peer<2>(mx));
  mx = fmax(mx, peer<1>(mx));
  if (l == 0) red[w] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int i = 1; i < ATT_WAVES; ++i) mx = fmax(mx, red[i]);
  for (int t = tid; t < n; t += NT) sc[t] = exp_f64(sc[t] - mx);
  __syncthreads();
  const double sum = pairwise_sum_block(sc, n, leaf);
  for (int t = tid; t < n; t += NT) sc[t] = sc[t] / sum;
  __syncthreads();

  double acc = 0.0;
  if constexpr (SHORT) {
    // attn_h = sum_t p[t] * V[t], ascending t from 0.0 (full.py:280-281):
    // every product rounded, then added, in t order.  Chunk c+1 is loaded
    // while wave 0 adds chunk c.  Row pos is this launch's V (vc): its writer
    // workgroup may not have stored it yet.
    const int nch = (n + AVC - 1) / AVC;
    for (int c = 0; c < nch; ++c) {
      BFP_ATT_LOAD_V(c + 1 < nch ? c + 1 : c)
      if (w == 0) {
        // 16 positions at a time: their LDS reads and products are independent
        // and issued together; only the adds form the chain
        // pos = n - 1 is the last position: it is added after the loop
        const int t0 = c * AVC, t1 = min(pos, t0 + AVC);
        const int16_t *vm = vsm + (c & 1) * AVC * 64 + l;
        const int8_t *ve = vse + (c & 1) * AVC * 4 + (l >> 4);
        int t = t0;
        for (; t + 16 <= t1; t += 16) {
          double pv[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = t + i - t0;
            pv[i] = sc[t + i] * ldexp((double)vm[r * 64], (int)ve[r * 4] - 15);
          }
#pragma unroll
          for (int i = 0; i < 16; ++i) acc = acc + pv[i];
        }
        for (; t < t1; ++t) {
          const int r = t - t0;
          acc = acc + sc[t] * ldexp((double)vm[r * 64], (int)ve[r * 4] - 15);
        }
        if (c == nch - 1) acc = acc + sc[pos] * vc[l];
      }
      if (c + 1 < nch) BFP_ATT_STORE_V(c + 1)
      __syncthreads();
    }
  } else {
    // attn_h = sum_t p[t] * V[t], ascending t from 0.0 (full.py:280-281),
    // for the tile's 16 dimensions.  Iteration k: the producers write the
    // products of block k into buf[k & 1] and refill their ring slot with
    // block k + AVL_DEPTH; lanes 0-15 of wave 0 add block k-1 from
    // buf[(k-1) & 1], one dimension per lane.  The blocks cover positions
    // 0 .. pos-1; row pos is this launch's V (vc, its writer workgroup may
    // not have stored it yet) and is added last.
    //
    // Product: p * (m * 2^(e-15)) is one rounding of the exact real
    // p*m*2^(e-15); so is ps * m with ps = p * 2^(e-15) whenever ps is exact,
    // i.e. a normal number (or p = 0).  A wave with any lane whose ps falls
    // below the normal range forms p * (m * 2^(e-15)) instead.  Positions
    // >= pos get ps = 0: adding +-0 leaves acc (never -0) unchanged.
    const int nb = (pos + TB - 1) / TB;
    double pt_nx[2];                       // p of the next block's rows, read a block ahead
#pragma unroll
    for (int r = 0; r < 2; ++r) pt_nx[r] = sc[tt0 + r < pos ? tt0 + r : 0];
    for (int k0 = 0; k0 <= nb; k0 += AVL_DEPTH) {
#pragma unroll
      for (int d = 0; d < AVL_DEPTH; ++d) {
        const int k = k0 + d;
        if (k <= nb) {                      // uniform: k0, d and nb are
          if (producer) {
            bool live[2], slow = false;
            double pt[2], s[2], ps[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
              const int t = k * TB + tt0 + r;
              live[r] = t < pos;
              pt[r] = pt_nx[r];
              pt_nx[r] = sc[t + TB < pos ? t + TB : 0];
              s[r] = ldexp(1.0, re[d][r] - 15);
              ps[r] = live[r] ? pt[r] * s[r] : 0.0;
              slow = slow || (live[r] && pt[r] != 0.0 && ps[r] < 0x1p-1022);
            }
            double pr[2][8];
            if (!__any(slow)) {
#pragma unroll
              for (int r = 0; r < 2; ++r) {
                const unsigned wv[4] = {rm[d][r].x, rm[d][r].y, rm[d][r].z, rm[d][r].w};
#pragma unroll
                for (int i = 0; i < 8; ++i)
                  pr[r][i] = ps[r] * (double)(int)(short)((wv[i >> 1] >> (16 * (i & 1))) & 0xffff);
              }
            } else {
#pragma unroll
              for (int r = 0; r < 2; ++r) {
                const unsigned wv[4] = {rm[d][r].x, rm[d][r].y, rm[d][r].z, rm[d][r].w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                  const double v = (double)(int)(short)((wv[i >> 1] >> (16 * (i & 1))) & 0xffff) * s[r];
                  pr[r][i] = live[r] ? pt[r] * v : 0.0;
                }
              }
            }
            double *bp = buf + (k & 1) * 16 * AVL_TBP + 8 * hh * AVL_TBP + tt0;
#pragma unroll
            for (int i = 0; i < 8; ++i)
              *reinterpret_cast<double2 *>(bp + i * AVL_TBP) = make_double2(pr[0][i], pr[1][i]);
          }
          if (w == 0 && l < 16 && k >= 1) {
            // block k-1 in full: its rows past pos - 1 hold products of +-0.
            // Groups of AV_G products; the reads of the next AV_AHEAD groups
            // are in flight while a group is added.  The scheduling barriers
            // keep that shape: left alone the compiler sinks the reads
            // toward their adds and the chain waits on each one.
            const double2 *lb =
                reinterpret_cast<const double2 *>(buf + ((k - 1) & 1) * 16 * AVL_TBP + l * AVL_TBP);
            constexpr int AV_G = AVL_G, AV_AHEAD = AVL_AHEAD, RING = AV_AHEAD + 1, NG = TB / AV_G;
            static_assert(TB % AV_G == 0 && AV_G % 2 == 0 && AV_AHEAD * AV_G / 2 <= 15, "AV read groups");
            double2 v[RING][AV_G / 2];
#pragma unroll
            for (int q = 0; q < AV_AHEAD; ++q)
#pragma unroll
              for (int i = 0; i < AV_G / 2; ++i) v[q][i] = lb[q * AV_G / 2 + i];
#pragma unroll
            for (int gq = 0; gq < NG; ++gq) {
              if (gq + AV_AHEAD < NG) {
#pragma unroll
                for (int i = 0; i < AV_G / 2; ++i)
                  v[(gq + AV_AHEAD) % RING][i] = lb[(gq + AV_AHEAD) * AV_G / 2 + i];
              }
              __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int i = 0; i < AV_G / 2; ++i) {
                acc = acc + v[gq % RING][i].x;
                acc = acc + v[gq % RING][i].y;
              }
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        }
        // outside the branch: a load in a branch makes the compiler drain
        // every outstanding load there
        load_blk(k + AVL_DEPTH, rm[d], re[d]);
        if (k <= nb) __syncthreads();
      }
    }
    if (w == 0) acc = acc + sc[pos] * vc[16 * dg + (l & 15)];
  }
#undef BFP_ATT_LOAD_V
#undef BFP_ATT_STORE_V
  if (w == 0) {
    // lanes 0-15 of the long form hold its tile; all 64 lanes take part
    int e;
    int m = quantize16_lanes(acc, e, true);   // tile_quantize(fp_quantize_vec(attn))
    const int idx = hq * HD + (SHORT ? l : 16 * dg + l);
    if (SHORT || l < 16) {
      a.att_m[b * a.D + idx] = (int16_t)m;
      if ((l & 15) == 0) a.att_e[b * (a.D / 16) + (idx >> 4)] = (int8_t)e;
    }
    if (a.dump && (SHORT || l < 16)) {
      a.dump->m[ST_ATTN][b * a.dump->mstride[ST_ATTN] + idx] = (int16_t)m;
      if ((l & 15) == 0)
        a.dump->e[ST_ATTN][b * (a.dump->mstride[ST_ATTN] / 16) + (idx >> 4)] = (int8_t)e;
    }
  }
}

// ----------------------------------------------------------------- o_res
template <int NW, int TPT>
__global__ __launch_bounds__(64 * NW) void k_o_res(LayerArgs a) {
  extern __shared__ int ism[];
  const int nT = a.D / 16;
  int *xs = ism;
  int *xes = ism + nT * 16;
  __shared__ int redM[NW * 16];
  __shared__ long long redA[NW * 16];
  const int c = blockIdx.x, b = blockIdx.y;
  ChunkRegs<TPT> R;
  load_chunk<NW, TPT>(R, a.w_o_m + (long long)c * nT * 32, a.w_o_e + (long long)c * nT * 16, nT);
  const int res_m = a.h_m[b * a.D + c * 16 + (threadIdx.x & 15)];   // residual, prefetched
  const int res_e = a.h_e[b * (a.D / 16) + c];
  stage_x_bfp(xs, xes, a.att_m + b * a.D, a.att_e + b * (a.D / 16), nT);
  __syncthreads();
  long long A;
  int M;
  chunk_AM<NW, TPT>(R, xs, xes, nT, redM, redA, A, M);
  if (threadIdx.x < 64) epi_ores(a, b, c, A, M, threadIdx.x < 16, res_m, res_e);
}

// -------------------------------------------------------------------- gu
template <int NW, int TPT>
__global__ __launch_bounds__(64 * NW) void k_gu(LayerArgs a) {
  extern __shared__ double dsm[];
  const int nT = a.D / 16;
  double *dbuf = dsm;             // 3*D
  double *leaf = dsm + 3 * a.D;
  int *xs = reinterpret_cast<int *>(leaf + PW_MAX_LEAVES);
  int *xes = xs + nT * 16;
  __shared__ int redM[NW * 16];
  __shared__ long long redA[NW * 16];
  const int c = blockIdx.x, b = blockIdx.y;
  ChunkRegs<TPT> RG, RU;
  load_chunk<NW, TPT>(RG, a.w_gu_m + (long long)(2 * c) * nT * 32,
                      a.w_gu_e + (long long)(2 * c) * nT * 16, nT);
  load_chunk<NW, TPT>(RU, a.w_gu_m + (long long)(2 * c + 1) * nT * 32,
                      a.w_gu_e + (long long)(2 * c + 1) * nT * 16, nT);
  int16_t *dm = nullptr;
  int8_t *de = nullptr;
  if (a.dump && c == 0) {
    dm = a.dump->m[ST_N2] + b * a.dump->mstride[ST_N2];
    de = a.dump->e[ST_N2] + b * (a.dump->mstride[ST_N2] / 16);
  }
  rmsnorm_to_x(a.h1_m + b * a.D, a.h1_e + b * (a.D / 16), a.g2, a.D, xs, xes, dbuf, leaf, dm, de);
  __syncthreads();
  long long Ag, Au;
  int Mg, Mu;
  chunk_AM<NW, TPT>(RG, xs, xes, nT, redM, redA, Ag, Mg);
  chunk_AM<NW, TPT>(RU, xs, xes, nT, redM, redA, Au, Mu);
  if (threadIdx.x < 64) epi_gu(a, b, c, Ag, Mg, Au, Mu, threadIdx.x < 16);
}

// ----------------------------------------------------------------- d_res
template <int NW, int TPT>
__global__ __launch_bounds__(64 * NW) void k_d_res(LayerArgs a) {
  extern __shared__ int ism[];
  const int nT = a.FFN / 16;
  int *xs = ism;
  int *xes = ism + nT * 16;
  __shared__ int redM[NW * 16];
  __shared__ long long redA[NW * 16];
  const int c = blockIdx.x, b = blockIdx.y;
  ChunkRegs<TPT> R;
  load_chunk<NW, TPT>(R, a.w_d_m + (long long)c * nT * 32, a.w_d_e + (long long)c * nT * 16, nT);
  const int res_m = a.h1_m[b * a.D + c * 16 + (threadIdx.x & 15)];   // residual, prefetched
  const int res_e = a.h1_e[b * (a.D / 16) + c];
  stage_x_bfp(xs, xes, a.mlp_m + b * a.FFN, a.mlp_e + b * (a.FFN / 16), nT);
  __syncthreads();
  long long A;
  int M;
  chunk_AM<NW, TPT>(R, xs, xes, nT, redM, redA, A, M);
  if (threadIdx.x < 64) epi_dres(a, b, c, A, M, threadIdx.x < 16, res_m, res_e);
}


// ------------------------------------------------- multi-sequence kernels
// For batch >= MULTI_MIN_BATCH the layer runs as norm -> matvec kernels in
// which a workgroup keeps its weight chunk in registers and loops over S
// sequences (grid.y = sequence groups), so weights are fetched once per
// group rather than once per sequence, and each RMSNorm is computed once per
// sequence rather than once per chunk.  Same arithmetic as the fused
// kernels: the outputs are bit-identical.

// n = tile_quantize(rmsnorm_fp(x, gamma)) of sequence blockIdx.x into xn
// (which = 1: h with g1 -> N1; which = 2: h1 with g2 -> N2).
__global__ __launch_bounds__(256) void k_norm_seq(LayerArgs a, int which) {
  extern __shared__ double dsm[];
  const int nT = a.D / 16;
  double *dbuf = dsm;             // 3*D
  double *leaf = dsm + 3 * a.D;
  int *xs = reinterpret_cast<int *>(leaf + PW_MAX_LEAVES);
  int *xes = xs + nT * 16;
  const int b = blockIdx.x;
  const int16_t *hm = (which == 1 ? a.h_m : a.h1_m) + b * a.D;
  const int8_t *he = (which == 1 ? a.h_e : a.h1_e) + b * (a.D / 16);
  int16_t *om = a.xn_m + b * a.D;
  int8_t *oe = a.xn_e + b * (a.D / 16);
  rmsnorm_to_x(hm, he, which == 1 ? a.g1 : a.g2, a.D, xs, xes, dbuf, leaf, om, oe);
  if (a.dump) {
    __syncthreads();   // om/oe written by other threads of this workgroup
    const int st = which == 1 ? ST_N1 : ST_N2;
    for (int i = threadIdx.x; i < a.D; i += blockDim.x) {
      a.dump->m[st][b * a.dump->mstride[st] + i] = om[i];
      if ((i & 15) == 0) a.dump->e[st][b * (a.dump->mstride[st] / 16) + (i >> 4)] = oe[i >> 4];
    }
  }
}

constexpr int MSEQ = 8;   // sequences per workgroup of the multi-sequence matvecs

// The epilogue of a multi-sequence chunk: wave 0, four sequences per pass
// (one per 16-lane group).
#define BFP_MULTI_EPI(CALL)                                                       \
  if (threadIdx.x < 64) {                                                         \
    const int r_ = threadIdx.x & 15;                                              \
    for (int p_ = 0; p_ < ns; p_ += 4) {                                          \
      const int s_ = p_ + (threadIdx.x >> 4);                                     \
      const bool wr_ = s_ < ns;                                                   \
      const int sc_ = wr_ ? s_ : 0;                                               \
      const int b = b0 + sc_;                                                     \
      CALL;                                                                       \
    }                                                                             \
  }

template <int NW, int TPT>
__global__ __launch_bounds__(64 * NW) void k_qkv_m(LayerArgs a) {
  extern __shared__ int ism[];
  const int nT = a.D / 16;
  int *xs = ism;
  int *xes = ism + MSEQ * nT * 16;
  __shared__ int redM[NW * 16 * MSEQ];
  __shared__ long long redA[NW * 16 * MSEQ];
  __shared__ long long Ao[16 * MSEQ];
  __shared__ int Mo[16 * MSEQ];
  const int c = blockIdx.x, b0 = blockIdx.y * MSEQ, ns = min(MSEQ, a.batch - b0);
  ChunkRegs<TPT> R;
  load_chunk<NW, TPT>(R, a.w_qkv_m + (long long)c * nT * 32, a.w_qkv_e + (long long)c * nT * 16, nT);
  stage_x_bfp(xs, xes, a.xn_m + b0 * a.D, a.xn_e + b0 * (a.D / 16), ns * nT);
  __syncthreads();
  chunk_AM_multi<NW, TPT, MSEQ>(R, xs, xes, nT, ns, redM, redA, Ao, Mo);
  BFP_MULTI_EPI(epi_qkv(a, b, c, Ao[r_ * MSEQ + sc_], Mo[r_ * MSEQ + sc_], wr_))
}

template <int NW, int TPT>
__global__ __launch_bounds__(64 * NW) void k_o_res_m(LayerArgs a) {
  extern __shared__ int ism[];
  const int nT = a.D / 16;
  int *xs = ism;
  int *xes = ism + MSEQ * nT * 16;
  __shared__ int redM[NW * 16 * MSEQ];
  __shared__ long long redA[NW * 16 * MSEQ];
  __shared__ long long Ao[16 * MSEQ];
  __shared__ int Mo[16 * MSEQ];
  const int c = blockIdx.x, b0 = blockIdx.y * MSEQ, ns = min(MSEQ, a.batch - b0);
  ChunkRegs<TPT> R;
  load_chunk<NW, TPT>(R, a.w_o_m + (long long)c * nT * 32, a.w_o_e + (long long)c * nT * 16, nT);
  stage_x_bfp(xs, xes, a.att_m + b0 * a.D, a.att_e + b0 * (a.D / 16), ns * nT);
  __syncthreads();
  chunk_AM_multi<NW, TPT, MSEQ>(R, xs, xes, nT, ns, redM, redA, Ao, Mo);
  BFP_MULTI_EPI(epi_ores(a, b, c, Ao[r_ * MSEQ + sc_], Mo[r_ * MSEQ + sc_], wr_,
                         a.h_m[b * a.D + c * 16 + r_], a.h_e[b * (a.D / 16) + c]))
}

template <int NW, int TPT>
__global__ __launch_bounds__(64 * NW) void k_gu_m(LayerArgs a) {
  extern __shared__ int ism[];
  const int nT = a.D / 16;
  int *xs = ism;
  int *xes = ism + MSEQ * nT * 16;
  __shared__ int redM[NW * 16 * MSEQ];
  __shared__ long long redA[NW * 16 * MSEQ];
  __shared__ long long Aog[16 * MSEQ], Aou[16 * MSEQ];
  __shared__ int Mog[16 * MSEQ], Mou[16 * MSEQ];
  const int c = blockIdx.x, b0 = blockIdx.y * MSEQ, ns = min(MSEQ, a.batch - b0);
  ChunkRegs<TPT> RG, RU;
  load_chunk<NW, TPT>(RG, a.w_gu_m + (long long)(2 * c) * nT * 32,
                      a.w_gu_e + (long long)(2 * c) * nT * 16, nT);
  load_chunk<NW, TPT>(RU, a.w_gu_m + (long long)(2 * c + 1) * nT * 32,
                      a.w_gu_e + (long long)(2 * c + 1) * nT * 16, nT);
  stage_x_bfp(xs, xes, a.xn_m + b0 * a.D, a.xn_e + b0 * (a.D / 16), ns * nT);
  __syncthreads();
  chunk_AM_multi<NW, TPT, MSEQ>(RG, xs, xes, nT, ns, redM, redA, Aog, Mog);
  chunk_AM_multi<NW, TPT, MSEQ>(RU, xs, xes, nT, ns, redM, redA, Aou, Mou);
  BFP_MULTI_EPI(epi_gu(a, b, c, Aog[r_ * MSEQ + sc_], Mog[r_ * MSEQ + sc_], Aou[r_ * MSEQ + sc_],
                       Mou[r_ * MSEQ + sc_], wr_))
}

template <int NW, int TPT>
__global__ __launch_bounds__(64 * NW) void k_d_res_m(LayerArgs a) {
  extern __shared__ int ism[];
  const int nT = a.FFN / 16;
  int *xs = ism;
  int *xes = ism + MSEQ * nT * 16;
  __shared__ int redM[NW * 16 * MSEQ];
  __shared__ long long redA[NW * 16 * MSEQ];
  __shared__ long long Ao[16 * MSEQ];
  __shared__ int Mo[16 * MSEQ];
  const int c = blockIdx.x, b0 = blockIdx.y * MSEQ, ns = min(MSEQ, a.batch - b0);
  ChunkRegs<TPT> R;
  load_chunk<NW, TPT>(R, a.w_d_m + (long long)c * nT * 32, a.w_d_e + (long long)c * nT * 16, nT);
  stage_x_bfp(xs, xes, a.mlp_m + b0 * a.FFN, a.mlp_e + b0 * (a.FFN / 16), ns * nT);
  __syncthreads();
  chunk_AM_multi<NW, TPT, MSEQ>(R, xs, xes, nT, ns, redM, redA, Ao, Mo);
  BFP_MULTI_EPI(epi_dres(a, b, c, Ao[r_ * MSEQ + sc_], Mo[r_ * MSEQ + sc_], wr_,
                         a.h1_m[b * a.D + c * 16 + r_], a.h1_e[b * (a.D / 16) + c]))
}

// ------------------------------------------ matrix-core multi-sequence path
// The four matvecs of a layer for 16 sequences per workgroup on the int8
// MFMA (bfp_mx.h); the epilogues are the multi-sequence path's.  blockIdx.x
// is a block of NC chunks, blockIdx.y a group of 16 sequences.  Each
// 16-lane group runs the epilogue of one (chunk, sequence) pair per pass.
#define BFP_MX_EPI(NPAIR, ...)                                                    \
  {                                                                              \
    const int r_ = threadIdx.x & 15, grp_ = threadIdx.x >> 4;                     \
    const int ngrp_ = blockDim.x >> 4;                                            \
    for (int p0_ = 0; p0_ < (NPAIR); p0_ += ngrp_) {                              \
      if (p0_ + 4 * (threadIdx.x >> 6) >= (NPAIR)) break; /* wave has no pair */ \
      const int p_ = p0_ + grp_;                                                  \
      const int pc_ = p_ < (NPAIR) ? p_ : 0;                                      \
      const int cc_ = pc_ / MX_SEQ, j_ = pc_ % MX_SEQ;                            \
      const bool wr_ = p_ < (NPAIR) && j_ < ns;                                   \
      const int b = b0 + (wr_ ? j_ : 0);                                          \
      __VA_ARGS__;                                                                \
    }                                                                             \
  }

// Q|K|V: two chunks per block.
__global__ __launch_bounds__(64 * MX_WAVES_MAX) void k_qkv_mx(LayerArgs a) {
  __shared__ long long Ao[2 * 16 * MX_SEQ];
  __shared__ int Mo[2 * 16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  const int nT = a.D / 16, c0 = 2 * blockIdx.x, b0 = blockIdx.y * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  mx_block<2>(a.w_qkv_m + (long long)c0 * nT * 32, a.w_qkv_e + (long long)c0 * nT * 16, nT,
              a.xn_m + (long long)b0 * a.D, a.xn_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex);
  BFP_MX_EPI(2 * MX_SEQ, {
    const int q_ = (cc_ * 16 + r_) * MX_SEQ + j_;
    epi_qkv(a, b, c0 + cc_, mx_A(Ao, q_), Mo[q_], wr_);
  })
}

// O and residual 1: one chunk per block.
__global__ __launch_bounds__(64 * MX_WAVES_MAX) void k_o_res_mx(LayerArgs a) {
  __shared__ long long Ao[16 * MX_SEQ];
  __shared__ int Mo[16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  const int nT = a.D / 16, c = blockIdx.x, b0 = blockIdx.y * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  mx_block<1>(a.w_o_m + (long long)c * nT * 32, a.w_o_e + (long long)c * nT * 16, nT,
              a.att_m + (long long)b0 * a.D, a.att_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex);
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_ores(a, b, c, mx_A(Ao, q_), Mo[q_], wr_, a.h_m[b * a.D + c * 16 + r_],
             a.h_e[b * (a.D / 16) + c]);
  })
}

// G and U: the G chunk (2x) and U chunk (2x+1) of FFN chunk x per block.
__global__ __launch_bounds__(64 * MX_WAVES_MAX) void k_gu_mx(LayerArgs a) {
  __shared__ long long Ao[2 * 16 * MX_SEQ];
  __shared__ int Mo[2 * 16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  const int nT = a.D / 16, c = blockIdx.x, b0 = blockIdx.y * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  mx_block<2>(a.w_gu_m + (long long)(2 * c) * nT * 32, a.w_gu_e + (long long)(2 * c) * nT * 16, nT,
              a.xn_m + (long long)b0 * a.D, a.xn_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex);
  BFP_MX_EPI(MX_SEQ, {
    const int qg_ = r_ * MX_SEQ + j_, qu_ = (16 + r_) * MX_SEQ + j_;
    (void)cc_;
    epi_gu(a, b, c, mx_A(Ao, qg_), Mo[qg_], mx_A(Ao, qu_), Mo[qu_], wr_);
  })
}

// D and residual 2: one chunk per block.
__global__ __launch_bounds__(64 * MX_WAVES_MAX) void k_d_res_mx(LayerArgs a) {
  __shared__ long long Ao[16 * MX_SEQ];
  __shared__ int Mo[16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  const int nT = a.FFN / 16, c = blockIdx.x, b0 = blockIdx.y * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  mx_block<1>(a.w_d_m + (long long)c * nT * 32, a.w_d_e + (long long)c * nT * 16, nT,
              a.mlp_m + (long long)b0 * a.FFN, a.mlp_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex);
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_dres(a, b, c, mx_A(Ao, q_), Mo[q_], wr_, a.h1_m[b * a.D + c * 16 + r_],
             a.h1_e[b * (a.D / 16) + c]);
  })
}

// ------------------------------------------------------------------ head
// One step of a (value, index) argmax over lanes: larger value wins, the
// lower index on ties (a total order, so any combining order gives the
// first index of the maximum).
template <int M>
__device__ __forceinline__ void argmax_step(double &best, int &besti) {
  const double ov = peer<M>(best);
  const int oi = peer<M>(besti);
  if (ov > best || (ov == best && oi < besti)) {
    best = ov;
    besti = oi;
  }
}

// The decode head's final norm (full.py:438): hn = (h / sqrt(mean(h*h) +
// 1e-5)) * w, float64, not re-quantised.  work: 3*D doubles of LDS, leaf:
// PW_MAX_LEAVES; hn may alias work (LDS) or be global.  Loads are issued in
// one batch per thread.  All threads call.
__device__ __forceinline__ void final_norm(const int16_t *__restrict__ hm, const int8_t *__restrict__ he,
                           const double *__restrict__ w, int D, double *work, double *leaf,
                           double *hn) {
  const int bs = blockDim.x, tid = threadIdx.x;
  double *sq = work, *xv = work + D, *wv = work + 2 * D;
  for (int i0 = tid; i0 < D; i0 += 4 * bs) {
    int m[4], e[4];
    double ww[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      int i = i0 + k * bs;
      i = i < D ? i : D - 1;
      m[k] = hm[i];
      e[k] = he[i >> 4];
      ww[k] = w[i];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = i0 + k * bs;
      if (i < D) {
        const double x = bfp_val(m[k], e[k]);
        sq[i] = x * x;
        xv[i] = x;
        wv[i] = ww[k];
      }
    }
  }
  __syncthreads();
  const double s = pairwise_sum_block(sq, D, leaf);
  const double rt = sqrt(s / (double)D + 1e-5);
  for (int i = tid; i < D; i += bs) hn[i] = (xv[i] / rt) * wv[i];
}

// logits = ((h / sqrt(mean(h*h) + 1e-5)) * w) @ embed.T in float64
// (full.py:438-440), with a per-workgroup first-index argmax.  Each row's
// dot product: 16 lanes, lane l sums k = 64i + 4l + c (i ascending, c =
// 0..3) with FMA, then a fixed 16-lane butterfly.  (BLAS dgemv's order is
// host-specific; the argmax differs only if the top two logits are within
// a few ulps.)
template <int MAXD64, bool EXACT>
__global__ __launch_bounds__(256) void k_head_logits(HeadArgs a) {
  extern __shared__ double dsm[];
  double *hn = dsm;                    // 3*D: the final norm's work space, then hn (D)
  double *leaf = dsm + 3 * a.D;        // PW_MAX_LEAVES
  __shared__ double bv[16];
  __shared__ int bi[16];
  const int b = blockIdx.y, wg = blockIdx.x, tid = threadIdx.x;
  const int l16 = tid & 15, sub = tid >> 4;      // 16 row slots per pass
  const int d64 = a.D / 64, r0 = wg * a.rows_per_wg;
  // a pass's embedding words, every load unconditional (a load behind a
  // branch is waited out there); the first pass is in flight during the
  // final norm, each later one during the previous pass's arithmetic.  The
  // prefetch past the last pass re-reads that pass's own rows (just
  // fetched, so it hits the caches; re-reading the first pass's rows cost a
  // quarter more HBM traffic than the table).
  float4 cur[MAXD64], nxt[MAXD64];
  auto load_rows = [&](int rr, float4 (&f)[MAXD64]) {
    rr = rr < a.rows_per_wg ? rr : rr - 16;
    const float4 *e4 = reinterpret_cast<const float4 *>(a.embed + (long long)(r0 + rr) * a.D);
#pragma unroll
    for (int i = 0; i < MAXD64; ++i) f[i] = e4[(EXACT || i < d64 ? i : d64 - 1) * 16 + l16];
  };
  load_rows(sub, cur);
  final_norm(a.h_m + b * a.D, a.h_e + b * (a.D / 16), a.norm_w, a.D, dsm, leaf, hn);
  __syncthreads();

  double best = -INFINITY;
  int besti = 0x7fffffff;
  for (int rr = sub; rr < a.rows_per_wg; rr += 16) {
    const int row = r0 + rr;
    load_rows(rr + 16, nxt);
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < MAXD64; ++i) {
      if (EXACT || i < d64) {
        const float4 f = cur[i];
        const double *hp = hn + i * 64 + 4 * l16;
        acc = fma((double)f.x, hp[0], acc);
        acc = fma((double)f.y, hp[1], acc);
        acc = fma((double)f.z, hp[2], acc);
        acc = fma((double)f.w, hp[3], acc);
      }
    }
#pragma unroll
    for (int i = 0; i < MAXD64; ++i) cur[i] = nxt[i];
    acc = psum<8>(acc);
    acc = psum<4>(acc);
    acc = psum<2>(acc);
    acc = psum<1>(acc);
    if (a.logits && l16 == 0) a.logits[(long long)b * a.VOCAB + row] = acc;
    if (acc > best || (acc == best && row < besti)) {
      best = acc;
      besti = row;
    }
  }
  // workgroup argmax, first index on ties
  argmax_step<16>(best, besti);
  argmax_step<32>(best, besti);
  if ((tid & 63) == 0) {
    bv[tid >> 6] = best;
    bi[tid >> 6] = besti;
  }
  __syncthreads();
  if (tid == 0) {
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k)
      if (bv[k] > best || (bv[k] == best && bi[k] < besti)) {
        best = bv[k];
        besti = bi[k];
      }
    a.part_v[b * a.n_wg + wg] = best;
    a.part_i[b * a.n_wg + wg] = besti;
  }
}


// Batch > 1 head: the final norm once per sequence (k_head_norm), then a GEMV
// in which each workgroup keeps its 32 embedding rows in registers as
// float64 and iterates over the sequences (16 at a time through LDS), so the
// 113 MB table is read once per step rather than once per sequence.  Each
// logit is summed in the same order as k_head_logits (lane l16 of a row's 16
// lanes accumulates k = 64i + 4*l16 + c, then the same butterfly), so the
// logits are bit-identical to the batch-1 kernel's.
__global__ __launch_bounds__(256) void k_head_norm(HeadArgs a) {
  extern __shared__ double dsm[];
  const int b = blockIdx.x;
  final_norm(a.h_m + b * a.D, a.h_e + b * (a.D / 16), a.norm_w, a.D, dsm, dsm + 3 * a.D,
             a.hn + (long long)b * a.D);
}

constexpr int HEAD_SEQ_GROUP = 16;   // most sequences staged in LDS at once

// Sequences per LDS stage for hidden size D (at most 96 KiB of LDS).
static int head_seq_group(int D) {
  int g = 98304 / (D * 8);
  return g < 1 ? 1 : (g > HEAD_SEQ_GROUP ? HEAD_SEQ_GROUP : g);
}

// EXACT: D == 64 * MAXD64, so every 64-column block is present and no load
// or LDS read sits behind a per-block branch (the compiler waits out every
// load at such a branch).
template <int MAXD64, int R, bool EXACT>
__global__ __launch_bounds__(256) void k_head_gemv(HeadArgs a, int sg) {
  extern __shared__ double hs[];       // sg x D
  __shared__ double bv[4][HEAD_SEQ_GROUP];
  __shared__ int bi[4][HEAD_SEQ_GROUP];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int slot = tid >> 4, l16 = tid & 15;
  const int d64 = a.D / 64;
  const int row0 = blockIdx.x * (16 * R);
  double eD[R][4 * MAXD64];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int row = row0 + slot + 16 * r;
    row = row < a.VOCAB ? row : a.VOCAB - 1;
    const float4 *e4 = reinterpret_cast<const float4 *>(a.embed + (long long)row * a.D);
#pragma unroll
    for (int i = 0; i < MAXD64; ++i) {
      float4 f = e4[(EXACT || i < d64 ? i : d64 - 1) * 16 + l16];   // unconditional load
      if (!EXACT && i >= d64) f = make_float4(0.f, 0.f, 0.f, 0.f);
      eD[r][4 * i] = (double)f.x;
      eD[r][4 * i + 1] = (double)f.y;
      eD[r][4 * i + 2] = (double)f.z;
      eD[r][4 * i + 3] = (double)f.w;
    }
  }
  for (int b0 = 0; b0 < a.batch; b0 += sg) {
    const int nb = min(sg, a.batch - b0);
    __syncthreads();
    {   // 16-byte loads, all of a group's (18 per thread at D 576) in flight before the LDS stores
      const double2 *src = reinterpret_cast<const double2 *>(a.hn + (long long)b0 * a.D);
      double2 *dst = reinterpret_cast<double2 *>(hs);
      const int n2 = nb * a.D / 2;
      constexpr int U = 18;
      for (int p0 = tid; p0 < n2; p0 += U * 256) {
        double2 v[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
          const int p = p0 + k * 256;
          v[k] = src[p < n2 ? p : n2 - 1];
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
          const int p = p0 + k * 256;
          if (p < n2) dst[p] = v[k];
        }
      }
    }
    __syncthreads();
    for (int bb = 0; bb < nb; ++bb) {
      const double *hp = hs + bb * a.D + 4 * l16;
      double acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.0;
#pragma unroll
      for (int i = 0; i < MAXD64; ++i) {
        if (EXACT || i < d64) {
          const double2 h01 = *reinterpret_cast<const double2 *>(hp + 64 * i);
          const double2 h23 = *reinterpret_cast<const double2 *>(hp + 64 * i + 2);
#pragma unroll
          for (int r = 0; r < R; ++r) {
            acc[r] = fma(eD[r][4 * i], h01.x, acc[r]);
            acc[r] = fma(eD[r][4 * i + 1], h01.y, acc[r]);
            acc[r] = fma(eD[r][4 * i + 2], h23.x, acc[r]);
            acc[r] = fma(eD[r][4 * i + 3], h23.y, acc[r]);
          }
        }
      }
      double best = -INFINITY;
      int besti = 0x7fffffff;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        double v = acc[r];
        v = psum<8>(v);
        v = psum<4>(v);
        v = psum<2>(v);
        v = psum<1>(v);
        const int row = row0 + slot + 16 * r;
        if (row < a.VOCAB) {
          if (a.logits && l16 == 0) a.logits[(long long)(b0 + bb) * a.VOCAB + row] = v;
          if (v > best || (v == best && row < besti)) {
            best = v;
            besti = row;
          }
        }
      }
      argmax_step<16>(best, besti);   // the wave's 4 row slots
      argmax_step<32>(best, besti);
      if (l == 0) {
        bv[w][bb] = best;
        bi[w][bb] = besti;
      }
    }
    __syncthreads();
    if (tid < nb) {
      double best = bv[0][tid];
      int besti = bi[0][tid];
      for (int k = 1; k < 4; ++k)
        if (bv[k][tid] > best || (bv[k][tid] == best && bi[k][tid] < besti)) {
          best = bv[k][tid];
          besti = bi[k][tid];
        }
      a.part_v[(b0 + tid) * a.n_wg + blockIdx.x] = best;
      a.part_i[(b0 + tid) * a.n_wg + blockIdx.x] = besti;
    }
  }
}

// Final argmax of each sequence and the token loop of full.py:432-443:
// at step s >= n_prompt the argmax is appended; the next input is
// prompt[s+1] while s+1 < n_prompt, prompt[n_prompt-1] again at
// s+1 == n_prompt (the reference feeds generated[-1], still the last prompt
// token), else the argmax.
// With rtl_loop, the policy of the FPGA driver (autoregress_bfp_top.sv
// :357-386): every step's argmax is recorded (result_buf[step]) and the
// next input is prompt[s+1] while s+1 < n_prompt, else this step's argmax.
__global__ __launch_bounds__(64) void k_ctl(CtlArgs a) {
  const int b = blockIdx.x, l = threadIdx.x;
  const int s = a.state[0];
  int nid = -1;
  if (a.head) {
    double best = -INFINITY;
    int besti = 0x7fffffff;
    for (int k = l; k < a.n_wg; k += 64) {
      double v = a.part_v[b * a.n_wg + k];
      int i = a.part_i[b * a.n_wg + k];
      if (v > best || (v == best && i < besti)) {
        best = v;
        besti = i;
      }
    }
    argmax_step<1>(best, besti);
    argmax_step<2>(best, besti);
    argmax_step<4>(best, besti);
    argmax_step<8>(best, besti);
    argmax_step<16>(best, besti);
    argmax_step<32>(best, besti);
    nid = besti;
  }
  if (l == 0) {
    if (a.head) a.last[b] = nid;
    int next;
    if (a.rtl_loop) {
      const int steps = a.n_prompt + a.n_gen;
      if (a.head && s < steps) a.out[b * steps + s] = nid;
      next = s + 1 < a.n_prompt ? a.prompt[b * a.n_prompt + s + 1] : nid;
    } else {
      if (a.head && s >= a.n_prompt && s - a.n_prompt < a.n_gen)
        a.out[b * a.n_gen + (s - a.n_prompt)] = nid;
      if (s + 1 < a.n_prompt)
        next = a.prompt[b * a.n_prompt + s + 1];
      else if (s + 1 == a.n_prompt)
        next = a.prompt[b * a.n_prompt + a.n_prompt - 1];
      else
        next = nid;
    }
    a.state[1 + b] = next;
  }
}

__global__ __launch_bounds__(64) void k_step_inc(int *state) {
  if (threadIdx.x == 0 && blockIdx.x == 0) state[0] += 1;
}

// Embedding lookup of the BFP table: embed_q[tid] = fp_quantize_vec(embed[tid])
// (full.py:411-412), quantised on the fly from the float32 table.
__global__ __launch_bounds__(256) void k_embed(EmbedArgs a) {
  const int b = blockIdx.x;
  int tok = a.state[1 + b];
  tok = tok < 0 ? 0 : (tok >= a.VOCAB ? a.VOCAB - 1 : tok);
  const float *row = a.embed + (long long)tok * a.D;
  for (int base = 0; base < a.D; base += blockDim.x) {
    int i = base + threadIdx.x;
    bool ok = i < a.D;
    double v = ok ? (double)row[i] : 0.0;
    int e;
    int m = quantize16_lanes(v, e);
    if (ok) {
      a.h_m[b * a.D + i] = (int16_t)m;
      if ((i & 15) == 0) a.h_e[b * (a.D / 16) + (i >> 4)] = (int8_t)e;
    }
  }
}

// --------------------------------------------------------------- launchers
typedef void (*lk_fn)(LayerArgs);

// Batches from this size on use the multi-sequence kernels, and from
// MX_MIN_BATCH on their matrix-core form (measured crossover: the MFMA form
// is ahead from 8 sequences; env BFP_MX_MIN_BATCH overrides).
constexpr int MULTI_MIN_BATCH = 4;
static int MX_MIN_BATCH = [] {
  const char *v = getenv("BFP_MX_MIN_BATCH");
  return v ? atoi(v) : 8;
}();

// The (waves, tiles per lane) pairs default_waves() produces for
// 4 <= in/16 <= 108, i.e. every supported D and FFN.
#define BFP_LAYER_SHAPES(X, KER) \
  X(KER, 1, 1) X(KER, 1, 2) X(KER, 1, 3) X(KER, 2, 2) X(KER, 2, 3) X(KER, 3, 3) X(KER, 4, 3) \
  X(KER, 6, 3) X(KER, 8, 3) X(KER, 9, 3)
#define BFP_CASE(KER, NW, TPT) \
  if (nw == NW && tpt == TPT) return KER<NW, TPT>;

static lk_fn pick_qkv(int nw, int tpt) { BFP_LAYER_SHAPES(BFP_CASE, k_qkv) return nullptr; }
static lk_fn pick_ores(int nw, int tpt) { BFP_LAYER_SHAPES(BFP_CASE, k_o_res) return nullptr; }
static lk_fn pick_gu(int nw, int tpt) { BFP_LAYER_SHAPES(BFP_CASE, k_gu) return nullptr; }
static lk_fn pick_dres(int nw, int tpt) { BFP_LAYER_SHAPES(BFP_CASE, k_d_res) return nullptr; }

typedef void (*lkm_fn)(LayerArgs);
static lkm_fn pick_qkv_m(int nw, int tpt) { BFP_LAYER_SHAPES(BFP_CASE, k_qkv_m) return nullptr; }
static lkm_fn pick_ores_m(int nw, int tpt) { BFP_LAYER_SHAPES(BFP_CASE, k_o_res_m) return nullptr; }
static lkm_fn pick_gu_m(int nw, int tpt) { BFP_LAYER_SHAPES(BFP_CASE, k_gu_m) return nullptr; }
static lkm_fn pick_dres_m(int nw, int tpt) { BFP_LAYER_SHAPES(BFP_CASE, k_d_res_m) return nullptr; }

// Attention variant by context capacity: products per producer wave and
// AV block (2 -> 14 positions, 4 -> 28, 8 -> 56); dynamic LDS may exceed
// 64 KiB at long contexts.
static void shape_for(int nT, int &nw, int &tpt) {
  nw = default_waves(nT);
  tpt = (nT + 4 * nw - 1) / (4 * nw);
}

static int attn_ppw(int max_ctx) {
  return max_ctx <= 128 ? 2 : (max_ctx <= 256 ? 3 : (max_ctx <= 512 ? 4 : 8));
}
static lk_fn attn_kernel(int ppw) {
  // max_ctx <= 512 = 64 * ATT_WAVES for ppw 2, 3 and 4: the short forms
  return ppw == 2 ? k_attn<2, true> : (ppw == 3 ? k_attn<3, true> : (ppw == 4 ? k_attn<4, true> : k_attn<8, false>));
}

// Raise a kernel's dynamic-LDS limit on the current device to at least
// `bytes`, never lowering it: the limit is process-wide per device, and
// another context may already launch the same kernel with a larger need.
static int raise_lds_limit(const void *f, int bytes) {
  static std::mutex mu;
  static std::map<std::pair<int, const void *>, int> limit;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  int &cur = limit[std::make_pair(dev, f)];
  if (bytes > cur) {
    HIP_TRY(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    cur = bytes;
  }
  return BFP_OK;
}

// Per device, before the first launch (outside any stream capture): allow
// the dynamic LDS the attention and multi-sequence kernels take.
int prepare_layer_kernels(int max_ctx, int D, int FFN) {
  const int ppw = attn_ppw(max_ctx);
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(attn_kernel(ppw)),
                          (int)attn_lds_bytes(max_ctx, ppw)));
  int nw, tpt, nwf, tptf;
  shape_for(D / 16, nw, tpt);
  shape_for(FFN / 16, nwf, tptf);
  const int shD = MSEQ * (D / 16) * 17 * 4, shF = MSEQ * (FFN / 16) * 17 * 4;
  const void *fs[4] = {reinterpret_cast<const void *>(pick_qkv_m(nw, tpt)),
                       reinterpret_cast<const void *>(pick_ores_m(nw, tpt)),
                       reinterpret_cast<const void *>(pick_gu_m(nw, tpt)),
                       reinterpret_cast<const void *>(pick_dres_m(nwf, tptf))};
  const int sh[4] = {shD, shD, shD, shF};
  for (int i = 0; i < 4; ++i)
    if (fs[i]) BFP_TRY(raise_lds_limit(fs[i], sh[i]));
  return BFP_OK;
}

static int launch_attn(const LayerArgs &a, hipStream_t s) {
  const int ppw = attn_ppw(a.max_ctx);
  // long contexts: ATT_DSPLIT workgroups per head, one 16-dimension tile each
  const int split = ppw == 8 ? ATT_DSPLIT : 1;
  hipLaunchKernelGGL(attn_kernel(ppw), dim3(a.H_Q * split, a.batch), dim3(64 * ATT_WAVES),
                     attn_lds_bytes(a.max_ctx, ppw), s, a);
  return launch_status("attn");
}

// Waves per workgroup of an MFMA matvec over nT tiles with n_blocks blocks:
// at most one resident round on the chip (two waves per SIMD), at least two
// tiles per wave.
static int mx_waves(int nT, int n_blocks) {
  int w = 2048 / n_blocks;
  w = w < (nT + 1) / 2 ? w : (nT + 1) / 2;
  w = w < MX_WAVES_MAX ? w : MX_WAVES_MAX;
  return w < 1 ? 1 : w;
}

static int launch_layer_mx(const LayerArgs &a, hipStream_t s) {
  const int nTD = a.D / 16, nTF = a.FFN / 16;
  const size_t sh_norm = (size_t)(3 * a.D + PW_MAX_LEAVES) * 8 + (size_t)nTD * 17 * 4;
  const int G = (a.batch + MX_SEQ - 1) / MX_SEQ;
  const int bq = (a.D + 2 * a.KV) / 32, bo = a.D / 16, bg = a.FFN / 16;
  hipLaunchKernelGGL(k_norm_seq, dim3(a.batch), dim3(256), sh_norm, s, a, 1);
  hipLaunchKernelGGL(k_qkv_mx, dim3(bq, G), dim3(64 * mx_waves(nTD, bq * G)),
                     mx_lds_bytes(2, nTD), s, a);
  BFP_TRY(launch_attn(a, s));
  hipLaunchKernelGGL(k_o_res_mx, dim3(bo, G), dim3(64 * mx_waves(nTD, bo * G)),
                     mx_lds_bytes(1, nTD), s, a);
  hipLaunchKernelGGL(k_norm_seq, dim3(a.batch), dim3(256), sh_norm, s, a, 2);
  hipLaunchKernelGGL(k_gu_mx, dim3(bg, G), dim3(64 * mx_waves(nTD, bg * G)),
                     mx_lds_bytes(2, nTD), s, a);
  hipLaunchKernelGGL(k_d_res_mx, dim3(bo, G), dim3(64 * mx_waves(nTF, bo * G)),
                     mx_lds_bytes(1, nTF), s, a);
  return launch_status("layer");
}

static int launch_layer_multi(const LayerArgs &a, hipStream_t s) {
  if (a.batch >= MX_MIN_BATCH) return launch_layer_mx(a, s);
  const int nTD = a.D / 16, nTF = a.FFN / 16;
  int nw, tpt, nwf, tptf;
  shape_for(nTD, nw, tpt);
  shape_for(nTF, nwf, tptf);
  lkm_fn fq = pick_qkv_m(nw, tpt), fo = pick_ores_m(nw, tpt), fg = pick_gu_m(nw, tpt);
  lkm_fn fd = pick_dres_m(nwf, tptf);
  if (!fq || !fo || !fg || !fd) return set_err(BFP_EINVAL, "no layer kernel for D=%d FFN=%d", a.D, a.FFN);
  const int nq = a.D + 2 * a.KV;
  const size_t sh_norm = (size_t)(3 * a.D + PW_MAX_LEAVES) * 8 + (size_t)nTD * 17 * 4;
  const int G = (a.batch + MSEQ - 1) / MSEQ;
  const size_t shD = (size_t)MSEQ * nTD * 17 * 4, shF = (size_t)MSEQ * nTF * 17 * 4;
  hipLaunchKernelGGL(k_norm_seq, dim3(a.batch), dim3(256), sh_norm, s, a, 1);
  hipLaunchKernelGGL(fq, dim3(nq / 16, G), dim3(64 * nw), shD, s, a);
  BFP_TRY(launch_attn(a, s));
  hipLaunchKernelGGL(fo, dim3(a.D / 16, G), dim3(64 * nw), shD, s, a);
  hipLaunchKernelGGL(k_norm_seq, dim3(a.batch), dim3(256), sh_norm, s, a, 2);
  hipLaunchKernelGGL(fg, dim3(a.FFN / 16, G), dim3(64 * nw), shD, s, a);
  hipLaunchKernelGGL(fd, dim3(a.D / 16, G), dim3(64 * nwf), shF, s, a);
  return launch_status("layer");
}

int launch_layer(const LayerArgs &a, hipStream_t s) {
  if (a.batch >= MULTI_MIN_BATCH && a.xn_m) return launch_layer_multi(a, s);
  const int nTD = a.D / 16, nTF = a.FFN / 16;
  int nw, tpt;
  shape_for(nTD, nw, tpt);
  const int nq = a.D + 2 * a.KV;
  const size_t sh_norm = (size_t)(3 * a.D + PW_MAX_LEAVES) * 8 + (size_t)nTD * 17 * 4;
  lk_fn f = pick_qkv(nw, tpt);
  lk_fn fo = pick_ores(nw, tpt), fg = pick_gu(nw, tpt);
  if (!f || !fo || !fg) return set_err(BFP_EINVAL, "no layer kernel for D=%d", a.D);
  hipLaunchKernelGGL(f, dim3(nq / 16, a.batch), dim3(64 * nw), sh_norm, s, a);
  BFP_TRY(launch_attn(a, s));
  hipLaunchKernelGGL(fo, dim3(a.D / 16, a.batch), dim3(64 * nw), (size_t)nTD * 17 * 4, s, a);
  hipLaunchKernelGGL(fg, dim3(a.FFN / 16, a.batch), dim3(64 * nw), sh_norm, s, a);
  int nwf, tptf;
  shape_for(nTF, nwf, tptf);
  f = pick_dres(nwf, tptf);
  if (!f) return set_err(BFP_EINVAL, "no down-proj kernel for FFN=%d", a.FFN);
  hipLaunchKernelGGL(f, dim3(a.D / 16, a.batch), dim3(64 * nwf), (size_t)nTF * 17 * 4, s, a);
  return launch_status("layer");
}

int launch_embed(const EmbedArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3(a.batch), dim3(256), 0, s, a);
  return launch_status("embed");
}

// Head workgroups for `batch` sequences: the batch-1 kernel covers
// rows_single rows per workgroup, the batch > 1 GEMV HEAD_ROWS_MULTI.
int head_workgroups(int vocab, int D, int rows_single, int batch) {
  const int rm = head_rows_multi(D);
  return batch == 1 ? vocab / rows_single : (vocab + rm - 1) / rm;
}

int prepare_head_kernels(int D) {
  const int sh = head_seq_group(D) * D * 8;
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(k_head_gemv<9, 2, true>), sh));
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(k_head_gemv<9, 2, false>), sh));
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(k_head_gemv<27, 1, false>), sh));
  return BFP_OK;
}

int launch_head(const HeadArgs &a, hipStream_t s) {
  size_t sh = (size_t)(3 * a.D + PW_MAX_LEAVES) * 8;
  if (a.batch == 1) {
    if (a.D == 576)
      hipLaunchKernelGGL((k_head_logits<9, true>), dim3(a.n_wg, a.batch), dim3(256), sh, s, a);
    else if (a.D < 576)
      hipLaunchKernelGGL((k_head_logits<9, false>), dim3(a.n_wg, a.batch), dim3(256), sh, s, a);
    else
      hipLaunchKernelGGL((k_head_logits<27, false>), dim3(a.n_wg, a.batch), dim3(256), sh, s, a);
    return launch_status("head");
  }
  if (!a.hn) return set_err(BFP_EINVAL, "head: no normed-hidden buffer for batch %d", a.batch);
  if (a.n_wg != head_workgroups(a.VOCAB, a.D, a.rows_per_wg, a.batch))
    return set_err(BFP_EINVAL, "head: %d workgroups for batch %d", a.n_wg, a.batch);
  hipLaunchKernelGGL(k_head_norm, dim3(a.batch), dim3(256), sh, s, a);
  const int sg = head_seq_group(a.D);
  const size_t shg = (size_t)sg * a.D * 8;
  if (a.D == 576)
    hipLaunchKernelGGL((k_head_gemv<9, 2, true>), dim3(a.n_wg), dim3(256), shg, s, a, sg);
  else if (a.D < 576)
    hipLaunchKernelGGL((k_head_gemv<9, 2, false>), dim3(a.n_wg), dim3(256), shg, s, a, sg);
  else
    hipLaunchKernelGGL((k_head_gemv<27, 1, false>), dim3(a.n_wg), dim3(256), shg, s, a, sg);
  return launch_status("head");
}

int launch_ctl(const CtlArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(k_ctl, dim3(a.batch), dim3(64), 0, s, a);
  hipLaunchKernelGGL(k_step_inc, dim3(1), dim3(64), 0, s, a.state);
  return launch_status("ctl");
}

}  // namespace bfp
