// Device code shared by the per-stage decode kernels (bfp_layer.hip) and
// the persistent decode kernel (bfp_persist.hip): the RMSNorm prologue, the
// matvec epilogues, the attention body and the head's final norm.  Both
// paths run these same functions, so their outputs are bit-identical.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bfp_device.h"
#include "bfp_f64.h"
#include "bfp_layer.h"
#include "bfp_mv.h"

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
// dbuf: 3*D doubles of LDS, leaf: PW_MAX_LEAVES doubles.  Thread tid keeps
// elements tid + k*bs (k < KE) and their gammas in registers from one batch
// of loads, so its up-to-KE divisions and tile quantisations are
// independent chains; the owners of numpy's pairwise leaves load their x
// elements themselves (pairwise_sum_block_g), so nothing is staged in LDS
// before the sum.  gamma(k, i): the gamma of element i, the thread's k-th
// (i = base + tid + k*bs).  All threads call.
template <int KE, class Gamma>
__device__ __forceinline__ void rmsnorm_to_x_g(const int16_t *__restrict__ hm, const int8_t *__restrict__ he,
                                               Gamma gamma, int D, int *xs, int *xes, double *dbuf,
                                               double *leaf, int16_t *dm, int8_t *de) {
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
      gg[k] = gamma(k, i);
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
  for (int base = 0; base < D; base += KE * bs) {   // one pass when D <= KE*bs
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
      // elements i and i ^ 1 sit in lanes l and l ^ 1 (bs is even): the even
      // lane writes the pair into the matvec's input form
      const int odd = __builtin_amdgcn_mov_dpp(mm[k], 0xB1, 0xf, 0xf, false);   // quad_perm 1,0,3,2
      if (i < D) {
        if ((i & 1) == 0) put_x_pair(xs, i >> 4, (i >> 1) & 7, mm[k], odd);
        if ((i & 15) == 0) xes[i >> 4] = ee[k];
        if (dm) {
          dm[i] = (int16_t)mm[k];
          if ((i & 15) == 0) de[i >> 4] = (int8_t)ee[k];
        }
      }
    }
  }
}

// The same RMSNorm with thread t on the adjacent elements 2t and 2t+1
// (D <= 2*blockDim): its two divisions and quantisations are one
// instruction stream, a tile's 16 elements sit in one 8-lane group, and the
// pair goes into the matvec's input form as it is.  The squares' pairwise
// sum: where numpy's leaves are at most 8 equal ones (every D % 64 == 0 up
// to 1024) each wave forms it alone from hm/he (sum_sq_wave: no barrier, no
// leaf buffer), else through sq (D doubles of LDS) and the block-wide sum.
// g0/g1: this thread's gammas.  All threads call.
// Core of it: returns this thread's quantised pair (m0, m1) and its tile's
// exponent e (every thread; meaningful where 2 * tid < D).
__device__ __forceinline__ void rmsnorm_pairs(const int16_t *__restrict__ hm, const int8_t *__restrict__ he,
                                              double g0, double g1, int D, double *sq, double *leaf,
                                              int &m0, int &m1, int &e) {
  const int i0 = 2 * (int)threadIdx.x;
  const bool on = i0 < D;
  const int j = on ? i0 : 0;
  const int e_in = he[j >> 4];
  const double x0 = bfp_val(hm[j], e_in), x1 = bfp_val(hm[j + 1], e_in);
  int nl, L;
  double s;
  if (pw_equal_leaves(D, nl, L)) {   // uniform: every wave forms the sum itself
    s = sum_sq_wave(hm, he, nl, L);
  } else {
    if (on) {
      sq[i0] = x0 * x0;
      sq[i0 + 1] = x1 * x1;
    }
    lds_barrier();
    s = pairwise_sum_block(sq, D, leaf);
  }
  const double rt = sqrt(s / (double)D + 1e-5);
  const double y0 = on ? (x0 * g0) / rt : 0.0;
  const double y1 = on ? (x1 * g1) / rt : 0.0;
  quantize16_pairs(y0, y1, m0, m1, e, true);   // tile_quantize(rmsnorm_fp(.)): canonical
}

__device__ __forceinline__ void rmsnorm_pairs_to_x(const int16_t *__restrict__ hm,
                                                   const int8_t *__restrict__ he, double g0, double g1,
                                                   int D, int *xs, int *xes, double *sq, double *leaf) {
  const int i0 = 2 * (int)threadIdx.x;
  const bool on = i0 < D;
  int m0, m1, e;
  rmsnorm_pairs(hm, he, g0, g1, D, sq, leaf, m0, m1, e);
  if (on) {
    put_x_pair(xs, i0 >> 4, (i0 >> 1) & 7, m0, m1);
    if ((i0 & 15) == 0) xes[i0 >> 4] = e;
  }
}

__device__ __forceinline__ void rmsnorm_to_x(const int16_t *__restrict__ hm, const int8_t *__restrict__ he,
                                             const double *__restrict__ g, int D, int *xs, int *xes,
                                             double *dbuf, double *leaf, int16_t *dm, int8_t *de) {
  rmsnorm_to_x_g<4>(hm, he, [g](int, int i) { return g[i]; }, D, xs, xes, dbuf, leaf, dm, de);
}

// ------------------------------------------------------------- epilogues
// Run by wave 0 (threads < 64) of a chunk's workgroup after chunk_AM: lane
// r + 16k holds row r of chunk c of sequence b (b may differ between the
// four 16-lane groups); only groups with wr set store.

// Tagged words between the workgroups of one launch: a BFP value with an
// 8-bit tag (1..255) of the (step, layer) that wrote it, stored and polled
// with device-scope (SC1) buffer accesses, which bypass the XCD's L2.
typedef __amdgpu_buffer_rsrc_t tw_rsrc;
constexpr int TW_SC1 = 16;
__device__ __forceinline__ tw_rsrc tw_make(const void *base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ unsigned tw_tag(int step, int layer, int NL) {
  return (unsigned)(((long long)step * NL + layer) % 255) + 1u;
}
__device__ __forceinline__ unsigned tw_word(int m, int e, unsigned tag) {
  return ((unsigned)m & 0xffffu) | (((unsigned)e & 0xffu) << 16) | (tag << 24);
}
// Bounded waits on tagged words: every 64 polls, give up (and set the flag
// word at rf) once the flag is set or TW_SPIN_TICKS have passed since t0.
constexpr unsigned long long TW_SPIN_TICKS = 200000000ull;   // 2 s at 100 MHz
__device__ __forceinline__ bool tw_give_up(tw_rsrc rf, unsigned it, unsigned long long t0) {
  if ((it & 63u) != 63u) return false;
  if (__builtin_amdgcn_raw_buffer_load_b32(rf, 0, 0, TW_SC1) != 0u ||
      __builtin_amdgcn_s_memrealtime() - t0 > TW_SPIN_TICKS) {
    __builtin_amdgcn_raw_buffer_store_b32(1u, rf, 0, 0, TW_SC1);
    return true;
  }
  return false;
}

// q|k|v rows: raw BFP out (V dumped here; Q and K post-RoPE by k_attn).
// tag != 0: the row also goes to a.t_qkv as a tagged word.
__device__ __forceinline__ void epi_qkv(const LayerArgs &a, int b, int c, long long A, int M,
                                        bool wr, unsigned tag = 0) {
  const int nq = a.D + 2 * a.KV;
  int m, e;
  chunk_quant(A, M, m, e);
  const int lane = threadIdx.x & 15;
  if (wr) a.qkv_m[b * nq + c * 16 + lane] = (int16_t)m;
  if (wr && lane == 0) a.qkv_e[b * (nq / 16) + c] = (int8_t)e;
  if (wr && tag)
    __builtin_amdgcn_raw_buffer_store_b32(tw_word(m, e, tag), tw_make(a.t_qkv, 0x7fffffff),
                                          4 * (b * nq + c * 16 + lane), 0, TW_SC1);
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
// tag != 0: h1 also goes to a.t_h1 as a tagged word.
__device__ __forceinline__ void epi_ores(const LayerArgs &a, int b, int c, long long A, int M,
                                         bool wr, int rm, int re, unsigned tag = 0) {
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
    if (tag)
      __builtin_amdgcn_raw_buffer_store_b32(tw_word(m, e, tag), tw_make(a.t_h1, 0x7fffffff), 4 * row, 0,
                                            TW_SC1);
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

// One lane of the SwiGLU: silu_fp(g) = fp_quantize_vec(g / (1 + exp(-g)))
// (full.py:241-242), then mlp = fp_quantize_vec(silu * u) (full.py:290), in
// the canonical form the down projection reads.  All 16 lanes of the tile
// call (the quantisations exchange the tile's maximum).
__device__ __forceinline__ int swiglu_lane(int gm, int ge, int um, int ue, int &me) {
  const double gv = bfp_val(gm, ge);
  int se;
  const int sm = quantize16_lanes(gv / (1.0 + exp_f64(-gv)), se);
  return quantize16_lanes(bfp_val(sm, se) * bfp_val(um, ue), me, true);
}

// g, u -> mlp = q(q(silu(g)) * u)   (full.py:241-242,288-290)
__device__ __forceinline__ void epi_gu(const LayerArgs &a, int b, int c, long long Ag, int Mg,
                                       long long Au, int Mu, bool wr) {
  const int r = threadIdx.x & 15;
  int gm, ge, um, ue;
  chunk_quant(Ag, Mg, gm, ge);
  chunk_quant(Au, Mu, um, ue);
  int me;
  const int mm = swiglu_lane(gm, ge, um, ue, me);   // D's input
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
// tag != 0: h also goes to a.t_h as a tagged word.
__device__ __forceinline__ void epi_dres(const LayerArgs &a, int b, int c, long long A, int M,
                                         bool wr, int rm, int re, unsigned tag = 0) {
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
    if (tag)
      __builtin_amdgcn_raw_buffer_store_b32(tw_word(m, e, tag), tw_make(a.t_h, 0x7fffffff), 4 * row, 0,
                                            TW_SC1);
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

// ------------------------------------------------------------------ attn
// Attention access through ordinary loads and stores: this sequence's q|k|v
// (D + 2KV, raw BFP) in, its attention output (D) out.
struct AttnPlainIO {
  // long form: every workgroup of a head scores all positions itself
  static constexpr bool kSplitScores = false;
  static constexpr int kAvBlock = 32;   // AV products: 16 KB of LDS, three workgroups a CU
  const int16_t *qm;
  const int8_t *qe;
  int16_t *om;
  int8_t *oe;
  __device__ __forceinline__ void qkv(int idx, int &m, int &e) const {
    m = qm[idx];
    e = qe[idx >> 4];
  }
  __device__ __forceinline__ uint4 k16(const int16_t *p) const { return *reinterpret_cast<const uint4 *>(p); }
  __device__ __forceinline__ uint4 v16(const int16_t *p) const { return *reinterpret_cast<const uint4 *>(p); }
  __device__ __forceinline__ int ke4(const int8_t *p) const { return *reinterpret_cast<const int *>(p); }
  __device__ __forceinline__ int ve4(const int8_t *p) const { return *reinterpret_cast<const int *>(p); }
  __device__ __forceinline__ int km1(const int16_t *p) const { return *p; }
  __device__ __forceinline__ int ke1(const int8_t *p) const { return *p; }
  __device__ __forceinline__ int ve1(const int8_t *p) const { return *p; }
  // loads of rows that may lie past the position (live false): read anyway,
  // the clamped row is a cache hit
  __device__ __forceinline__ uint4 k16l(const int16_t *p, bool) const { return k16(p); }
  __device__ __forceinline__ int ke4l(const int8_t *p, bool) const { return ke4(p); }
  __device__ __forceinline__ uint4 v16l(const int16_t *p, bool) const { return v16(p); }
  __device__ __forceinline__ int ve1l(const int8_t *p, bool) const { return ve1(p); }
  __device__ __forceinline__ void k_put(int16_t *pm, int8_t *pe, int m, int e, bool we) const {
    *pm = (int16_t)m;
    if (we) *pe = (int8_t)e;
  }
  __device__ __forceinline__ void v_put(int16_t *pm, int8_t *pe, int m, int e, bool we) const {
    k_put(pm, pe, m, e, we);
  }
  __device__ __forceinline__ void before_out() const {}
  __device__ __forceinline__ void out(int idx, int m, int e, bool we) const {
    om[idx] = (int16_t)m;
    if (we) oe[idx >> 4] = (int8_t)e;
  }
  // phase stamps of a traced decode (ATT_MARK_*); none on this path
  __device__ __forceinline__ void mark(int) const {}
  // the (cos, sin) of RoPE pair j from the row at cs
  __device__ __forceinline__ void rope_cs(const double *cs, int j, double &c, double &s) const {
    c = cs[2 * j];
    s = cs[2 * j + 1];
  }
};

// The attention's phase stamps (IO::mark), in the order they are taken.
constexpr int ATT_MARK_ROPE = 0;      // q|k|v in, RoPE done, the cache row stored
constexpr int ATT_MARK_SCORES = 1;    // every score in LDS (after the long form's exchange)
constexpr int ATT_MARK_SOFTMAX = 2;   // probabilities in LDS
constexpr int ATT_MARK_AV = 3;        // the AV chains done
constexpr int ATT_MARK_QKV = 4;       // wave 0's q|k|v input in (its q head)

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
// ATT_DSPLIT, attn_sc_block, attn_sc_stride: bfp_layer.h
constexpr int AVL_PW = 3;
constexpr int AVL_TB = AVL_PW * 64;
constexpr int AVL_TBP = AVL_TB + 2;
constexpr int AVL_DEPTH = 4;
constexpr int AVL_G = 8;        // chain: positions per group of LDS reads
constexpr int AVL_AHEAD = 3;    // chain: groups of reads in flight ahead of the adds
// av_block: rows of the short forms' AV products held in LDS at once
// (IO::kAvBlock)
// The long form with split scores (IO::kSplitScores) stages a pass of K rows
// (64 * ATT_WAVES of them, ATT_KS mantissas and 4 exponents a row) in the
// AV buffers' space before the AV phase: kstage.
constexpr int ATT_KS = 72;   // 144-byte rows: 8 consecutive rows' 16-byte reads hit distinct bank groups
inline size_t attn_lds_bytes(int max_ctx, int ppw, int av_block, bool kstage = false) {
  const size_t sc_len = (size_t)((max_ctx + 1) & ~1);
  size_t av = ppw <= 4 ? (size_t)2 * ATT_AVC * (64 * 2 + 4) : (size_t)2 * 16 * AVL_TBP * 8;
  const size_t ks = (size_t)64 * ATT_WAVES * (ATT_KS * 2 + 4);
  if (ppw > 4 && kstage && ks > av) av = ks;
  const size_t pr = ppw <= 4 ? (size_t)av_block * 64 * 8 : 0;
  return (256 + sc_len) * 8 + av + pr;
}

// One K row of the cache (64 mantissas, 4 tile exponents) in registers.
struct KRow {
  uint4 m[8];
  int e4;
};
// live: the row is at or before the position (else the IO may skip the
// memory request: the values are never used)
template <class IO>
__device__ __forceinline__ void load_krow(const IO &io, KRow &r, const int16_t *Km, const int8_t *Ke,
                                          long long o, bool live) {
#pragma unroll
  for (int i = 0; i < 8; ++i) r.m[i] = io.k16l(Km + o + 8 * i, live);
  r.e4 = io.ke4l(Ke + (o >> 4), live);
}

// The attention of one head (or one tile of it) for one sequence.  The body
// runs in workgroup `bx` of sequence b's launch (head bx, or head
// bx / ATT_DSPLIT and tile bx % ATT_DSPLIT in the long form) over KV slots
// 0..pos with RoPE position rpos.  `io` carries every access to the q|k|v
// input, the KV cache and the output (AttnPlainIO: ordinary loads and
// stores; the persistent decode kernel's form reads and writes at the
// device-coherent level).  dsm: attn_lds_bytes(a.max_ctx, PPW, IO::kAvBlock) of LDS.
template <int PPW, bool SHORT, class IO, class PosF>
__device__ __forceinline__ void attn_body(const LayerArgs &a, IO &io, int bx, int b, PosF posf,
                                          double *dsm) {
  constexpr int NT = 64 * ATT_WAVES;
  constexpr int AVC = ATT_AVC;                 // V rows per staged chunk (short)
  constexpr int VL = AVC * 8 / NT;             // 16-byte V loads per thread and chunk
  constexpr int TB = AVL_TB;                   // positions per AV block (long)
  static_assert(SHORT || PPW == 8, "the long form is instantiated as PPW 8");
  static_assert(AVL_PW + 1 <= ATT_WAVES && AVL_TB % 8 == 0 && AVL_TBP % 2 == 0, "long AV geometry");
  double *q = dsm;                  // 64
  double *kc = dsm + 64;            // 64 (current position, post-rope)
  double *vc = dsm + 128;           // 64
  double *leaf = dsm + 192;         // PW_MAX_LEAVES (= 64)
  double *sc = dsm + 256;           // max_ctx, rounded up to even
  // short: staged V, 2 x AVC x 64 mantissas and 2 x AVC x 4 exponents;
  // long: product double buffer, 2 x 16 dimensions x AVL_TBP doubles
  int16_t *vsm = reinterpret_cast<int16_t *>(sc + ((a.max_ctx + 1) & ~1));
  int8_t *vse = reinterpret_cast<int8_t *>(vsm + 2 * AVC * 64);
  double *prod = reinterpret_cast<double *>(vse + 2 * AVC * 4);   // IO::kAvBlock x 64
  double *buf = sc + ((a.max_ctx + 1) & ~1);
  __shared__ double red[ATT_WAVES];
  const int hq = SHORT ? bx : bx / ATT_DSPLIT;
  const int dg = SHORT ? 0 : bx % ATT_DSPLIT;   // long: the tile of dimensions 16dg ..
  const bool lead = dg == 0;                             // stores the cache row and the dumps
  const int grp = a.H_Q / a.H_KV, g = hq / grp;
  const int HD = 64;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const long long kv_tok = (long long)a.H_KV * HD;     // elements per position
  int16_t *Km = a.k_m + (long long)b * a.max_ctx * kv_tok;
  int8_t *Ke = a.k_e + (long long)b * a.max_ctx * (kv_tok / 16);
  int16_t *Vm = a.v_m + (long long)b * a.max_ctx * kv_tok;
  int8_t *Ve = a.v_e + (long long)b * a.max_ctx * (kv_tok / 16);
  const bool writer = (hq % grp) == 0 && lead;

  // contexts of at most 128 (PPW 2) or 256 (PPW 3) positions: each 32-lane
  // half-wave scores one position, lane j (of 32) holding elements j and
  // 32 + j of its K row, in passes of 2*ATT_WAVES positions.  The elements
  // of LS_PRE passes (128 positions) are in registers at once: the first
  // group's are loaded before the position is read (rows clamped to the
  // cache's last slot: their values past n - 1 are never used), a second
  // group's (PPW 3, more than 128 positions) after the first is scored.
  // (Eight passes keep the PPW 3 form within 80 registers: three workgroups
  // per CU.  Staging the rows through LDS with 16-byte loads instead, and
  // reading the lanes' elements from there, measured slower: config 5
  // 33.1k -> 32.8k tokens/s.)
  constexpr bool LANE_SPLIT = SHORT && (PPW == 2 || PPW == 3);
  constexpr int LS_PASS = LANE_SPLIT ? (PPW == 2 ? 128 : 256) / (2 * ATT_WAVES) : 1;
  constexpr int LS_PRE = LS_PASS < 8 ? LS_PASS : 8;
  int lsm[LS_PRE][2], lse[LS_PRE][2];
  auto ls_load = [&](int g0, int last) {   // passes g0 .. g0 + LS_PRE - 1, rows up to `last`
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
  if constexpr (LANE_SPLIT) ls_load(0, a.max_ctx - 1);
  // this wave's q|k|v input: q head hq (wave 0), k head g (1), v head g (2
  // and the rest, which do not use it)
  int in_m, in_e;
  io.qkv(w == 0 ? hq * HD + l : (w == 1 ? a.D + g * HD + l : a.D + a.KV + g * HD + l), in_m, in_e);
  io.mark(ATT_MARK_QKV);
  // the position is read after the loads that do not depend on it are issued
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const int2 pp = posf();   // (KV slot, RoPE position)
  const int pos = pp.x, rpos = pp.y;
  const int n = pos + 1;
  const double *cs = a.rope_row ? a.rope_row                 // (HD/2) x (cos, sin)
                                : a.rope + (long long)rpos * HD;
  // this lane's (cos, sin), read before the K rows below are requested (the
  // persistent kernel's row is in LDS and is read as such: through a generic
  // pointer it is a FLAT load, and a wait on one also waits for every vector
  // load issued before it, which cost the long form 3 us)
  double rcos = 0.0, rsin = 0.0;
  if (w < 2) io.rope_cs(cs, l & 31, rcos, rsin);

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
      vr[j] = io.v16(Vg + t_ * vstride);               \
    }                                                                            \
    int t_ = (c) * AVC + (tid < AVC ? tid : 0);                                  \
    t_ = t_ < n ? t_ : n - 1;                                                    \
    ver = io.ve4(Veg + t_ * (vstride / 16));             \
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
      const bool live = t < n;
      t = live ? t : n - 1;
      const long long o = ((long long)t * a.H_KV + g) * HD + 16 * dg + 8 * hh;
      m[r] = io.v16l(Vm + o, live);
      e[r] = io.ve1l(Ve + (o >> 4), live);
    }
  };

  // the first K row of this thread's scores, in flight during the RoPE phase
  // (long contexts: KR rows per thread in flight, the first since the RoPE
  // phase, so a pass over 64 * ATT_WAVES * KR positions waits for memory once)
  constexpr int KR = SHORT ? 1 : 2;
  KRow kr[KR];
  // long form with IO::kSplitScores: the head's ATT_DSPLIT workgroups split
  // the scores, workgroup dg taking rows t = ATT_DSPLIT u + dg (u < nu),
  // and exchange them (see below); else every workgroup takes every row
  constexpr int RS = (!SHORT && IO::kSplitScores) ? ATT_DSPLIT : 1;
  const int r0 = RS > 1 ? dg : 0;
  const int nu = (n - r0 + RS - 1) / RS;
  // long form with split scores: each pass of the workgroup's rows (u0 ..
  // u0 + NT - 1) is staged through LDS with coalesced loads -- 8 lanes per
  // row, lane l part l % 8 of row l / 8 + 8i of its wave's 64 -- instead of
  // each thread loading its own row (the same bytes at a third of the rate
  // per CU); rows from pos on are never loaded (row pos is scored from kc)
  constexpr bool KST = !SHORT && IO::kSplitScores;
  int16_t *kst = reinterpret_cast<int16_t *>(buf);          // NT x ATT_KS
  int8_t *kex = reinterpret_cast<int8_t *>(kst + NT * ATT_KS);   // NT x 4
  uint4 ks[KST ? 8 : 1];
  int kse = 0;
  auto kst_load = [&](int u0) {
#pragma unroll
    for (int i = 0; i < (KST ? 8 : 1); ++i) {
      const int t = RS * (u0 + 64 * w + 8 * i + (l >> 3)) + r0;
      const bool live = t < pos;
      ks[i] = io.k16l(Km + ((long long)(live ? t : 0) * a.H_KV + g) * HD + 8 * (l & 7), live);
    }
    const int t = RS * (u0 + tid) + r0;
    const bool live = t < pos;
    kse = io.ke4l(Ke + ((((long long)(live ? t : 0) * a.H_KV + g) * HD) >> 4), live);
  };
  auto kst_store = [&]() {
#pragma unroll
    for (int i = 0; i < (KST ? 8 : 1); ++i)
      *reinterpret_cast<uint4 *>(kst + (64 * w + 8 * i + (l >> 3)) * ATT_KS + 8 * (l & 7)) = ks[i];
    *reinterpret_cast<int *>(kex + 4 * tid) = kse;
  };
  if constexpr (KST) {
    kst_load(0);
  } else if constexpr (!LANE_SPLIT) {
    const int t = RS * tid + r0;
    load_krow(io, kr[0], Km, Ke, ((long long)(t < n ? t : n - 1) * a.H_KV + g) * HD, t < n);
  }

  if (w == 0) {            // q head hq
    int idx = hq * HD + l;
    int e;
    int m = rope_lane(bfp_val(in_m, in_e), rcos, rsin, e);
    q[l] = bfp_val(m, e);
    if (a.dump && lead) {
      int cm, ce;
      canon_copy(m, e, cm, ce);
      a.dump->m[ST_Q][b * a.dump->mstride[ST_Q] + idx] = (int16_t)cm;
      if ((l & 15) == 0) a.dump->e[ST_Q][b * (a.dump->mstride[ST_Q] / 16) + (idx >> 4)] = (int8_t)ce;
    }
  } else if (w == 1) {     // k head g
    int e;
    int m = rope_lane(bfp_val(in_m, in_e), rcos, rsin, e);
    kc[l] = bfp_val(m, e);
    long long o = ((long long)pos * a.H_KV + g) * HD + l;
    if (writer) {
      io.k_put(Km + o, Ke + (o >> 4), m, e, (l & 15) == 0);
    }
    if (a.dump && writer) {
      int cm, ce;
      canon_copy(m, e, cm, ce);
      int r = g * HD + l;
      a.dump->m[ST_K][b * a.dump->mstride[ST_K] + r] = (int16_t)cm;
      if ((l & 15) == 0) a.dump->e[ST_K][b * (a.dump->mstride[ST_K] / 16) + (r >> 4)] = (int8_t)ce;
    }
  } else if (w == 2) {     // v head g (not rotated)
    const int m = in_m, e = in_e;
    vc[l] = bfp_val(m, e);
    long long o = ((long long)pos * a.H_KV + g) * HD + l;
    if (writer) {
      io.v_put(Vm + o, Ve + (o >> 4), m, e, (l & 15) == 0);
    }
  }
  if constexpr (KST) kst_store();   // the first pass's K rows
  lds_barrier();
  io.mark(ATT_MARK_ROPE);

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
      if (g0 > 0) ls_load(g0, n - 1);
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
        if (j == 31 && t < n) sc[t] = tot * a.score_mul;
      }
    }
  } else if constexpr (SHORT) {
    // contexts of at most NT positions: one row per thread, the one in
    // flight since the RoPE phase
    if (tid < n) sc[tid] = ddot64_skx_bfp(q, kr[0].m, kr[0].e4) * a.score_mul;
    if (tid == pos) sc[pos] = ddot64_skx(q, kc) * a.score_mul;
  } else if constexpr (KST) {
    // one staged row per thread and pass (the first pass's rows were
    // written to LDS before the RoPE barrier)
    for (int u0 = 0; u0 < nu; u0 += NT) {   // uniform
      if (u0 > 0) {
        lds_barrier();   // the previous pass's rows are read
        kst_load(u0);
        kst_store();
        lds_barrier();
      }
      const int t = RS * (u0 + tid) + r0;
      const double sj = ddot64_skx_bfp(q, reinterpret_cast<const uint4 *>(kst + tid * ATT_KS),
                                       *reinterpret_cast<const int *>(kex + 4 * tid)) * a.score_mul;
      if (t < n) sc[t] = sj;
    }
    if ((pos - r0) % RS == 0 && tid == ((pos - r0) / RS) % NT) sc[pos] = ddot64_skx(q, kc) * a.score_mul;
    if constexpr (RS > 1) {
      // exchange: publish this workgroup's rows (each thread the rows it
      // scored), then read the other workgroups' (the same q, K rows and
      // ddot order, so the same bits); each workgroup's block is contiguous
      // (attn_sc_block), and a thread's reads are all issued before the
      // first is used
      for (int u = tid; u < nu; u += NT) io.score_put(hq, r0, u, sc[RS * u + r0]);
      const int nb = (n + RS - 1) / RS;   // rows of the longest block
      constexpr int GL = 4;
      for (int i0 = 0; i0 < RS * nb; i0 += GL * NT) {   // uniform
        uint4 v[GL];
#pragma unroll
        for (int k = 0; k < GL; ++k) {
          const int i = min(i0 + tid + k * NT, RS * nb - 1);
          v[k] = io.score_raw(hq, i / nb, i % nb);
        }
#pragma unroll
        for (int k = 0; k < GL; ++k) {
          const int i = i0 + tid + k * NT, d_ = i / nb, t = RS * (i % nb) + d_;
          if (i < RS * nb && d_ != r0 && t < n) sc[t] = io.score_val(v[k], hq, d_, i % nb);
        }
      }
    }
  } else {
    // passes of KR rows per thread: rows t = RS u + r0, u = u0 + tid + j*NT;
    // kr[0] of the next pass is loaded as soon as this pass's kr[0] is
    // consumed
    const int last = n - 1;
    for (int u0 = 0; u0 < nu; u0 += KR * NT) {
#pragma unroll
      for (int j = 1; j < KR; ++j) {
        const int t = RS * (u0 + tid + j * NT) + r0;
        load_krow(io, kr[j], Km, Ke, ((long long)(t < n ? t : last) * a.H_KV + g) * HD, t < n);
      }
#pragma unroll
      for (int j = 0; j < KR; ++j) {
        const int t = RS * (u0 + tid + j * NT) + r0;
        const double sj = ddot64_skx_bfp(q, kr[j].m, kr[j].e4) * a.score_mul;
        if (j == 0) {
          const int tn = t + RS * KR * NT;
          load_krow(io, kr[0], Km, Ke, ((long long)(tn < n ? tn : last) * a.H_KV + g) * HD, tn < n);
        }
        if (t < n) sc[t] = sj;
      }
    }
    // row pos from LDS, by the thread that scored it from the cache
    if ((pos - r0) % RS == 0 && tid == ((pos - r0) / RS) % NT) sc[pos] = ddot64_skx(q, kc) * a.score_mul;
  }
  if constexpr (SHORT) {
    BFP_ATT_STORE_V(0)
  } else {
#pragma unroll
    for (int d = 0; d < AVL_DEPTH; ++d) load_blk(d, rm[d], re[d]);   // overlaps the softmax
  }
  lds_barrier();
  io.mark(ATT_MARK_SCORES);
  // softmax_fp (full.py:245-247): e = exp(s - max); p = e / pairwise_sum(e)
  if (SHORT && n <= 128) {
    // wave 0 alone (only it reads p in the short forms' AV chain): lane l
    // holds positions l and l + 64; numpy's sum of n <= 128 is one block --
    // n < 8 added in order from 0.0, else accumulators r_j (lanes 0-7,
    // positions j, j + 8, ... in order) combined
    // ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the last n % 8 in order --
    // plus the reduction's initial 0.0.  No barrier: the wave reads back
    // only its own LDS writes.
    if (w == 0) {
      const double s0 = l < n ? sc[l] : -INFINITY, s1 = l + 64 < n ? sc[l + 64] : -INFINITY;
      double mx = fmax(s0, s1);
      mx = fmax(mx, peer<32>(mx));
      mx = fmax(mx, peer<16>(mx));
      mx = fmax(mx, peer<8>(mx));
      mx = fmax(mx, peer<4>(mx));
      mx = fmax(mx, peer<2>(mx));
      mx = fmax(mx, peer<1>(mx));
      const double e0 = exp_f64(s0 - mx), e1 = exp_f64(s1 - mx);
      if (l < n) sc[l] = e0;
      if (l + 64 < n) sc[l + 64] = e1;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      double res;
      if (n < 8) {
        res = 0.0;
        for (int t = 0; t < n; ++t) res += sc[t];
      } else {
        const int top = n - n % 8, j = l & 7;
        double r = sc[j];
        for (int t = 8 + j; t < top; t += 8) r = r + sc[t];
        r = r + dpp_f64(r, 0xB1);
        r = r + dpp_f64(r, 0x4E);
        r = r + dpp_f64(r, 0x141);
        const long long rb = __double_as_longlong(r);
        res = __longlong_as_double(
            (long long)(((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)(rb >> 32), 0) << 32) |
                        (unsigned)__builtin_amdgcn_readlane((int)(rb & 0xffffffffLL), 0)));
        for (int t = top; t < n; ++t) res += sc[t];
      }
      const double sum = 0.0 + res;
      if (l < n) sc[l] = e0 / sum;
      if (l + 64 < n) sc[l + 64] = e1 / sum;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
  } else {
    double mx = -INFINITY;
    for (int t = tid; t < n; t += NT) mx = fmax(mx, sc[t]);
    mx = fmax(mx, peer<32>(mx));
    mx = fmax(mx, peer<16>(mx));
    mx = fmax(mx, peer<8>(mx));
    mx = fmax(mx, peer<4>(mx));
    mx = fmax(mx, peer<2>(mx));
    mx = fmax(mx, peer<1>(mx));
    if (l == 0) red[w] = mx;
    lds_barrier();
    mx = red[0];
#pragma unroll
    for (int i = 1; i < ATT_WAVES; ++i) mx = fmax(mx, red[i]);
    for (int t = tid; t < n; t += NT) sc[t] = exp_f64(sc[t] - mx);
    lds_barrier();
    const double sum = pairwise_sum_block(sc, n, leaf);
    for (int t = tid; t < n; t += NT) sc[t] = sc[t] / sum;
    lds_barrier();
  }

  io.mark(ATT_MARK_SOFTMAX);
  double acc = 0.0;
  if constexpr (SHORT) {
    // attn_h = sum_t p[t] * V[t], ascending t from 0.0 (full.py:280-281):
    // every product rounded, then added, in t order.  Every thread forms a
    // block of IO::kAvBlock rows' products p[t] * (m * 2^(e-15)) into LDS,
    // one per position and dimension; wave 0 then only reads and adds them,
    // one dimension per lane.  (Wave 0 forming each product itself cost
    // about 70 cycles per position.)  Chunk c+1 of V is loaded while chunk c
    // is used.  Row pos is this launch's V (vc): its writer workgroup may not
    // have stored it yet; it is added last.
    constexpr int PB = IO::kAvBlock;
    static_assert(PB >= 16 && PB % 16 == 0 && PB <= AVC, "AV product block");
    const int nch = (n + AVC - 1) / AVC;
    if (n <= 128) lds_barrier();   // wave 0's softmax wrote p without a barrier
    for (int c = 0; c < nch; ++c) {
      BFP_ATT_LOAD_V(c + 1 < nch ? c + 1 : c)
      const int t0 = c * AVC, t1 = min(pos, t0 + AVC);   // rows t0 .. t1-1
      const int16_t *vmc = vsm + (c & 1) * AVC * 64;
      const int8_t *vec = vse + (c & 1) * AVC * 4;
      for (int r0 = 0; r0 < t1 - t0; r0 += PB) {         // uniform
        const int nr = min(PB, t1 - t0 - r0);
        for (int q = tid; q < nr * 64; q += NT) {
          const int r = r0 + (q >> 6), dd = q & 63;
          prod[q] = sc[t0 + r] * ldexp((double)vmc[r * 64 + dd], (int)vec[r * 4 + (dd >> 4)] - 15);
        }
        lds_barrier();
        if (w == 0) {
          // 16 positions at a time: their LDS reads are issued together;
          // only the adds form the chain
          const double *pl = prod + l;
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
      if (w == 0 && c == nch - 1) acc = acc + sc[pos] * vc[l];
      if (c + 1 < nch) BFP_ATT_STORE_V(c + 1)
      lds_barrier();
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
        if (k <= nb) lds_barrier();
      }
    }
    if (w == 0) acc = acc + sc[pos] * vc[16 * dg + (l & 15)];
  }
#undef BFP_ATT_LOAD_V
#undef BFP_ATT_STORE_V
  io.mark(ATT_MARK_AV);
  io.before_out();   // the cache row stored above is visible before the output is
  if (w == 0) {
    // lanes 0-15 of the long form hold its tile; all 64 lanes take part
    int e;
    int m = quantize16_lanes(acc, e, true);   // tile_quantize(fp_quantize_vec(attn))
    const int idx = hq * HD + (SHORT ? l : 16 * dg + l);
    if (SHORT || l < 16) {
      io.out(idx, m, e, (l & 15) == 0);
    }
    if (a.dump && (SHORT || l < 16)) {
      a.dump->m[ST_ATTN][b * a.dump->mstride[ST_ATTN] + idx] = (int16_t)m;
      if ((l & 15) == 0)
        a.dump->e[ST_ATTN][b * (a.dump->mstride[ST_ATTN] / 16) + (idx >> 4)] = (int8_t)e;
    }
  }
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
  lds_barrier();
  const double s = pairwise_sum_block(sq, D, leaf);
  const double rt = sqrt(s / (double)D + 1e-5);
  for (int i = tid; i < D; i += bs) hn[i] = (xv[i] / rt) * wv[i];
}

// One logit of the decode head: lane l16 of the row's 16 lanes sums
// k = 64i + 4*l16 + c (i ascending, c = 0..3) with FMA from the float32
// row f (f[i] holds k = 64i + 4*l16 .. +3) and the normed hidden hn, then a
// fixed 16-lane butterfly (every lane ends with the total).  MAXD64 >= D/64
// (d64); EXACT when they are equal.
template <int MAXD64, bool EXACT>
__device__ __forceinline__ double head_row_dot(const float4 (&f)[MAXD64], const double *hn, int l16,
                                               int d64) {
  double acc = 0.0;
#pragma unroll
  for (int i = 0; i < MAXD64; ++i) {
    if (EXACT || i < d64) {
      const double *hp = hn + i * 64 + 4 * l16;
      acc = fma((double)f[i].x, hp[0], acc);
      acc = fma((double)f[i].y, hp[1], acc);
      acc = fma((double)f[i].z, hp[2], acc);
      acc = fma((double)f[i].w, hp[3], acc);
    }
  }
  acc = psum<8>(acc);
  acc = psum<4>(acc);
  acc = psum<2>(acc);
  return psum<1>(acc);
}

// The token loop after step s's head (argmax nid).  The simulator's loop
// (full.py:432-443) records the argmax of steps n_prompt .. n_prompt+n_gen-1
// and feeds prompt[s+1] during the prompt, then the last prompt token once
// more (its loop re-reads ids[-1] at step n_prompt), then the argmax.  The
// FPGA's loop (autoregress_bfp_top.sv:357-386) records every step's argmax
// and feeds prompt[s+1], then the argmax.
__device__ __forceinline__ int ctl_out_len(int n_prompt, int n_gen, int rtl_loop) {
  return rtl_loop ? n_prompt + n_gen : n_gen;
}
// Slot of out[] that step s's argmax goes to, or -1.
__device__ __forceinline__ int ctl_out_slot(int s, int n_prompt, int n_gen, int rtl_loop) {
  if (rtl_loop) return s < n_prompt + n_gen ? s : -1;
  return s >= n_prompt && s - n_prompt < n_gen ? s - n_prompt : -1;
}
// The input token of step s + 1.
__device__ __forceinline__ int ctl_next(int s, int nid, int n_prompt, const int *prompt, int rtl_loop) {
  if (s + 1 < n_prompt) return prompt[s + 1];
  if (!rtl_loop && s + 1 == n_prompt) return prompt[n_prompt - 1];
  return nid;
}

}  // namespace bfp
