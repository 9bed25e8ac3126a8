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

#include "bfp_attn_grp.h"
#include "bfp_layer_dev.h"

namespace bfp {

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
// One launch per layer step: grid (H_Q, batch) for the short forms,
// (H_Q * ATT_DSPLIT, batch) for the long one (attn_body has the phases).
// SHORT: max_ctx <= 64 * ATT_WAVES, at most one score per thread (PPW 4) or
// one per 32-lane half-wave (PPW 2: max_ctx <= 128, PPW 3: <= 256); fewer
// registers -- at most 80 for PPW 3, so three workgroups fit a CU (many
// sequences at short context), two for PPW 2 and 4 (PPW 2 at 80 registers
// measured 1.6% slower at batch 1).
template <int PPW, bool SHORT>
__global__ __launch_bounds__(64 * ATT_WAVES, (SHORT ? (PPW == 3 ? 6 : 4) : 2)) void k_attn(LayerArgs a) {
  extern __shared__ double dsm[];
  const int b = blockIdx.y, nq = a.D + 2 * a.KV;
  AttnPlainIO io{a.qkv_m + b * nq, a.qkv_e + b * (nq / 16), a.att_m + b * a.D,
                 a.att_e + b * (a.D / 16)};
  attn_body<PPW, SHORT>(a, io, blockIdx.x, b, [&] { return make_int2(cur_kv_pos(a), cur_pos(a)); }, dsm);
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
  __shared__ int redM[2 * NW * 16];
  __shared__ long long redA[2 * NW * 16];
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
  chunk_AM2<NW, TPT>(RG, RU, xs, xes, nT, redM, redA, Ag, Mg, Au, Mu);   // G and U in one pass
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

// xn (and the stage dump) of sequence b from rmsnorm_pairs' (m0, m1, e).
__device__ __forceinline__ void norm_pairs_out(const LayerArgs &a, int b, int which, int m0, int m1,
                                               int e) {
  const int i0 = 2 * (int)threadIdx.x, nT = a.D / 16;
  const bool on = i0 < a.D;
  if (on) {
    int16_t *om = a.xn_m + (long long)b * a.D;
    int8_t *oe = a.xn_e + (long long)b * nT;
    *reinterpret_cast<int *>(om + i0) = (m0 & 0xffff) | (m1 << 16);
    if ((i0 & 15) == 0) oe[i0 >> 4] = (int8_t)e;
    if (a.dump) {
      const int st = which == 1 ? ST_N1 : ST_N2;
      const StageDump *d = a.dump;
      d->m[st][b * d->mstride[st] + i0] = (int16_t)m0;
      d->m[st][b * d->mstride[st] + i0 + 1] = (int16_t)m1;
      if ((i0 & 15) == 0) d->e[st][b * (d->mstride[st] / 16) + (i0 >> 4)] = (int8_t)e;
    }
  }
}

// The same with thread t on elements 2t, 2t + 1 (rmsnorm_pairs; blockDim
// >= D / 2): one division pair and one tile quantisation per thread, the
// squares' pairwise sum over LDS.  dsm: D + PW_MAX_LEAVES doubles.
__global__ __launch_bounds__(512) void k_norm_pairs(LayerArgs a, int which) {
  extern __shared__ double dsm[];
  const int b = blockIdx.x, nT = a.D / 16;
  const int16_t *hm = (which == 1 ? a.h_m : a.h1_m) + (long long)b * a.D;
  const int8_t *he = (which == 1 ? a.h_e : a.h1_e) + (long long)b * nT;
  const double *g = which == 1 ? a.g1 : a.g2;
  const int i0 = 2 * (int)threadIdx.x;
  const double2 gg = *reinterpret_cast<const double2 *>(g + (i0 < a.D ? i0 : 0));
  int m0, m1, e;
  rmsnorm_pairs(hm, he, gg.x, gg.y, a.D, dsm, dsm + a.D, m0, m1, e);
  norm_pairs_out(a, b, which, m0, m1, e);
}

// The RMSNorm launch of the multi-sequence paths: the pair form up to
// D = 1024, else one thread per 4 elements (k_norm_seq).
static void launch_norm_seq(const LayerArgs &a, int which, hipStream_t s) {
  if (a.D <= 1024) {
    const int nt = (a.D / 2 + 63) / 64 * 64;
    hipLaunchKernelGGL(k_norm_pairs, dim3(a.batch), dim3(nt), (size_t)(a.D + PW_MAX_LEAVES) * 8, s,
                       a, which);
  } else {
    const size_t sh = (size_t)(3 * a.D + PW_MAX_LEAVES) * 8 + (size_t)(a.D / 16) * 17 * 4;
    hipLaunchKernelGGL(k_norm_seq, dim3(a.batch), dim3(256), sh, s, a, which);
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
// The phase stamps of a traced batched decode (MX_TRACE_KERNELS x
// MX_TRACE_BLOCKS x MX_TRACE_STAMPS), set by set_mx_trace.  Only the kernel
// instances launched for a traced decode (TR) read it, so an untraced launch
// carries no stamp code and no extra argument (a null test per phase cost
// config 5 2.7%, a trace pointer in LayerArgs 0.4%).
__device__ unsigned long long *g_mx_trace;
int set_mx_trace(unsigned long long *p) {
  HIP_TRY(hipMemcpyToSymbol(HIP_SYMBOL(g_mx_trace), &p, sizeof p));
  return BFP_OK;
}

// The trace slice of matvec kernel k in a traced launch.
template <bool TR>
__device__ __forceinline__ unsigned long long *mx_tr(const LayerArgs &, int k) {
  if constexpr (TR) return g_mx_trace + (size_t)k * MX_TRACE_BLOCKS * MX_TRACE_STAMPS;
  return nullptr;
}

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

// Q|K|V: one chunk per block (two chunks per block, half the blocks,
// measured 8.5 against 6.6 us for the 960 x 576 block of 64 sequences).
template <bool TR>
__global__ __launch_bounds__(64 * MX_WAVES_MAX) void k_qkv_mx(LayerArgs a) {
  __shared__ long long Ao[16 * MX_SEQ];
  __shared__ int Mo[16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  const int nT = a.D / 16, c = blockIdx.x, b0 = blockIdx.y * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  mx_block<1>(a.w_qkv_m + (long long)c * nT * 32, a.w_qkv_e + (long long)c * nT * 16, nT,
              a.xn_m + (long long)b0 * a.D, a.xn_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex, mx_tr<TR>(a, MX_K_QKV));
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_qkv(a, b, c, mx_A(Ao, q_), Mo[q_], wr_);
  })
  mx_mark(mx_tr<TR>(a, MX_K_QKV), 5);
}

// The attention's q|k|v input from tagged words that the Q|K|V blocks of the
// same launch store, polled with a bounded wait (tw_give_up); everything
// else as AttnPlainIO.
struct AttnTagIO : AttnPlainIO {
  tw_rsrc rq, rf;   // this sequence's q|k|v words, the abort flag
  unsigned tag;
  __device__ __forceinline__ void qkv(int idx, int &m, int &e) const {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    unsigned v;
    for (unsigned it = 0;; ++it) {
      v = __builtin_amdgcn_raw_buffer_load_b32(rq, 4 * idx, 0, TW_SC1);
      if ((v >> 24) == tag || tw_give_up(rf, it, t0)) break;
      __builtin_amdgcn_s_sleep(2);
    }
    m = (int)(short)(v & 0xffffu);
    e = (int)(signed char)((v >> 16) & 0xffu);
  }
};

// k_qkv_mx's blocks (ids below nblk: chunk id % ((D + 2KV) / 16), sequence
// group id / that) and a short attention form's k_attn (H_Q x batch
// workgroups from nblk: head id % H_Q, sequence id / H_Q) in one launch.
// The blocks also store q|k|v as tagged words, which the attention
// workgroups poll (AttnTagIO).  Workgroups are dispatched in id order and
// the blocks never wait, so every block an attention workgroup waits for
// has been dispatched before it.  blockDim = 64 * ATT_WAVES; the blocks'
// Ao / Mo sit in the dynamic LDS after their exponents, so the attention
// keeps k_attn's LDS and occupancy.
template <int PPW, bool TR>
__global__ __launch_bounds__(64 * ATT_WAVES, (PPW == 3 ? 6 : 4)) void k_qkv_attn_mx(LayerArgs a, int nblk) {
  extern __shared__ double dsm[];
  const int nq = a.D + 2 * a.KV;
  const unsigned tag = tw_tag(cur_pos(a), a.layer, a.NL);
  if ((int)blockIdx.x >= nblk) {
    const int L = blockIdx.x - nblk, hq = L % a.H_Q, b = L / a.H_Q;
    AttnTagIO io{{a.qkv_m + b * nq, a.qkv_e + b * (nq / 16), a.att_m + b * a.D, a.att_e + b * (a.D / 16)},
                 tw_make(a.t_qkv + (long long)b * nq, nq * 4), tw_make(a.t_abort, 4), tag};
    attn_body<PPW, true>(a, io, hq, b, [&] { return make_int2(cur_kv_pos(a), cur_pos(a)); }, dsm);
    return;
  }
  const int nT = a.D / 16, bq = nq / 16, c = blockIdx.x % bq, b0 = blockIdx.x / bq * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  int8_t *mx_ex = reinterpret_cast<int8_t *>(dsm);
  long long *Ao = reinterpret_cast<long long *>(mx_ex + mx_lds_bytes(1, nT));   // 32 nT bytes
  int *Mo = reinterpret_cast<int *>(Ao + 16 * MX_SEQ);
  mx_block<1>(a.w_qkv_m + (long long)c * nT * 32, a.w_qkv_e + (long long)c * nT * 16, nT,
              a.xn_m + (long long)b0 * a.D, a.xn_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex, mx_tr<TR>(a, MX_K_QKV));
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_qkv(a, b, c, mx_A(Ao, q_), Mo[q_], wr_, tag);
  })
  mx_mark(mx_tr<TR>(a, MX_K_QKV), 5);
}

// K 16-byte loads of thread i (of n) over the byte ranges [m, m + mb) and
// one over [e, e + eb), offsets clamped into them (no load in a branch): a
// later launch's weights brought into the memory-side cache, which every
// XCD shares, by workgroups that would otherwise only wait.  Returns a value
// the caller keeps alive to its end.  At config 5 the O, G/U and D launches
// averaged 0.3-0.45 us less each and the decode 0.25% more tokens/s (three
// alternated runs of each form on one box).
template <int K>
__device__ __forceinline__ unsigned mall_touch(const void *m, size_t mb, const void *e, size_t eb, int i, int n) {
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(m), (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t re = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(e), (short)0, 0x7fffffff, 0x00020000);
  unsigned acc = 0;
#pragma unroll
  for (int k = 0; k < K; ++k) {   // K x n x 16 bytes >= mb for the callers' sizes
    size_t off = ((size_t)i + (size_t)k * n) * 16;
    off = off < mb ? off : mb - 16;
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rm, (int)off, 0, 0);
    acc ^= v[0];
  }
  const size_t oe = (size_t)i * 16 < eb ? (size_t)i * 16 : eb - 16;
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(re, (int)oe, 0, 0);
  return acc ^ v[0];
}

// AttnTagIO whose phase stamps, in a traced launch (TR), go to the Q|K|V
// kernel's trace rows at the workgroup's id (past the matvec blocks'):
// 0 entry, 1 wave 0's q|k|v in, 2 RoPE and the staged rows in LDS, 3
// scores, 4 wave 0's softmax, 5 wave 0's AV chains.
template <bool TR>
struct AttnTagIOT : AttnTagIO {
  unsigned long long *tr;
  __device__ __forceinline__ void mark(int k) const {
    if constexpr (TR) mx_mark(tr, k == ATT_MARK_QKV ? 1 : 2 + k);
  }
};

// The same launch with one attention workgroup per (KV group, sequence):
// all the group's query heads (bfp_attn_grp.h), H_KV x batch workgroups
// from nblk (group id % H_KV, sequence id / H_KV).
template <int PPW, bool TR>
__global__ __launch_bounds__(64 * ATT_WAVES, 2) void k_qkv_attng_mx(LayerArgs a, int nblk) {
  extern __shared__ double dsm[];
  const int nq = a.D + 2 * a.KV;
  const unsigned tag = tw_tag(cur_pos(a), a.layer, a.NL);
  if ((int)blockIdx.x >= nblk) {
    const int L = blockIdx.x - nblk, gk = L % a.H_KV, b = L / a.H_KV;
    mx_mark(mx_tr<TR>(a, MX_K_QKV), 0);
    // the O launch's weights, touched while these workgroups wait for their
    // q|k|v words, so the O blocks find them in the memory-side cache
    const unsigned pf = mall_touch<1>(a.w_o_m, (size_t)a.D * a.D * 2, a.w_o_e, (size_t)a.D * a.D / 16,
                                   L * blockDim.x + threadIdx.x, (gridDim.x - nblk) * blockDim.x);
    AttnTagIOT<TR> io{{{a.qkv_m + b * nq, a.qkv_e + b * (nq / 16), a.att_m + b * a.D, a.att_e + b * (a.D / 16)},
                       tw_make(a.t_qkv + (long long)b * nq, nq * 4), tw_make(a.t_abort, 4), tag},
                      mx_tr<TR>(a, MX_K_QKV)};
    attn_group_body<PPW>(a, io, gk, b, [&] { return make_int2(cur_kv_pos(a), cur_pos(a)); }, dsm);
    asm volatile("" ::"v"(pf));
    return;
  }
  const int nT = a.D / 16, bq = nq / 16, c = blockIdx.x % bq, b0 = blockIdx.x / bq * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  int8_t *mx_ex = reinterpret_cast<int8_t *>(dsm);
  long long *Ao = reinterpret_cast<long long *>(mx_ex + mx_lds_bytes(1, nT));   // 32 nT bytes
  int *Mo = reinterpret_cast<int *>(Ao + 16 * MX_SEQ);
  mx_block<1>(a.w_qkv_m + (long long)c * nT * 32, a.w_qkv_e + (long long)c * nT * 16, nT,
              a.xn_m + (long long)b0 * a.D, a.xn_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex, mx_tr<TR>(a, MX_K_QKV));
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_qkv(a, b, c, mx_A(Ao, q_), Mo[q_], wr_, tag);
  })
  mx_mark(mx_tr<TR>(a, MX_K_QKV), 5);
}
// BFP_ATT_GROUP=0 keeps the one-head-per-workgroup form (read per launch).
static int att_group_env() {
  const char *v = getenv("BFP_ATT_GROUP");
  return v ? atoi(v) : 1;
}

typedef void (*qa_fn)(LayerArgs, int);
static qa_fn qkv_attn_kernel(int ppw, bool tr = false) {
  if (tr) return ppw == 2 ? k_qkv_attn_mx<2, true> : (ppw == 3 ? k_qkv_attn_mx<3, true> : k_qkv_attn_mx<4, true>);
  return ppw == 2 ? k_qkv_attn_mx<2, false> : (ppw == 3 ? k_qkv_attn_mx<3, false> : k_qkv_attn_mx<4, false>);
}
static qa_fn qkv_attng_kernel(int ppw, bool tr) {
  if (tr) return ppw == 2 ? k_qkv_attng_mx<2, true> : k_qkv_attng_mx<3, true>;
  return ppw == 2 ? k_qkv_attng_mx<2, false> : k_qkv_attng_mx<3, false>;
}
// Grouped attention in the joined launch: the lane-split short forms, at
// most AG_MAXG heads a group (and BFP_ATT_GROUP set).
static bool mx_attn_grouped(const LayerArgs &a) {
  const int grp = a.H_Q / a.H_KV;
  return att_group_env() && attn_ppw(a.max_ctx) <= 3 && grp <= AG_MAXG && grp + 2 <= ATT_WAVES;
}
inline size_t qkv_attng_lds(const LayerArgs &a) {
  const size_t sha = attn_grp_lds_bytes(a.max_ctx, a.H_Q / a.H_KV);
  const size_t shq = (size_t)mx_lds_bytes(1, a.D / 16) + 16 * MX_SEQ * 12;
  return sha > shq ? sha : shq;
}
inline size_t qkv_attn_lds(const LayerArgs &a) {
  const size_t sha = attn_lds_bytes(a.max_ctx, attn_ppw(a.max_ctx), AttnPlainIO::kAvBlock);
  const size_t shq = (size_t)mx_lds_bytes(1, a.D / 16) + 16 * MX_SEQ * 12;
  return sha > shq ? sha : shq;
}

// O and residual 1: one chunk per block.
template <bool TR>
__global__ __launch_bounds__(64 * MX_WAVES_MAX) void k_o_res_mx(LayerArgs a) {
  __shared__ long long Ao[16 * MX_SEQ];
  __shared__ int Mo[16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  const int nT = a.D / 16, c = blockIdx.x, b0 = blockIdx.y * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  mx_block<1>(a.w_o_m + (long long)c * nT * 32, a.w_o_e + (long long)c * nT * 16, nT,
              a.att_m + (long long)b0 * a.D, a.att_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex, mx_tr<TR>(a, MX_K_O));
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_ores(a, b, c, mx_A(Ao, q_), Mo[q_], wr_, a.h_m[b * a.D + c * 16 + r_],
             a.h_e[b * (a.D / 16) + c]);
  })
  mx_mark(mx_tr<TR>(a, MX_K_O), 5);
}

// An RMSNorm of sequence b (k_norm_pairs' arithmetic and output; which = 1:
// norm 1 with gamma g, 2: norm 2) from tagged words that the blocks of the
// same launch store (words: the sequence's D words): each thread polls whole
// quads until all four carry this (step, layer)'s tag.  The wait is
// bounded (tw_give_up): one that gives up sets *t_abort and goes on (the
// host then reports the decode as failed).
__device__ __forceinline__ void norm_tagged(const LayerArgs &a, int b, int which, const unsigned *words,
                                            const double *g, double *dsm) {
  const int D = a.D;
  int16_t *hm = reinterpret_cast<int16_t *>(dsm + D + PW_MAX_LEAVES);
  int8_t *he = reinterpret_cast<int8_t *>(hm + D);
  const unsigned tag = tw_tag(cur_pos(a), a.layer, a.NL);
  const tw_rsrc r = tw_make(words + (long long)b * D, D * 4), rf = tw_make(a.t_abort, 4);
  const int i0 = 2 * (int)threadIdx.x;
  const double2 gg = *reinterpret_cast<const double2 *>(g + (i0 < D ? i0 : 0));
  for (int q = threadIdx.x; q < D / 4; q += blockDim.x) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    uint4 v;
    for (unsigned it = 0;; ++it) {
      typedef unsigned v4u __attribute__((ext_vector_type(4)));
      const v4u u = __builtin_amdgcn_raw_buffer_load_b128(r, 16 * q, 0, TW_SC1);
      v = make_uint4(u.x, u.y, u.z, u.w);
      if ((v.x >> 24) == tag && (v.y >> 24) == tag && (v.z >> 24) == tag && (v.w >> 24) == tag) break;
      if (tw_give_up(rf, it, t0)) break;
      __builtin_amdgcn_s_sleep(2);
    }
    hm[4 * q] = (int16_t)(v.x & 0xffffu);
    hm[4 * q + 1] = (int16_t)(v.y & 0xffffu);
    hm[4 * q + 2] = (int16_t)(v.z & 0xffffu);
    hm[4 * q + 3] = (int16_t)(v.w & 0xffffu);
    if ((q & 3) == 0) he[q >> 2] = (int8_t)((v.x >> 16) & 0xffu);
  }
  __syncthreads();
  int m0, m1, e;
  rmsnorm_pairs(hm, he, gg.x, gg.y, D, dsm, dsm + D, m0, m1, e);
  norm_pairs_out(a, b, which, m0, m1, e);
}

// k_o_res_mx's blocks (ids below nblk: chunk id % (D/16), sequence group
// id / (D/16)) and RMSNorm 2 (one workgroup per sequence, ids from nblk) in
// one launch.  The blocks also store h1 as tagged words, which the norm
// workgroups poll.  Workgroups are dispatched in id order and the blocks
// never wait, so every block a norm workgroup waits for has been dispatched
// before it.  blockDim >= D / 2.
template <bool TR>
__global__ __launch_bounds__(64 * MX_WAVES_MAX) void k_o_res_norm_mx(LayerArgs a, int nblk) {
  __shared__ long long Ao[16 * MX_SEQ];
  __shared__ int Mo[16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  if ((int)blockIdx.x >= nblk) {
    // the G/U launch's weights, touched while these workgroups wait for h1
    const unsigned pf = mall_touch<8>(a.w_gu_m, (size_t)a.FFN * a.D * 4, a.w_gu_e, (size_t)a.FFN * a.D / 8,
                                      (blockIdx.x - nblk) * blockDim.x + threadIdx.x, (gridDim.x - nblk) * blockDim.x);
    norm_tagged(a, blockIdx.x - nblk, 2, a.t_h1, a.g2, reinterpret_cast<double *>(mx_ex));
    asm volatile("" ::"v"(pf));
    return;
  }
  const int nT = a.D / 16, c = blockIdx.x % nT, b0 = blockIdx.x / nT * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  const unsigned tag = tw_tag(cur_pos(a), a.layer, a.NL);
  mx_block<1>(a.w_o_m + (long long)c * nT * 32, a.w_o_e + (long long)c * nT * 16, nT,
              a.att_m + (long long)b0 * a.D, a.att_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex, mx_tr<TR>(a, MX_K_O));
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_ores(a, b, c, mx_A(Ao, q_), Mo[q_], wr_, a.h_m[b * a.D + c * 16 + r_],
             a.h_e[b * (a.D / 16) + c], tag);
  })
  mx_mark(mx_tr<TR>(a, MX_K_O), 5);
}

// G and U: the G chunk (2x) and U chunk (2x+1) of FFN chunk x per block.
template <bool TR>
__global__ __launch_bounds__(64 * MX_WAVES_MAX) void k_gu_mx(LayerArgs a) {
  __shared__ long long Ao[2 * 16 * MX_SEQ];
  __shared__ int Mo[2 * 16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  const int nT = a.D / 16, c = blockIdx.x, b0 = blockIdx.y * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  mx_block<2>(a.w_gu_m + (long long)(2 * c) * nT * 32, a.w_gu_e + (long long)(2 * c) * nT * 16, nT,
              a.xn_m + (long long)b0 * a.D, a.xn_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex, mx_tr<TR>(a, MX_K_GU));
  BFP_MX_EPI(MX_SEQ, {
    const int qg_ = r_ * MX_SEQ + j_, qu_ = (16 + r_) * MX_SEQ + j_;
    (void)cc_;
    epi_gu(a, b, c, mx_A(Ao, qg_), Mo[qg_], mx_A(Ao, qu_), Mo[qu_], wr_);
  })
  mx_mark(mx_tr<TR>(a, MX_K_GU), 5);
}

// D and residual 2: one chunk per block, up to 12 waves (the FFN-input
// block has 96 tiles: 12 waves measured 9.7 against 10.2 us for 8).
constexpr int MX_WAVES_D = 12;
template <bool TR>
__global__ __launch_bounds__(64 * MX_WAVES_D) void k_d_res_mx(LayerArgs a) {
  __shared__ long long Ao[16 * MX_SEQ];
  __shared__ int Mo[16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  const int nT = a.FFN / 16, c = blockIdx.x, b0 = blockIdx.y * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  mx_block<1>(a.w_d_m + (long long)c * nT * 32, a.w_d_e + (long long)c * nT * 16, nT,
              a.mlp_m + (long long)b0 * a.FFN, a.mlp_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex, mx_tr<TR>(a, MX_K_D));
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_dres(a, b, c, mx_A(Ao, q_), Mo[q_], wr_, a.h1_m[b * a.D + c * 16 + r_],
             a.h1_e[b * (a.D / 16) + c]);
  })
  mx_mark(mx_tr<TR>(a, MX_K_D), 5);
}


// k_d_res_mx's blocks (ids below nblk) and the next layer's RMSNorm 1 (one
// workgroup per sequence, ids from nblk, gamma g1_next) in one launch, as
// k_o_res_norm_mx: the blocks also store h as tagged words.
template <bool TR>
__global__ __launch_bounds__(64 * MX_WAVES_D) void k_d_res_norm_mx(LayerArgs a, int nblk) {
  __shared__ long long Ao[16 * MX_SEQ];
  __shared__ int Mo[16 * MX_SEQ];
  extern __shared__ int8_t mx_ex[];
  if ((int)blockIdx.x >= nblk) {
    // the next layer's Q|K|V weights, touched while these workgroups wait for h
    const size_t nq = (size_t)a.D + 2 * (size_t)a.KV;
    const unsigned pf = mall_touch<4>(a.w_qkv_next_m, nq * a.D * 2, a.w_qkv_next_e, nq * a.D / 16,
                                      (blockIdx.x - nblk) * blockDim.x + threadIdx.x, (gridDim.x - nblk) * blockDim.x);
    norm_tagged(a, blockIdx.x - nblk, 1, a.t_h, a.g1_next, reinterpret_cast<double *>(mx_ex));
    asm volatile("" ::"v"(pf));
    return;
  }
  const int nT = a.FFN / 16, nc = a.D / 16, c = blockIdx.x % nc, b0 = blockIdx.x / nc * MX_SEQ;
  const int ns = min(MX_SEQ, a.batch - b0);
  const unsigned tag = tw_tag(cur_pos(a), a.layer, a.NL);
  mx_block<1>(a.w_d_m + (long long)c * nT * 32, a.w_d_e + (long long)c * nT * 16, nT,
              a.mlp_m + (long long)b0 * a.FFN, a.mlp_e + (long long)b0 * nT, ns, Ao, Mo, mx_ex, mx_tr<TR>(a, MX_K_D));
  BFP_MX_EPI(MX_SEQ, {
    const int q_ = r_ * MX_SEQ + j_;
    (void)cc_;
    epi_dres(a, b, c, mx_A(Ao, q_), Mo[q_], wr_, a.h1_m[b * a.D + c * 16 + r_],
             a.h1_e[b * (a.D / 16) + c], tag);
  })
  mx_mark(mx_tr<TR>(a, MX_K_D), 5);
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
    for (int i = 0; i < MAXD64; ++i) f[i] = ld_nt(e4 + (EXACT || i < d64 ? i : d64 - 1) * 16 + l16);
  };
  load_rows(sub, cur);
  final_norm(a.h_m + b * a.D, a.h_e + b * (a.D / 16), a.norm_w, a.D, dsm, leaf, hn);
  __syncthreads();

  double best = -INFINITY;
  int besti = 0x7fffffff;
  for (int rr = sub; rr < a.rows_per_wg; rr += 16) {
    const int row = r0 + rr;
    load_rows(rr + 16, nxt);
    const double acc = head_row_dot<MAXD64, EXACT>(cur, hn, l16, d64);
#pragma unroll
    for (int i = 0; i < MAXD64; ++i) cur[i] = nxt[i];
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
//
// With the bounded head (a.hq_x set) the workgroup also quantises its
// normed hidden h for k_headq_mx: q = rint(h / 2^eh) with the power of two
// 2^eh that puts max |h| in (16383, 32767], so |h - 2^eh q| <= 2^eh / 2 and
// |q| <= 32767; q goes out as split bytes (q = 256 qh + ql + 128) in
// k_embq_build's layout with sequence b % 16 in place of the row (word
// (((b / 16) * G + g) * 2 + p) * 64 + 16 kg + b % 16), with eh, sum q and
// an upper bound of sum |h| (any summation order is within 575 rounding
// units, so the sum times 1 + 2^-40 bounds it).
__global__ __launch_bounds__(256) void k_head_norm(HeadArgs a) {
  extern __shared__ double dsm[];
  const int b = blockIdx.x, D = a.D, tid = threadIdx.x;
  if (!a.hq_x) {
    final_norm(a.h_m + b * D, a.h_e + b * (D / 16), a.norm_w, D, dsm, dsm + 3 * D,
               a.hn + (long long)b * D);
    return;
  }
  __shared__ double rmax[4], rsum[4];
  __shared__ int rq[4];
  final_norm(a.h_m + b * D, a.h_e + b * (D / 16), a.norm_w, D, dsm, dsm + 3 * D, dsm);
  lds_barrier();
  double mx = 0.0, s1 = 0.0;
  for (int i = tid; i < D; i += 256) {
    const double v = dsm[i];
    a.hn[(long long)b * D + i] = v;
    mx = fmax(mx, fabs(v));
    s1 += fabs(v);
  }
  for (int o = 32; o; o >>= 1) {
    mx = fmax(mx, __shfl_xor(mx, o));
    s1 += __shfl_xor(s1, o);
  }
  if ((tid & 63) == 0) {
    rmax[tid >> 6] = mx;
    rsum[tid >> 6] = s1;
  }
  lds_barrier();
  mx = fmax(fmax(rmax[0], rmax[1]), fmax(rmax[2], rmax[3]));
  int eh = 0;
  if (mx > 0.0) {
    eh = ilogb(mx) - 14;
    if (ldexp(mx, -eh) > 32767.0) ++eh;
  }
  const int G = D / 64;
  int sx = 0;
  for (int sl = tid; sl < D / 16; sl += 256) {   // slot sl: elements 16sl .. +15, group sl / 4
    unsigned hw[4] = {0, 0, 0, 0}, lw[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int v = (int)rint(ldexp(dsm[16 * sl + j], -eh));
      sx += v;
      hw[j >> 2] |= ((unsigned)(v >> 8) & 0xffu) << (8 * (j & 3));
      lw[j >> 2] |= ((unsigned)((v & 255) - 128) & 0xffu) << (8 * (j & 3));
    }
    uint4 *o = a.hq_x + ((long long)(b / 16) * G + (sl >> 2)) * 128 + 16 * (sl & 3) + (b & 15);
    o[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    o[64] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  }
  for (int o = 32; o; o >>= 1) sx += __shfl_xor(sx, o);
  if ((tid & 63) == 0) rq[tid >> 6] = sx;
  lds_barrier();
  if (tid == 0) {
    const double h1 = ((rsum[0] + rsum[1]) + (rsum[2] + rsum[3])) * (1.0 + 0x1p-40);
    a.hq_seq[b] = HeadQSeq{h1, eh, (rq[0] + rq[1]) + (rq[2] + rq[3])};
  }
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
      float4 f = ld_nt(e4 + (EXACT || i < d64 ? i : d64 - 1) * 16 + l16);   // unconditional load
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
// Argmax over the head's per-workgroup maxima of sequence b, the token
// record and the next input (wave 0; returns the next input in every lane).
__device__ __forceinline__ int ctl_body(const CtlArgs &a, int b, int s) {
  const int l = threadIdx.x & 63;
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
  const int next = ctl_next(s, nid, a.n_prompt, a.prompt + b * a.n_prompt, a.rtl_loop);
  if (l == 0) {
    if (a.head) a.last[b] = nid;
    const int k = ctl_out_slot(s, a.n_prompt, a.n_gen, a.rtl_loop);
    if (a.head && k >= 0) a.out[b * ctl_out_len(a.n_prompt, a.n_gen, a.rtl_loop) + k] = nid;
    a.state[1 + b] = next;
  }
  return next;
}

__global__ __launch_bounds__(64) void k_ctl(CtlArgs a) {
  ctl_body(a, blockIdx.x, a.state[0]);
}

__global__ __launch_bounds__(64) void k_step_inc(int *state) {
  if (threadIdx.x == 0 && blockIdx.x == 0) state[0] += 1;
}

// Embedding lookup of the BFP table: embed_q[tid] = fp_quantize_vec(embed[tid])
// (full.py:411-412), quantised on the fly from the float32 table, into h of
// sequence b.
__device__ __forceinline__ void embed_body(const EmbedArgs &a, int b, int tok) {
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

__global__ __launch_bounds__(256) void k_embed(EmbedArgs a) {
  embed_body(a, blockIdx.x, a.state[1 + blockIdx.x]);
}

// The end of a batched decode step in one launch: k_ctl, the step increment
// and the next step's k_embed.  Sequence b's workgroup picks its next input
// and embeds it into h (the head has read h already).  The step counter
// moves once every workgroup has read it: each counts itself in at
// state[1 + batch] (device-scope, after its read), and the last one resets
// that count and advances state[0].
__global__ __launch_bounds__(256) void k_ctl_embed(CtlArgs a, EmbedArgs e) {
  __shared__ int tok_s;
  const int b = blockIdx.x;
  const int s = a.state[0];
  if (threadIdx.x < 64) {
    const int next = ctl_body(a, b, s);
    if (threadIdx.x == 0) tok_s = next;
  }
  __syncthreads();
  embed_body(e, b, tok_s);
  if (threadIdx.x == 0) {
    const int n = __hip_atomic_fetch_add(a.state + 1 + a.batch, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (n == a.batch - 1) {
      a.state[1 + a.batch] = 0;
      a.state[0] = s + 1;
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

// Waves and tiles per lane of a matvec over nT input tiles.
static void shape_for(int nT, int &nw, int &tpt) {
  nw = default_waves(nT);
  tpt = (nT + 4 * nw - 1) / (4 * nw);
}

static lk_fn attn_kernel(int ppw) {
  // max_ctx <= 512 = 64 * ATT_WAVES for ppw 2, 3 and 4: the short forms
  return ppw == 2 ? k_attn<2, true> : (ppw == 3 ? k_attn<3, true> : (ppw == 4 ? k_attn<4, true> : k_attn<8, false>));
}

// Raise a kernel's dynamic-LDS limit on the current device to at least
// `bytes`, never lowering it: the limit is process-wide per device, and
// another context may already launch the same kernel with a larger need.
int raise_lds_limit(const void *f, int bytes) {
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
                          (int)attn_lds_bytes(max_ctx, ppw, AttnPlainIO::kAvBlock)));
  if (ppw <= 4) {
    LayerArgs la{};
    la.max_ctx = max_ctx;
    la.D = D;
    BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(qkv_attn_kernel(ppw)), (int)qkv_attn_lds(la)));
    BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(qkv_attn_kernel(ppw, true)), (int)qkv_attn_lds(la)));
  }
  if (ppw <= 3) {   // the grouped form, for up to AG_MAXG heads a group
    LayerArgs la{};
    la.max_ctx = max_ctx;
    la.D = D;
    la.H_Q = AG_MAXG;
    la.H_KV = 1;
    for (bool tr : {false, true})
      BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(qkv_attng_kernel(ppw, tr)), (int)qkv_attng_lds(la)));
  }
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
                     attn_lds_bytes(a.max_ctx, ppw, AttnPlainIO::kAvBlock), s, a);
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

// Waves per workgroup of k_d_res_mx (up to MX_WAVES_D).
static int mx_waves_d(const LayerArgs &a) {
  const int nTF = a.FFN / 16, n_blocks = a.D / 16 * ((a.batch + MX_SEQ - 1) / MX_SEQ);
  int wd = 2048 / n_blocks;
  wd = wd < (nTF + 1) / 2 ? wd : (nTF + 1) / 2;
  return wd < MX_WAVES_D ? (wd < 1 ? 1 : wd) : MX_WAVES_D;
}

// The batched decode's RMSNorms in the O and D launches: when the tagged
// buffers are given, no stage dump is asked for, and both launches' blocks
// have at least D / 2 threads (rmsnorm_pairs).  The same for every layer
// of a decode, so a layer skips its norm 1 exactly when the layer before
// ran it.
static bool mx_fused_norms(const LayerArgs &a) {
  const int G = (a.batch + MX_SEQ - 1) / MX_SEQ, bo = a.D / 16;
  return a.t_h1 && a.t_h && a.t_abort && !a.dump && 128 * mx_waves(a.D / 16, bo * G) >= a.D &&
         128 * mx_waves_d(a) >= a.D;
}

// Q|K|V and a short attention form in one launch (k_qkv_attn_mx): when the
// tagged q|k|v buffer is given, no stage dump is asked for, and the Q|K|V
// blocks run with the attention's wave count.
static bool mx_joined_qkv_attn(const LayerArgs &a) {
  const int G = (a.batch + MX_SEQ - 1) / MX_SEQ, bq = (a.D + 2 * a.KV) / 16;
  return a.t_qkv && a.t_abort && !a.dump && attn_ppw(a.max_ctx) <= 4 &&
         mx_waves(a.D / 16, bq * G) == ATT_WAVES;
}

int layer_form(const LayerArgs &a) {
  if (!(a.batch >= MULTI_MIN_BATCH && a.xn_m)) return BFP_FORM_SINGLE;
  if (a.batch < MX_MIN_BATCH) return BFP_FORM_MULTI;
  return BFP_FORM_MX | (mx_joined_qkv_attn(a) ? BFP_FORM_QKV_ATTN : 0) |
         (mx_joined_qkv_attn(a) && mx_attn_grouped(a) ? BFP_FORM_ATT_GROUP : 0) |
         (mx_fused_norms(a) ? BFP_FORM_NORM_FUSED : 0);
}

static int launch_layer_mx(const LayerArgs &a, hipStream_t s, bool mx_traced) {
  const int nTD = a.D / 16, nTF = a.FFN / 16;
  const int G = (a.batch + MX_SEQ - 1) / MX_SEQ;
  const int bq = (a.D + 2 * a.KV) / 16, bo = a.D / 16, bg = a.FFN / 16;
  const bool fused = mx_fused_norms(a);
  const bool tr = mx_traced;
  if (!(fused && a.layer > 0)) launch_norm_seq(a, 1, s);   // else the last layer's D launch ran it
  if (mx_joined_qkv_attn(a) && mx_attn_grouped(a)) {
    // Q|K|V + attention by KV group in one launch
    hipLaunchKernelGGL(qkv_attng_kernel(attn_ppw(a.max_ctx), tr), dim3(bq * G + a.H_KV * a.batch),
                       dim3(64 * ATT_WAVES), qkv_attng_lds(a), s, a, bq * G);
  } else if (mx_joined_qkv_attn(a)) {
    // Q|K|V + attention in one launch (batched decode, short forms)
    hipLaunchKernelGGL(qkv_attn_kernel(attn_ppw(a.max_ctx), tr), dim3(bq * G + a.H_Q * a.batch),
                       dim3(64 * ATT_WAVES), qkv_attn_lds(a), s, a, bq * G);
  } else {
    hipLaunchKernelGGL((tr ? k_qkv_mx<true> : k_qkv_mx<false>), dim3(bq, G), dim3(64 * mx_waves(nTD, bq * G)),
                       mx_lds_bytes(1, nTD), s, a);
    BFP_TRY(launch_attn(a, s));
  }
  const int wo = mx_waves(nTD, bo * G);
  if (fused) {
    // O + RMSNorm 2 in one launch (batched decode)
    const size_t shn = (size_t)(a.D + PW_MAX_LEAVES) * 8 + (size_t)a.D * 3;
    const size_t sho = mx_lds_bytes(1, nTD);
    hipLaunchKernelGGL((tr ? k_o_res_norm_mx<true> : k_o_res_norm_mx<false>), dim3(bo * G + a.batch), dim3(64 * wo), sho > shn ? sho : shn, s,
                       a, bo * G);
  } else {
    hipLaunchKernelGGL((tr ? k_o_res_mx<true> : k_o_res_mx<false>), dim3(bo, G), dim3(64 * wo), mx_lds_bytes(1, nTD), s, a);
    launch_norm_seq(a, 2, s);
  }
  hipLaunchKernelGGL((tr ? k_gu_mx<true> : k_gu_mx<false>), dim3(bg, G), dim3(64 * mx_waves(nTD, bg * G)),
                     mx_lds_bytes(2, nTD), s, a);
  const int wd = mx_waves_d(a);
  if (fused && a.g1_next) {
    // D + the next layer's RMSNorm 1 in one launch (batched decode)
    const size_t shn = (size_t)(a.D + PW_MAX_LEAVES) * 8 + (size_t)a.D * 3;
    const size_t shd = mx_lds_bytes(1, nTF);
    hipLaunchKernelGGL((tr ? k_d_res_norm_mx<true> : k_d_res_norm_mx<false>), dim3(bo * G + a.batch), dim3(64 * wd), shd > shn ? shd : shn, s,
                       a, bo * G);
  } else {
    hipLaunchKernelGGL((tr ? k_d_res_mx<true> : k_d_res_mx<false>), dim3(bo, G), dim3(64 * wd), mx_lds_bytes(1, nTF), s, a);
  }
  return launch_status("layer");
}

static int launch_layer_multi(const LayerArgs &a, hipStream_t s, bool mx_traced) {
  if (a.batch >= MX_MIN_BATCH) return launch_layer_mx(a, s, mx_traced);
  const int nTD = a.D / 16, nTF = a.FFN / 16;
  int nw, tpt, nwf, tptf;
  shape_for(nTD, nw, tpt);
  shape_for(nTF, nwf, tptf);
  lkm_fn fq = pick_qkv_m(nw, tpt), fo = pick_ores_m(nw, tpt), fg = pick_gu_m(nw, tpt);
  lkm_fn fd = pick_dres_m(nwf, tptf);
  if (!fq || !fo || !fg || !fd) return set_err(BFP_EINVAL, "no layer kernel for D=%d FFN=%d", a.D, a.FFN);
  const int nq = a.D + 2 * a.KV;
  const int G = (a.batch + MSEQ - 1) / MSEQ;
  const size_t shD = (size_t)MSEQ * nTD * 17 * 4, shF = (size_t)MSEQ * nTF * 17 * 4;
  launch_norm_seq(a, 1, s);
  hipLaunchKernelGGL(fq, dim3(nq / 16, G), dim3(64 * nw), shD, s, a);
  BFP_TRY(launch_attn(a, s));
  hipLaunchKernelGGL(fo, dim3(a.D / 16, G), dim3(64 * nw), shD, s, a);
  launch_norm_seq(a, 2, s);
  hipLaunchKernelGGL(fg, dim3(a.FFN / 16, G), dim3(64 * nw), shD, s, a);
  hipLaunchKernelGGL(fd, dim3(a.D / 16, G), dim3(64 * nwf), shF, s, a);
  return launch_status("layer");
}

int launch_layer(const LayerArgs &a, hipStream_t s, bool mx_traced) {
  if (a.batch >= MULTI_MIN_BATCH && a.xn_m) return launch_layer_multi(a, s, mx_traced);
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
// Batched head on the float64 matrix cores (batch >= HEAD_SEQ_MIN).
// v_mfma_f64_16x16x4f64 computes every output as four FMAs in k order, each
// rounded (checked on the GPU against FMA chains over a million outputs:
// bit-equal, while separate multiply-adds or other orders differ), so
// partial l of a logit -- the FMA chain over k = 64i + 4l + c, i then c
// ascending, of k_head_logits / k_head_gemv -- is one accumulator fed by
// NB MFMAs (one per 64-column block i, c on the instruction's k axis).
// Tiles of 16 rows x 16 sequences: accumulator l holds partial l of all 256
// logits; the 16 partials are then summed in the butterfly order of those
// kernels (q and q + 8, then 4 apart, 2, 1), so the logits are bit-identical
// to theirs.
// Operands: B (lane L: c = L / 16, sequence L % 16) is a group of 16 normed
// hidden vectors, held in registers for the whole kernel; A (lane L: row
// L % 16, c = L / 16) comes from the 16-row tile of the embedding in LDS,
// staged as float32 from a copy permuted at load time (ep, below) into two
// LDS buffers by tile parity.  Output (lane L, element v) is row
// 4v + L / 16, sequence L % 16.
// Workgroup: 8 waves, 32 sequences (blockIdx.y), rows [x * rpw, + rpw) in
// 16-row tiles.  Wave w takes sequence group g = w & 1 (16 sequences) and
// partials h, h + 4, h + 8, h + 12 with h = w >> 1 (NB x 4 doubles of B a
// lane), so the butterfly's first two levels stay in the wave: a_h =
// p_h + p_(h+8), a_(h+4) = p_(h+4) + p_(h+12), b_h = a_h + a_(h+4).  Waves
// h = 1..3 hand b_h over through LDS and wave h = 0 forms (b0 + b2) +
// (b1 + b3) and keeps the per-sequence first-index argmax, which goes to
// part_v / part_i.  The two h = 0 waves (w = 0, 1) run on different SIMDs
// (waves go to the four SIMDs in turn).
// The hand-over is double-buffered by tile parity, so one barrier a tile
// orders both it and the embedding buffers.  A tile's embedding loads are
// issued two tiles ahead (two register sets) and stored to LDS after the
// MFMAs of the tile before it.  ep holds a wave's four partials
// contiguously: ep[row][(4i + c) * 16 + 4h + j] = embed[row][64i + 4(h + 4j) + c].
typedef double head_d4 __attribute__((ext_vector_type(4)));
constexpr int HEAD_ROW_PAD = 4;   // floats: rows 16 B apart in the LDS banks
constexpr int HEAD_XCH = 2 * 3 * 4 * 64;   // doubles of one hand-over buffer
inline int head_mx_lds(int D) { return 2 * 16 * (D + HEAD_ROW_PAD) * 4 + 2 * HEAD_XCH * 8; }

// one tile's staging registers, by name (an array of them, indexed in the
// lambdas, stayed in scratch memory)
struct HeadStage {
  float4 v0, v1, v2, v3, v4;
};

template <int NB>
__global__ __launch_bounds__(512) void k_head_mx(HeadArgs a, int rpw) {
  constexpr int D = 64 * NB, RS = D + HEAD_ROW_PAD, F4 = D / 4;   // float4 per row
  constexpr int TQ = 16 * F4, KQ = (TQ + 511) / 512;               // float4 per tile, per thread
  static_assert(KQ <= 5, "at most 5 staging registers");
  extern __shared__ float esm[];          // 2 x 16 rows x RS floats, then the hand-over
  double *xch = reinterpret_cast<double *>(esm + 2 * 16 * RS);     // [parity][group][h - 1][v][lane]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = w & 1, h = w >> 1;
  const int sl = blockIdx.y * 32 + 16 * g + (lane & 15);
  const bool live = sl < a.batch;
  const int sc = live ? sl : a.batch - 1;
  const int c = lane >> 4;
  double bq[NB][4];
  {
    const double *hp = a.hn + (long long)sc * D + c + 4 * h;   // partial h + 4j
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) bq[i][j] = hp[64 * i + 16 * j];
  }
  const int row_lo = blockIdx.x * rpw;
  const int row_hi = row_lo + rpw < a.VOCAB ? row_lo + rpw : a.VOCAB;
  const int ntile = (row_hi - row_lo) / 16;
  auto load_tile = [&](HeadStage &st, int t) {
    const float4 *src = reinterpret_cast<const float4 *>(a.embedp + (long long)(row_lo + 16 * t) * D);
    auto ld = [&](int k) {
      const int q = k * 512 + tid;
      return ld_nt(src + (q < TQ ? q : TQ - 1));
    };
    st.v0 = ld(0);
    if constexpr (KQ > 1) st.v1 = ld(1);
    if constexpr (KQ > 2) st.v2 = ld(2);
    if constexpr (KQ > 3) st.v3 = ld(3);
    if constexpr (KQ > 4) st.v4 = ld(4);
  };
  auto store_tile = [&](const HeadStage &st, int buf) {
    float *dst = esm + buf * 16 * RS;
    auto stq = [&](int k, float4 v) {
      const int q = k * 512 + tid, r = q / F4, j = q - r * F4;
      if (q < TQ) *reinterpret_cast<float4 *>(dst + r * RS + 4 * j) = v;
    };
    stq(0, st.v0);
    if constexpr (KQ > 1) stq(1, st.v1);
    if constexpr (KQ > 2) stq(2, st.v2);
    if constexpr (KQ > 3) stq(3, st.v3);
    if constexpr (KQ > 4) stq(4, st.v4);
  };
  double bv = -INFINITY;
  int bi = 0x7fffffff;
  HeadStage s0, s1;
  if (ntile > 0) {
    load_tile(s0, 0);
    store_tile(s0, 0);
  }
  if (ntile > 1) load_tile(s1, 1);
  lds_barrier();
  double *xg = xch + g * (3 * 4 * 64) + lane;   // + parity * HEAD_XCH + ((h - 1) * 4 + v) * 64
  // tile t: `nxt` holds tile t + 1 (loaded a tile ago), `fut` takes t + 2
  auto tile = [&](int t, HeadStage &nxt, HeadStage &fut) {
    if (t + 2 < ntile) load_tile(fut, t + 2);
    const float *ar = esm + (t & 1) * 16 * RS + (lane & 15) * RS + 16 * c + 4 * h;
    head_d4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = head_d4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const float4 f = *reinterpret_cast<const float4 *>(ar + 64 * i);
      acc[0] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)f.x, bq[i][0], acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)f.y, bq[i][1], acc[1], 0, 0, 0);
      acc[2] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)f.z, bq[i][2], acc[2], 0, 0, 0);
      acc[3] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)f.w, bq[i][3], acc[3], 0, 0, 0);
    }
    double b4[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) b4[v] = (acc[0][v] + acc[2][v]) + (acc[1][v] + acc[3][v]);
    double *xb = xg + (t & 1) * HEAD_XCH;
    if (h) {
#pragma unroll
      for (int v = 0; v < 4; ++v) xb[((h - 1) * 4 + v) * 64] = b4[v];
    }
    if (t + 1 < ntile) store_tile(nxt, (t + 1) & 1);
    // Orders this tile's hand-over before wave h = 0 reads it, the store of
    // tile t + 1 before its MFMAs, and every read of buffer t & 1 (embedding
    // and hand-over) before tile t + 2 writes it.
    lds_barrier();
    if (!h) {
      const int rbase = row_lo + 16 * t + (lane >> 4);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const double x = (b4[v] + xb[(4 + v) * 64]) + (xb[v * 64] + xb[(8 + v) * 64]);
        const int row = rbase + 4 * v;
        if (a.logits && live) a.logits[(long long)sl * a.VOCAB + row] = x;
        if (x > bv || (x == bv && row < bi)) {
          bv = x;
          bi = row;
        }
      }
    }
  };
  for (int t = 0; t < ntile; t += 2) {
    tile(t, s1, s0);
    if (t + 1 < ntile) tile(t + 1, s0, s1);
  }
  if (!h) {
    argmax_step<16>(bv, bi);   // the four lanes of a sequence (lane / 16)
    argmax_step<32>(bv, bi);
    if (lane < 16 && live) {
      a.part_v[(long long)sl * a.n_wg + blockIdx.x] = bv;
      a.part_i[(long long)sl * a.n_wg + blockIdx.x] = bi;
    }
  }
}

// ------------------------------------------------------------ bounded head
// The batched head's argmax without every float64 logit.  L(s, r), the
// logit k_head_mx forms (FMA chains and butterfly of k_head_logits), is
// bracketed for every (sequence, row) by an exact integer dot product of
// the two operands quantised to int16: with h = 2^eh qh + dh, |dh| <= 2^eh/2
// (k_head_norm) and e_r = 2^er qe + de, |de| <= 2^er/2 (k_embq_build),
//   |h.e_r - 2^(eh+er) qh.qe| <= 2^er/2 |h|_1 + 2^(eh+er)/2 |qe|_1,
// and |L - h.e_r| <= 40 rounding units of sum |h_k e_k| <= |h|_1 max|e_r|
// (a chain of 36 FMAs and 4 adds per term; 2^-45 is taken).  qh.qe is exact
// (|qh.qe| < 2^40) and 2^(eh+er) qh.qe is exact in float64, so with B the
// bound (rounded outward) every logit lies in [A - B, A + B].  B is formed
// as |h|_1 r1 + 2^eh r2 with the row's r1 = 2^(er-1) + 2^-45 max|e_r| and
// r2 = 2^(er-1) |qe|_1, then enlarged by 2^-20 of itself (far more than its
// few roundings) and 2^-50 |A| (the roundings of A - B and A + B).  The row with
// the largest L (first index on ties) has A + B >= L >= every other row's
// A - B, so it lies in a 16-row block whose largest upper bound reaches the
// largest lower bound T of all rows: k_headq_pick forms the exact logits of
// those blocks only (usually one) and takes their argmax, which is the
// argmax of all of them.

// The embedding as the bounded head reads it: row r as int16 q with its own
// scale 2^er (max |e_r| / 2^er in (16383, 32767]), split bytes (q = 256 qh +
// ql + 128, qh = q >> 8, ql = (q & 255) - 128) in the operand layout of
// v_mfma_i32_16x16x64_i8 (lane L: row L % 16, columns 16 (L / 16) .. +15 of
// a 64-column group, byte j = column 16 (L / 16) + j; checked on the GPU):
// 16-byte word ((((r / 16) * G + g) * 2 + p) * 64 + 16 kg + r % 16 holds the
// high (p = 0) or low (p = 1) bytes of elements 64g + 16kg .. +15, so each
// plane of a group is 1 KB read by one wave-wide load.  meta[r]: the row's
// record (HeadQRow).  One workgroup per 16 rows.
__global__ __launch_bounds__(256) void k_embq_build(const float *__restrict__ E, int D,
                                                    uint4 *__restrict__ q, HeadQRow *__restrict__ meta) {
  const int chunk = blockIdx.x, tid = threadIdx.x, i = tid >> 4, l16 = tid & 15;
  const long long r = (long long)chunk * 16 + i;
  const int G = D / 64;
  const float *row = E + r * D;
  float mx = 0.f;
  for (int k = l16; k < D; k += 16) mx = fmaxf(mx, fabsf(row[k]));
  for (int o = 8; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
  int er = 0;
  if (mx > 0.f) {
    er = ilogb((double)mx) - 14;
    if (ldexp((double)mx, -er) > 32767.0) ++er;
  }
  int sw = 0, s1 = 0;
  for (int sl = l16; sl < D / 16; sl += 16) {   // 16-element slot sl: group sl / 4, kg sl % 4
    unsigned hw[4] = {0, 0, 0, 0}, lw[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int v = (int)rint(ldexp((double)row[16 * sl + j], -er));
      sw += v;
      s1 += v < 0 ? -v : v;
      hw[j >> 2] |= ((unsigned)(v >> 8) & 0xffu) << (8 * (j & 3));
      lw[j >> 2] |= ((unsigned)((v & 255) - 128) & 0xffu) << (8 * (j & 3));
    }
    uint4 *o = q + ((long long)chunk * G + (sl >> 2)) * 128 + 16 * (sl & 3) + i;
    o[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    o[64] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  }
  for (int o = 8; o; o >>= 1) {
    sw += __shfl_xor(sw, o, 16);
    s1 += __shfl_xor(s1, o, 16);
  }
  if (l16 == 0) {
    const bool z = mx == 0.f;
    meta[r] = HeadQRow{er, sw, z ? 0.0 : ldexp(1.0, er - 1) + 0x1p-45 * (double)mx,
                       z ? 0.0 : ldexp((double)s1, er - 1)};
  }
}

// Lower and upper bounds of the logits, per (sequence, 16-row block): each
// wave one block of rows against the workgroup's (up to) 64 sequences, in
// groups of 16 (the matrix-core tile).  With W = 256 Wh + Wl + 128 and
// x = 256 xh + xl + 128 over the D products,
//   sum W x = 65536 P(Wh, xh) + 256 (P(Wh, xl) + P(Wl, xh)) + P(Wl, xl)
//             + 128 (sum W + sum x) - 16384 D,
// each P one v_mfma_i32_16x16x64_i8 per 64 columns (|P| < 2^24 in int32).
// Lane L owns rows 4 (L / 16) + v of the block and sequence L % 16 of the
// group; the block's maxima over its rows go to hq_blk[s][block].
typedef int headq_v4 __attribute__((ext_vector_type(4)));
constexpr int HEADQ_PD = 4;   // weight groups in flight ahead of the one in use
template <int G>
__global__ __launch_bounds__(512, 4) void k_headq_mx(HeadArgs a) {
  extern __shared__ uint4 xq[];   // [4 groups][G][2 planes][64 lanes]
  __shared__ HeadQSeq sq[HEADQ_SEQ];
  __shared__ HeadQRow rq[8 * 16];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, kg = lane >> 4, i = lane & 15;
  const int b0 = blockIdx.y * HEADQ_SEQ;
  const int nq = min(4, (a.batch - b0 + 15) / 16);
  const int nch = a.VOCAB / 16;
  const int c = min(blockIdx.x * 8 + w, nch - 1);   // past the end: block nch-1 again, not stored
  // the first weight groups of this wave's block, then the stage: the
  // quantised hidden of the workgroup's sequences (groups past the batch are
  // left unwritten and their products unused) and the records
  const uint4 *pw = a.embq + (long long)c * G * 128 + lane;
  uint4 Wr[HEADQ_PD][2];
#pragma unroll
  for (int p = 0; p < HEADQ_PD; ++p) {
    Wr[p][0] = ld_nt(pw + 128 * (p < G ? p : G - 1));
    Wr[p][1] = ld_nt(pw + 128 * (p < G ? p : G - 1) + 64);
  }
  {
    // every staging load of a thread before its stores (one after another,
    // load then store, the stage took 6 us)
    constexpr int SPT = (4 * G * 128 + 511) / 512;
    const int lim = nq * G * 128;
    const uint4 *src = a.hq_x + (long long)(b0 / 16) * G * 128;
    uint4 st[SPT];
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const int k = tid + 512 * j;
      st[j] = src[k < lim ? k : lim - 1];
    }
    const int r = blockIdx.x * 128 + (tid & 127);   // the rows' records (the last block again past the end)
    const HeadQRow rr = a.embq_meta[r < a.VOCAB ? r : a.VOCAB - 16 + (r & 15)];
    const int bs = b0 + (tid & (HEADQ_SEQ - 1));
    const HeadQSeq ss = a.hq_seq[bs < a.batch ? bs : a.batch - 1];
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const int k = tid + 512 * j;
      if (k < lim) xq[k] = st[j];
    }
    if (tid < 8 * 16) rq[tid] = rr;
    if (tid < HEADQ_SEQ) sq[tid] = ss;
  }
  __syncthreads();
  // the four sequence groups' products side by side: 16 independent
  // accumulators, one group of 64 columns at a time
  headq_v4 acc[4][4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[q][k] = headq_v4{0, 0, 0, 0};
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4 wh4 = Wr[g % HEADQ_PD][0], wl4 = Wr[g % HEADQ_PD][1];
    if (g + HEADQ_PD < G) {
      Wr[g % HEADQ_PD][0] = ld_nt(pw + 128 * (g + HEADQ_PD));
      Wr[g % HEADQ_PD][1] = ld_nt(pw + 128 * (g + HEADQ_PD) + 64);
    }
    const headq_v4 wh = {(int)wh4.x, (int)wh4.y, (int)wh4.z, (int)wh4.w};
    const headq_v4 wl = {(int)wl4.x, (int)wl4.y, (int)wl4.z, (int)wl4.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 xh4 = xq[(q * G + g) * 128 + lane], xl4 = xq[(q * G + g) * 128 + 64 + lane];
      const headq_v4 xh = {(int)xh4.x, (int)xh4.y, (int)xh4.z, (int)xh4.w};
      const headq_v4 xl = {(int)xl4.x, (int)xl4.y, (int)xl4.z, (int)xl4.w};
      acc[q][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh, xh, acc[q][0], 0, 0, 0);
      acc[q][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh, xl, acc[q][1], 0, 0, 0);
      acc[q][2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl, xh, acc[q][2], 0, 0, 0);
      acc[q][3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl, xl, acc[q][3], 0, 0, 0);
    }
  }
  const bool store = blockIdx.x * 8 + w < nch;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int s = b0 + 16 * q + i;
    const HeadQSeq Q = sq[(16 * q + i) < HEADQ_SEQ ? 16 * q + i : 0];
    const long long sx = 128LL * Q.sumx - 16384LL * a.D;
    double mlo = -INFINITY, mhi = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const HeadQRow &Mv = rq[16 * w + 4 * kg + v];
      // a zero row (r1 = r2 = 0): S = 0, so lo = hi = +0, its exact logit
      const long long S = ((long long)acc[q][0][v] << 16) + ((long long)(acc[q][1][v] + acc[q][2][v]) << 8) +
                          acc[q][3][v] + 128LL * Mv.sumw + sx;
      const double A = ldexp((double)S, Mv.er + Q.eh);
      double B = fma(Q.h1, Mv.r1, ldexp(Mv.r2, Q.eh));
      B = fma(B, 0x1p-20, B) + 0x1p-50 * fabs(A);
      double lo = A - B, hi = A + B;
      if (Mv.er + Q.eh < -1000) {   // near the underflow range: always a candidate
        lo = -INFINITY;
        hi = INFINITY;
      }
      mlo = fmax(mlo, lo);
      mhi = fmax(mhi, hi);
    }
    mlo = fmax(mlo, __shfl_xor(mlo, 16));
    mhi = fmax(mhi, __shfl_xor(mhi, 16));
    mlo = fmax(mlo, __shfl_xor(mlo, 32));
    mhi = fmax(mhi, __shfl_xor(mhi, 32));
    if (q < nq && store && kg == 0 && s < a.batch) a.hq_blk[(long long)s * nch + c] = make_double2(mlo, mhi);
  }
}

// Sequence b's argmax from the bounds: T = the largest lower bound; the
// blocks whose upper bound reaches T get their 16 exact logits
// (k_head_logits' FMA chains and butterfly: the values k_head_mx forms) and
// the argmax over them, first index on ties (a rule that does not depend on
// the order the blocks are taken in), is the head's (part_v / part_i [b],
// one entry a sequence).  All of a thread's bound loads are issued at once;
// the candidate blocks go to an LDS list, two at a time through the
// workgroup (16 lanes a row).
constexpr int HEADQ_PICK_T = 512;
constexpr int HEADQ_PICK_PER = 8;   // blocks a thread kept in registers (VOCAB / 16 <= 4096)
template <int MAXD64, bool EXACT>
__global__ __launch_bounds__(HEADQ_PICK_T) void k_headq_pick(HeadArgs a) {
  extern __shared__ double hs[];   // D, then the candidate list (VOCAB / 16 ints)
  __shared__ double rv[HEADQ_PICK_T / 64];
  __shared__ int ri[HEADQ_PICK_T / 64];
  __shared__ int ncand;
  const int b = blockIdx.x, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int nch = a.VOCAB / 16, d64 = a.D / 64, l16 = tid & 15;
  int *cand = reinterpret_cast<int *>(hs + a.D);
  if (tid == 0) ncand = 0;
  // the normed hidden (D <= 2 * HEADQ_PICK_T) with the bounds' loads below,
  // stored once they are all issued
  const double *hb = a.hn + (long long)b * a.D;
  const double h0 = hb[tid < a.D ? tid : 0], h1v = hb[tid + HEADQ_PICK_T < a.D ? tid + HEADQ_PICK_T : 0];
  const double2 *blk = a.hq_blk + (long long)b * nch;
  // the first HEADQ_PICK_PER blocks of the thread stay in registers (all of
  // them up to 4096 blocks); any further ones are read again below
  double t = -INFINITY, hv[HEADQ_PICK_PER];
  {
    double2 v[HEADQ_PICK_PER];
#pragma unroll
    for (int k = 0; k < HEADQ_PICK_PER; ++k) {
      const int c = tid + HEADQ_PICK_T * k;
      v[k] = blk[c < nch ? c : nch - 1];
    }
#pragma unroll
    for (int k = 0; k < HEADQ_PICK_PER; ++k) {
      t = fmax(t, v[k].x);   // clamped entries repeat one
      hv[k] = v[k].y;
    }
  }
  if (tid < a.D) hs[tid] = h0;
  if (tid + HEADQ_PICK_T < a.D) hs[tid + HEADQ_PICK_T] = h1v;
  for (int c = tid + HEADQ_PICK_T * HEADQ_PICK_PER; c < nch; c += HEADQ_PICK_T) t = fmax(t, blk[c].x);
  for (int o = 32; o; o >>= 1) t = fmax(t, __shfl_xor(t, o));
  if (l == 0) rv[w] = t;
  __syncthreads();
  double T = rv[0];
#pragma unroll
  for (int k = 1; k < HEADQ_PICK_T / 64; ++k) T = fmax(T, rv[k]);
#pragma unroll
  for (int k = 0; k < HEADQ_PICK_PER; ++k) {
    const int c = tid + HEADQ_PICK_T * k;
    if (c < nch && hv[k] >= T) cand[atomicAdd(&ncand, 1)] = c;
  }
  for (int c = tid + HEADQ_PICK_T * HEADQ_PICK_PER; c < nch; c += HEADQ_PICK_T)
    if (blk[c].y >= T) cand[atomicAdd(&ncand, 1)] = c;
  __syncthreads();
  const int n = ncand;
  double best = -INFINITY;
  int besti = 0x7fffffff;
  for (int k0 = 0; k0 < n; k0 += HEADQ_PICK_T / 256) {   // uniform
    const int k = k0 + (tid >> 8);
    const int row = cand[k < n ? k : n - 1] * 16 + ((tid >> 4) & 15);
    const float4 *e4 = reinterpret_cast<const float4 *>(a.embed + (long long)row * a.D);
    float4 f[MAXD64];
#pragma unroll
    for (int j = 0; j < MAXD64; ++j) f[j] = e4[(EXACT || j < d64 ? j : d64 - 1) * 16 + l16];
    const double x = head_row_dot<MAXD64, EXACT>(f, hs, l16, d64);
    if (k < n && (x > best || (x == best && row < besti))) {
      best = x;
      besti = row;
    }
  }
  argmax_step<1>(best, besti);
  argmax_step<2>(best, besti);
  argmax_step<4>(best, besti);
  argmax_step<8>(best, besti);
  argmax_step<16>(best, besti);
  argmax_step<32>(best, besti);
  if (l == 0) {
    rv[w] = best;
    ri[w] = besti;
  }
  __syncthreads();
  if (tid == 0) {
    for (int k = 1; k < HEADQ_PICK_T / 64; ++k)
      if (rv[k] > best || (rv[k] == best && ri[k] < besti)) {
        best = rv[k];
        besti = ri[k];
      }
    a.part_v[b] = best;
    a.part_i[b] = besti;
  }
}
inline size_t headq_pick_lds(int D, int VOCAB) { return (size_t)D * 8 + (size_t)(VOCAB / 16) * 4; }

typedef void (*headq_mx_fn)(HeadArgs);
static headq_mx_fn headq_mx_kernel(int G) {
  switch (G) {
    case 1: return k_headq_mx<1>;
    case 2: return k_headq_mx<2>;
    case 3: return k_headq_mx<3>;
    case 4: return k_headq_mx<4>;
    case 5: return k_headq_mx<5>;
    case 6: return k_headq_mx<6>;
    case 7: return k_headq_mx<7>;
    case 8: return k_headq_mx<8>;
    default: return k_headq_mx<9>;
  }
}
inline int headq_mx_lds(int D) { return 4 * (D / 64) * 64 * 32; }

int launch_embq_build(const float *embed, int VOCAB, int D, uint4 *q, HeadQRow *meta, hipStream_t s) {
  hipLaunchKernelGGL(k_embq_build, dim3(VOCAB / 16), dim3(256), 0, s, embed, D, q, meta);
  return launch_status("embedding quantisation");
}

typedef void (*head_mx_fn)(HeadArgs, int);
static head_mx_fn head_mx_kernel(int nb) {
  switch (nb) {
    case 1: return k_head_mx<1>;
    case 2: return k_head_mx<2>;
    case 3: return k_head_mx<3>;
    case 4: return k_head_mx<4>;
    case 5: return k_head_mx<5>;
    case 6: return k_head_mx<6>;
    case 7: return k_head_mx<7>;
    case 8: return k_head_mx<8>;
    default: return k_head_mx<9>;
  }
}

int head_workgroups(int vocab, int D, int rows_single, int batch, bool have64) {
  if (batch == 1) return vocab / rows_single;
  if (head_seq_form(D, batch, have64)) {
    const int r = head_seq_rows(vocab);
    return (vocab + r - 1) / r;
  }
  const int rm = head_rows_multi(D);
  return (vocab + rm - 1) / rm;
}

int prepare_head_kernels(int D) {
  const int sh = head_seq_group(D) * D * 8;
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(k_head_gemv<9, 2, true>), sh));
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(k_head_gemv<9, 2, false>), sh));
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(k_head_gemv<27, 1, false>), sh));
  if (D % 64 == 0 && D <= 576) {
    BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(head_mx_kernel(D / 64)), head_mx_lds(D)));
    BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(headq_mx_kernel(D / 64)), headq_mx_lds(D)));
  }
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
  const bool seqf = head_seq_form(a.D, a.batch, a.embedp != nullptr);
  if (a.hq_blk) {
    // the bounded head: one (value, index) a sequence
    if (!seqf || a.logits || !a.embq || !a.embq_meta || !a.hq_x || !a.hq_seq || a.n_wg != 1)
      return set_err(BFP_EINVAL, "head: bounded form without its buffers");
    hipLaunchKernelGGL(k_head_norm, dim3(a.batch), dim3(256), sh, s, a);
    hipLaunchKernelGGL(headq_mx_kernel(a.D / 64), dim3((a.VOCAB / 16 + 7) / 8, (a.batch + HEADQ_SEQ - 1) / HEADQ_SEQ),
                       dim3(512), headq_mx_lds(a.D), s, a);
    const size_t shp = headq_pick_lds(a.D, a.VOCAB);
    if (shp > 64 * 1024) return set_err(BFP_EINVAL, "head: vocabulary %d too large for the bounded form", a.VOCAB);
    if (a.D == 576)
      hipLaunchKernelGGL((k_headq_pick<9, true>), dim3(a.batch), dim3(HEADQ_PICK_T), shp, s, a);
    else
      hipLaunchKernelGGL((k_headq_pick<9, false>), dim3(a.batch), dim3(HEADQ_PICK_T), shp, s, a);
    return launch_status("bounded head");
  }
  if (a.n_wg != head_workgroups(a.VOCAB, a.D, a.rows_per_wg, a.batch, a.embedp != nullptr))
    return set_err(BFP_EINVAL, "head: %d workgroups for batch %d", a.n_wg, a.batch);
  hipLaunchKernelGGL(k_head_norm, dim3(a.batch), dim3(256), sh, s, a);
  if (seqf) {
    hipLaunchKernelGGL(head_mx_kernel(a.D / 64), dim3(a.n_wg, (a.batch + 31) / 32), dim3(512),
                       head_mx_lds(a.D), s, a, head_seq_rows(a.VOCAB));
    return launch_status("head");
  }
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

int launch_ctl_embed(const CtlArgs &a, const EmbedArgs &e, hipStream_t s) {
  if (e.batch != a.batch || e.state != a.state)
    return set_err(BFP_EINVAL, "ctl_embed: batch %d / %d or state differ", a.batch, e.batch);
  hipLaunchKernelGGL(k_ctl_embed, dim3(a.batch), dim3(256), 0, s, a, e);
  return launch_status("ctl_embed");
}

}  // namespace bfp
