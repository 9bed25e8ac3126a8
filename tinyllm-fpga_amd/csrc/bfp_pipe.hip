// Pipelined batched decode step: every layer of one decode step for a batch
// of sequences (rtl/vc707/host/gen_smollm_blockfp_full.py:261-293, the
// layer loop of :432-443) as ONE launch of one workgroup per compute unit.
//
// Why: the per-stage launches of a batch-64 step (five a layer) each start
// cold -- their exponents and weights are fetched after the kernel boundary
// -- and each waits for its slowest block before the next stage can begin.
// Here the sequences pass the stages in groups of 16 (the matrix-core
// block), so one group's attention runs while the next group's Q|K|V and
// the previous group's G/U run, and every matvec workgroup keeps its weight
// chunk in registers for all groups of a layer, prefetching the next
// layer's chunk as soon as its last group is done.
//
//   role (fixed)   workgroups         per layer
//   Q|K|V chunk c  nq16               the chunk for each group
//   O chunk c      nd16               the chunk + residual -> h1
//   G/U chunk c    nf16               G and U chunks + SwiGLU -> mlp
//   D chunk c      nd16               the chunk + residual -> h
//   (any)                             RMSNorm 1 / 2 of one sequence, and the
//                                     attention of one (KV group, sequence):
//                                     all the group's query heads
//                                     (bfp_attn_grp.h), spread over the
//                                     workgroups by the host's schedule
//                                     (pipe_plan)
//
// Group g runs stage s of layer L at beat 7L + s + g.  Every dependency of a
// job lies on an earlier beat and each workgroup runs its jobs in beat
// order, so the earliest unfinished job can always proceed: no cycle of
// waits can form (all workgroups are resident at once: the grid is the
// compute-unit count and one workgroup of each fits a unit).
//
// Hand-off: every activation element travels as one 32-bit word m (16) | e
// (8) | tag (8), stored and loaded at the device-coherent level (SC1: the
// eight XCDs' L2 caches are not coherent with one another), the tag being
// (step * NL + layer) % 255 + 1; a consumer polls the words it needs until
// each carries the tag it wants, so a word validates itself (no flag and no
// wait for stores to complete).  The words are cleared before each decode
// and every word is rewritten every layer; every reader of a buffer lies
// upstream, in its group's stage chain, of the buffer's next writer, so no
// read can see a later write.  The KV cache row of this step is stored with
// ordinary stores: within the step no job reads it (each attention takes
// row pos from its q|k|v input), and the next step is another launch.
//
// Every wait is bounded (2 s of the 100 MHz clock); one that gives up sets
// the abort flag, which every later wait sees, so all waves reach the end
// of the kernel and the host reports the decode as failed.  The arithmetic
// is the batched launches' own (bfp_mx.h tile sums, bfp_layer_dev.h norms,
// epilogues and attention), so the outputs are bit-identical to them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <set>
#include <type_traits>
#include <vector>

#include "bfp.h"
#include "bfp_attn_grp.h"
#include "bfp_coh.h"
#include "bfp_device.h"
#include "bfp_f64.h"
#include "bfp_internal.h"
#include "bfp_layer.h"
#include "bfp_layer_dev.h"
#include "bfp_mv.h"
#include "bfp_mx.h"
#include "bfp_pipe.h"

namespace bfp {

constexpr int PP_NW = PIPE_THREADS / 64;
constexpr int PP_TPW_D = 5;    // input tiles per wave of a D-input chunk (D <= 640)
constexpr int PP_TPW_F = 12;   // of an FFN-input chunk (FFN <= 1536)

// ------------------------------------------------------------ hand-off
// The tagged words q = tid + k * PIPE_THREADS < nq (16-byte quads of r),
// NQ per thread: every thread's loads are issued together; then, in rounds,
// every quad that does not carry the tag yet is loaded again, all of them
// at once (one round trip a round, not one per quad: a job that starts
// before its inputs are complete would otherwise wait for its NQ quads one
// after another), the rounds bounded like Wait's; put(q, v) receives each
// quad.  (Ordinary first loads, re-polling only the words without the tag
// at the device-coherent level, left a stale copy cached that the re-polls
// kept returning: the waits gave up.)
template <int NQ, int POL = CPOL_SC1, class Put>
__device__ __forceinline__ void pp_poll_quads(Wait &w, rsrc_t r, int nq, unsigned tag, Put put) {
  static_assert(NQ <= 32, "pending-quad mask");
  uint4 v[NQ];
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int q = threadIdx.x + k * PIPE_THREADS;
    v[k] = ld_b128<POL>(r, 16 * (q < nq ? q : nq - 1));
  }
  unsigned pend = 0;
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int q = threadIdx.x + k * PIPE_THREADS;
    if (q < nq && !Wait::ok4(v[k], tag)) pend |= 1u << k;
  }
  if (pend != 0u && !w.aborted) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    for (unsigned it = 1;; ++it) {
      __builtin_amdgcn_s_sleep(2);
#pragma unroll
      for (int k = 0; k < NQ; ++k)
        if ((pend >> k) & 1u) v[k] = ld_b128<POL>(r, 16 * (threadIdx.x + k * PIPE_THREADS));
#pragma unroll
      for (int k = 0; k < NQ; ++k)
        if (((pend >> k) & 1u) && Wait::ok4(v[k], tag)) pend &= ~(1u << k);
      if (pend == 0u || w.give_up(it, t0)) break;
    }
  }
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int q = threadIdx.x + k * PIPE_THREADS;
    if (q < nq) put(q, v[k]);
  }
}

// Trace stamp k of the current job (thread 0; a buffer store, so it does
// not hold up LDS waits as a generic store would).
__device__ __forceinline__ void pp_stamp(unsigned long long *tr, int k, unsigned long long v) {
  if (tr && threadIdx.x == 0) {
    typedef unsigned v2u __attribute__((ext_vector_type(2)));
    v2u x;
    x.x = (unsigned)v;
    x.y = (unsigned)(v >> 32);
    __builtin_amdgcn_raw_buffer_store_b64(x, rsrc(tr + k, 8), 0, 0, 0);
  }
}
__device__ __forceinline__ void pp_clock(unsigned long long *tr, int k) {
  if (tr) pp_stamp(tr, k, __builtin_amdgcn_s_memrealtime());
}

// ------------------------------------------------------------- weights
// A matvec role's weights of one layer, this lane's share: for tile t0 + k
// of its wave (tiles t0 .. t0 + tpw - 1, tpw = ceil(nT / 8)) and chunk c,
// the 16 bytes of row lane % 16, half (lane / 16) & 1 -- after the first
// group's job of the layer, split in place into its high bytes (x, y) and
// offset low bytes (z, w) -- and the exponents of rows 4 (lane / 16) .. +3.
template <int NC, int TPW>
struct PipeW {
  uint4 m[TPW][NC];
  int e[TPW][NC];
};

// The loads of a layer's weights (pm / pe: the block's first chunk, device
// layout), every one unconditional: tiles past the wave's range read a
// valid tile that is never used.
template <int NC, int TPW>
__device__ __forceinline__ void pw_load(PipeW<NC, TPW> &W, const void *pm, const void *pe, int nT) {
  const rsrc_t rm = rsrc(pm, NC * nT * 512), re = rsrc(pe, NC * nT * 16);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i = lane & 15, kg = lane >> 4, h = kg & 1;
  const int tpw = (nT + PP_NW - 1) / PP_NW, t0 = w * tpw;
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    int t = t0 + k;
    t = t < nT ? t : nT - 1;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      W.m[k][c] = ld_b128<0>(rm, ((c * nT + t) * 32 + h * 16 + i) * 16);
      W.e[k][c] = (int)__builtin_amdgcn_raw_buffer_load_b32(re, (c * nT + t) * 16 + 4 * kg, 0, 0);
    }
  }
}

template <int NC, int TPW>
__device__ __forceinline__ void pw_split(PipeW<NC, TPW> &W) {
#pragma unroll
  for (int k = 0; k < TPW; ++k)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      long hi, lo;
      mx_split(W.m[k][c], hi, lo);
      W.m[k][c] = make_uint4((unsigned)hi, (unsigned)((unsigned long)hi >> 32), (unsigned)lo,
                             (unsigned)((unsigned long)lo >> 32));
    }
}

// LDS of a matvec job: the group's inputs [t][s][16] (int16), their tile
// exponents [t][s], and the (A, M) of every (row, sequence).
struct MvLds {
  int16_t *xs;
  int8_t *xex;
  long long *Ao;
  int *Mo;
};
__device__ __forceinline__ MvLds mv_lds(double *dsm, int nT, int NC) {
  MvLds m;
  m.xs = lds(reinterpret_cast<int16_t *>(dsm));
  m.xex = lds(reinterpret_cast<int8_t *>(m.xs + 16 * nT * 16));
  m.Ao = lds(reinterpret_cast<long long *>(dsm + (16 * nT * 32 + 16 * nT + 7) / 8));
  m.Mo = lds(reinterpret_cast<int *>(m.Ao + NC * 256));
  return m;
}

// The group's inputs into LDS from tagged words: ns sequences of n_in words
// from wbase (the group's first sequence), NQ quads per thread, and the
// block's (A, M) cleared.  Sequences past ns are not staged: the passes
// read sequence min(s, ns - 1) for them.
template <int NQ, int NC>
__device__ __forceinline__ void pp_stage_x(Wait &w, const unsigned *wbase, int n_in, int ns, unsigned tag,
                                           const MvLds &S) {
  const int q4 = n_in / 4;   // quads a sequence
  pp_poll_quads<NQ>(w, rsrc(wbase), ns * q4, tag, [&](int q, const uint4 &v) {
    const int s = q / q4, k = 4 * (q - s * q4);   // sequence, first element
    const int t = k >> 4, j = k & 15;
    typedef unsigned v2u __attribute__((ext_vector_type(2)));
    v2u m;
    m.x = (v.x & 0xffffu) | (v.y << 16);
    m.y = (v.z & 0xffffu) | (v.w << 16);
    *reinterpret_cast<v2u *>(S.xs + (t * 16 + s) * 16 + j) = m;
    if (j == 0) S.xex[t * 16 + s] = (int8_t)tw_e(v.x);
  });
  for (int q = threadIdx.x; q < NC * 16 * 16; q += PIPE_THREADS) {
    S.Ao[q] = 0;
    S.Mo[q] = -(1 << 29);
  }
}

// The (A, M) of the block's NC chunks against the group's ns sequences,
// staged in LDS (pp_stage_x); the tile sums are bfp_mx.h's select-free
// form.  On return (after a barrier) Ao[row*16 + s] and Mo[row*16 + s]
// hold the pair of (row, s).
template <int NC, int TPW>
__device__ __forceinline__ void pipe_mv(const PipeW<NC, TPW> &W, int nT, int ns, const MvLds &S,
                                        unsigned long long *tr) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i = lane & 15, kg = lane >> 4, h = kg & 1;
  const int sc = i < ns ? i : ns - 1;
  lds_barrier();
  pp_clock(tr, 2);
  const int tpw = (nT + PP_NW - 1) / PP_NW, t0 = w * tpw;
  const int nk = nT - t0 < tpw ? nT - t0 : tpw;   // this wave's tiles (may be <= 0)
  // pass 1: M over the tiles, reduced in LDS, and each output's smallest E
  // (for the window test below)
  int M[NC][4], Emin[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      M[c][v] = -(1 << 29);
      Emin[c][v] = 1 << 29;
    }
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    if (k < nk) {
      const int xv = S.xex[(t0 + k) * 16 + sc];
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int E = ((W.e[k][c] << (24 - 8 * v)) >> 24) + xv;
          M[c][v] = E > M[c][v] ? E : M[c][v];
          Emin[c][v] = E < Emin[c][v] ? E : Emin[c][v];
        }
    }
  }
  if (nk > 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) atomicMax(&S.Mo[(c * 16 + 4 * kg + v) * 16 + i], M[c][v]);
  }
  lds_barrier();
  pp_clock(tr, 5);
  bool wide = false;   // some tile of this lane lies past the 47-bit window
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      M[c][v] = S.Mo[(c * 16 + 4 * kg + v) * 16 + i] + 1;   // + 1: the shift of 2S
      wide = wide || M[c][v] - Emin[c][v] > ALIGN_MAX + 1;
    }
  // pass 2: the aligned tile sums (bfp_mx.h's select-free form)
  long long A[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) A[c][v] = 0;
  const long k1 = mx_k1();
  auto pass2 = [&](auto win) {
    constexpr bool WIN = decltype(win)::value;
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
      if (k < nk) {
        const int t = t0 + k;
        const uint4 xw = *reinterpret_cast<const uint4 *>(S.xs + (t * 16 + sc) * 16 + 8 * h);
        const int xev = S.xex[t * 16 + sc];
        long xh, xl;
        mx_split(xw, xh, xl);
        mx_v4 sh, sl;
        mx_xsum(xh, xl, k1, sh, sl);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const long wh = (long)(((unsigned long)W.m[k][c].y << 32) | W.m[k][c].x);
          const long wl = (long)(((unsigned long)W.m[k][c].w << 32) | W.m[k][c].z);
          mx_v4 hh, lo;
          mx_tile2(wh, wl, xh, xl, k1, sh, sl, hh, lo);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int E = ((W.e[k][c] << (24 - 8 * v)) >> 24) + xev;
            A[c][v] += mx_align2<WIN>(hh[v], lo[v], M[c][v] - E);
          }
        }
      }
    }
  };
  if (__any(wide)) pass2(std::true_type{});
  else pass2(std::false_type{});
  if (nk > 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        atomicAdd(reinterpret_cast<unsigned long long *>(&S.Ao[(c * 16 + 4 * kg + v) * 16 + i]),
                  (unsigned long long)A[c][v]);
  }
  lds_barrier();
  pp_clock(tr, 6);
}

__device__ __forceinline__ long long pp_A(const MvLds &S, int q) {
  const long long A = S.Ao[q];
  return A < SAT_LO ? SAT_LO : (A > SAT_HI ? SAT_HI : A);
}

// ---------------------------------------------------------- attention IO
// attn_body's accesses for this kernel: q|k|v and the output as tagged
// words, the KV cache -- rows 0..pos-1 written by earlier launches, row pos
// by this job for later ones -- with ordinary buffer accesses.
struct AttnPipeIO {
  rsrc_t rq, ro;                  // this sequence's q|k|v and attention output words
  unsigned tag;
  Wait *w;
  rsrc_t rkm, rke, rvm, rve, rrope;
  const int16_t *km0, *vm0;
  const int8_t *ke0, *ve0;
  const double *rope0;
  __device__ __forceinline__ void qkv(int idx, int &m, int &e) const {
    const unsigned v = w->word(rq, 4 * idx, tag);
    m = tw_m(v);
    e = tw_e(v);
  }
  __device__ __forceinline__ uint4 k16(const int16_t *p) const { return ld_b128<0>(rkm, (int)(p - km0) * 2); }
  __device__ __forceinline__ uint4 v16(const int16_t *p) const { return ld_b128<0>(rvm, (int)(p - vm0) * 2); }
  __device__ __forceinline__ int ke4(const int8_t *p) const {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(rke, (int)(p - ke0), 0, 0);
  }
  __device__ __forceinline__ int ve4(const int8_t *p) const {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(rve, (int)(p - ve0), 0, 0);
  }
  __device__ __forceinline__ int km1(const int16_t *p) const {
    return (int)(short)__builtin_amdgcn_raw_buffer_load_b16(rkm, (int)(p - km0) * 2, 0, 0);
  }
  __device__ __forceinline__ int ke1(const int8_t *p) const {
    return (int)(signed char)__builtin_amdgcn_raw_buffer_load_b8(rke, (int)(p - ke0), 0, 0);
  }
  __device__ __forceinline__ int ve1(const int8_t *p) const {
    return (int)(signed char)__builtin_amdgcn_raw_buffer_load_b8(rve, (int)(p - ve0), 0, 0);
  }
  __device__ __forceinline__ void k_put(int16_t *pm, int8_t *pe, int m, int e, bool we) const {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)m, rkm, (int)(pm - km0) * 2, 0, 0);
    if (we) __builtin_amdgcn_raw_buffer_store_b8((unsigned char)e, rke, (int)(pe - ke0), 0, 0);
  }
  __device__ __forceinline__ void v_put(int16_t *pm, int8_t *pe, int m, int e, bool we) const {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)m, rvm, (int)(pm - vm0) * 2, 0, 0);
    if (we) __builtin_amdgcn_raw_buffer_store_b8((unsigned char)e, rve, (int)(pe - ve0), 0, 0);
  }
  __device__ __forceinline__ void before_out() const {}
  __device__ __forceinline__ void out(int idx, int m, int e, bool) const { st_coh(ro, 4 * idx, tagged(m, e, tag)); }
  unsigned long long *tr;          // traced launch: this job's stamps
  __device__ __forceinline__ void mark(int k) const {
    if (k == ATT_MARK_QKV) pp_clock(tr, 2);   // wave 0's q|k|v input in
    else pp_clock(tr, 4 + k);                 // RoPE, scores, softmax, AV chains done
  }
  __device__ __forceinline__ void rope_cs(const double *cs, int j, double &c, double &s) const {
    const uint4 u = ld_b128<0>(rrope, (int)((cs - rope0) + 2 * j) * 8);
    c = __longlong_as_double((long long)(((unsigned long long)u.y << 32) | u.x));
    s = __longlong_as_double((long long)(((unsigned long long)u.w << 32) | u.z));
  }
};

// --------------------------------------------------------------- jobs
#define PP_ENTER()                                  \
  pp = uniform_ptr(pp);                             \
  const PipeArgs p = cload(pp);                     \
  Wait w{rsrc(p.abort_flag, 4), false};             \
  dsm = lds(dsm);                                   \
  const PT_CONST LayerArgs *LA = (const PT_CONST LayerArgs *)p.L

// RMSNorm `which` (1: h with gamma 1 -> x1; 2: h1 with gamma 2 -> x2) of
// sequence b at layer l (k_norm_pairs' arithmetic).
__device__ __forceinline__ void job_norm(const PipeArgs &p, const PT_CONST LayerArgs *LA, Wait &w, int l, int b,
                                         int which, int pos, double *dsm, unsigned long long *tr) {
  const int D = p.D, nd16 = p.nd16, tid = threadIdx.x;
  const unsigned tag = tag_of(pos, l, p.NL);
  double *sq = dsm, *leaf = dsm + D;
  int16_t *hm = lds(reinterpret_cast<int16_t *>(dsm + D + PW_MAX_LEAVES));
  int8_t *he = lds(reinterpret_cast<int8_t *>(hm + D));
  const double *gam = which == 1 ? LA[l].g1 : LA[l].g2;
  const int i0 = 2 * tid;
  const uint4 gu = ld_b128<0>(rsrc(gam, D * 8), i0 * 8);   // past D: zeros
  lds_barrier();   // the previous job's LDS reads are done
  if (which == 1 && l == 0) {
    // layer 0's input: the embedding k_ctl_embed stored (an earlier launch)
    if (tid < D / 8) {
      *reinterpret_cast<uint4 *>(hm + 8 * tid) = ld_b128<0>(rsrc(p.h_m), (b * D + 8 * tid) * 2);
    } else if (tid < D / 8 + D / 64) {
      const int q = tid - D / 8;
      *reinterpret_cast<int *>(he + 4 * q) =
          (int)__builtin_amdgcn_raw_buffer_load_b32(rsrc(p.h_e), b * nd16 + 4 * q, 0, 0);
    }
  } else {
    const unsigned *wi = which == 1 ? p.w_h : p.w_h1;
    const unsigned tin = which == 1 ? tag_of(pos, l - 1, p.NL) : tag;
    pp_poll_quads<1>(w, rsrc(wi + (long long)b * D), D / 4, tin, [&](int q, const uint4 &v) {
      typedef unsigned v2u __attribute__((ext_vector_type(2)));
      v2u m;
      m.x = (v.x & 0xffffu) | (v.y << 16);
      m.y = (v.z & 0xffffu) | (v.w << 16);
      *reinterpret_cast<v2u *>(hm + 4 * q) = m;
      if ((q & 3) == 0) he[q >> 2] = (int8_t)tw_e(v.x);
    });
  }
  lds_barrier();
  pp_clock(tr, 2);
  const double g0 = __longlong_as_double((long long)(((unsigned long long)gu.y << 32) | gu.x));
  const double g1 = __longlong_as_double((long long)(((unsigned long long)gu.w << 32) | gu.z));
  int m0, m1, e;
  rmsnorm_pairs(hm, he, g0, g1, D, sq, leaf, m0, m1, e);
  if (i0 < D) {
    typedef unsigned v2u __attribute__((ext_vector_type(2)));
    v2u x;
    x.x = tagged(m0, e, tag);
    x.y = tagged(m1, e, tag);
    __builtin_amdgcn_raw_buffer_store_b64(x, rsrc((which == 1 ? p.w_x1 : p.w_x2) + (long long)b * D), 4 * i0, 0,
                                          CPOL_SC1);
  }
}

// The attention of KV group gk (all its query heads) of sequence b at
// layer l.  A function of its own: inlined into the role functions, its
// scalar values spilled into vector-register lanes and the job took 12.2 us
// at position 135 of config 5 instead of 8.0.
template <int PPW>
__device__ __noinline__ void job_attn(const PipeArgs &p, const PT_CONST LayerArgs *LA, Wait &w, int l, int gk,
                                         int b, int pos, double *dsm, unsigned long long *tr) {
  const int nq = p.D + 2 * p.KV;
  LayerArgs a = cload(LA + l);
  a.dump = nullptr;
  a.rope_row = nullptr;
  AttnPipeIO io;
  io.rq = rsrc(p.w_qkv + (long long)b * nq);
  io.ro = rsrc(p.w_att + (long long)b * p.D);
  io.tag = tag_of(pos, l, p.NL);
  io.w = &w;
  io.km0 = a.k_m;
  io.ke0 = a.k_e;
  io.vm0 = a.v_m;
  io.ve0 = a.v_e;
  io.rkm = rsrc(a.k_m);
  io.rke = rsrc(a.k_e);
  io.rvm = rsrc(a.v_m);
  io.rve = rsrc(a.v_e);
  io.rope0 = a.rope;
  io.rrope = rsrc(a.rope);
  io.tr = tr;
  lds_barrier();   // the previous job's LDS reads are done
  attn_group_body<PPW>(a, io, gk, b, [pos] { return make_int2(pos, pos); }, dsm);
}

// The epilogue pairs of a block: 16-lane group j (waves 0-3) owns sequence
// j of the group, lane r row r of each chunk.
#define PP_EPI(...)                                           \
  if (threadIdx.x < 16 * PIPE_SEQ) {                          \
    const int r = threadIdx.x & 15, j = threadIdx.x >> 4;     \
    const bool wr = j < ns;                                   \
    const int b = b0 + (wr ? j : 0);                          \
    __VA_ARGS__;                                              \
  }

// Matvec stage ST (chunk c, group g) of layer l with the role's weights.
template <int ST, int NC, int TPW>
__device__ __forceinline__ void job_mv(const PipeArgs &p, const PT_CONST LayerArgs *LA, Wait &w, int l, int c,
                                       int g, int pos, const PipeW<NC, TPW> &W, double *dsm,
                                       unsigned long long *tr) {
  const int D = p.D, b0 = g * PIPE_SEQ, ns = min(PIPE_SEQ, p.batch - b0);
  const unsigned tag = tag_of(pos, l, p.NL);
  constexpr bool FIN = ST == PS_D;                    // FFN-wide input
  const int nT = FIN ? p.FFN / 16 : p.nd16;
  const int n_in = nT * 16;
  const unsigned *xw = ST == PS_QKV ? p.w_x1 : (ST == PS_O ? p.w_att : (ST == PS_GU ? p.w_x2 : p.w_mlp));
  const MvLds S = mv_lds(dsm, nT, NC);
  // this lane's residual word (O: h of the layer input; D: h1), loaded now
  // and checked in the epilogue
  const int r_ = threadIdx.x & 15, j_ = threadIdx.x >> 4;
  const int bres = b0 + (j_ < ns ? j_ : 0);
  rsrc_t rres = rsrc(ST == PS_O ? p.w_h : p.w_h1);
  unsigned tres = ST == PS_O ? tag_of(pos, l - 1, p.NL) : tag;
  unsigned res = 0;
  if constexpr (ST == PS_O || ST == PS_D) {
    if (ST == PS_O && l == 0) {   // layer 0's input: k_ctl_embed's BFP (an earlier launch)
      const int m = (int)(short)__builtin_amdgcn_raw_buffer_load_b16(rsrc(p.h_m), 2 * (bres * D + c * 16 + r_), 0, 0);
      const int e = (int)(signed char)__builtin_amdgcn_raw_buffer_load_b8(rsrc(p.h_e), bres * p.nd16 + c, 0, 0);
      res = tagged(m, e, 0);
    } else {
      res = ld_coh(rres, 4 * (bres * D + c * 16 + r_));
    }
  }
  lds_barrier();   // the previous job's LDS reads are done
  // quads a thread stages: 16 sequences of at most PP_NW * TPW tiles
  constexpr int NQ = (PIPE_SEQ * PP_NW * TPW * 16 / 4 + PIPE_THREADS - 1) / PIPE_THREADS;
  pp_stage_x<NQ, NC>(w, xw + (long long)b0 * n_in, n_in, ns, tag, S);
  pipe_mv<NC, TPW>(W, nT, ns, S, tr);
  auto residual = [&](int &rm, int &re) {
    if ((ST == PS_D || l > 0) && (res >> 24) != tres) res = w.word(rres, 4 * (bres * D + c * 16 + r_), tres);
    rm = tw_m(res);
    re = tw_e(res);
  };
  if constexpr (ST == PS_QKV) {
    const int nq = D + 2 * p.KV;
    const rsrc_t ro = rsrc(p.w_qkv);
    PP_EPI({
      int m, e;
      const int q = r * 16 + j;
      chunk_quant(pp_A(S, q), S.Mo[q], m, e);
      if (wr) st_coh(ro, 4 * (b * nq + c * 16 + r), tagged(m, e, tag));
    })
  } else if constexpr (ST == PS_O) {
    const rsrc_t ro = rsrc(p.w_h1);
    PP_EPI({
      int rm, re;
      residual(rm, re);
      int om, oe, e;
      const int q = r * 16 + j;
      chunk_quant(pp_A(S, q), S.Mo[q], om, oe);
      const int m = residual_lane(om, oe, rm, re, e);
      if (wr) st_coh(ro, 4 * (b * D + c * 16 + r), tagged(m, e, tag));
    })
  } else if constexpr (ST == PS_GU) {
    const int F = p.FFN;
    const rsrc_t ro = rsrc(p.w_mlp);
    PP_EPI({
      const int qg = r * 16 + j, qu = (16 + r) * 16 + j;
      int gm, ge, um, ue, me;
      chunk_quant(pp_A(S, qg), S.Mo[qg], gm, ge);
      chunk_quant(pp_A(S, qu), S.Mo[qu], um, ue);
      const int mm = swiglu_lane(gm, ge, um, ue, me);
      if (wr) st_coh(ro, 4 * (b * F + c * 16 + r), tagged(mm, me, tag));
    })
  } else {
    const int nd16 = p.nd16;
    const rsrc_t ro = rsrc(p.w_h), rhm = rsrc(p.h_m), rhe = rsrc(p.h_e);
    const bool last = l == p.NL - 1;
    PP_EPI({
      int rm, re;
      residual(rm, re);
      int dm, de, e;
      const int q = r * 16 + j;
      chunk_quant(pp_A(S, q), S.Mo[q], dm, de);
      const int m = residual_lane(dm, de, rm, re, e);
      int chm = m, che = e;
      if (p.hist_m) canon16_lanes(chm, che);
      if (wr) {
        st_coh(ro, 4 * (b * D + c * 16 + r), tagged(m, e, tag));
        if (last) {   // the head's input (read after the launch)
          __builtin_amdgcn_raw_buffer_store_b16((unsigned short)m, rhm, 2 * (b * D + c * 16 + r), 0, 0);
          if (r == 0) __builtin_amdgcn_raw_buffer_store_b8((unsigned char)e, rhe, b * nd16 + c, 0, 0);
        }
        if (p.hist_m && pos < p.hist_steps) {
          const long long o = (((long long)b * p.hist_steps + pos) * p.NL + l) * D;
          p.hist_m[o + c * 16 + r] = (int16_t)chm;
          if (r == 0) p.hist_e[(o >> 4) + c] = (int8_t)che;
        }
      }
    })
  }
  pp_clock(tr, 7);
}
#undef PP_EPI

// ---------------------------------------------------------------- roles
// The base of chunk c's block (device layout) in layer l for role ST.
template <int ST>
__device__ __forceinline__ void role_block(const PT_CONST LayerArgs *LA, int l, int c, int nT, const void *&pm,
                                           const void *&pe) {
  if constexpr (ST == PS_QKV) {
    pm = LA[l].w_qkv_m + (long long)c * nT * 32;
    pe = LA[l].w_qkv_e + (long long)c * nT * 16;
  } else if constexpr (ST == PS_O) {
    pm = LA[l].w_o_m + (long long)c * nT * 32;
    pe = LA[l].w_o_e + (long long)c * nT * 16;
  } else if constexpr (ST == PS_GU) {
    pm = LA[l].w_gu_m + (long long)(2 * c) * nT * 32;
    pe = LA[l].w_gu_e + (long long)(2 * c) * nT * 16;
  } else {
    pm = LA[l].w_d_m + (long long)c * nT * 32;
    pe = LA[l].w_d_e + (long long)c * nT * 16;
  }
}

// A workgroup's whole step: its jobs in beat order, layer by layer, with
// the weights of its matvec role ST (-1: none) for chunk c.
template <int ST, int PPW>
__device__ __noinline__ void pipe_role(const PT_CONST PipeArgs *pp, double *dsm, int c) {
  PP_ENTER();
  c = uniform_int(c);
  constexpr bool MV = ST >= 0;
  constexpr int NC = ST == PS_GU ? 2 : 1;
  constexpr int TPW = ST == PS_D ? PP_TPW_F : PP_TPW_D;
  const int nT = ST == PS_D ? p.FFN / 16 : p.nd16;
  const int pos = *(const PT_CONST int *)p.state;
  PipeW<NC, MV ? TPW : 1> W;
  bool fresh = false;   // W holds loads not yet split
  if constexpr (MV) {
    const void *pm, *pe;
    role_block<ST>(LA, 0, c, nT, pm, pe);
    pw_load(W, pm, pe, nT);
    fresh = true;
  }
  const PT_CONST int *js = (const PT_CONST int *)p.jobs;
  const int j0 = ((const PT_CONST int *)p.jstart)[blockIdx.x], j1 = ((const PT_CONST int *)p.jstart)[blockIdx.x + 1];
  unsigned long long *trw = p.trace ? p.trace + (long long)blockIdx.x * PIPE_TRACE_JOBS * PIPE_TRACE_W : nullptr;
  for (int j = j0; j < j1; ++j) {
    const int code = js[j];
    const int l = code >> 26, st = (code >> 23) & 7, g = (code >> 16) & 127, idx = code & 0xffff;
    unsigned long long *tr = (trw && j - j0 < PIPE_TRACE_JOBS) ? trw + (j - j0) * PIPE_TRACE_W : nullptr;
    pp_stamp(tr, 0, (unsigned)code + 1u);
    pp_clock(tr, 1);
    if (st == PS_N1 || st == PS_N2) {
      job_norm(p, LA, w, l, idx, st == PS_N1 ? 1 : 2, pos, dsm, tr);
    } else if (st == PS_ATT) {
      job_attn<PPW>(p, LA, w, l, idx % p.H_KV, idx / p.H_KV, pos, dsm, tr);
    } else if constexpr (MV) {
      if (fresh) {
        pw_split(W);
        fresh = false;
      }
      job_mv<ST, NC, TPW>(p, LA, w, l, c, g, pos, W, dsm, tr);
      if (g == p.ngrp - 1 && l + 1 < p.NL) {   // the layer's last group: prefetch the next
        const void *pm, *pe;
        role_block<ST>(LA, l + 1, c, nT, pm, pe);
        pw_load(W, pm, pe, nT);
        fresh = true;
      }
    }
    pp_clock(tr, 3);
  }
}

// gp: the argument block in device memory (read through the constant
// address space as scalars).
template <int PPW>
__global__ __launch_bounds__(PIPE_THREADS, 1) void k_pipe_step(const PipeArgs *gp) {
  extern __shared__ double dsm[];
  const PT_CONST PipeArgs *pp = (const PT_CONST PipeArgs *)gp;
  const int role = ((const PT_CONST int *)cload(pp).role)[blockIdx.x];
  const int st = role >> 16, c = role & 0xffff;
  if (role < 0) pipe_role<-1, PPW>(pp, dsm, 0);
  else if (st == PS_QKV) pipe_role<PS_QKV, PPW>(pp, dsm, c);
  else if (st == PS_O) pipe_role<PS_O, PPW>(pp, dsm, c);
  else if (st == PS_GU) pipe_role<PS_GU, PPW>(pp, dsm, c);
  else pipe_role<PS_D, PPW>(pp, dsm, c);
}

// ------------------------------------------------------------------ host
typedef void (*pp_fn)(const PipeArgs *);
static pp_fn pipe_kernel(int ppw) { return ppw == 2 ? k_pipe_step<2> : k_pipe_step<3>; }

int pipe_plan(const bfp_dims &d, int batch, int max_ctx, int cus, PipePlan &pl) {
  const int ppw = attn_ppw(max_ctx);
  const int nq16 = (d.D + 2 * d.H_KV * d.HD) / 16, nd16 = d.D / 16, nf16 = d.FFN / 16;
  const int ngrp = (batch + PIPE_SEQ - 1) / PIPE_SEQ;
  const int roles = nq16 + nd16 + nf16 + nd16;
  const int NL = d.NL, HKV = d.H_KV, KVC = d.H_KV * d.HD / 16, grp = d.H_Q / d.H_KV;
  if (d.HD != 64 || ppw > 3 || grp > AG_MAXG || grp + 2 > ATT_WAVES || d.D % 64 || d.FFN % 64 ||
      nd16 > PP_NW * PP_TPW_D ||
      nf16 > PP_NW * PP_TPW_F || d.D > 2 * PIPE_THREADS || batch < 1 || (long long)batch * d.H_KV > 65535 ||
      ngrp > PIPE_MAX_GROUPS || roles > cus || NL < 1 || NL > PIPE_MAX_LAYERS)
    return 0;
  pl.batch = batch;
  pl.ngrp = ngrp;
  pl.grid = cus;
  pl.ppw = ppw;
  // The jobs of a step, each workgroup's list in the order of a simulated
  // run: job durations and the hand-off latency are config 5's measured
  // medians (us); matvec jobs run on their role's workgroup in (layer,
  // group) order; a free workgroup takes its own next matvec job when that
  // is ready, else the oldest ready RMSNorm or attention job.  Each list is
  // in simulated start order, and every job starts after its inputs' jobs
  // end, so in any run the earliest unfinished job can proceed.  A job's
  // time is its inputs' poll (once they are complete) plus its work, as
  // measured with the job trace at config 5.
  const double t_lat = 0.3, t_n = 2.8, t_att = 8.3;
  const double t_mv[PS_COUNT] = {0, 4.5, 0, 5.2, 0, 7.2, 10.8};
  struct Job {
    int code = 0, npend = 0;
    double dur = 0.0, ready = 0.0, end = 0.0;
    std::vector<int> out;   // jobs that read this one's outputs
  };
  std::vector<Job> J;
  // job ids: per (layer, group): N1 ns, QKV nq16, ATT ns*HKV, O nd16, N2 ns, GU nf16, D nd16
  std::vector<int> base((size_t)NL * ngrp + 1);
  auto nsg = [&](int g) { return std::min(PIPE_SEQ, batch - g * PIPE_SEQ); };
  {
    int n = 0;
    for (int l = 0; l < NL; ++l)
      for (int g = 0; g < ngrp; ++g) {
        base[(size_t)l * ngrp + g] = n;
        n += 2 * nsg(g) + nsg(g) * HKV + nq16 + 2 * nd16 + nf16;
      }
    base[(size_t)NL * ngrp] = n;
    J.resize(n);
  }
  auto id_of = [&](int l, int st, int g, int idx) -> int {
    const int ns = nsg(g), b0 = g * PIPE_SEQ;
    int o = base[(size_t)l * ngrp + g];
    switch (st) {
      case PS_N1: return o + (idx - b0);
      case PS_QKV: return o + ns + idx;
      case PS_ATT: return o + ns + nq16 + (idx - b0 * HKV);
      case PS_O: return o + ns + nq16 + ns * HKV + idx;
      case PS_N2: return o + ns + nq16 + ns * HKV + nd16 + (idx - b0);
      case PS_GU: return o + 2 * ns + nq16 + ns * HKV + nd16 + idx;
      default: return o + 2 * ns + nq16 + ns * HKV + nd16 + nf16 + idx;
    }
  };
  auto dep = [&](int from, int to) { J[from].out.push_back(to); };
  for (int l = 0; l < NL; ++l)
    for (int g = 0; g < ngrp; ++g) {
      const int b0 = g * PIPE_SEQ, b1 = b0 + nsg(g);
      for (int b = b0; b < b1; ++b) {
        const int j = id_of(l, PS_N1, g, b);
        J[j].code = pipe_job(l, PS_N1, g, b);
        J[j].dur = t_n;
        if (l > 0)
          for (int c = 0; c < nd16; ++c) dep(id_of(l - 1, PS_D, g, c), j);
      }
      for (int c = 0; c < nq16; ++c) {
        const int j = id_of(l, PS_QKV, g, c);
        J[j].code = pipe_job(l, PS_QKV, g, c);
        J[j].dur = t_mv[PS_QKV];
        for (int b = b0; b < b1; ++b) dep(id_of(l, PS_N1, g, b), j);
      }
      for (int b = b0; b < b1; ++b)
        for (int kv = 0; kv < HKV; ++kv) {
          const int j = id_of(l, PS_ATT, g, b * HKV + kv);
          J[j].code = pipe_job(l, PS_ATT, g, b * HKV + kv);
          J[j].dur = t_att;
          for (int k = 0; k < 4; ++k) {   // its heads' q rows, its k and v rows: 64 each
            for (int h = kv * grp; h < kv * grp + grp; ++h) dep(id_of(l, PS_QKV, g, 4 * h + k), j);
            dep(id_of(l, PS_QKV, g, nd16 + 4 * kv + k), j);
            dep(id_of(l, PS_QKV, g, nd16 + KVC + 4 * kv + k), j);
          }
        }
      for (int c = 0; c < nd16; ++c) {
        const int j = id_of(l, PS_O, g, c);
        J[j].code = pipe_job(l, PS_O, g, c);
        J[j].dur = t_mv[PS_O];
        for (int b = b0; b < b1; ++b)
          for (int kv = 0; kv < HKV; ++kv) dep(id_of(l, PS_ATT, g, b * HKV + kv), j);
      }
      for (int b = b0; b < b1; ++b) {
        const int j = id_of(l, PS_N2, g, b);
        J[j].code = pipe_job(l, PS_N2, g, b);
        J[j].dur = t_n;
        for (int c = 0; c < nd16; ++c) dep(id_of(l, PS_O, g, c), j);
      }
      for (int c = 0; c < nf16; ++c) {
        const int j = id_of(l, PS_GU, g, c);
        J[j].code = pipe_job(l, PS_GU, g, c);
        J[j].dur = t_mv[PS_GU];
        for (int b = b0; b < b1; ++b) dep(id_of(l, PS_N2, g, b), j);
      }
      for (int c = 0; c < nd16; ++c) {
        const int j = id_of(l, PS_D, g, c);
        J[j].code = pipe_job(l, PS_D, g, c);
        J[j].dur = t_mv[PS_D];
        for (int c2 = 0; c2 < nf16; ++c2) dep(id_of(l, PS_GU, g, c2), j);
      }
    }
  // roles: the workgroup of each matvec chunk; its jobs in (layer, group)
  // order.  (Two workgroups a D chunk taking alternate groups, with the
  // Q|K|V chunks in pairs to free them, made the simulated step longer: the
  // stage chain of a group, not the D role, bounds the layer.)
  pl.role.assign(cus, -1);
  std::vector<std::vector<int>> pinned(cus);
  std::vector<size_t> pnext(cus, 0);
  {
    int w = 0;
    const int rs[4] = {PS_QKV, PS_O, PS_GU, PS_D}, rn[4] = {nq16, nd16, nf16, nd16};
    for (int k = 0; k < 4; ++k)
      for (int c = 0; c < rn[k]; ++c, ++w) {
        pl.role[w] = (rs[k] << 16) | c;
        for (int l = 0; l < NL; ++l)
          for (int g = 0; g < ngrp; ++g) pinned[w].push_back(id_of(l, rs[k], g, c));
      }
  }
  // event simulation; a workgroup with a matvec role takes an RMSNorm or
  // attention job only when it would end before the role's next matvec job
  // became ready in the previous pass (none in the first pass): the best of
  // a few passes is kept
  auto is_mv = [](int st) { return st == PS_QKV || st == PS_O || st == PS_GU || st == PS_D; };
  std::vector<double> est(J.size(), 1e300), best_est;
  std::vector<std::vector<int>> lst(cus), best_lst;
  double best_len = 1e300;
  for (int pass = 0; pass < 4; ++pass) {
    for (Job &x : J) {
      x.npend = 0;
      x.ready = 0.0;
      x.end = 0.0;
    }
    for (const Job &x : J)
      for (int o : x.out) ++J[o].npend;
    std::vector<double> wfree(cus, 0.0);
    std::fill(pnext.begin(), pnext.end(), 0);
    for (auto &v : lst) v.clear();
    std::set<std::pair<double, int>> flex;   // ready RMSNorm / attention jobs, oldest first
    for (size_t j = 0; j < J.size(); ++j)
      if (J[j].npend == 0 && !is_mv((J[j].code >> 23) & 7)) flex.insert({0.0, (int)j});
    size_t left = J.size();
    bool stuck = false;
    while (left > 0) {
      double best_t = 1e300;
      int best_w = -1, best_j = -1;
      for (int w = 0; w < cus; ++w) {
        double t = 1e300, limit = 1e300;
        int jj = -1;
        if (pnext[w] < pinned[w].size()) {
          const int j = pinned[w][pnext[w]];
          limit = est[j];
          if (J[j].npend == 0) {
            t = std::max(wfree[w], J[j].ready);
            jj = j;
          }
        }
        if (!flex.empty()) {
          const int f = flex.begin()->second;
          const double tf = std::max(wfree[w], flex.begin()->first);
          if (tf < t && tf + J[f].dur <= limit) {
            t = tf;
            jj = -2;
          }
        }
        if (jj != -1 && t < best_t) {
          best_t = t;
          best_w = w;
          best_j = jj;
        }
      }
      if (best_w < 0) {   // every ready job is held back by the estimates
        stuck = true;
        break;
      }
      int j = best_j;
      if (j == -2) {
        j = flex.begin()->second;
        flex.erase(flex.begin());
      } else {
        ++pnext[best_w];
      }
      J[j].end = best_t + J[j].dur;
      wfree[best_w] = J[j].end;
      lst[best_w].push_back(j);
      for (int o : J[j].out) {
        J[o].ready = std::max(J[o].ready, J[j].end + t_lat);
        if (--J[o].npend == 0 && !is_mv((J[o].code >> 23) & 7)) flex.insert({J[o].ready, o});
      }
      --left;
    }
    if (stuck) continue;
    double len = 0.0;
    for (const Job &x : J) len = std::max(len, x.end);
    if (len < best_len) {
      best_len = len;
      best_lst = lst;
    }
    for (size_t j = 0; j < J.size(); ++j) est[j] = J[j].ready;
  }
  if (best_lst.empty()) return 0;
  lst = best_lst;
  pl.sim_step_us = best_len;
  pl.jstart.assign((size_t)cus + 1, 0);
  pl.jobs.clear();
  for (int w = 0; w < cus; ++w) {
    pl.jstart[w] = (int)pl.jobs.size();
    for (int j : lst[w]) pl.jobs.push_back(J[j].code);
  }
  pl.jstart[cus] = (int)pl.jobs.size();
  // LDS: the attention's, a matvec job's (inputs, exponents, A and M) and
  // an RMSNorm's
  const int nTmax = std::max(nd16, nf16);
  const size_t att = attn_grp_lds_bytes(max_ctx, grp);
  const size_t mv = ((size_t)16 * nTmax * 32 + 16 * nTmax + 7) / 8 * 8 + (size_t)2 * 256 * 12;
  const size_t nrm = (size_t)(d.D + PW_MAX_LEAVES) * 8 + (size_t)d.D * 2 + nd16;
  pl.lds = (std::max(att, std::max(mv, nrm)) + 15) & ~(size_t)15;
  return 1;
}

int pipe_prepare(const PipePlan &pl) {
  const pp_fn f = pipe_kernel(pl.ppw);
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(f), (int)pl.lds));
  int nb = 0;
  HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(f), PIPE_THREADS,
                                                       pl.lds));
  if (nb < 1) return set_err(BFP_EINVAL, "pipelined step: %zu bytes of LDS do not fit a compute unit", pl.lds);
  return BFP_OK;
}

int launch_pipe_step(const PipePlan &pl, const PipeArgs *dev_args, hipStream_t s) {
  // grid = the compute units and one workgroup fits each (pipe_prepare):
  // every workgroup is resident at once
  hipLaunchKernelGGL(pipe_kernel(pl.ppw), dim3(pl.grid), dim3(PIPE_THREADS), pl.lds, s, dev_args);
  return launch_status("pipelined step");
}

}  // namespace bfp
