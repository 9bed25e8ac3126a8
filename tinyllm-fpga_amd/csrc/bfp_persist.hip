// Persistent decode kernel: the whole batch-1 greedy decode
// (rtl/vc707/host/gen_smollm_blockfp_full.py:426-443) as ONE launch of one
// workgroup per compute unit.
//
// The workgroups wait on one another, so all of them must be resident at
// once.  The grid is the compute-unit count and the launch is refused unless
// the occupancy calculator fits at least one workgroup per compute unit;
// the library runs nothing else on the device meanwhile (its calls are
// synchronous), so the dispatcher places every workgroup at once.  This is
// an ordinary launch, not hipLaunchCooperativeKernel: the kernel uses no
// grid barrier, and every process that had made a cooperative launch ended
// in a segmentation fault inside exit() under rocprofv3 (after the
// profiler's own finalisation), while processes without one exited cleanly.
// Should a workgroup ever not be placed, the bounded waits below give up
// and the decode reports BFP_EIO instead of hanging.
//
// Why: a decode step is 5 dependent stages per layer x 30 layers + the
// head.  As separate kernels each stage pays a launch and the reload of its
// inputs (about 3.7 us of fixed cost per graph node on MI355X, against
// 0.2-3.5 MB of weights per stage).  Here every workgroup keeps one role for
// the whole decode and the stages hand their outputs over through memory:
//
//   role       workgroups        job per layer step
//   Q|K|V      0 .. nq-1         chunk c of q|k|v (RMSNorm prologue); the
//                                first n_att of them also run attention job c
//   O          o0 ..             chunk c of o + residual -> h1
//   G/U        g0 ..             chunks (2c, 2c+1) of g|u + SwiGLU -> mlp
//   D          d0 ..             chunk c of d + residual -> h (layer output)
//   (all)                        the head: a slice of the vocabulary, then
//                                the argmax over all slices -> next token
//
// Each workgroup issues the loads of its next job's weights as soon as its
// current job is done, so the weight stream overlaps the other stages.
//
// Hand-off: every activation element travels as one 32-bit word
// m (16 bits) | e (8 bits) | tag (8 bits), stored and loaded at the
// device-coherent level (the SC1 cache policy: the eight XCDs' L2 caches
// are not coherent with one another).  A consumer spins until every word it
// needs carries the tag of the (step, layer) it wants, so no flag, counter
// or fence is needed: each word validates itself.  Buffers are
// double-buffered by step parity; tags are (step*NL + layer) % 255 + 1, and
// the buffers start at 0.  Ordering argument (one write ahead at most):
// every producer's next write into a buffer of the same parity depends,
// through the stage chain, on every consumer of its previous write having
// read it.  The KV cache rows are stored and read at the coherent level
// too; the writer waits for its row stores to complete before it stores
// its attention output, and every reader of that row at a later step
// depends on that output (for NL >= 2).
//
// Every wait is bounded (2 s on the 100 MHz clock); a wait that gives up
// raises a device abort flag which every other wait then sees, so all waves
// run to the end of the kernel and the host reports the abort.  The
// arithmetic is the per-stage kernels' own (bfp_layer_dev.h, bfp_mv.h):
// the outputs are bit-identical to the graph path.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <vector>

#include "bfp.h"
#include "bfp_device.h"
#include "bfp_f64.h"
#include "bfp_internal.h"
#include "bfp_layer.h"
#include "bfp_layer_dev.h"
#include "bfp_mv.h"
#include "bfp_persist.h"
#include "bfp_coh.h"

namespace bfp {

constexpr int PT_THREADS = 512;   // 8 waves: the attention body's workgroup size
constexpr int PT_NW = PT_THREADS / 64;
constexpr int PT_HEAD_D64 = 9;    // head rows of at most 576 elements

// A weight chunk (nT tiles: mantissas nT x 512 bytes at wm, exponents nT x 16
// at we) into registers, every load unconditional: tiles past nT read 0 and
// the engine ignores them.
template <int TPT>
__device__ __forceinline__ void load_chunk_rs(ChunkRegs<TPT> &R, const void *wm, const void *we, int nT) {
  const rsrc_t rm = rsrc(wm, nT * 512), re = rsrc(we, nT * 16);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, tq = lane >> 4;
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const int t = tq + 4 * (w + PT_NW * j);
    R.a[j] = ld_b128<0>(rm, (t * 32 + r) * 16);
    R.b[j] = ld_b128<0>(rm, (t * 32 + 16 + r) * 16);
    R.e[j] = (int)(signed char)__builtin_amdgcn_raw_buffer_load_b8(re, t * 16 + r, 0, 0);
  }
}

// This thread's gammas (elements 2t and 2t + 1; D <= 2 * PT_THREADS) of one
// norm, prefetched with the layer's weights (one 16-byte load).
struct Gammas {
  double v[2];
};
__device__ __forceinline__ void load_gammas(Gammas &G, const double *g, int D) {
  const uint4 u = ld_b128<0>(rsrc(g, D * 8), threadIdx.x * 16);   // past D: zeros
  G.v[0] = __longlong_as_double((long long)(((unsigned long long)u.y << 32) | u.x));
  G.v[1] = __longlong_as_double((long long)(((unsigned long long)u.w << 32) | u.z));
}

// A tagged BFP vector of n elements (n % 16 == 0) into (m, e) arrays.
__device__ __forceinline__ void wait_bfp(Wait &w, rsrc_t r, int n, unsigned tag, int16_t *hm,
                                         int8_t *he) {
  for (int q = threadIdx.x; q < n / 4; q += blockDim.x) {
    const uint4 v = w.quad(r, 16 * q, tag);
    hm[4 * q] = (int16_t)tw_m(v.x);
    hm[4 * q + 1] = (int16_t)tw_m(v.y);
    hm[4 * q + 2] = (int16_t)tw_m(v.z);
    hm[4 * q + 3] = (int16_t)tw_m(v.w);
    if ((q & 3) == 0) he[q >> 2] = (int8_t)tw_e(v.x);
  }
}

// A tagged BFP vector into the matvec's LDS input form (xs, xes).
__device__ __forceinline__ void wait_x(Wait &w, rsrc_t r, int n, unsigned tag, int *xs, int *xes) {
  for (int q = threadIdx.x; q < n / 4; q += blockDim.x) {
    const uint4 v = w.quad(r, 16 * q, tag);
    const int p0 = 2 * q;
    put_x_pair(xs, p0 >> 3, p0 & 7, tw_m(v.x), tw_m(v.y));
    put_x_pair(xs, (p0 + 1) >> 3, (p0 + 1) & 7, tw_m(v.z), tw_m(v.w));
    if ((q & 3) == 0) xes[q >> 2] = tw_e(v.x);
  }
}

// embed_q[tok] = fp_quantize_vec(embed[tok]) (full.py:411-412) into (m, e)
// arrays; all threads call (16-lane groups hold whole tiles).
__device__ __forceinline__ void embed_vec(const PersistArgs &p, int tok, int16_t *hm, int8_t *he) {
  const float *row = p.embed + (long long)tok * p.D;
  for (int base = 0; base < p.D; base += blockDim.x) {
    const int i = base + threadIdx.x;
    const bool ok = i < p.D;
    int e;
    const int m = quantize16_lanes(ok ? (double)row[i] : 0.0, e);
    if (ok) {
      hm[i] = (int16_t)m;
      if ((i & 15) == 0) he[i >> 4] = (int8_t)e;
    }
  }
}

// Tile c of embed_q[tok]: lane r of each 16-lane group holds element 16c + r.
__device__ __forceinline__ void embed_tile(const PersistArgs &p, int tok, int c, int &m, int &e) {
  const float *row = p.embed + (long long)tok * p.D;
  m = quantize16_lanes((double)row[c * 16 + (threadIdx.x & 15)], e);
}

// A device-clock stamp into 64-bit slot k of buf (a buffer store: it does
// not hold up the workgroup's LDS waits as a generic store would).
__device__ __forceinline__ void put_clock(unsigned long long *buf, size_t k) {
  const unsigned long long t = __builtin_amdgcn_s_memrealtime();
  typedef unsigned v2u __attribute__((ext_vector_type(2)));
  v2u v;
  v.x = (unsigned)t;
  v.y = (unsigned)(t >> 32);
  __builtin_amdgcn_raw_buffer_store_b64(v, rsrc(buf + k, 8), 0, 0, 0);
}
// Stage trace stamp k of (step s, layer l) by thread 0 of the role's first
// workgroup (lead), when tracing.
__device__ __forceinline__ void stamp(const PersistArgs &p, bool lead, int s, int l, int k) {
  if (p.trace && lead && threadIdx.x == 0) put_clock(p.trace, ((size_t)s * p.NL + l) * PT_TRACE_LAYER + k);
}
__device__ __forceinline__ void stamp_head(const PersistArgs &p, int s, int k) {
  if (p.trace && blockIdx.x == 0 && threadIdx.x == 0)
    put_clock(p.trace, (size_t)p.steps * p.NL * PT_TRACE_LAYER + (size_t)s * PT_TRACE_STEP + k);
}

__device__ __forceinline__ int clamp_tok(const PersistArgs &p, int t) {
  return t < 0 ? 0 : (t >= p.VOCAB ? p.VOCAB - 1 : t);
}

// Attention access at the device-coherent level: q|k|v and the output as
// tagged words, the KV cache through SC1 buffer loads and stores.
struct AttnCohIO {
  // long form: the head's ATT_DSPLIT workgroups split the scores and
  // exchange them through sc_buf (rsc: head hq's at hq * sc_stride entries,
  // in blocks per workgroup, attn_sc_stride), each score as four tagged
  // words, which the readers poll: no flag, no wait for the stores'
  // completion
  static constexpr bool kSplitScores = true;
  static constexpr int kAvBlock = ATT_AVC;   // a whole staged chunk's products (one workgroup a CU)
  rsrc_t rq, ro;                  // this step's q|k|v and attention output words
  unsigned tag;
  Wait *w;
  rsrc_t rsc;
  int sc_stride, sc_block;
  rsrc_t rkm, rke, rvm, rve;      // this layer's KV cache
  const int16_t *km0, *vm0;
  const int8_t *ke0, *ve0;
  // the step's RoPE row: role_qkv's copy in LDS (rope_s), read as LDS
  const double *rope_s;
  __device__ __forceinline__ void rope_cs(const double *, int j, double &c, double &s) const {
    const double *ls = lds(rope_s);
    c = ls[2 * j];
    s = ls[2 * j + 1];
  }
  unsigned long long *trace;      // traced decode, first attention job: its (step, layer) stamps
  __device__ __forceinline__ void mark(int k) const {
    // ATT_MARK_ROPE .. ATT_MARK_AV at PT_TRACE_ATT + k, the q|k|v arrival in slot 2
    if (trace && threadIdx.x == 0) put_clock(trace, k == ATT_MARK_QKV ? 2 : PT_TRACE_ATT + k);
  }
  __device__ __forceinline__ void qkv(int idx, int &m, int &e) const {
    const unsigned v = w->word(rq, 4 * idx, tag);
    m = tw_m(v);
    e = tw_e(v);
  }
  __device__ __forceinline__ uint4 k16(const int16_t *p) const { return ld_b128<CPOL_SC1>(rkm, (int)(p - km0) * 2); }
  __device__ __forceinline__ uint4 v16(const int16_t *p) const { return ld_b128<CPOL_SC1>(rvm, (int)(p - vm0) * 2); }
  __device__ __forceinline__ int ke4(const int8_t *p) const {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(rke, (int)(p - ke0), 0, CPOL_SC1);
  }
  __device__ __forceinline__ int ve4(const int8_t *p) const {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(rve, (int)(p - ve0), 0, CPOL_SC1);
  }
  __device__ __forceinline__ int km1(const int16_t *p) const {
    return (int)(short)__builtin_amdgcn_raw_buffer_load_b16(rkm, (int)(p - km0) * 2, 0, CPOL_SC1);
  }
  __device__ __forceinline__ int ke1(const int8_t *p) const {
    return (int)(signed char)__builtin_amdgcn_raw_buffer_load_b8(rke, (int)(p - ke0), 0, CPOL_SC1);
  }
  __device__ __forceinline__ int ve1(const int8_t *p) const {
    return (int)(signed char)__builtin_amdgcn_raw_buffer_load_b8(rve, (int)(p - ve0), 0, CPOL_SC1);
  }
  // loads of rows that may lie past the position (live false): those go to
  // an offset past the buffer's end (kDead >= the descriptors' 0x7fffffff
  // bytes), where a buffer load returns zeros without a memory request --
  // device-coherent loads are not cached, and the clamped row the callers
  // name would cost as much as a live one
  static constexpr int kDead = (int)0x80000000u;
  __device__ __forceinline__ uint4 k16l(const int16_t *p, bool live) const {
    return ld_b128<CPOL_SC1>(rkm, live ? (int)(p - km0) * 2 : kDead);
  }
  __device__ __forceinline__ int ke4l(const int8_t *p, bool live) const {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(rke, live ? (int)(p - ke0) : kDead, 0, CPOL_SC1);
  }
  __device__ __forceinline__ uint4 v16l(const int16_t *p, bool live) const {
    return ld_b128<CPOL_SC1>(rvm, live ? (int)(p - vm0) * 2 : kDead);
  }
  __device__ __forceinline__ int ve1l(const int8_t *p, bool live) const {
    return (int)(signed char)__builtin_amdgcn_raw_buffer_load_b8(rve, live ? (int)(p - ve0) : kDead, 0, CPOL_SC1);
  }
  __device__ __forceinline__ void k_put(int16_t *pm, int8_t *pe, int m, int e, bool we) const {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)m, rkm, (int)(pm - km0) * 2, 0, CPOL_SC1);
    if (we) __builtin_amdgcn_raw_buffer_store_b8((unsigned char)e, rke, (int)(pe - ke0), 0, CPOL_SC1);
  }
  __device__ __forceinline__ void v_put(int16_t *pm, int8_t *pe, int m, int e, bool we) const {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)m, rvm, (int)(pm - vm0) * 2, 0, CPOL_SC1);
    if (we) __builtin_amdgcn_raw_buffer_store_b8((unsigned char)e, rve, (int)(pe - ve0), 0, CPOL_SC1);
  }
  // the cache row's stores complete (vmcnt 0 in the waves that made them)
  // before any wave stores the output
  __device__ __forceinline__ void before_out() const {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    lds_barrier();
  }
  __device__ __forceinline__ void out(int idx, int m, int e, bool) const { st_coh(ro, 4 * idx, tagged(m, e, tag)); }
  // row u of workgroup dg's block (its position ATT_DSPLIT u + dg): bits
  // 16k .. 16k+15 of the score in word k, with the (step, layer) tag
  __device__ __forceinline__ int sc_off(int hq, int dg, int u) const { return 16 * (hq * sc_stride + dg * sc_block + u); }
  __device__ __forceinline__ void score_put(int hq, int dg, int u, double v) const {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned tg = tag << 24;
    v4u x;
    x.x = (unsigned)(b & 0xffffu) | tg;
    x.y = (unsigned)((b >> 16) & 0xffffu) | tg;
    x.z = (unsigned)((b >> 32) & 0xffffu) | tg;
    x.w = (unsigned)((b >> 48) & 0xffffu) | tg;
    __builtin_amdgcn_raw_buffer_store_b128(x, rsc, sc_off(hq, dg, u), 0, CPOL_SC1);
  }
  // a first read of the entry (issued with the others before any is used),
  // then its value, waiting (bounded) while its words carry another tag
  __device__ __forceinline__ uint4 score_raw(int hq, int dg, int u) const {
    return ld_b128<CPOL_SC1>(rsc, sc_off(hq, dg, u));
  }
  __device__ __forceinline__ double score_val(uint4 v, int hq, int dg, int u) const {
    if (!Wait::ok4(v, tag)) v = w->quad(rsc, sc_off(hq, dg, u), tag);
    const unsigned long long b = (unsigned long long)(v.x & 0xffffu) | ((unsigned long long)(v.y & 0xffffu) << 16) |
                                 ((unsigned long long)(v.z & 0xffffu) << 32) |
                                 ((unsigned long long)(v.w & 0xffffu) << 48);
    return __longlong_as_double((long long)b);
  }
};

// Role entry: the argument block (device memory) as scalars, the wait
// state in registers, the dynamic LDS as LDS.
#define PT_ENTER()                                  \
  pp = uniform_ptr(pp);                             \
  const PersistArgs p = cload(pp);                  \
  Wait w{rsrc(p.abort_flag, 4), false};             \
  dsm = lds(dsm);                                   \
  const PT_CONST LayerArgs *L = (const PT_CONST LayerArgs *)p.L

// ------------------------------------------------------------------ head
// Step s's head on this workgroup's slice of the vocabulary, then the
// argmax over every slice (full.py:438-440; first index on ties).  Every
// workgroup returns the same token.
__device__ __forceinline__ int persist_head(const PersistArgs &p, int s, double *dsm, Wait &w) {
  const int D = p.D, G = gridDim.x, g = blockIdx.x, tid = threadIdx.x;
  const int l16 = tid & 15, sub = tid >> 4, slots = PT_THREADS / 16;
  const int r0 = (int)((long long)g * p.VOCAB / G), r1 = (int)((long long)(g + 1) * p.VOCAB / G);
  const int nrows = r1 - r0, d64 = D / 64;
  double *work = dsm;                       // 3*D: final norm, then hn (aliases its start)
  double *leaf = dsm + 3 * D;
  int16_t *hm = reinterpret_cast<int16_t *>(leaf + PW_MAX_LEAVES);
  int8_t *he = reinterpret_cast<int8_t *>(hm + D);
  __shared__ double bv[PT_NW];
  __shared__ int bi[PT_NW];
  const rsrc_t re = rsrc(p.embed + (long long)r0 * D, nrows * D * 4);
  float4 cur[PT_HEAD_D64], nxt[PT_HEAD_D64];
  auto load_rows = [&](int rr, float4 (&f)[PT_HEAD_D64]) {
    rr = rr < nrows ? rr : nrows - 1;       // past the slice: re-read its last row
#pragma unroll
    for (int i = 0; i < PT_HEAD_D64; ++i) {
      const uint4 u = ld_b128<CPOL_NT>(re, (rr * D + ((i < d64 ? i : d64 - 1) * 16 + l16) * 4) * 4);
      f[i] = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                         __uint_as_float(u.w));
    }
  };
  load_rows(sub, cur);                      // in flight while h arrives
  const unsigned tg = tag_of(s, p.NL - 1, p.NL);
  wait_bfp(w, rsrc(p.t_h + (s & 1) * D), D, tg, hm, he);
  lds_barrier();
  stamp_head(p, s, 0);
  final_norm(hm, he, p.norm_w, D, work, leaf, work);
  lds_barrier();
  double best = -INFINITY;
  int besti = 0x7fffffff;
  for (int rr = sub; rr < nrows; rr += slots) {
    load_rows(rr + slots, nxt);
    const double acc = head_row_dot<PT_HEAD_D64, false>(cur, work, l16, d64);
#pragma unroll
    for (int i = 0; i < PT_HEAD_D64; ++i) cur[i] = nxt[i];
    const int row = r0 + rr;
    if (acc > best || (acc == best && row < besti)) {
      best = acc;
      besti = row;
    }
  }
  argmax_step<16>(best, besti);
  argmax_step<32>(best, besti);
  if ((tid & 63) == 0) {
    bv[tid >> 6] = best;
    bi[tid >> 6] = besti;
  }
  lds_barrier();
  const unsigned ptag = (unsigned)(s % 255) + 1u;
  const rsrc_t rp = rsrc(p.t_part + (size_t)(s & 1) * G * 4);
  if (tid == 0) {
    for (int k = 1; k < PT_NW; ++k)
      if (bv[k] > best || (bv[k] == best && bi[k] < besti)) {
        best = bv[k];
        besti = bi[k];
      }
    const unsigned long long u = (unsigned long long)__double_as_longlong(best);
    st_coh(rp, 16 * g, (unsigned)(u & 0xffffffu) | (ptag << 24));
    st_coh(rp, 16 * g + 4, (unsigned)((u >> 24) & 0xffffffu) | (ptag << 24));
    st_coh(rp, 16 * g + 8, (unsigned)(u >> 48) | (ptag << 24));
    st_coh(rp, 16 * g + 12, ((unsigned)besti & 0xffffffu) | (ptag << 24));
  }
  stamp_head(p, s, 1);
  // every slice's (value, index): one per thread
  best = -INFINITY;
  besti = 0x7fffffff;
  if (tid < G) {
    const uint4 v = w.quad(rp, tid * 16, ptag);
    const unsigned long long u = (unsigned long long)(v.x & 0xffffffu) |
                                 ((unsigned long long)(v.y & 0xffffffu) << 24) |
                                 ((unsigned long long)(v.z & 0xffffu) << 48);
    best = __longlong_as_double((long long)u);
    besti = (int)(v.w & 0xffffffu);
  }
  argmax_step<1>(best, besti);
  argmax_step<2>(best, besti);
  argmax_step<4>(best, besti);
  argmax_step<8>(best, besti);
  argmax_step<16>(best, besti);
  argmax_step<32>(best, besti);
  lds_barrier();   // bv/bi reuse
  if ((tid & 63) == 0) {
    bv[tid >> 6] = best;
    bi[tid >> 6] = besti;
  }
  lds_barrier();
  best = bv[0];
  besti = bi[0];
  for (int k = 1; k < PT_NW; ++k)
    if (bv[k] > best || (bv[k] == best && bi[k] < besti)) {
      best = bv[k];
      besti = bi[k];
    }
  lds_barrier();   // bv/bi and the LDS work space are reused by the next step
  stamp_head(p, s, 2);
  return besti;
}

// After step s: the head (when the loop evaluates it), the record of its
// argmax (workgroup 0) and the next step's input token.
__device__ __forceinline__ int end_of_step(const PersistArgs &p, int s, double *dsm, Wait &w) {
  const bool head = p.rtl_loop || s >= p.n_prompt - 1;
  int nid = -1;
  if (head) nid = persist_head(p, s, dsm, w);
  if (head && blockIdx.x == 0 && threadIdx.x == 0) {
    p.last[0] = nid;
    const int k = ctl_out_slot(s, p.n_prompt, p.n_gen, p.rtl_loop);
    if (k >= 0) p.out[k] = nid;
  }
  return ctl_next(s, nid, p.n_prompt, p.prompt, p.rtl_loop);
}

// ------------------------------------------------------------------ roles
// Q|K|V chunk c (and attention job c when c < n_att).
template <int PPW, bool SHORT>
__device__ void role_qkv(const PT_CONST PersistArgs *pp, double *dsm, int c) {
  PT_ENTER();
  c = uniform_int(c);
  const int D = p.D, nT = D / 16, nq = D + 2 * p.KV;
  // the step's RoPE row (HD/2 x (cos, sin)) for the attention, in LDS ahead
  // of the norm and attention work space
  double *rope_s = dsm;
  dsm += 64;
  double *dbuf = dsm;
  double *leaf = dsm + 3 * D;
  int *xs = reinterpret_cast<int *>(leaf + PW_MAX_LEAVES);
  int *xes = xs + nT * 16;
  int16_t *hm = reinterpret_cast<int16_t *>(xes + nT);
  int8_t *he = reinterpret_cast<int8_t *>(hm + D);
  __shared__ int redM[PT_NW * 16];
  __shared__ long long redA[PT_NW * 16];
  ChunkRegs<2> R;
  Gammas G1;
  load_chunk_rs(R, L[0].w_qkv_m + (long long)c * nT * 32, L[0].w_qkv_e + (long long)c * nT * 16, nT);
  load_gammas(G1, L[0].g1, D);
  int tok = clamp_tok(p, p.prompt[0]);
  for (int s = 0; s < p.steps; ++s) {
    if (c == 0 && threadIdx.x == 0 && p.clock) put_clock(p.clock, s);
    const rsrc_t rq = rsrc(p.t_qkv + (s & 1) * nq);
    for (int l = 0; l < p.NL; ++l) {
      LayerArgs a = cload(L + l);
      const unsigned tg = tag_of(s, l, p.NL);
      double rope_v = 0.0;   // loaded now, stored to LDS before the attention
      if (c < p.n_att && threadIdx.x < 64) rope_v = a.rope[(long long)s * 64 + threadIdx.x];
      if (l == 0)
        embed_vec(p, tok, hm, he);
      else
        wait_bfp(w, rsrc(p.t_h + (s & 1) * D), D, tag_of(s, l - 1, p.NL), hm, he);
      lds_barrier();
      stamp(p, c == 0, s, l, 0);
      rmsnorm_pairs_to_x(hm, he, G1.v[0], G1.v[1], D, xs, xes, dbuf + D, leaf);
      lds_barrier();
      stamp(p, c == 0, s, l, 10);
      long long A;
      int M;
      chunk_AM<PT_NW, 2>(R, xs, xes, nT, redM, redA, A, M);
      stamp(p, c == 0, s, l, 11);
      if (threadIdx.x < 64) {
        int m, e;
        chunk_quant(A, M, m, e);
        if (threadIdx.x < 16) st_coh(rq, 4 * (c * 16 + threadIdx.x), tagged(m, e, tg));
      }
      stamp(p, c == 0, s, l, 1);
      if (c < p.n_att) {
        if (threadIdx.x < 64) rope_s[threadIdx.x] = rope_v;
        a.rope_row = rope_s;
        lds_barrier();   // the attention reuses the LDS
        AttnCohIO io;
        io.rq = rq;
        io.ro = rsrc(p.t_att + (s & 1) * D);
        io.tag = tg;
        io.w = &w;
        io.km0 = a.k_m;
        io.ke0 = a.k_e;
        io.vm0 = a.v_m;
        io.ve0 = a.v_e;
        io.rkm = rsrc(a.k_m);
        io.rke = rsrc(a.k_e);
        io.rvm = rsrc(a.v_m);
        io.rve = rsrc(a.v_e);
        io.rsc = rsrc(p.sc_buf);
        io.sc_stride = attn_sc_stride(a.max_ctx);
        io.sc_block = attn_sc_block(a.max_ctx);
        io.rope_s = rope_s;
        io.trace = (p.trace && c == 0) ? p.trace + ((size_t)s * p.NL + l) * PT_TRACE_LAYER : nullptr;
        attn_body<PPW, SHORT>(a, io, c, 0, [s] { return make_int2(s, s); }, dsm);
        stamp(p, c == 0, s, l, 3);
      }
      const int ln = l + 1 < p.NL ? l + 1 : 0;
      load_chunk_rs(R, L[ln].w_qkv_m + (long long)c * nT * 32, L[ln].w_qkv_e + (long long)c * nT * 16, nT);
      load_gammas(G1, L[ln].g1, D);
      lds_barrier();
    }
    tok = clamp_tok(p, end_of_step(p, s, dsm, w));
  }
  if (c == 0 && threadIdx.x == 0 && p.clock) put_clock(p.clock, p.steps);
}

// O chunk c: h1 = q(h + Wo att).
__device__ void role_o(const PT_CONST PersistArgs *pp, double *dsm, int c) {
  PT_ENTER();
  c = uniform_int(c);
  const int D = p.D, nT = D / 16;
  int *xs = reinterpret_cast<int *>(dsm);
  int *xes = xs + nT * 16;
  __shared__ int redM[PT_NW * 16];
  __shared__ long long redA[PT_NW * 16];
  ChunkRegs<2> R;
  load_chunk_rs(R, L[0].w_o_m + (long long)c * nT * 32, L[0].w_o_e + (long long)c * nT * 16, nT);
  int tok = clamp_tok(p, p.prompt[0]);
  for (int s = 0; s < p.steps; ++s) {
    const rsrc_t rh = rsrc(p.t_h + (s & 1) * D), ra = rsrc(p.t_att + (s & 1) * D);
    const rsrc_t r1 = rsrc(p.t_h1 + (s & 1) * D);
    for (int l = 0; l < p.NL; ++l) {
      const unsigned tg = tag_of(s, l, p.NL);
      int rm = 0, re = 0;
      if (threadIdx.x < 64) {   // this lane's row of h, the residual
        if (l == 0) {
          embed_tile(p, tok, c, rm, re);
        } else {
          const unsigned v = w.word(rh, 4 * (c * 16 + (threadIdx.x & 15)), tag_of(s, l - 1, p.NL));
          rm = tw_m(v);
          re = tw_e(v);
        }
      }
      wait_x(w, ra, D, tg, xs, xes);
      lds_barrier();
      stamp(p, c == 0, s, l, 4);
      long long A;
      int M;
      chunk_AM<PT_NW, 2>(R, xs, xes, nT, redM, redA, A, M);
      stamp(p, c == 0, s, l, 15);
      if (threadIdx.x < 64) {
        int om, oe, e;
        chunk_quant(A, M, om, oe);
        const int m = residual_lane(om, oe, rm, re, e);
        if (threadIdx.x < 16) st_coh(r1, 4 * (c * 16 + threadIdx.x), tagged(m, e, tg));
      }
      stamp(p, c == 0, s, l, 5);
      const int ln = l + 1 < p.NL ? l + 1 : 0;
      load_chunk_rs(R, L[ln].w_o_m + (long long)c * nT * 32, L[ln].w_o_e + (long long)c * nT * 16, nT);
      lds_barrier();
    }
    tok = clamp_tok(p, end_of_step(p, s, dsm, w));
  }
}

// G/U chunks (2c, 2c+1): mlp = q(q(silu(g)) * u) of n2 = rmsnorm(h1, g2).
__device__ void role_gu(const PT_CONST PersistArgs *pp, double *dsm, int c) {
  PT_ENTER();
  c = uniform_int(c);
  const int D = p.D, nT = D / 16;
  double *dbuf = dsm;
  double *leaf = dsm + 3 * D;
  int *xs = reinterpret_cast<int *>(leaf + PW_MAX_LEAVES);
  int *xes = xs + nT * 16;
  int16_t *hm = reinterpret_cast<int16_t *>(xes + nT);
  int8_t *he = reinterpret_cast<int8_t *>(hm + D);
  __shared__ int redM[2 * PT_NW * 16];        // G and U
  __shared__ long long redA[2 * PT_NW * 16];
  ChunkRegs<2> RG, RU;
  Gammas G2;
  auto load_w = [&](int l) {
    load_gammas(G2, L[l].g2, D);
    load_chunk_rs(RG, L[l].w_gu_m + (long long)(2 * c) * nT * 32, L[l].w_gu_e + (long long)(2 * c) * nT * 16, nT);
    load_chunk_rs(RU, L[l].w_gu_m + (long long)(2 * c + 1) * nT * 32,
                  L[l].w_gu_e + (long long)(2 * c + 1) * nT * 16, nT);
  };
  load_w(0);
  for (int s = 0; s < p.steps; ++s) {
    const rsrc_t r1 = rsrc(p.t_h1 + (s & 1) * D), rmlp = rsrc(p.t_mlp + (s & 1) * p.FFN);
    for (int l = 0; l < p.NL; ++l) {
      const unsigned tg = tag_of(s, l, p.NL);
      wait_bfp(w, r1, D, tg, hm, he);
      lds_barrier();
      stamp(p, c == 0, s, l, 6);
      rmsnorm_pairs_to_x(hm, he, G2.v[0], G2.v[1], D, xs, xes, dbuf + D, leaf);
      lds_barrier();
      stamp(p, c == 0, s, l, 12);
      long long Ag, Au;
      int Mg, Mu;
      chunk_AM2<PT_NW, 2>(RG, RU, xs, xes, nT, redM, redA, Ag, Mg, Au, Mu);
      stamp(p, c == 0, s, l, 13);
      if (threadIdx.x < 64) {
        int gm, ge, um, ue, me;
        chunk_quant(Ag, Mg, gm, ge);
        chunk_quant(Au, Mu, um, ue);
        const int mm = swiglu_lane(gm, ge, um, ue, me);
        if (threadIdx.x < 16) st_coh(rmlp, 4 * (c * 16 + threadIdx.x), tagged(mm, me, tg));
      }
      stamp(p, c == 0, s, l, 7);
      load_w(l + 1 < p.NL ? l + 1 : 0);
      lds_barrier();
    }
    (void)end_of_step(p, s, dsm, w);
  }
}

// D chunk c: h = q(h1 + Wd mlp), the layer's output (and its history row).
__device__ void role_d(const PT_CONST PersistArgs *pp, double *dsm, int c) {
  PT_ENTER();
  c = uniform_int(c);
  const int D = p.D, nT = p.FFN / 16;
  int *xs = reinterpret_cast<int *>(dsm);
  int *xes = xs + nT * 16;
  __shared__ int redM[PT_NW * 16];
  __shared__ long long redA[PT_NW * 16];
  ChunkRegs<3> R;
  load_chunk_rs(R, L[0].w_d_m + (long long)c * nT * 32, L[0].w_d_e + (long long)c * nT * 16, nT);
  for (int s = 0; s < p.steps; ++s) {
    const rsrc_t r1 = rsrc(p.t_h1 + (s & 1) * D), rmlp = rsrc(p.t_mlp + (s & 1) * p.FFN);
    const rsrc_t rh = rsrc(p.t_h + (s & 1) * D);
    for (int l = 0; l < p.NL; ++l) {
      const unsigned tg = tag_of(s, l, p.NL);
      int rm = 0, re = 0;
      if (threadIdx.x < 64) {   // this lane's row of h1, the residual
        const unsigned v = w.word(r1, 4 * (c * 16 + (threadIdx.x & 15)), tg);
        rm = tw_m(v);
        re = tw_e(v);
      }
      wait_x(w, rmlp, p.FFN, tg, xs, xes);
      lds_barrier();
      stamp(p, c == 0, s, l, 8);
      long long A;
      int M;
      chunk_AM<PT_NW, 3>(R, xs, xes, nT, redM, redA, A, M);
      stamp(p, c == 0, s, l, 14);
      if (threadIdx.x < 64) {
        const int r = threadIdx.x & 15;
        int dm, de, e;
        chunk_quant(A, M, dm, de);
        const int m = residual_lane(dm, de, rm, re, e);
        if (threadIdx.x < 16) st_coh(rh, 4 * (c * 16 + r), tagged(m, e, tg));
        if (p.hist_m) {
          int chm = m, che = e;
          canon16_lanes(chm, che);
          if (threadIdx.x < 16 && s < p.hist_steps) {
            const long long o = ((long long)s * p.NL + l) * D;
            p.hist_m[o + c * 16 + r] = (int16_t)chm;
            if (r == 0) p.hist_e[(o >> 4) + c] = (int8_t)che;
          }
        }
      }
      stamp(p, c == 0, s, l, 9);
      const int ln = l + 1 < p.NL ? l + 1 : 0;
      load_chunk_rs(R, L[ln].w_d_m + (long long)c * nT * 32, L[ln].w_d_e + (long long)c * nT * 16, nT);
      lds_barrier();
    }
    (void)end_of_step(p, s, dsm, w);
  }
}

// Workgroups past the layer roles: the head only.
__device__ void role_head_only(const PT_CONST PersistArgs *pp, double *dsm) {
  PT_ENTER();
  (void)L;
  for (int s = 0; s < p.steps; ++s) (void)end_of_step(p, s, dsm, w);
}

// gp: the argument block in device memory (a global address, so it can be
// read through the constant address space; the kernel's own by-value
// arguments may be copied to private memory).
template <int PPW, bool SHORT>
__global__ __launch_bounds__(PT_THREADS, 1) void k_decode_persist(const PersistArgs *gp) {
  extern __shared__ double dsm[];
  const PT_CONST PersistArgs *pp = (const PT_CONST PersistArgs *)gp;
  const PersistArgs p = cload(pp);
  const int g = blockIdx.x;
  if (g < p.n_qkv) {
    role_qkv<PPW, SHORT>(pp, dsm, g);
  } else if (g < p.g0) {
    role_o(pp, dsm, g - p.o0);
  } else if (g < p.d0) {
    role_gu(pp, dsm, g - p.g0);
  } else if (g < p.d0 + p.n_d) {
    role_d(pp, dsm, g - p.d0);
  } else {
    role_head_only(pp, dsm);
  }
}

// ------------------------------------------------------------------- host
typedef void (*pk_fn)(const PersistArgs *);

static pk_fn persist_kernel(int ppw) {
  return ppw == 2 ? k_decode_persist<2, true>
                  : (ppw == 3 ? k_decode_persist<3, true>
                              : (ppw == 4 ? k_decode_persist<4, true> : k_decode_persist<8, false>));
}

static size_t persist_lds(const PersistArgs &p, int max_ctx) {
  const int D = p.D, nT = D / 16, nTF = p.FFN / 16;
  const size_t norm = (size_t)(3 * D + PW_MAX_LEAVES) * 8 + (size_t)nT * 17 * 4 + (size_t)D * 2 + nT;
  const size_t dx = (size_t)nTF * 17 * 4;
  const size_t head = (size_t)(3 * D + PW_MAX_LEAVES) * 8 + (size_t)D * 2 + nT;
  // the Q|K|V role keeps the step's RoPE row (64 doubles) ahead of both its
  // norm work space and the attention's
  size_t lds = attn_lds_bytes(max_ctx, attn_ppw(max_ctx), AttnCohIO::kAvBlock, AttnCohIO::kSplitScores) + 64 * 8;
  lds = lds > norm + 64 * 8 ? lds : norm + 64 * 8;
  lds = lds > dx ? lds : dx;
  lds = lds > head ? lds : head;
  return (lds + 15) & ~(size_t)15;
}

int persist_plan(const bfp_dims &d, int max_ctx, int device, PersistArgs &p, int &grid) {
  int cus = 0;
  HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  const int nq = (d.D + 2 * d.H_KV * d.HD) / 16, no = d.D / 16, ngu = d.FFN / 16, nd = d.D / 16;
  const int ppw = attn_ppw(max_ctx);
  const int natt = ppw == 8 ? d.H_Q * ATT_DSPLIT : d.H_Q;
  if (d.HD != 64 || d.D > 576 || d.D % 64 || d.FFN > 1536 || d.NL < 2 || (d.NL + 1) % 255 == 0 ||
      d.VOCAB >= (1 << 24) || d.VOCAB < cus || natt > nq || nq + no + ngu + nd > cus || cus > PT_THREADS)
    return 0;
  p.D = d.D;
  p.FFN = d.FFN;
  p.KV = d.H_KV * d.HD;
  p.NL = d.NL;
  p.VOCAB = d.VOCAB;
  p.n_qkv = nq;
  p.n_att = natt;
  p.o0 = nq;
  p.g0 = nq + no;
  p.d0 = nq + no + ngu;
  p.n_d = nd;
  grid = cus;
  return 1;
}

int launch_decode_persist(const PersistArgs &p, PersistArgs *dev_args, int grid, int max_ctx,
                          hipStream_t s) {
  const pk_fn f = persist_kernel(attn_ppw(max_ctx));
  const size_t lds = persist_lds(p, max_ctx);
  BFP_TRY(raise_lds_limit(reinterpret_cast<const void *>(f), (int)lds));
  int nb = 0;
  HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(f), PT_THREADS, lds));
  if (nb < 1) return set_err(BFP_EINVAL, "persistent decode: %zu bytes of LDS do not fit a compute unit", lds);
  HIP_TRY(hipMemcpyAsync(dev_args, &p, sizeof p, hipMemcpyHostToDevice, s));
  HIP_TRY(hipStreamSynchronize(s));   // p is the caller's stack copy
  // grid = the compute units (persist_plan) and nb >= 1: every workgroup
  // is resident at once
  hipLaunchKernelGGL(f, dim3(grid), dim3(PT_THREADS), lds, s, dev_args);
  return launch_status("persistent decode");
}

}  // namespace bfp
