// Model context: HBM-resident BFP weights and KV cache, the layer step and the
// autoregressive decode driver (rtl/vc707/host/gen_smollm_blockfp_full.py
// :411-443), replayed step by step as HIP graphs.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <vector>

#include "bfp.h"
#include "bfp_internal.h"
#include "bfp_layer.h"
#include "bfp_mx.h"
#include "bfp_persist.h"
#include "bfp_pipe.h"

using namespace bfp;

// The copy of the embedding the batched head reads, permuted within each
// row of D = 64 NB columns: vp[row][(4i + c) * 16 + 4h + j] =
// v[row][64i + 4(h + 4j) + c] (partials h, h + 4, h + 8, h + 12 of block i,
// k-index c, contiguous).
__global__ void permute_embed_kernel(const float *__restrict__ v, long long n, int D,
                                     float *__restrict__ vp) {
  const long long q = blockIdx.x * (long long)blockDim.x + threadIdx.x;   // destination index
  if (q >= n) return;
  const long long row = q / D;
  const int jj = (int)(q - row * D);
  const int j = jj & 3, h = (jj >> 2) & 3, c = (jj >> 4) & 3, i = jj >> 6;
  vp[q] = v[row * D + 64 * i + 4 * (h + 4 * j) + c];
}

// Two word-granular copies in one launch (n0, n1 32-bit words): the
// single-layer boundary call's input from pinned host memory into the
// device activations, and its output back.
__global__ void copy_words2_kernel(const unsigned *__restrict__ s0, unsigned *__restrict__ d0, int n0,
                                   const unsigned *__restrict__ s1, unsigned *__restrict__ d1, int n1) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n0 + n1; i += gridDim.x * blockDim.x) {
    if (i < n0) d0[i] = s0[i];
    else d1[i - n0] = s1[i - n0];
  }
}

struct bfp_ctx {
  bfp_dims d{};
  int device = 0, max_batch = 1, max_ctx = 0;
  hipStream_t stream = nullptr;
  // weights (device layout); per layer at base + layer * stride
  uint8_t *qkv_m = nullptr, *o_m = nullptr, *gu_m = nullptr, *d_m = nullptr;
  int8_t *qkv_e = nullptr, *o_e = nullptr, *gu_e = nullptr, *d_e = nullptr;
  size_t s_qkv_m = 0, s_o_m = 0, s_gu_m = 0, s_d_m = 0;
  size_t s_qkv_e = 0, s_o_e = 0, s_gu_e = 0, s_d_e = 0;
  double *g1 = nullptr, *g2 = nullptr, *norm_w = nullptr, *rope = nullptr;
  double *rope_row = nullptr;   // one (cos, sin) row for a position past the table
  float *embed = nullptr;
  float *embedp = nullptr;     // the embedding permuted per row for the batched head
                               // (made when max_batch >= HEAD_SEQ_MIN)
  // the bounded head (made with embedp): the embedding as split int16 with
  // per-row meta, and per step the quantised hidden, its per-sequence
  // record and the per-block bounds
  uint4 *embq = nullptr, *hq_x = nullptr;
  HeadQRow *embq_meta = nullptr;
  HeadQSeq *hq_seq = nullptr;
  double2 *hq_blk = nullptr;
  // activations (max_batch sequences)
  int16_t *h_m = nullptr, *h1_m = nullptr, *qkv_am = nullptr, *att_m = nullptr, *mlp_m = nullptr;
  int8_t *h_e = nullptr, *h1_e = nullptr, *qkv_ae = nullptr, *att_e = nullptr, *mlp_e = nullptr;
  int16_t *xn_m = nullptr;   // RMSNorm output, multi-sequence layer path
  int8_t *xn_e = nullptr;
  double *hn = nullptr;      // normed final hidden, batch > 1 head
  // KV cache: NL x max_batch x max_ctx x KV
  int16_t *k_m = nullptr, *v_m = nullptr;
  int8_t *k_e = nullptr, *v_e = nullptr;
  size_t s_kv_m = 0, s_kv_e = 0;   // per layer
  // head / driver state
  int head_wg = 0, head_rows = 0;
  double *part_v = nullptr;
  int *part_i = nullptr, *state = nullptr, *last = nullptr;
  unsigned *t_h1 = nullptr, *t_h = nullptr;   // batched decode: h1, h as tagged words (max_batch x D)
  unsigned *t_qkv = nullptr;   // batched decode: q|k|v as tagged words (max_batch x (D + 2KV))
  int *t_abort = nullptr;    // set by a tagged wait that gave up
  StageDump *dump_dev = nullptr;
  // engine tables of the composed RTL layer, made on its first use
  uint16_t *rtl_exp = nullptr;
  int16_t *rtl_silu = nullptr;
  unsigned *rtl_freq = nullptr;
  // the RTL decode head's buffers, made on its first use
  uint4 *rtl_emb_m = nullptr;
  int8_t *rtl_emb_e = nullptr, *rtl_lg_e = nullptr, *rtl_xn_e = nullptr;
  int16_t *rtl_lg_m = nullptr, *rtl_xn_m = nullptr;
  int *rtl_work = nullptr, *rtl_tok = nullptr;
  // the persistent decode's tagged hand-off words, per-layer argument blocks
  // and step clock, made on its first use
  unsigned *pt_words = nullptr;
  size_t pt_nwords = 0;
  LayerArgs *pt_layers = nullptr;
  PersistArgs *pt_args = nullptr;
  unsigned long long *pt_clock = nullptr;
  unsigned *pt_scores = nullptr;   // the long attention form's score exchange (tagged words)
  // the pipelined batched step (bfp_pipe.hip), made on its first use: its
  // tagged hand-off words, the layer blocks, the argument block, and one
  // schedule per batch size
  unsigned *pp_words = nullptr;
  size_t pp_nwords = 0;
  LayerArgs *pp_layers = nullptr;
  PipeArgs *pp_args = nullptr;
  struct PipeSched {
    PipePlan pl;
    int *role = nullptr, *jstart = nullptr, *jobs = nullptr;
    bool ok = false;
  };
  std::vector<PipeSched> pp_sched;   // by batch size (index batch - 1)
  std::vector<void *> allocs;
  // pinned, mapped host memory through which the single-layer boundary call
  // (bfp_layer_step_kv) passes its input and output, read and written by
  // copy kernels on the stream (made on first use)
  uint8_t *pin = nullptr, *pin_dev = nullptr;
  size_t pin_bytes = 0;
  int last_path = -1;   // BFP_PATH_* of the last decode
  int last_form = -1;   // BFP_FORM_* of the last decode
  float last_decode_ms = 0.f, last_gen_ms = 0.f;
  std::vector<float> step_ms;   // per-step device time of the last decode (BFP_DECODE_STEP_TIMES)
  std::vector<unsigned long long> trace;   // stage stamps of the last traced persistent decode

  int alloc(void **p, size_t bytes) {
    *p = nullptr;
    hipError_t e = hipMalloc(p, bytes ? bytes : 16);
    if (e != hipSuccess) {
      *p = nullptr;
      return set_err(BFP_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    allocs.push_back(*p);
    return BFP_OK;
  }
  // Fine-grained device memory: device-coherent (SC1) accesses to it are
  // faster than to ordinary allocations (a cross-XCD hand-off measured
  // 396 ns one way against 580 ns).
  int alloc_fine(void **p, size_t bytes) {
    *p = nullptr;
    hipError_t e = hipExtMallocWithFlags(p, bytes ? bytes : 16, hipDeviceMallocFinegrained);
    if (e != hipSuccess) {
      *p = nullptr;
      return set_err(BFP_ENOMEM, "hipExtMallocWithFlags(%zu, fine-grained): %s", bytes,
                     hipGetErrorString(e));
    }
    allocs.push_back(*p);
    return BFP_OK;
  }
  int pinned(size_t bytes) {
    if (bytes <= pin_bytes) return BFP_OK;
    if (pin) {
      HIP_TRY(hipStreamSynchronize(stream));
      (void)hipHostFree(pin);
      pin = pin_dev = nullptr;
      pin_bytes = 0;
    }
    void *p = nullptr, *dp = nullptr;
    hipError_t e = hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocCoherent);
    if (e != hipSuccess) return set_err(BFP_ENOMEM, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
    e = hipHostGetDevicePointer(&dp, p, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(p);
      return set_err(BFP_EIO, "hipHostGetDevicePointer: %s", hipGetErrorString(e));
    }
    pin = static_cast<uint8_t *>(p);
    pin_dev = static_cast<uint8_t *>(dp);
    pin_bytes = bytes;
    return BFP_OK;
  }
  ~bfp_ctx() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (pin) (void)hipHostFree(pin);
    for (void *p : allocs) (void)hipFree(p);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace {

int check_dims(const bfp_dims &d) {
  if (d.D <= 0 || d.H_Q <= 0 || d.H_KV <= 0 || d.HD <= 0 || d.FFN <= 0 || d.NL <= 0 ||
      d.MAX_CTX <= 0 || d.VOCAB <= 0)
    return set_err(BFP_EINVAL, "dims must be positive");
  if (d.HD != 64) return set_err(BFP_EINVAL, "HD=%d: the attention kernel is built for HD=64", d.HD);
  if (d.H_Q % d.H_KV) return set_err(BFP_EINVAL, "H_Q=%d not a multiple of H_KV=%d", d.H_Q, d.H_KV);
  if (d.H_Q * d.HD != d.D) return set_err(BFP_EINVAL, "H_Q*HD=%d != D=%d", d.H_Q * d.HD, d.D);
  if (d.D % 64 || d.D < 64 || d.D > 1728)
    return set_err(BFP_EINVAL, "D=%d must be a multiple of 64 in [64, 1728]", d.D);
  if (d.FFN % 16 || d.FFN < 64 || d.FFN > 1728)
    return set_err(BFP_EINVAL, "FFN=%d must be a multiple of 16 in [64, 1728]", d.FFN);
  if (d.VOCAB % 16) return set_err(BFP_EINVAL, "VOCAB=%d not a multiple of 16", d.VOCAB);
  if (d.MAX_CTX > 4096) return set_err(BFP_EINVAL, "MAX_CTX=%d > 4096", d.MAX_CTX);
  return BFP_OK;
}

// RoPE table of positions 0 .. max_ctx-1 with the reference's own float
// expressions (full.py:253-254, rope_row).
void rope_table(std::vector<double> &t, int max_ctx, int HD) {
  t.resize((size_t)max_ctx * HD);
  for (int pos = 0; pos < max_ctx; ++pos) rope_row(t.data() + (size_t)pos * HD, pos, HD, 10000.0);
}

// Workgroups of the head for `batch` sequences, and the most any batch uses.
int head_nwg(const bfp_ctx *c, int batch) {
  return head_workgroups(c->d.VOCAB, c->d.D, c->head_rows, batch, c->embedp != nullptr);
}
int head_part_max(const bfp_ctx *c) {
  int m = 0;
  for (int b : {1, 2, c->max_batch}) m = std::max(m, head_nwg(c, b));
  return m;
}

// The bounded head (argmax only) where its copy exists, no logits are asked
// for and the batch takes the float64 matrix-core form; BFP_HEAD_BOUNDED=0
// keeps k_head_mx.
bool head_bounded(const bfp_ctx *c, int batch, const double *logits) {
  const char *v = getenv("BFP_HEAD_BOUNDED");
  return c->embq && !logits && head_seq_form(c->d.D, batch, c->embedp != nullptr) && !(v && atoi(v) == 0);
}

HeadArgs head_args(bfp_ctx *c, int batch, double *logits) {
  const bfp_dims &d = c->d;
  const bool bq = head_bounded(c, batch, logits);
  HeadArgs ha{d.D, d.VOCAB, batch, c->head_rows, bq ? 1 : head_nwg(c, batch), c->h_m, c->h_e, c->norm_w,
              c->embed, c->part_v, c->part_i, logits, c->hn, c->embedp};
  if (bq) {
    ha.embq = c->embq;
    ha.embq_meta = c->embq_meta;
    ha.hq_x = c->hq_x;
    ha.hq_seq = c->hq_seq;
    ha.hq_blk = c->hq_blk;
  }
  return ha;
}

LayerArgs layer_args(bfp_ctx *c, int layer, int batch) {
  const bfp_dims &d = c->d;
  LayerArgs a;
  memset(&a, 0, sizeof a);
  a.D = d.D;
  a.H_Q = d.H_Q;
  a.H_KV = d.H_KV;
  a.HD = d.HD;
  a.FFN = d.FFN;
  a.KV = d.H_KV * d.HD;
  a.max_ctx = c->max_ctx;
  a.batch = batch;
  a.inv_sqrt_hd_div = sqrt((double)d.HD);
  {
    int ex = 0;   // score_mul is exact only for a power-of-two divisor (check_dims: HD = 64)
    if (frexp(a.inv_sqrt_hd_div, &ex) != 0.5) abort();
    a.score_mul = 1.0 / a.inv_sqrt_hd_div;
  }
  a.w_qkv_m = reinterpret_cast<const uint4 *>(c->qkv_m + layer * c->s_qkv_m);
  a.w_qkv_e = c->qkv_e + layer * c->s_qkv_e;
  {
    const int ln = layer + 1 < c->d.NL ? layer + 1 : layer;
    a.w_qkv_next_m = reinterpret_cast<const uint4 *>(c->qkv_m + ln * c->s_qkv_m);
    a.w_qkv_next_e = c->qkv_e + ln * c->s_qkv_e;
  }
  a.w_o_m = reinterpret_cast<const uint4 *>(c->o_m + layer * c->s_o_m);
  a.w_o_e = c->o_e + layer * c->s_o_e;
  a.w_gu_m = reinterpret_cast<const uint4 *>(c->gu_m + layer * c->s_gu_m);
  a.w_gu_e = c->gu_e + layer * c->s_gu_e;
  a.w_d_m = reinterpret_cast<const uint4 *>(c->d_m + layer * c->s_d_m);
  a.w_d_e = c->d_e + layer * c->s_d_e;
  a.g1 = c->g1 + (size_t)layer * d.D;
  a.g2 = c->g2 + (size_t)layer * d.D;
  a.rope = c->rope;
  a.h_m = c->h_m;
  a.h_e = c->h_e;
  a.h1_m = c->h1_m;
  a.h1_e = c->h1_e;
  a.qkv_m = c->qkv_am;
  a.qkv_e = c->qkv_ae;
  a.att_m = c->att_m;
  a.att_e = c->att_e;
  a.mlp_m = c->mlp_m;
  a.mlp_e = c->mlp_e;
  a.xn_m = c->xn_m;
  a.xn_e = c->xn_e;
  a.k_m = c->k_m + layer * c->s_kv_m;
  a.k_e = c->k_e + layer * c->s_kv_e;
  a.v_m = c->v_m + layer * c->s_kv_m;
  a.v_e = c->v_e + layer * c->s_kv_e;
  a.layer = layer;
  a.NL = d.NL;
  a.kv_pos_const = -1;
  return a;
}

void stage_lens(const bfp_dims &d, int len[ST_COUNT]) {
  const int KV = d.H_KV * d.HD;
  const int L[ST_COUNT] = {d.D, d.D, KV, KV, d.D, d.D, d.D, d.D, d.FFN, d.FFN, d.FFN, d.D, d.D};
  for (int i = 0; i < ST_COUNT; ++i) len[i] = L[i];
}

// BFP_PERSIST=0 keeps batch-1 decodes on the per-stage graph.
bool persist_enabled() {
  const char *v = getenv("BFP_PERSIST");
  return !(v && v[0] == '0');
}

// Batches from BFP_PIPE_MIN_BATCH sequences (0, the default: none; the
// BFP_DECODE_PIPE flag: every batch the plan covers) run each decode step
// as one pipelined launch (bfp_pipe.hip).
int pipe_min_batch() {
  const char *v = getenv("BFP_PIPE_MIN_BATCH");
  const int n = v ? atoi(v) : 0;
  return n > 0 ? n : 1 << 30;
}

// The pipelined step's schedule for `batch` sequences and its buffers, or
// null (*out) when the plan does not cover the dimensions.
int pipe_get(bfp_ctx *c, int batch, bfp_ctx::PipeSched **out) {
  *out = nullptr;
  const bfp_dims &d = c->d;
  if ((int)c->pp_sched.size() < c->max_batch) c->pp_sched.resize(c->max_batch);
  bfp_ctx::PipeSched &ps = c->pp_sched[batch - 1];
  if (!ps.ok) {
    int cus = 0;
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->device));
    if (!pipe_plan(d, batch, c->max_ctx, cus, ps.pl)) return BFP_OK;
    BFP_TRY(pipe_prepare(ps.pl));
    if (!c->pp_words) {
      c->pp_nwords = pipe_words(d, c->max_batch);
      // fine-grained, like the other tagged words (coarse-grained measured the
      // same: the hand-off loads and stores bypass the L2 either way)
      BFP_TRY(c->alloc_fine((void **)&c->pp_words, c->pp_nwords * 4));
      BFP_TRY(c->alloc((void **)&c->pp_layers, sizeof(LayerArgs) * d.NL));
      BFP_TRY(c->alloc((void **)&c->pp_args, sizeof(PipeArgs)));
      std::vector<LayerArgs> la(d.NL);
      for (int l = 0; l < d.NL; ++l) la[l] = layer_args(c, l, c->max_batch);
      HIP_TRY(hipMemcpy(c->pp_layers, la.data(), sizeof(LayerArgs) * d.NL, hipMemcpyHostToDevice));
    }
    BFP_TRY(c->alloc((void **)&ps.role, sizeof(int) * ps.pl.role.size()));
    BFP_TRY(c->alloc((void **)&ps.jstart, sizeof(int) * ps.pl.jstart.size()));
    BFP_TRY(c->alloc((void **)&ps.jobs, sizeof(int) * std::max<size_t>(ps.pl.jobs.size(), 1)));
    HIP_TRY(hipMemcpy(ps.role, ps.pl.role.data(), sizeof(int) * ps.pl.role.size(), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(ps.jstart, ps.pl.jstart.data(), sizeof(int) * ps.pl.jstart.size(), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(ps.jobs, ps.pl.jobs.data(), sizeof(int) * ps.pl.jobs.size(), hipMemcpyHostToDevice));
    ps.ok = true;
  }
  *out = &ps;
  return BFP_OK;
}

// The pipelined step's argument block for this decode (its flags cleared),
// copied to the device.
int pipe_args(bfp_ctx *c, const bfp_ctx::PipeSched &ps, int batch, int16_t *dhm, int8_t *dhe, int steps,
              unsigned long long *trace) {
  const bfp_dims &d = c->d;
  hipStream_t s = c->stream;
  PipeArgs pa{};
  pa.L = c->pp_layers;
  pa.D = d.D;
  pa.FFN = d.FFN;
  pa.KV = d.H_KV * d.HD;
  pa.NL = d.NL;
  pa.H_Q = d.H_Q;
  pa.H_KV = d.H_KV;
  pa.batch = batch;
  pa.ngrp = ps.pl.ngrp;
  pa.nq16 = (d.D + 2 * pa.KV) / 16;
  pa.nd16 = d.D / 16;
  pa.nf16 = d.FFN / 16;
  pa.state = c->state;
  pa.h_m = c->h_m;
  pa.h_e = c->h_e;
  const size_t B = c->max_batch, D = d.D, nq = D + 2 * (size_t)pa.KV;
  unsigned *w = c->pp_words;
  pa.w_h = w;
  pa.w_x1 = (w += B * D);
  pa.w_qkv = (w += B * D);
  pa.w_att = (w += B * nq);
  pa.w_h1 = (w += B * D);
  pa.w_x2 = (w += B * D);
  pa.w_mlp = (w += B * D);
  pa.abort_flag = c->t_abort;
  pa.role = ps.role;
  pa.jstart = ps.jstart;
  pa.jobs = ps.jobs;
  pa.hist_m = dhm;
  pa.hist_e = dhe;
  pa.hist_steps = dhm ? steps : 0;
  pa.trace = trace;
  // no word of an earlier decode may carry a tag of this one
  HIP_TRY(hipMemsetAsync(c->pp_words, 0, c->pp_nwords * 4, s));
  HIP_TRY(hipMemcpyAsync(c->pp_args, &pa, sizeof pa, hipMemcpyHostToDevice, s));
  HIP_TRY(hipStreamSynchronize(s));   // pa is a stack copy
  return BFP_OK;
}

// The whole batch-1 decode as one persistent launch (bfp_persist.hip).
int decode_persist(bfp_ctx *c, PersistArgs pa, int grid, const int *dprompt, int n_prompt,
                   int n_gen, int *dout, int16_t *dhm, int8_t *dhe, bool rtl_loop, bool trace,
                   bool abort_test) {
  const bfp_dims &d = c->d;
  hipStream_t s = c->stream;
  const int steps = n_prompt + n_gen;
  DevBuf tmp;
  unsigned long long *dtrace = nullptr;
  const size_t ntrace = persist_trace_len(steps, d.NL);
  c->trace.clear();
  if (trace) {
    BFP_TRY(tmp.alloc((void **)&dtrace, ntrace * sizeof(unsigned long long)));
    HIP_TRY(hipMemsetAsync(dtrace, 0, ntrace * sizeof(unsigned long long), s));
  }
  if (!c->pt_words) {
    const size_t nw = persist_words(d, grid);
    BFP_TRY(c->alloc_fine((void **)&c->pt_words, nw * 4));
    BFP_TRY(c->alloc((void **)&c->pt_layers, sizeof(LayerArgs) * d.NL));
    BFP_TRY(c->alloc((void **)&c->pt_args, sizeof(PersistArgs)));
    BFP_TRY(c->alloc((void **)&c->pt_clock, sizeof(unsigned long long) * (c->max_ctx + 1)));
    BFP_TRY(c->alloc_fine((void **)&c->pt_scores, 16 * (size_t)d.H_Q * attn_sc_stride(c->max_ctx)));
    std::vector<LayerArgs> la(d.NL);
    for (int l = 0; l < d.NL; ++l) la[l] = layer_args(c, l, 1);
    HIP_TRY(hipMemcpy(c->pt_layers, la.data(), sizeof(LayerArgs) * d.NL, hipMemcpyHostToDevice));
    c->pt_nwords = nw;
  }
  const size_t D = d.D, nq = D + 2 * (size_t)d.H_KV * d.HD, F = d.FFN;
  unsigned *w = c->pt_words;
  pa.t_h = w;
  pa.t_h1 = (w += 2 * D);
  pa.t_att = (w += 2 * D);
  pa.t_qkv = (w += 2 * D);
  pa.t_mlp = (w += 2 * nq);
  pa.t_part = (w += 2 * F);
  pa.sc_buf = c->pt_scores;
  pa.abort_flag = (w += 2 * 4 * (size_t)grid);
  pa.L = c->pt_layers;
  pa.steps = steps;
  pa.n_prompt = n_prompt;
  pa.n_gen = n_gen;
  pa.rtl_loop = rtl_loop ? 1 : 0;
  pa.prompt = dprompt;
  pa.out = dout;
  pa.last = c->last;
  pa.embed = c->embed;
  pa.norm_w = c->norm_w;
  pa.clock = c->pt_clock;
  pa.hist_m = dhm;
  pa.hist_e = dhe;
  pa.hist_steps = dhm ? steps : 0;
  pa.trace = dtrace;
  HIP_TRY(hipMemsetAsync(c->pt_words, 0, c->pt_nwords * 4, s));
  // the score words too: their tags repeat from one decode to the next
  HIP_TRY(hipMemsetAsync(c->pt_scores, 0, 16 * (size_t)d.H_Q * attn_sc_stride(c->max_ctx), s));
  if (abort_test) HIP_TRY(hipMemsetD32Async((hipDeviceptr_t)pa.abort_flag, 1, 1, s));
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  HIP_TRY(hipEventCreate(&ev0));
  HIP_TRY(hipEventCreate(&ev1));
  (void)hipEventRecord(ev0, s);
  int rc = launch_decode_persist(pa, c->pt_args, grid, c->max_ctx, s);
  (void)hipEventRecord(ev1, s);
  if (!rc) {
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = set_err(BFP_EIO, "persistent decode: %s", hipGetErrorString(e));
  }
  unsigned aborted = 0;
  std::vector<unsigned long long> clk(steps + 1);
  if (!rc) {
    hipError_t e = hipMemcpy(&aborted, pa.abort_flag, 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess)
      e = hipMemcpy(clk.data(), c->pt_clock, sizeof(unsigned long long) * (steps + 1),
                    hipMemcpyDeviceToHost);
    if (e != hipSuccess) rc = set_err(BFP_EIO, "persistent decode read-back: %s", hipGetErrorString(e));
    else if (aborted) rc = set_err(BFP_EIO, "persistent decode: a hand-off wait timed out");
  }
  if (!rc) {
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, ev0, ev1);
    int khz = 0;
    (void)hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, c->device);
    const double tick_ms = khz > 0 ? 1.0 / khz : 1e-5;   // the clock runs at 100 MHz
    c->last_decode_ms = ms;
    c->last_gen_ms = n_gen > 0 ? (float)((double)(clk[steps] - clk[n_prompt]) * tick_ms) : 0.f;
    c->step_ms.resize(steps);
    for (int k = 0; k < steps; ++k) c->step_ms[k] = (float)((double)(clk[k + 1] - clk[k]) * tick_ms);
    c->last_path = BFP_PATH_PERSIST;
    c->last_form = BFP_FORM_PERSIST;
    if (dtrace) {
      c->trace.resize(ntrace);
      hipError_t e = hipMemcpy(c->trace.data(), dtrace, ntrace * sizeof(unsigned long long),
                               hipMemcpyDeviceToHost);
      if (e != hipSuccess) rc = set_err(BFP_EIO, "persistent decode trace: %s", hipGetErrorString(e));
    }
  }
  (void)hipEventDestroy(ev0);
  (void)hipEventDestroy(ev1);
  return rc;
}

// Tokens and the optional history back to the host.
int decode_copy_out(bfp_ctx *c, int batch, int steps, int n_out, const int *dout, int32_t *tokens_out,
                    const int16_t *dhm, const int8_t *dhe, int16_t *hist_m, int8_t *hist_e) {
  const bfp_dims &d = c->d;
  if (n_out > 0)
    HIP_TRY(hipMemcpy(tokens_out, dout, sizeof(int) * batch * n_out, hipMemcpyDeviceToHost));
  if (dhm) {
    HIP_TRY(hipMemcpy(hist_m, dhm, (size_t)batch * steps * d.NL * d.D * 2, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(hist_e, dhe, (size_t)batch * steps * d.NL * d.D / 16, hipMemcpyDeviceToHost));
  }
  return BFP_OK;
}

}  // namespace

extern "C" {

bfp_ctx *bfp_create(const bfp_dims *dims, int device, int max_batch) {
  if (!dims) {
    set_err(BFP_EINVAL, "null dims");
    return nullptr;
  }
  if (check_dims(*dims)) return nullptr;
  if (max_batch <= 0 || max_batch > 1024) {
    set_err(BFP_EINVAL, "max_batch=%d out of range", max_batch);
    return nullptr;
  }
  if (hipSetDevice(device) != hipSuccess) {
    set_err(BFP_EIO, "hipSetDevice(%d) failed", device);
    return nullptr;
  }
  bfp_ctx *c = new bfp_ctx();
  c->d = *dims;
  c->device = device;
  c->max_batch = max_batch;
  c->max_ctx = dims->MAX_CTX;
  const bfp_dims &d = c->d;
  const int KV = d.H_KV * d.HD;
  const size_t nq = (size_t)d.D + 2 * KV;
  c->s_qkv_m = nq * d.D * 2;
  c->s_qkv_e = nq * d.D / 16;
  c->s_o_m = (size_t)d.D * d.D * 2;
  c->s_o_e = (size_t)d.D * d.D / 16;
  c->s_gu_m = (size_t)2 * d.FFN * d.D * 2;
  c->s_gu_e = (size_t)2 * d.FFN * d.D / 16;
  c->s_d_m = (size_t)d.D * d.FFN * 2;
  c->s_d_e = (size_t)d.D * d.FFN / 16;
  c->s_kv_m = (size_t)max_batch * c->max_ctx * KV;
  c->s_kv_e = c->s_kv_m / 16;
  c->head_rows = (d.VOCAB % 64 == 0) ? 64 : 16;
  c->head_wg = d.VOCAB / c->head_rows;
  const size_t B = max_batch;
  int rc = 0;
  std::vector<double> rope;
  rope_table(rope, c->max_ctx, d.HD);
  if ((rc = hipStreamCreate(&c->stream)) != hipSuccess) {
    set_err(BFP_EIO, "hipStreamCreate failed");
    delete c;
    return nullptr;
  }
  if ((rc = c->alloc((void **)&c->qkv_m, c->s_qkv_m * d.NL)) ||
      (rc = c->alloc((void **)&c->qkv_e, c->s_qkv_e * d.NL)) ||
      (rc = c->alloc((void **)&c->o_m, c->s_o_m * d.NL)) ||
      (rc = c->alloc((void **)&c->o_e, c->s_o_e * d.NL)) ||
      (rc = c->alloc((void **)&c->gu_m, c->s_gu_m * d.NL)) ||
      (rc = c->alloc((void **)&c->gu_e, c->s_gu_e * d.NL)) ||
      (rc = c->alloc((void **)&c->d_m, c->s_d_m * d.NL)) ||
      (rc = c->alloc((void **)&c->d_e, c->s_d_e * d.NL)) ||
      (rc = c->alloc((void **)&c->g1, sizeof(double) * d.D * d.NL)) ||
      (rc = c->alloc((void **)&c->g2, sizeof(double) * d.D * d.NL)) ||
      (rc = c->alloc((void **)&c->norm_w, sizeof(double) * d.D)) ||
      (rc = c->alloc((void **)&c->rope, sizeof(double) * rope.size())) ||
      (rc = c->alloc((void **)&c->rope_row, sizeof(double) * d.HD)) ||
      (rc = c->alloc((void **)&c->embed, sizeof(float) * (size_t)d.VOCAB * d.D)) ||
      (max_batch >= HEAD_SEQ_MIN && d.D % 64 == 0 && d.D <= 576 &&
       ((rc = c->alloc((void **)&c->embedp, sizeof(float) * (size_t)d.VOCAB * d.D)) ||
        (rc = c->alloc((void **)&c->embq, (size_t)d.VOCAB * d.D * 2)) ||
        (rc = c->alloc((void **)&c->embq_meta, sizeof(HeadQRow) * (size_t)d.VOCAB)) ||
        (rc = c->alloc((void **)&c->hq_x, (size_t)(B + 15) / 16 * (d.D / 64) * 64 * 32)) ||
        (rc = c->alloc((void **)&c->hq_seq, sizeof(HeadQSeq) * B)) ||
        (rc = c->alloc((void **)&c->hq_blk, sizeof(double2) * B * (d.VOCAB / 16))))) ||
      (rc = c->alloc((void **)&c->h_m, 2 * B * d.D)) || (rc = c->alloc((void **)&c->h_e, B * d.D / 16)) ||
      (rc = c->alloc((void **)&c->h1_m, 2 * B * d.D)) ||
      (rc = c->alloc((void **)&c->h1_e, B * d.D / 16)) ||
      (rc = c->alloc((void **)&c->qkv_am, 2 * B * nq)) ||
      (rc = c->alloc((void **)&c->qkv_ae, B * nq / 16)) ||
      (rc = c->alloc((void **)&c->att_m, 2 * B * d.D)) ||
      (rc = c->alloc((void **)&c->att_e, B * d.D / 16)) ||
      (rc = c->alloc((void **)&c->mlp_m, 2 * B * d.FFN)) ||
      (rc = c->alloc((void **)&c->mlp_e, B * d.FFN / 16)) ||
      (rc = c->alloc((void **)&c->k_m, 2 * c->s_kv_m * d.NL)) ||
      (rc = c->alloc((void **)&c->k_e, c->s_kv_e * d.NL)) ||
      (rc = c->alloc((void **)&c->v_m, 2 * c->s_kv_m * d.NL)) ||
      (rc = c->alloc((void **)&c->v_e, c->s_kv_e * d.NL)) ||
      (rc = c->alloc((void **)&c->xn_m, 2 * B * d.D)) ||
      (rc = c->alloc((void **)&c->xn_e, B * d.D / 16)) ||
      (rc = c->alloc((void **)&c->hn, sizeof(double) * B * d.D)) ||
      (rc = c->alloc((void **)&c->part_v, sizeof(double) * B * head_part_max(c))) ||
      (rc = c->alloc((void **)&c->part_i, sizeof(int) * B * head_part_max(c))) ||
      (rc = c->alloc((void **)&c->state, sizeof(int) * (B + 2))) ||   // + k_ctl_embed's count
      (rc = c->alloc((void **)&c->last, sizeof(int) * B)) ||
      (rc = c->alloc((void **)&c->t_h1, sizeof(unsigned) * B * d.D)) ||
      (rc = c->alloc((void **)&c->t_h, sizeof(unsigned) * B * d.D)) ||
      (rc = c->alloc((void **)&c->t_qkv, sizeof(unsigned) * B * (d.D + 2 * d.H_KV * d.HD))) ||
      (rc = c->alloc((void **)&c->t_abort, sizeof(int))) ||
      (rc = c->alloc((void **)&c->dump_dev, sizeof(StageDump)))) {
    delete c;
    return nullptr;
  }
  if (prepare_layer_kernels(c->max_ctx, d.D, d.FFN) || prepare_head_kernels(d.D)) {
    delete c;
    return nullptr;
  }
  // s_kv_m counts elements; the mantissa arrays are int16
  if (hipMemcpy(c->rope, rope.data(), sizeof(double) * rope.size(), hipMemcpyHostToDevice) !=
          hipSuccess ||
      hipMemset(c->k_m, 0, 2 * c->s_kv_m * d.NL) != hipSuccess ||
      hipMemset(c->v_m, 0, 2 * c->s_kv_m * d.NL) != hipSuccess ||
      hipMemset(c->k_e, 0, c->s_kv_e * d.NL) != hipSuccess ||
      hipMemset(c->v_e, 0, c->s_kv_e * d.NL) != hipSuccess) {
    set_err(BFP_EIO, "context initialisation copy failed");
    delete c;
    return nullptr;
  }
  return c;
}

void bfp_destroy(bfp_ctx *c) { delete c; }

int bfp_get_dims(const bfp_ctx *c, bfp_dims *out) {
  if (!c || !out) return set_err(BFP_EINVAL, "null argument");
  *out = c->d;
  return BFP_OK;
}

// Load one weight tensor.  Matrices: from float32 (quantize_W on the device,
// full.py:110-119) or from the reference layout (m, e).  Gammas / final norm
// weight: float32 (quantised to BFP-exact float64 as fp_quantize_vec does,
// full.py:322-323,413) or (m, e).  The embedding must be float32: the head
// uses the raw table (full.py:439).
int bfp_load_weights_wide(bfp_ctx *c, int which, int layer, const void *wide_m,
                          const void *wide_e) {
  if (!c || !wide_m || !wide_e) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  const int KV = d.H_KV * d.HD;
  if (which < BFP_WQ || which > BFP_WD)
    return set_err(BFP_EINVAL, "wide layout is for matrices BFP_WQ..BFP_WD, not slot %d", which);
  if (layer < 0 || layer >= d.NL) return set_err(BFP_EINVAL, "layer %d out of range [0, %d)", layer, d.NL);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  int n_out = d.D, n_in = d.D, cstride = 1;
  uint8_t *Pm = nullptr;
  int8_t *Pe = nullptr;
  switch (which) {
    case BFP_WQ: case BFP_WK: case BFP_WV: {
      const int row0 = which == BFP_WQ ? 0 : (which == BFP_WK ? d.D : d.D + KV);
      n_out = which == BFP_WQ ? d.D : KV;
      Pm = c->qkv_m + layer * c->s_qkv_m + (size_t)row0 * d.D * 2;
      Pe = c->qkv_e + layer * c->s_qkv_e + (size_t)row0 * d.D / 16;
      break;
    }
    case BFP_WO:
      Pm = c->o_m + layer * c->s_o_m;
      Pe = c->o_e + layer * c->s_o_e;
      break;
    case BFP_WG: case BFP_WU: {
      n_out = d.FFN;
      cstride = 2;
      const size_t off = which == BFP_WG ? 0 : 1;   // chunks interleaved G0 U0 G1 U1 ...
      Pm = c->gu_m + layer * c->s_gu_m + off * (size_t)16 * d.D * 2;
      Pe = c->gu_e + layer * c->s_gu_e + off * (size_t)16 * d.D / 16;
      break;
    }
    default:   // BFP_WD
      n_in = d.FFN;
      Pm = c->d_m + layer * c->s_d_m;
      Pe = c->d_e + layer * c->s_d_e;
      break;
  }
  const size_t bm = (size_t)n_out * n_in * 2, be = (size_t)n_out * n_in / 16;
  DevBuf tmp;
  void *dm, *de;
  BFP_TRY(tmp.alloc(&dm, bm));
  BFP_TRY(tmp.alloc(&de, be));
  HIP_TRY(hipMemcpyAsync(dm, wide_m, bm, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(de, wide_e, be, hipMemcpyHostToDevice, s));
  BFP_TRY(pack_wide(dm, de, n_out, n_in, Pm, Pe, s, cstride));
  HIP_TRY(hipStreamSynchronize(s));
  return BFP_OK;
}

int bfp_load_weights(bfp_ctx *c, int which, int layer, const float *fp32, const int16_t *m,
                     const int8_t *e) {
  if (!c) return set_err(BFP_EINVAL, "null context");
  const bfp_dims &d = c->d;
  const int KV = d.H_KV * d.HD;
  if (which != BFP_EMBED && which != BFP_NORM_W && (layer < 0 || layer >= d.NL))
    return set_err(BFP_EINVAL, "layer %d out of range [0, %d)", layer, d.NL);
  if (!fp32 && (!m || !e)) return set_err(BFP_EINVAL, "need fp32 or (m, e)");
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  int n_out = 0, n_in = d.D, cstride = 1;
  uint8_t *Pm = nullptr;
  int8_t *Pe = nullptr;
  switch (which) {
    case BFP_WQ: case BFP_WK: case BFP_WV: {
      int row0 = which == BFP_WQ ? 0 : (which == BFP_WK ? d.D : d.D + KV);
      n_out = which == BFP_WQ ? d.D : KV;
      Pm = c->qkv_m + layer * c->s_qkv_m + (size_t)row0 * d.D * 2;
      Pe = c->qkv_e + layer * c->s_qkv_e + (size_t)row0 * d.D / 16;
      break;
    }
    case BFP_WO:
      n_out = d.D;
      Pm = c->o_m + layer * c->s_o_m;
      Pe = c->o_e + layer * c->s_o_e;
      break;
    case BFP_WG: case BFP_WU: {
      n_out = d.FFN;
      cstride = 2;
      size_t off = which == BFP_WG ? 0 : 1;   // chunks interleaved G0 U0 G1 U1 ...
      Pm = c->gu_m + layer * c->s_gu_m + off * (size_t)16 * d.D * 2;
      Pe = c->gu_e + layer * c->s_gu_e + off * (size_t)16 * d.D / 16;
      break;
    }
    case BFP_WD:
      n_out = d.D;
      n_in = d.FFN;
      Pm = c->d_m + layer * c->s_d_m;
      Pe = c->d_e + layer * c->s_d_e;
      break;
    case BFP_G1: case BFP_G2: case BFP_NORM_W: {
      double *dst = which == BFP_NORM_W ? c->norm_w
                                        : (which == BFP_G1 ? c->g1 : c->g2) + (size_t)layer * d.D;
      DevBuf tmp;
      int16_t *qm;
      int8_t *qe;
      BFP_TRY(tmp.alloc((void **)&qm, (size_t)d.D * 2));
      BFP_TRY(tmp.alloc((void **)&qe, (size_t)d.D / 16));
      if (fp32) {
        float *f;
        BFP_TRY(tmp.alloc((void **)&f, (size_t)d.D * 4));
        HIP_TRY(hipMemcpyAsync(f, fp32, (size_t)d.D * 4, hipMemcpyHostToDevice, s));
        BFP_TRY(bfp_tile_quantize_f32_d(f, d.D, qm, qe, s));
      } else {
        HIP_TRY(hipMemcpyAsync(qm, m, (size_t)d.D * 2, hipMemcpyHostToDevice, s));
        HIP_TRY(hipMemcpyAsync(qe, e, (size_t)d.D / 16, hipMemcpyHostToDevice, s));
      }
      BFP_TRY(bfp_tile_decode_d(qm, qe, d.D, dst, s));
      HIP_TRY(hipStreamSynchronize(s));
      return BFP_OK;
    }
    case BFP_EMBED: {
      if (!fp32) return set_err(BFP_EINVAL, "the embedding must be given as float32");
      // The head's bounds hold for finite values only: with a NaN or an
      // infinity no block's bounds would bracket the largest logit, so such
      // an embedding is refused here.
      for (size_t i = 0, n = (size_t)d.VOCAB * d.D; i < n; ++i)
        if (!std::isfinite(fp32[i]))
          return set_err(BFP_EINVAL, "embedding value (%zu, %zu) is not finite", i / d.D, i % d.D);
      HIP_TRY(hipMemcpy(c->embed, fp32, sizeof(float) * (size_t)d.VOCAB * d.D,
                        hipMemcpyHostToDevice));
      if (c->embedp) {
        const long long n = (long long)d.VOCAB * d.D;
        hipLaunchKernelGGL(permute_embed_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           s, c->embed, n, d.D, c->embedp);
        BFP_TRY(launch_status("embed permute"));
        BFP_TRY(launch_embq_build(c->embed, d.VOCAB, d.D, c->embq, c->embq_meta, s));
        HIP_TRY(hipStreamSynchronize(s));
      }
      return BFP_OK;
    }
    default:
      return set_err(BFP_EINVAL, "unknown weight slot %d", which);
  }
  DevBuf tmp;
  if (fp32) {
    float *f;
    size_t bytes = (size_t)n_out * n_in * 4;
    BFP_TRY(tmp.alloc((void **)&f, bytes));
    HIP_TRY(hipMemcpyAsync(f, fp32, bytes, hipMemcpyHostToDevice, s));
    BFP_TRY(quantize_pack_f32(f, n_out, n_in, Pm, Pe, s, cstride));
  } else {
    int16_t *dm;
    int8_t *de;
    size_t bm = (size_t)n_out * n_in * 2, be = (size_t)n_out * n_in / 16;
    BFP_TRY(tmp.alloc((void **)&dm, bm));
    BFP_TRY(tmp.alloc((void **)&de, be));
    HIP_TRY(hipMemcpyAsync(dm, m, bm, hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(de, e, be, hipMemcpyHostToDevice, s));
    BFP_TRY(pack(dm, de, n_out, n_in, Pm, Pe, s, cstride));
  }
  HIP_TRY(hipStreamSynchronize(s));
  return BFP_OK;
}

int bfp_reset_kv(bfp_ctx *c) {
  if (!c) return set_err(BFP_EINVAL, "null context");
  const bfp_dims &d = c->d;
  HIP_TRY(hipMemsetAsync(c->k_m, 0, 2 * c->s_kv_m * d.NL, c->stream));
  HIP_TRY(hipMemsetAsync(c->v_m, 0, 2 * c->s_kv_m * d.NL, c->stream));
  HIP_TRY(hipMemsetAsync(c->k_e, 0, c->s_kv_e * d.NL, c->stream));
  HIP_TRY(hipMemsetAsync(c->v_e, 0, c->s_kv_e * d.NL, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return BFP_OK;
}

int bfp_kv_io(bfp_ctx *c, int layer, int seq, int t0, int n, int16_t *k_m, int8_t *k_e,
              int16_t *v_m, int8_t *v_e, int write) {
  if (!c || !k_m || !k_e || !v_m || !v_e) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  if (layer < 0 || layer >= d.NL || seq < 0 || seq >= c->max_batch || t0 < 0 || n < 0 ||
      t0 + n > c->max_ctx)
    return set_err(BFP_ERANGE, "kv_io: layer %d seq %d positions [%d, %d) out of range", layer, seq,
                   t0, t0 + n);
  if (n == 0) return BFP_OK;
  HIP_TRY(hipSetDevice(c->device));
  const size_t KV = (size_t)d.H_KV * d.HD;
  const size_t om = layer * c->s_kv_m + ((size_t)seq * c->max_ctx + t0) * KV;
  const size_t oe = layer * c->s_kv_e + ((size_t)seq * c->max_ctx + t0) * KV / 16;
  const size_t bm = (size_t)n * KV * 2, be = (size_t)n * KV / 16;
  hipStream_t s = c->stream;
  if (write) {
    HIP_TRY(hipMemcpyAsync(c->k_m + om, k_m, bm, hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(c->k_e + oe, k_e, be, hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(c->v_m + om, v_m, bm, hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(c->v_e + oe, v_e, be, hipMemcpyHostToDevice, s));
  } else {
    HIP_TRY(hipMemcpyAsync(k_m, c->k_m + om, bm, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipMemcpyAsync(k_e, c->k_e + oe, be, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipMemcpyAsync(v_m, c->v_m + om, bm, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipMemcpyAsync(v_e, c->v_e + oe, be, hipMemcpyDeviceToHost, s));
  }
  HIP_TRY(hipStreamSynchronize(s));
  return BFP_OK;
}

// fwd_layer (full.py:261-293) for `batch` sequences: RoPE at position pos,
// K/V written at slot kv_pos, attention over slots 0..kv_pos.  h in/out are
// host arrays (batch x D mantissas, batch x D/16 exponents); dump (optional)
// receives every stage.
int bfp_layer_step_kv(bfp_ctx *c, int layer, int pos, int kv_pos, int batch, const int16_t *h_m,
                      const int8_t *h_e, int16_t *out_m, int8_t *out_e, bfp_stage_dump *dump) {
  if (!c || !h_m || !h_e || !out_m || !out_e) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  if (layer < 0 || layer >= d.NL) return set_err(BFP_EINVAL, "layer %d out of range", layer);
  if (batch <= 0 || batch > c->max_batch) return set_err(BFP_EINVAL, "batch %d out of range", batch);
  if (kv_pos < 0 || kv_pos >= c->max_ctx)
    return set_err(BFP_ERANGE, "kv_pos %d outside the KV capacity %d", kv_pos, c->max_ctx);
  if (pos < 0) return set_err(BFP_ERANGE, "pos %d is negative", pos);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  // h in and out through pinned host memory (four pageable hipMemcpyAsync
  // took most of a call's time); D % 64 == 0, so both parts are whole
  // 32-bit words.  At batch 1 the layer's kernels read h from the mapped
  // buffer and write the output back into it; larger batches move it to
  // and from the device activations with copy kernels.
  const size_t bm = (size_t)batch * d.D * 2, be = (size_t)batch * d.D / 16;
  BFP_TRY(c->pinned(2 * (bm + be)));
  memcpy(c->pin, h_m, bm);
  memcpy(c->pin + bm, h_e, be);
  const bool direct = batch == 1;
  const int nw = (int)((bm + be) / 4), cgrid = std::min((nw + 255) / 256, 64);
  if (!direct) {
    hipLaunchKernelGGL(copy_words2_kernel, dim3(cgrid), dim3(256), 0, s,
                       reinterpret_cast<const unsigned *>(c->pin_dev), reinterpret_cast<unsigned *>(c->h_m),
                       (int)(bm / 4), reinterpret_cast<const unsigned *>(c->pin_dev + bm),
                       reinterpret_cast<unsigned *>(c->h_e), (int)(be / 4));
    BFP_TRY(launch_status("layer input"));
  }
  LayerArgs a = layer_args(c, layer, batch);
  if (direct) {
    a.h_m = reinterpret_cast<int16_t *>(c->pin_dev);
    a.h_e = reinterpret_cast<int8_t *>(c->pin_dev + bm);
  }
  a.pos_const = pos;
  a.kv_pos_const = kv_pos;
  std::vector<double> row;
  if (pos >= c->max_ctx) {   // past the table: this position's row, same expressions
    row.resize(d.HD);
    rope_row(row.data(), pos, d.HD, 10000.0);
    HIP_TRY(hipMemcpyAsync(c->rope_row, row.data(), sizeof(double) * d.HD, hipMemcpyHostToDevice, s));
    a.rope_row = c->rope_row;
  }
  DevBuf tmp;
  StageDump sd;
  int len[ST_COUNT];
  stage_lens(d, len);
  if (dump) {
    for (int i = 0; i < ST_COUNT; ++i) {
      BFP_TRY(tmp.alloc((void **)&sd.m[i], (size_t)batch * len[i] * 2));
      BFP_TRY(tmp.alloc((void **)&sd.e[i], (size_t)batch * len[i] / 16));
      sd.mstride[i] = len[i];
    }
    HIP_TRY(hipMemcpyAsync(c->dump_dev, &sd, sizeof sd, hipMemcpyHostToDevice, s));
    a.dump = c->dump_dev;
  }
  BFP_TRY(launch_layer(a, s));
  uint8_t *po = direct ? c->pin : c->pin + bm + be, *po_dev = c->pin_dev + bm + be;
  if (!direct) {
    hipLaunchKernelGGL(copy_words2_kernel, dim3(cgrid), dim3(256), 0, s,
                       reinterpret_cast<const unsigned *>(c->h_m), reinterpret_cast<unsigned *>(po_dev),
                       (int)(bm / 4), reinterpret_cast<const unsigned *>(c->h_e),
                       reinterpret_cast<unsigned *>(po_dev + bm), (int)(be / 4));
    BFP_TRY(launch_status("layer output"));
  }
  if (dump) {
    for (int i = 0; i < ST_COUNT; ++i) {
      if (dump->m[i])
        HIP_TRY(hipMemcpyAsync(dump->m[i], sd.m[i], (size_t)batch * len[i] * 2,
                               hipMemcpyDeviceToHost, s));
      if (dump->e[i])
        HIP_TRY(hipMemcpyAsync(dump->e[i], sd.e[i], (size_t)batch * len[i] / 16,
                               hipMemcpyDeviceToHost, s));
    }
  }
  HIP_TRY(hipStreamSynchronize(s));
  memcpy(out_m, po, bm);
  memcpy(out_e, po + bm, be);
  return BFP_OK;
}

int bfp_layer_step(bfp_ctx *c, int layer, int pos, int batch, const int16_t *h_m,
                   const int8_t *h_e, int16_t *out_m, int8_t *out_e, bfp_stage_dump *dump) {
  return bfp_layer_step_kv(c, layer, pos, pos, batch, h_m, h_e, out_m, out_e, dump);
}

int bfp_kv_io_f64(bfp_ctx *c, int layer, int seq, int t0, int n, double *k, double *v,
                  int write) {
  if (!c || (n > 0 && (!k || !v))) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  if (layer < 0 || layer >= d.NL || seq < 0 || seq >= c->max_batch || t0 < 0 || n < 0 ||
      t0 + n > c->max_ctx)
    return set_err(BFP_ERANGE, "kv_io_f64: layer %d seq %d positions [%d, %d) out of range",
                   layer, seq, t0, t0 + n);
  if (n == 0) return BFP_OK;
  HIP_TRY(hipSetDevice(c->device));
  const size_t KV = (size_t)d.H_KV * d.HD, cnt = (size_t)n * KV;
  const size_t om = layer * c->s_kv_m + ((size_t)seq * c->max_ctx + t0) * KV;
  const size_t oe = layer * c->s_kv_e + ((size_t)seq * c->max_ctx + t0) * KV / 16;
  hipStream_t s = c->stream;
  DevBuf tmp;
  double *dk, *dv;
  int *flag;
  BFP_TRY(tmp.alloc((void **)&dk, cnt * sizeof(double)));
  BFP_TRY(tmp.alloc((void **)&dv, cnt * sizeof(double)));
  BFP_TRY(tmp.alloc((void **)&flag, sizeof(int)));
  if (write) {
    int inexact = 0;
    HIP_TRY(hipMemcpyAsync(flag, &inexact, sizeof(int), hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(dk, k, cnt * sizeof(double), hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(dv, v, cnt * sizeof(double), hipMemcpyHostToDevice, s));
    BFP_TRY(tile_encode_f64(dk, cnt, c->k_m + om, c->k_e + oe, flag, s));
    BFP_TRY(tile_encode_f64(dv, cnt, c->v_m + om, c->v_e + oe, flag, s));
    HIP_TRY(hipMemcpyAsync(&inexact, flag, sizeof(int), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (inexact)
      return set_err(BFP_EINVAL, "kv_io_f64: positions [%d, %d) hold values that are not BFP tiles",
                     t0, t0 + n);
    return BFP_OK;
  } else {
    BFP_TRY(bfp_tile_decode_d(c->k_m + om, c->k_e + oe, cnt, dk, s));
    BFP_TRY(bfp_tile_decode_d(c->v_m + om, c->v_e + oe, cnt, dv, s));
    HIP_TRY(hipMemcpyAsync(k, dk, cnt * sizeof(double), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipMemcpyAsync(v, dv, cnt * sizeof(double), hipMemcpyDeviceToHost, s));
  }
  HIP_TRY(hipStreamSynchronize(s));
  return BFP_OK;
}

int bfp_matvec(bfp_ctx *c, const int16_t *x_m, const int8_t *x_e, int which, int layer,
               int batch, int16_t *y_m, int8_t *y_e) {
  if (!c || !x_m || !x_e || !y_m || !y_e) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  const int KV = d.H_KV * d.HD;
  if (layer < 0 || layer >= d.NL) return set_err(BFP_EINVAL, "layer %d out of range", layer);
  if (batch <= 0) return set_err(BFP_EINVAL, "batch %d must be positive", batch);
  int n_out = d.D, n_in = d.D, cstride = 1;
  const uint8_t *Pm = nullptr;
  const int8_t *Pe = nullptr;
  switch (which) {
    case BFP_WQ: case BFP_WK: case BFP_WV: {
      const int row0 = which == BFP_WQ ? 0 : (which == BFP_WK ? d.D : d.D + KV);
      n_out = which == BFP_WQ ? d.D : KV;
      Pm = c->qkv_m + layer * c->s_qkv_m + (size_t)row0 * d.D * 2;
      Pe = c->qkv_e + layer * c->s_qkv_e + (size_t)row0 * d.D / 16;
      break;
    }
    case BFP_WO:
      Pm = c->o_m + layer * c->s_o_m;
      Pe = c->o_e + layer * c->s_o_e;
      break;
    case BFP_WG: case BFP_WU: {
      n_out = d.FFN;
      cstride = 2;                                  // chunks interleaved G0 U0 G1 U1 ...
      const size_t off = which == BFP_WG ? 0 : 1;
      Pm = c->gu_m + layer * c->s_gu_m + off * (size_t)16 * d.D * 2;
      Pe = c->gu_e + layer * c->s_gu_e + off * (size_t)16 * d.D / 16;
      break;
    }
    case BFP_WD:
      n_in = d.FFN;
      Pm = c->d_m + layer * c->s_d_m;
      Pe = c->d_e + layer * c->s_d_e;
      break;
    default:
      return set_err(BFP_EINVAL, "matvec: slot %d is not a matrix (BFP_WQ .. BFP_WD)", which);
  }
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  DevBuf tmp;
  int16_t *dxm, *dym;
  int8_t *dxe, *dye;
  BFP_TRY(tmp.alloc((void **)&dxm, (size_t)batch * n_in * 2));
  BFP_TRY(tmp.alloc((void **)&dxe, (size_t)batch * n_in / 16));
  BFP_TRY(tmp.alloc((void **)&dym, (size_t)batch * n_out * 2));
  BFP_TRY(tmp.alloc((void **)&dye, (size_t)batch * n_out / 16));
  HIP_TRY(hipMemcpyAsync(dxm, x_m, (size_t)batch * n_in * 2, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(dxe, x_e, (size_t)batch * n_in / 16, hipMemcpyHostToDevice, s));
  BFP_TRY(launch_matvec(Pm, Pe, n_out, n_in, batch, 1, 0, 0, dxm, dxe, n_in, dym, dye, n_out, 0, s,
                        cstride));
  HIP_TRY(hipMemcpyAsync(y_m, dym, (size_t)batch * n_out * 2, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(y_e, dye, (size_t)batch * n_out / 16, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return BFP_OK;
}

// The engine tables of the composed RTL layer, made on their first use.
static int rtl_tables_ready(bfp_ctx *c) {
  if (c->rtl_exp) return BFP_OK;
  const bfp_dims &d = c->d;
  std::vector<uint16_t> ex(1024);
  std::vector<int16_t> si(65536);
  std::vector<uint32_t> fr(d.HD / 2);
  BFP_TRY(bfp_rtl_tables(ex.data(), si.data(), fr.data(), d.HD, 10000.0));
  uint16_t *de;
  int16_t *ds;
  unsigned *df;
  BFP_TRY(c->alloc((void **)&de, ex.size() * 2));
  BFP_TRY(c->alloc((void **)&ds, si.size() * 2));
  BFP_TRY(c->alloc((void **)&df, fr.size() * 4));
  HIP_TRY(hipMemcpy(de, ex.data(), ex.size() * 2, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(ds, si.data(), si.size() * 2, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(df, fr.data(), fr.size() * 4, hipMemcpyHostToDevice));
  c->rtl_exp = de, c->rtl_silu = ds, c->rtl_freq = df;
  return BFP_OK;
}

static RtlArgs rtl_args(bfp_ctx *c, int layer, int pos, int kv_pos) {
  RtlArgs a;
  a.L = layer_args(c, layer, 1);
  a.exp_lut = c->rtl_exp;
  a.silu_lut = c->rtl_silu;
  a.freq = c->rtl_freq;
  a.pos = pos;
  a.kv_pos = kv_pos;
  a.pos_ptr = nullptr;
  return a;
}

// The RTL head's buffers (made once) and its tile-quantised embedding in the
// device layout (re-made on every call, so it follows the loaded weights).
static int rtl_head_ready(bfp_ctx *c, RtlHeadArgs &ha) {
  const bfp_dims &d = c->d;
  if (d.D % 64 || d.VOCAB % 16)
    return set_err(BFP_EINVAL, "rtl head: D %d must be a multiple of 64, VOCAB %d of 16", d.D, d.VOCAB);
  if (!c->rtl_emb_m) {
    BFP_TRY(c->alloc((void **)&c->rtl_emb_m, (size_t)d.VOCAB * d.D * 2));
    BFP_TRY(c->alloc((void **)&c->rtl_emb_e, (size_t)d.VOCAB * d.D / 16));
    BFP_TRY(c->alloc((void **)&c->rtl_lg_m, (size_t)d.VOCAB * 2));
    BFP_TRY(c->alloc((void **)&c->rtl_lg_e, (size_t)d.VOCAB));
    BFP_TRY(c->alloc((void **)&c->rtl_xn_m, (size_t)d.D * 2));
    BFP_TRY(c->alloc((void **)&c->rtl_xn_e, (size_t)d.D / 16));
    BFP_TRY(c->alloc((void **)&c->rtl_work, sizeof(int) * 3 * (size_t)(d.VOCAB / 16)));
    BFP_TRY(c->alloc((void **)&c->rtl_tok, sizeof(int)));
  }
  BFP_TRY(bfp_quantize_pack_f32_d(c->embed, d.VOCAB, d.D, c->rtl_emb_m, c->rtl_emb_e, c->stream));
  ha = RtlHeadArgs{d.D, d.VOCAB, c->h_m, c->h_e, c->norm_w, c->rtl_xn_m, c->rtl_xn_e,
                   c->rtl_emb_m, c->rtl_emb_e, c->rtl_lg_m, c->rtl_lg_e, c->rtl_work, c->rtl_tok};
  return BFP_OK;
}

// The composed RTL-exact layer (smollm_layer_bfp.sv:1603-2600) on one
// sequence: RoPE at pos, KV slot kv_pos, attention over slots 0..kv_pos.
int bfp_rtl_layer_step(bfp_ctx *c, int layer, int pos, int kv_pos, const int16_t *h_m,
                       const int8_t *h_e, int16_t *out_m, int8_t *out_e, bfp_stage_dump *dump) {
  if (!c || !h_m || !h_e || !out_m || !out_e) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  if (layer < 0 || layer >= d.NL) return set_err(BFP_EINVAL, "layer %d out of range", layer);
  if (pos < 0 || pos > 2047)
    return set_err(BFP_EINVAL, "pos %d outside the RTL position range 0..2047", pos);
  if (kv_pos < 0 || kv_pos >= c->max_ctx)
    return set_err(BFP_ERANGE, "kv_pos %d outside the KV capacity %d", kv_pos, c->max_ctx);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  BFP_TRY(rtl_tables_ready(c));
  HIP_TRY(hipMemcpyAsync(c->h_m, h_m, (size_t)d.D * 2, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(c->h_e, h_e, (size_t)d.D / 16, hipMemcpyHostToDevice, s));
  RtlArgs a = rtl_args(c, layer, pos, kv_pos);
  DevBuf tmp;
  StageDump sd;
  int len[ST_COUNT];
  stage_lens(d, len);
  if (dump) {
    for (int i = 0; i < ST_COUNT; ++i) {
      BFP_TRY(tmp.alloc((void **)&sd.m[i], (size_t)len[i] * 2));
      BFP_TRY(tmp.alloc((void **)&sd.e[i], (size_t)len[i] / 16));
      sd.mstride[i] = len[i];
    }
    HIP_TRY(hipMemcpyAsync(c->dump_dev, &sd, sizeof sd, hipMemcpyHostToDevice, s));
    a.L.dump = c->dump_dev;
  }
  BFP_TRY(launch_rtl_layer(a, s));
  HIP_TRY(hipMemcpyAsync(out_m, c->h_m, (size_t)d.D * 2, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(out_e, c->h_e, (size_t)d.D / 16, hipMemcpyDeviceToHost, s));
  if (dump) {
    for (int i = 0; i < ST_COUNT; ++i) {
      if (dump->m[i])
        HIP_TRY(hipMemcpyAsync(dump->m[i], sd.m[i], (size_t)len[i] * 2, hipMemcpyDeviceToHost, s));
      if (dump->e[i])
        HIP_TRY(hipMemcpyAsync(dump->e[i], sd.e[i], (size_t)len[i] / 16, hipMemcpyDeviceToHost, s));
    }
  }
  HIP_TRY(hipStreamSynchronize(s));
  return BFP_OK;
}

// The FPGA decode head (smollm_decode_head_bfp.sv) on one hidden state.
int bfp_rtl_head(bfp_ctx *c, const int16_t *h_m, const int8_t *h_e, int16_t *logit_m,
                 int8_t *logit_e, int32_t *token) {
  if (!c || !h_m || !h_e || !token) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  RtlHeadArgs ha;
  BFP_TRY(rtl_head_ready(c, ha));
  HIP_TRY(hipMemcpyAsync(c->h_m, h_m, (size_t)d.D * 2, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(c->h_e, h_e, (size_t)d.D / 16, hipMemcpyHostToDevice, s));
  BFP_TRY(launch_rtl_head(ha, s));
  if (logit_m) HIP_TRY(hipMemcpyAsync(logit_m, c->rtl_lg_m, (size_t)d.VOCAB * 2, hipMemcpyDeviceToHost, s));
  if (logit_e) HIP_TRY(hipMemcpyAsync(logit_e, c->rtl_lg_e, (size_t)d.VOCAB, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(token, c->rtl_tok, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return BFP_OK;
}

// The FPGA's token loop over the composed RTL layer and head, sequence 0.
int bfp_rtl_decode(bfp_ctx *c, const int32_t *prompt, int n_prompt, int n_gen, int32_t *preds,
                   int16_t *hist_m, int8_t *hist_e) {
  if (!c || !prompt || !preds) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  if (n_prompt < 1 || n_gen < 0) return set_err(BFP_EINVAL, "n_prompt %d, n_gen %d", n_prompt, n_gen);
  const int steps = n_prompt + n_gen;
  if (steps > c->max_ctx || steps > 2048)
    return set_err(BFP_ERANGE, "%d steps beyond the KV capacity %d or the RTL position range 2048",
                   steps, c->max_ctx);
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= d.VOCAB)
      return set_err(BFP_EINVAL, "prompt id %d out of range", prompt[i]);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  BFP_TRY(rtl_tables_ready(c));
  RtlHeadArgs ha;
  BFP_TRY(rtl_head_ready(c, ha));
  // The loop runs on the device: one step (embedding row, NL layers at the
  // device step, the head, k_rtl_ctl) is captured as a graph and replayed
  // `steps` times; predictions (and the history) are read back once.
  DevBuf tmp;
  int *dprompt, *dpreds;
  BFP_TRY(tmp.alloc((void **)&dprompt, sizeof(int) * n_prompt));
  BFP_TRY(tmp.alloc((void **)&dpreds, sizeof(int) * steps));
  int16_t *dhm = nullptr;
  int8_t *dhe = nullptr;
  if (hist_m && hist_e) {
    BFP_TRY(tmp.alloc((void **)&dhm, (size_t)steps * d.D * 2));
    BFP_TRY(tmp.alloc((void **)&dhe, (size_t)steps * d.D / 16));
  }
  HIP_TRY(hipMemcpyAsync(dprompt, prompt, sizeof(int) * n_prompt, hipMemcpyHostToDevice, s));
  const int st0[2] = {0, prompt[0]};
  HIP_TRY(hipMemcpyAsync(c->state, st0, sizeof st0, hipMemcpyHostToDevice, s));
  const EmbedArgs ea{d.D, 1, d.VOCAB, c->embed, c->state, c->h_m, c->h_e};
  const RtlCtlArgs ca{c->state, dprompt, n_prompt, dpreds, c->rtl_tok, c->h_m, c->h_e, dhm, dhe, d.D};
  hipGraph_t gr = nullptr;
  hipGraphExec_t ex = nullptr;
  HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int rc = launch_embed(ea, s);
  for (int l = 0; l < d.NL && !rc; ++l) {
    RtlArgs ra = rtl_args(c, l, 0, 0);
    ra.pos_ptr = c->state;
    rc = launch_rtl_layer(ra, s);
  }
  if (!rc) rc = launch_rtl_head(ha, s);
  if (!rc) rc = launch_rtl_ctl(ca, s);
  const hipError_t e1 = hipStreamEndCapture(s, &gr);
  if (!rc && e1 != hipSuccess) rc = set_err(BFP_EIO, "graph capture: %s", hipGetErrorString(e1));
  if (!rc) {
    const hipError_t e2 = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
    if (e2 != hipSuccess) rc = set_err(BFP_EIO, "graph instantiate: %s", hipGetErrorString(e2));
  }
  for (int step = 0; step < steps && !rc; ++step) {
    const hipError_t e = hipGraphLaunch(ex, s);
    if (e != hipSuccess) rc = set_err(BFP_EIO, "graph launch: %s", hipGetErrorString(e));
  }
  if (!rc) {
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = set_err(BFP_EIO, "rtl decode: %s", hipGetErrorString(e));
  }
  if (ex) (void)hipGraphExecDestroy(ex);
  if (gr) (void)hipGraphDestroy(gr);
  if (rc) return rc;
  HIP_TRY(hipMemcpy(preds, dpreds, sizeof(int) * steps, hipMemcpyDeviceToHost));
  if (dhm) {
    HIP_TRY(hipMemcpy(hist_m, dhm, (size_t)steps * d.D * 2, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(hist_e, dhe, (size_t)steps * d.D / 16, hipMemcpyDeviceToHost));
  }
  return BFP_OK;
}

// Final norm + float64 logits + first-index argmax for `batch` hidden states
// (full.py:438-440).  logits (optional): batch x VOCAB.
int bfp_head(bfp_ctx *c, int batch, const int16_t *h_m, const int8_t *h_e, double *logits,
             int32_t *argmax) {
  if (!c || !h_m || !h_e || !argmax) return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  if (batch <= 0 || batch > c->max_batch) return set_err(BFP_EINVAL, "batch %d out of range", batch);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  DevBuf tmp;
  double *dl = nullptr;
  if (logits) BFP_TRY(tmp.alloc((void **)&dl, sizeof(double) * batch * d.VOCAB));
  HIP_TRY(hipMemcpyAsync(c->h_m, h_m, (size_t)batch * d.D * 2, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(c->h_e, h_e, (size_t)batch * d.D / 16, hipMemcpyHostToDevice, s));
  HeadArgs ha = head_args(c, batch, dl);
  BFP_TRY(launch_head(ha, s));
  // reuse the controller's reduction with an empty prompt schedule
  std::vector<int> st(batch + 1, 0);
  st[0] = 1 << 30;   // step beyond any prompt: no token bookkeeping
  HIP_TRY(hipMemcpyAsync(c->state, st.data(), sizeof(int) * (batch + 1), hipMemcpyHostToDevice, s));
  int *dprompt, *dout;
  BFP_TRY(tmp.alloc((void **)&dprompt, sizeof(int) * batch));
  BFP_TRY(tmp.alloc((void **)&dout, sizeof(int) * batch));
  CtlArgs ca{batch, 1, 0, ha.n_wg, 1, c->state, dprompt, dout, c->part_v, c->part_i, c->last};
  BFP_TRY(launch_ctl(ca, s));
  HIP_TRY(hipMemcpyAsync(argmax, c->last, sizeof(int) * batch, hipMemcpyDeviceToHost, s));
  if (logits)
    HIP_TRY(hipMemcpyAsync(logits, dl, sizeof(double) * batch * d.VOCAB, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return BFP_OK;
}

// The golden-token loop of full.py:426-443 for `batch` independent
// sequences (prompt: batch x n_prompt, tokens_out: batch x n_gen).  All
// steps run on the device: each step is embed -> NL layers -> (head from
// step n_prompt-1 on) -> controller, captured once as a HIP graph and
// replayed (flags & BFP_DECODE_NO_GRAPH launches the kernels directly).
// hist_m/hist_e (optional): every layer's h_out at every step, laid out
// (batch, n_prompt + n_gen, NL, D) and (..., D/16).
int bfp_decode(bfp_ctx *c, const int32_t *prompt, int n_prompt, int n_gen, int batch,
               int32_t *tokens_out, int16_t *hist_m, int8_t *hist_e, int flags) {
  if (!c || !prompt || (!tokens_out && (n_gen > 0 || (flags & BFP_DECODE_RTL_LOOP))))
    return set_err(BFP_EINVAL, "null argument");
  const bfp_dims &d = c->d;
  if (n_prompt < 1 || n_gen < 0) return set_err(BFP_EINVAL, "n_prompt=%d n_gen=%d", n_prompt, n_gen);
  if (batch <= 0 || batch > c->max_batch) return set_err(BFP_EINVAL, "batch %d out of range", batch);
  const int steps = n_prompt + n_gen;
  if (steps > c->max_ctx)
    return set_err(BFP_ERANGE, "n_prompt + n_gen = %d exceeds the KV capacity %d", steps,
                   c->max_ctx);
  for (int i = 0; i < batch * n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= d.VOCAB)
      return set_err(BFP_EINVAL, "prompt token %d out of range [0, %d)", prompt[i], d.VOCAB);
  HIP_TRY(hipSetDevice(c->device));
  hipStream_t s = c->stream;
  DevBuf tmp;
  int *dprompt, *dout;
  BFP_TRY(tmp.alloc((void **)&dprompt, sizeof(int) * batch * n_prompt));
  const bool rtl_loop = (flags & BFP_DECODE_RTL_LOOP) != 0;
  const int n_out = rtl_loop ? steps : n_gen;   // tokens recorded per sequence
  BFP_TRY(tmp.alloc((void **)&dout, sizeof(int) * batch * (n_out > 0 ? n_out : 1)));
  int16_t *dhm = nullptr;
  int8_t *dhe = nullptr;
  if (hist_m && hist_e) {
    BFP_TRY(tmp.alloc((void **)&dhm, (size_t)batch * steps * d.NL * d.D * 2));
    BFP_TRY(tmp.alloc((void **)&dhe, (size_t)batch * steps * d.NL * d.D / 16));
  }
  HIP_TRY(hipMemcpyAsync(dprompt, prompt, sizeof(int) * batch * n_prompt, hipMemcpyHostToDevice, s));
  std::vector<int> st(batch + 2, 0);   // step, next inputs, k_ctl_embed's arrival count
  for (int b = 0; b < batch; ++b) st[1 + b] = prompt[b * n_prompt];
  HIP_TRY(hipMemcpyAsync(c->state, st.data(), sizeof(int) * (batch + 2), hipMemcpyHostToDevice, s));

  PersistArgs pa{};
  int grid = 0;
  if (batch == 1 && !(flags & (BFP_DECODE_NO_GRAPH | BFP_DECODE_NO_PERSIST)) && persist_enabled() &&
      persist_plan(d, c->max_ctx, c->device, pa, grid)) {
    BFP_TRY(decode_persist(c, pa, grid, dprompt, n_prompt, n_gen, dout, dhm, dhe, rtl_loop,
                           (flags & BFP_DECODE_TRACE) != 0, (flags & BFP_DECODE_ABORT_TEST) != 0));
    return decode_copy_out(c, batch, steps, n_out, dout, tokens_out, dhm, dhe, hist_m, hist_e);
  }
  c->last_path = (flags & BFP_DECODE_NO_GRAPH) ? BFP_PATH_EAGER : BFP_PATH_GRAPH;
  // the pipelined step (one launch for the step's layers) unless the
  // per-stage launches are asked for or traced
  bfp_ctx::PipeSched *pipe = nullptr;
  if (((flags & BFP_DECODE_PIPE) || batch >= pipe_min_batch()) && !(flags & BFP_DECODE_NO_PIPE))
    BFP_TRY(pipe_get(c, batch, &pipe));
  c->trace.clear();
  // traced pipelined step: every job's stamps of the last step's launch
  unsigned long long *pptr = nullptr;
  const size_t npp = pipe ? (size_t)pipe->pl.grid * PIPE_TRACE_JOBS * PIPE_TRACE_W : 0;
  if (pipe && (flags & BFP_DECODE_TRACE)) {
    BFP_TRY(tmp.alloc((void **)&pptr, npp * sizeof(unsigned long long)));
    HIP_TRY(hipMemsetAsync(pptr, 0, npp * sizeof(unsigned long long), s));
  }
  if (pipe) BFP_TRY(pipe_args(c, *pipe, batch, dhm, dhe, steps, pptr));
  // traced batched decode: the matrix-core blocks' phase stamps
  unsigned long long *mxtr = nullptr;
  const size_t nmx = (size_t)MX_TRACE_KERNELS * MX_TRACE_BLOCKS * MX_TRACE_STAMPS;
  if (!pipe && (flags & BFP_DECODE_TRACE)) {
    BFP_TRY(tmp.alloc((void **)&mxtr, nmx * sizeof(unsigned long long)));
    HIP_TRY(hipMemsetAsync(mxtr, 0, nmx * sizeof(unsigned long long), s));
    BFP_TRY(set_mx_trace(mxtr));
  }
  // no tagged word of an earlier decode may carry a tag of this one
  HIP_TRY(hipMemsetAsync(c->t_h1, 0, sizeof(unsigned) * batch * d.D, s));
  HIP_TRY(hipMemsetAsync(c->t_h, 0, sizeof(unsigned) * batch * d.D, s));
  HIP_TRY(hipMemsetAsync(c->t_qkv, 0, sizeof(unsigned) * batch * (d.D + 2 * d.H_KV * d.HD), s));
  HIP_TRY(hipMemsetAsync(c->t_abort, 0, sizeof(int), s));
  if (flags & BFP_DECODE_ABORT_TEST) HIP_TRY(hipMemsetD32Async((hipDeviceptr_t)c->t_abort, 1, 1, s));

  EmbedArgs ea{d.D, batch, d.VOCAB, c->embed, c->state, c->h_m, c->h_e};
  HeadArgs ha = head_args(c, batch, nullptr);
  CtlArgs ca{batch, n_prompt, n_gen, ha.n_wg, 0, c->state, dprompt, dout, c->part_v,
             c->part_i, c->last, rtl_loop ? 1 : 0};
  // A step: the layers, the head, then k_ctl_embed (the token loop, the step
  // increment and the next step's embedding); step 0's embedding goes first.
  auto enqueue_step = [&](bool head) -> int {
    if (pipe) {
      BFP_TRY(launch_pipe_step(pipe->pl, c->pp_args, s));
      c->last_form = BFP_FORM_PIPE;
    }
    for (int l = 0; l < d.NL && !pipe; ++l) {
      LayerArgs a = layer_args(c, l, batch);
      a.pos_ptr = c->state;
      a.hist_m = dhm;
      a.hist_e = dhe;
      a.hist_steps = steps;
      a.t_h1 = c->t_h1;   // tags are unique per (step, layer) within a decode
      a.t_h = c->t_h;
      a.t_qkv = c->t_qkv;
      a.g1_next = l + 1 < d.NL ? c->g1 + (size_t)(l + 1) * d.D : nullptr;
      a.t_abort = c->t_abort;
      c->last_form = layer_form(a);
      BFP_TRY(launch_layer(a, s, mxtr != nullptr));
    }
    CtlArgs cc = ca;
    cc.head = head ? 1 : 0;
    if (head) BFP_TRY(launch_head(ha, s));
    BFP_TRY(launch_ctl_embed(cc, ea, s));
    return BFP_OK;
  };
  const bool use_graph = !(flags & BFP_DECODE_NO_GRAPH);
  hipGraphExec_t ex[2] = {nullptr, nullptr};
  hipGraph_t gr[2] = {nullptr, nullptr};
  int rc = BFP_OK;
  if (use_graph) {
    for (int k = 0; k < 2 && !rc; ++k) {
      HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
      rc = enqueue_step(k == 1);
      hipError_t e1 = hipStreamEndCapture(s, &gr[k]);
      if (!rc && e1 != hipSuccess) rc = set_err(BFP_EIO, "graph capture: %s", hipGetErrorString(e1));
      if (!rc) {
        hipError_t e2 = hipGraphInstantiate(&ex[k], gr[k], nullptr, nullptr, 0);
        if (e2 != hipSuccess) rc = set_err(BFP_EIO, "graph instantiate: %s", hipGetErrorString(e2));
      }
    }
  }
  hipEvent_t ev0 = nullptr, ev1 = nullptr, evg = nullptr;
  const bool per_step = (flags & BFP_DECODE_STEP_TIMES) != 0;
  std::vector<hipEvent_t> sev;
  if (per_step) {
    sev.resize(steps + 1, nullptr);
    for (auto &e : sev) (void)hipEventCreate(&e);
  }
  if (!rc) {
    (void)hipEventCreate(&ev0);
    (void)hipEventCreate(&ev1);
    (void)hipEventCreate(&evg);
    (void)hipEventRecord(ev0, s);
    if (steps > 0) rc = launch_embed(ea, s);
    for (int step = 0; step < steps && !rc; ++step) {
      const bool head = rtl_loop || step >= n_prompt - 1;
      if (step == n_prompt) (void)hipEventRecord(evg, s);
      if (per_step) (void)hipEventRecord(sev[step], s);
      if (use_graph) {
        hipError_t e = hipGraphLaunch(ex[head ? 1 : 0], s);
        if (e != hipSuccess) rc = set_err(BFP_EIO, "graph launch: %s", hipGetErrorString(e));
      } else {
        rc = enqueue_step(head);
      }
    }
    if (n_gen == 0) (void)hipEventRecord(evg, s);
    if (per_step) (void)hipEventRecord(sev[steps], s);
    (void)hipEventRecord(ev1, s);
  }
  if (!rc) {
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = set_err(BFP_EIO, "decode: %s", hipGetErrorString(e));
  }
  if (!rc) {
    int ab = 0;
    hipError_t e = hipMemcpy(&ab, c->t_abort, sizeof ab, hipMemcpyDeviceToHost);
    if (e != hipSuccess) rc = set_err(BFP_EIO, "decode: %s", hipGetErrorString(e));
    else if (ab) rc = set_err(BFP_EIO, "decode: a wait for tagged words gave up");
  }
  if (!rc) {
    float ms = 0.f, gms = 0.f;
    (void)hipEventElapsedTime(&ms, ev0, ev1);
    (void)hipEventElapsedTime(&gms, evg, ev1);
    c->last_decode_ms = ms;
    c->last_gen_ms = gms;
    if (mxtr) {
      c->trace.resize(nmx);
      hipError_t e = hipMemcpy(c->trace.data(), mxtr, nmx * sizeof(unsigned long long), hipMemcpyDeviceToHost);
      if (e != hipSuccess) rc = set_err(BFP_EIO, "decode trace: %s", hipGetErrorString(e));
    }
    if (pptr) {
      c->trace.resize(npp);
      hipError_t e = hipMemcpy(c->trace.data(), pptr, npp * sizeof(unsigned long long), hipMemcpyDeviceToHost);
      if (e != hipSuccess) rc = set_err(BFP_EIO, "decode trace: %s", hipGetErrorString(e));
    }
    c->step_ms.clear();
    if (per_step) {
      c->step_ms.resize(steps);
      for (int k = 0; k < steps; ++k) (void)hipEventElapsedTime(&c->step_ms[k], sev[k], sev[k + 1]);
    }
  }
  for (auto &e : sev)
    if (e) (void)hipEventDestroy(e);
  for (int k = 0; k < 2; ++k) {
    if (ex[k]) (void)hipGraphExecDestroy(ex[k]);
    if (gr[k]) (void)hipGraphDestroy(gr[k]);
  }
  if (ev0) (void)hipEventDestroy(ev0);
  if (ev1) (void)hipEventDestroy(ev1);
  if (evg) (void)hipEventDestroy(evg);
  if (rc) return rc;
  return decode_copy_out(c, batch, steps, n_out, dout, tokens_out, dhm, dhe, hist_m, hist_e);
}

int bfp_decode_path(const bfp_ctx *c) { return c ? c->last_path : -1; }
int bfp_decode_form(const bfp_ctx *c) { return c ? c->last_form : -1; }

int bfp_decode_trace(const bfp_ctx *c, uint64_t *out, size_t n) {
  if (!c || (!out && n > 0)) return set_err(BFP_EINVAL, "null argument");
  const size_t k = c->trace.size();
  for (size_t i = 0; i < k && i < n; ++i) out[i] = c->trace[i];
  return (int)k;
}

// Per-step device times of the last bfp_decode run with BFP_DECODE_STEP_TIMES:
// copies min(n, steps) values and returns how many were recorded.
int bfp_decode_step_times(const bfp_ctx *c, float *ms, int n) {
  if (!c || (!ms && n > 0)) return set_err(BFP_EINVAL, "null argument");
  const int k = (int)c->step_ms.size();
  for (int i = 0; i < k && i < n; ++i) ms[i] = c->step_ms[i];
  return k;
}

// Device time of the last bfp_decode: all steps, and the steps from
// n_prompt on (the generated tokens).
int bfp_decode_time(const bfp_ctx *c, float *total_ms, float *gen_ms) {
  if (!c || !total_ms || !gen_ms) return set_err(BFP_EINVAL, "null argument");
  *total_ms = c->last_decode_ms;
  *gen_ms = c->last_gen_ms;
  return BFP_OK;
}

}  // extern "C"
