// Argument block, schedule and host entry points of the pipelined batched
// decode step (bfp_pipe.hip): one persistent launch runs every layer of one
// decode step for a batch of sequences, the sequences flowing through the
// layer's stages in groups of 16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "bfp.h"
#include "bfp_layer.h"

namespace bfp {

// The stages of one layer (rtl/vc707/host/gen_smollm_blockfp_full.py
// :261-293) in the order a sequence group passes them.
enum PipeStage { PS_N1 = 0, PS_QKV, PS_ATT, PS_O, PS_N2, PS_GU, PS_D, PS_COUNT };
constexpr int PIPE_SEQ = 16;            // sequences per group (the matrix-core block)
constexpr int PIPE_THREADS = 512;       // 8 waves: the attention body's workgroup size
constexpr int PIPE_MAX_LAYERS = 32, PIPE_MAX_GROUPS = 128;

// A job: (layer << 26) | (stage << 23) | (group << 16) | index, where index
// is the sequence (RMSNorms), the chunk (matvecs: q|k|v, O and D 16-row
// chunks; G/U the FFN chunk whose G and U halves are adjacent chunks of the
// interleaved block), or sequence * H_KV + KV group (attention: every query
// head of the group).
inline int pipe_job(int layer, int stage, int g, int idx) {
  return (layer << 26) | (stage << 23) | (g << 16) | idx;
}

struct PipeArgs {
  const LayerArgs *L;          // NL layer blocks (device memory): weights, gammas, RoPE, KV cache
  int D, FFN, KV, NL, H_Q, H_KV, batch, ngrp;
  int nq16, nd16, nf16;        // 16-row chunks of q|k|v, of D, of FFN
  const int *state;            // state[0]: the step (its position)
  // BFP (batch-major): layer 0's input, which k_ctl_embed stores, and the
  // last layer's output, which the head reads
  int16_t *h_m;   int8_t *h_e;
  // the stages' outputs as tagged words (m 16 | e 8 | tag 8 bits, the tag
  // of the (step, layer) that stored it), batch-major: h (layer output,
  // D), x1 (RMSNorm 1, D), qkv (D + 2KV), att (D), h1 (D), x2 (RMSNorm 2,
  // D), mlp (FFN)
  unsigned *w_h, *w_x1, *w_qkv, *w_att, *w_h1, *w_x2, *w_mlp;
  int *abort_flag;             // set by a wait that gave up
  // the schedule: per workgroup its matvec role ((stage << 16) | chunk, or
  // -1) and its jobs of the step in order, jobs[jstart[w] .. jstart[w + 1])
  const int *role, *jstart, *jobs;
  int16_t *hist_m;             // optional per-(sequence, step, layer) outputs
  int8_t *hist_e;
  int hist_steps;
  // optional job trace of the launch (each step's launch overwrites the
  // last): per workgroup PIPE_TRACE_JOBS slots of PIPE_TRACE_W words -- the
  // job code + 1, then the 100 MHz clock at the job's start,
  // when its inputs were in (LDS), and when its outputs were stored; a matvec
  // job also stamps its row maxima (5), its tile sums (6) and its
  // epilogue's stores issued (7), an attention job its RoPE and cache row
  // (4), scores (5), softmax (6) and AV chains (7)
  unsigned long long *trace;
};
constexpr int PIPE_TRACE_JOBS = 1024, PIPE_TRACE_W = 8;

// The schedule of one batch size.
struct PipePlan {
  int batch = 0, ngrp = 0, grid = 0, ppw = 0;
  size_t lds = 0;
  double sim_step_us = 0.0;   // the step's length in the schedule's simulation
  std::vector<int> role, jstart, jobs;
};

// Fills pl for `batch` sequences on `cus` compute units and returns 1 when
// the pipelined step covers these dimensions and context, else 0 (the
// caller then runs the per-stage launches).
int pipe_plan(const bfp_dims &d, int batch, int max_ctx, int cus, PipePlan &pl);
// Prepares the kernel for pl (its LDS limit; one workgroup per compute unit
// must fit).
int pipe_prepare(const PipePlan &pl);
// One launch of a decode step on stream s; dev_args holds the PipeArgs.
int launch_pipe_step(const PipePlan &pl, const PipeArgs *dev_args, hipStream_t s);

}  // namespace bfp

namespace bfp {
// Tagged words of the pipelined step for max_batch sequences.
inline size_t pipe_words(const bfp_dims &d, int max_batch) {
  const size_t nq = (size_t)d.D + 2 * (size_t)d.H_KV * d.HD;
  return (size_t)max_batch * (5 * (size_t)d.D + nq + (size_t)d.FFN);
}
}  // namespace bfp
