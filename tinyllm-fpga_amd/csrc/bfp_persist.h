// Argument block and host entry points of the persistent batch-1 decode
// kernel (bfp_persist.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bfp.h"
#include "bfp_layer.h"

namespace bfp {

struct PersistArgs {
  const LayerArgs *L;            // NL per-layer argument blocks (device memory)
  int D, FFN, KV, NL, VOCAB;
  int n_qkv, n_att;              // Q|K|V chunks; attention jobs per layer step
  int o0, g0, d0, n_d;           // first workgroup of the O, G/U and D roles; D chunks
  int steps, n_prompt, n_gen, rtl_loop;
  const int *prompt;             // device, n_prompt ids
  int *out, *last;               // recorded argmaxes; the last head's argmax
  const float *embed;            // (VOCAB, D) float32, tied embedding and head
  const double *norm_w;          // (D,) final norm weight
  // tagged activation words, two of each (step parity): h, h1, att (D),
  // q|k|v (D + 2KV), mlp (FFN); the head's per-workgroup argmax, 4 words each
  unsigned *t_h, *t_h1, *t_att, *t_qkv, *t_mlp, *t_part;
  // the long attention form's score exchange: per head attn_sc_stride
  // entries of 4 tagged words (16 bits of a float64 score each)
  unsigned *sc_buf;
  unsigned *abort_flag;          // set by a wait that gave up
  unsigned long long *clock;     // steps + 1 stamps of the 100 MHz clock, or null
  int16_t *hist_m;               // optional per-(step, layer) outputs
  int8_t *hist_e;
  int hist_steps;
  // optional stage trace (100 MHz clock), written by the first workgroup of
  // each role: per (step, layer) PT_TRACE_LAYER stamps -- 0/1 Q|K|V input
  // ready / output stored, 2 attention job 0's q|k|v input in (wave 0), 3
  // attention output stored, 4/5 O, 6/7 G/U, 8/9 D
  // ready / stored, 10/11 Q|K|V norm / matvec done, 12/13 G/U norm / matvecs
  // done, 14 D matvec done, 15 O matvec done, and attention job 0's phases
  // 16 RoPE (and its q|k|v input) done, 17 scores, 18 softmax, 19 AV chains
  // done -- then per step PT_TRACE_STEP stamps of the head (h ready, slice
  // argmax stored, token known)
  unsigned long long *trace;
};
constexpr int PT_TRACE_LAYER = 20;
constexpr int PT_TRACE_ATT = 16;        // first attention phase stamp (ATT_MARK_* follow)
constexpr int PT_TRACE_STEP = 3;
inline size_t persist_trace_len(int steps, int NL) {
  return (size_t)steps * NL * PT_TRACE_LAYER + (size_t)steps * PT_TRACE_STEP;
}

// Words of tagged device memory the kernel needs (all of it cleared to 0
// before each launch; the abort flag is the last word).
inline size_t persist_words(const bfp_dims &d, int grid) {
  const size_t nq = (size_t)d.D + 2 * (size_t)d.H_KV * d.HD;
  return 2 * (3 * (size_t)d.D + nq + (size_t)d.FFN) + 2 * 4 * (size_t)grid + 1;
}

// Fills the shape fields of p and the grid (one workgroup per compute unit)
// and returns 1 when the persistent kernel covers these dimensions, else 0
// (the caller then decodes through the per-stage graph).
int persist_plan(const bfp_dims &d, int max_ctx, int device, PersistArgs &p, int &grid);
// One launch of the whole decode on stream s, one workgroup per compute
// unit; the argument block is copied to dev_args (device memory,
// sizeof(PersistArgs)) first.
int launch_decode_persist(const PersistArgs &p, PersistArgs *dev_args, int grid, int max_ctx,
                          hipStream_t s);

}  // namespace bfp
