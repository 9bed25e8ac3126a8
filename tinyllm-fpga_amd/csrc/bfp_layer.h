// Device-side argument blocks of the fused decoder-layer and head kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bfp {

enum Stage { ST_N1 = 0, ST_Q, ST_K, ST_V, ST_ATTN, ST_O, ST_H1, ST_N2, ST_G, ST_U, ST_MLP, ST_D,
             ST_HOUT, ST_COUNT };

// Per-sequence stage dump (BFP m/e of every intermediate of one layer
// step, named as gen_smollm_blockfp_bfp.py:398-409 dumps them).  Sequence b
// writes stage s at m[s] + b*mstride[s], e[s] + b*(mstride[s]/16).
struct StageDump {
  int16_t *m[ST_COUNT];
  int8_t *e[ST_COUNT];
  int mstride[ST_COUNT];
};

struct LayerArgs {
  int D, H_Q, H_KV, HD, FFN, KV, max_ctx, batch;
  double inv_sqrt_hd_div;   // math.sqrt(HD), the divisor of the scores
  // 1 / math.sqrt(HD), exact: sqrt(HD) is a power of two (HD = 64: 8), so
  // score / sqrt(HD) == score * score_mul for every score (both round the
  // same real, a power-of-two scaling of the score, subnormals included)
  // and the kernels multiply instead of dividing (a float64 division is a
  // sequence of about ten instructions per score)
  double score_mul;
  // weights of this layer, device layout
  const uint4 *w_qkv_m;     // (D + 2KV) x D   rows: q | k | v
  const int8_t *w_qkv_e;
  const uint4 *w_o_m;       // D x D
  const int8_t *w_o_e;
  const uint4 *w_gu_m;      // 2FFN x D, chunks interleaved G0 U0 G1 U1 ...
  const int8_t *w_gu_e;
  const uint4 *w_d_m;       // D x FFN
  const int8_t *w_d_e;
  const double *g1, *g2;    // (D,) BFP-exact gammas
  const double *rope;       // (max_ctx, HD/2, 2): cos, sin of theta_j(pos)
  // activations, sequence b at base + b*len (m) and base + b*len/16 (e)
  int16_t *h_m;   int8_t *h_e;     // D, layer input and output
  int16_t *h1_m;  int8_t *h1_e;    // D
  int16_t *qkv_m; int8_t *qkv_e;   // D + 2KV, pre-rope
  int16_t *att_m; int8_t *att_e;   // D
  int16_t *mlp_m; int8_t *mlp_e;   // FFN
  int16_t *xn_m;  int8_t *xn_e;    // D, RMSNorm output (multi-sequence path)
  // this layer's KV cache: sequence b, position t, kv head g at
  // ((b*max_ctx + t)*H_KV + g)*HD mantissas and /16 exponents
  int16_t *k_m; int8_t *k_e;
  int16_t *v_m; int8_t *v_e;
  const int *pos_ptr;       // device position (== kv_pos); read when non-null
  int pos_const;            // RoPE position when pos_ptr is null
  int kv_pos_const;         // KV slot when pos_ptr is null and >= 0 (attention over
                            // slots 0..kv_pos); -1: kv_pos = pos
  const double *rope_row;   // when non-null: the (HD/2) x (cos, sin) row of this
                            // launch's RoPE position (positions past the table)
  const StageDump *dump;    // device pointer or null
  // h_out history for per-(step, layer) checks: ((b*hist_steps + pos)*NL + layer)*D
  int16_t *hist_m; int8_t *hist_e;
  int hist_steps, layer, NL;
  // batched decode: h1 and h also as tagged words (batch x D each), read by
  // the RMSNorm workgroups of the O and D launches (k_o_res_norm_mx: norm 2;
  // k_d_res_norm_mx: the next layer's norm 1, with its gamma g1_next), or
  // null; t_abort is set when one of their bounded waits gives up
  unsigned *t_h1, *t_h;
  const double *g1_next;
  // the next layer's Q|K|V weights (the D launch's RMSNorm workgroups touch
  // them while they wait), or this layer's for the last layer
  const uint4 *w_qkv_next_m;
  const int8_t *w_qkv_next_e;
  // batched decode: q|k|v also as tagged words (batch x (D + 2KV)), read by
  // the attention workgroups of the Q|K|V launch (k_qkv_attn_mx), or null
  unsigned *t_qkv;
  int *t_abort;
};

// The composed RTL-exact layer (smollm_layer_bfp.sv) on one sequence: the
// layer's buffers (L.batch == 1; xn holds NORM1 and NORM2 outputs, qkv the
// Q/K/V tiles, att the attention output) plus the engines' tables.
struct RtlArgs {
  LayerArgs L;
  const uint16_t *exp_lut;    // EXP_LUT[1024]
  const int16_t *silu_lut;    // SILU_LUT[65536], indexed by code & 0xFFFF
  const unsigned *freq;       // FREQ_TURNS_Q31[HD/2]
  int pos, kv_pos;            // RoPE position, KV slot (attention over 0..kv_pos)
  const int *pos_ptr;         // device step counter; when set, pos = kv_pos = *pos_ptr
};

// The RTL token loop's per-step control (after the head): record the
// prediction (and the last layer's output), then the next step's input.
struct RtlCtlArgs {
  int *state;                                // {step, token id}: the next step's input
  const int *prompt; int n_prompt;           // device prompt ids
  int *preds;                                // preds[step] = the head's token
  const int *tok;                            // the head's token (device)
  const int16_t *h_m; const int8_t *h_e;     // the last layer's output
  int16_t *hist_m; int8_t *hist_e;           // optional per-step copies of it
  int D;
};

// The FPGA decode head (smollm_decode_head_bfp.sv) on one sequence.
struct RtlHeadArgs {
  int D, VOCAB;
  const int16_t *h_m; const int8_t *h_e;     // final hidden state
  const double *norm_w;                      // final norm gamma (tile_quantize'd on the device)
  int16_t *xn_m; int8_t *xn_e;               // normed hidden
  const uint4 *emb_m; const int8_t *emb_e;   // tile-quantised tied embedding, device layout
  int16_t *lg_m; int8_t *lg_e;               // per-row logits (VOCAB of each)
  int *work;                                 // 3 * VOCAB / 16 ints
  int *token;                                // argmax out (device)
};

// One sequence of the bounded head (k_head_norm's quantised hidden): the
// scale exponent eh (hidden = 2^eh * q up to 2^eh / 2 an element), the sum
// of q, and an upper bound of the hidden's 1-norm.
struct HeadQSeq {
  double h1;
  int eh, sumx;
};
// One embedding row of the bounded head: its scale exponent er (row =
// 2^er * q up to 2^er / 2 an element), sum q, and the row's parts of the
// bound, r1 = 2^(er-1) + 2^-45 max |row| and r2 = 2^(er-1) sum |q| (both 0
// for a zero row).
struct HeadQRow {
  int er, sumw;
  double r1, r2;
};

struct HeadArgs {
  int D, VOCAB, batch, rows_per_wg, n_wg;
  const int16_t *h_m; const int8_t *h_e;   // final hidden (BFP)
  const double *norm_w;                    // (D,) quantised final norm weight
  const float *embed;                      // (VOCAB, D) raw float32 (exact in f64)
  double *part_v; int *part_i;             // (batch, n_wg) per-workgroup argmax
  double *logits;                          // optional (batch, VOCAB)
  double *hn;                              // (batch, D) normed hidden, batch > 1 path
  const float *embedp;                     // (VOCAB, D) the embedding permuted per row, or null:
                                           // [row][(4i + c) * 16 + 4h + j] = embed[row][64i + 4(h + 4j) + c]
  // the bounded head (k_headq_mx + k_headq_pick; all null: not used)
  const uint4 *embq;                       // the embedding as int16, split bytes, matrix-core layout
  const HeadQRow *embq_meta;               // (VOCAB,)
  uint4 *hq_x;                             // the quantised hidden, split bytes, matrix-core layout
  HeadQSeq *hq_seq;                        // (batch,)
  double2 *hq_blk;                         // (batch, VOCAB / 16) per 16-row block: max lower, max upper bound
};

// The bounded head runs from HEAD_SEQ_MIN sequences (with the permuted
// copy's conditions, D % 64 == 0 and D <= 576) unless logits are asked for.
constexpr int HEADQ_SEQ = 64;   // sequences per k_headq_mx workgroup

// Batches from HEAD_SEQ_MIN sequences on run the head on the float64 matrix
// cores (k_head_mx), when the embedding's permuted copy exists and
// D % 64 == 0, D <= 576.
constexpr int HEAD_SEQ_MIN = 32;
inline bool head_seq_form(int D, int batch, bool havep) {
  return havep && batch >= HEAD_SEQ_MIN && D % 64 == 0 && D <= 576;
}
// Rows per workgroup of k_head_mx: the vocabulary over about 128 row groups
// (x 2 workgroups of 32 sequences at batch 64: one per CU), in whole 16-row
// tiles.
inline int head_seq_rows(int vocab) {
  const int r = (vocab + 127) / 128;
  return (r + 15) / 16 * 16;
}

// Attention form by KV capacity: products per producer wave and AV block
// (2 -> 14 positions, 4 -> 28, 8 -> 56); 2, 3 and 4 are the short forms (one
// workgroup per head), 8 the long one (four workgroups per head).
inline int attn_ppw(int max_ctx) {
  return max_ctx <= 128 ? 2 : (max_ctx <= 256 ? 3 : (max_ctx <= 512 ? 4 : 8));
}

// Long attention form: workgroups per head, each owning 16 dimensions.
constexpr int ATT_DSPLIT = 4;
// Doubles per head of the long form's score exchange: workgroup dg's rows
// t = ATT_DSPLIT u + dg at dg * ceil(max_ctx / ATT_DSPLIT) + u, so each
// workgroup's stores and each block of another's loads are contiguous.
__host__ __device__ inline int attn_sc_block(int max_ctx) { return (max_ctx + ATT_DSPLIT - 1) / ATT_DSPLIT; }
__host__ __device__ inline int attn_sc_stride(int max_ctx) { return ATT_DSPLIT * attn_sc_block(max_ctx); }

// Rows per workgroup of the batch > 1 head: 16 row slots x 2 rows for
// D <= 576, x 1 row above (register budget).
inline int head_rows_multi(int D) { return D <= 576 ? 32 : 16; }

struct CtlArgs {
  int batch, n_prompt, n_gen, n_wg, head;
  int *state;                 // [0] = step; [1 + b] = next input token of sequence b
  const int *prompt;          // (batch, n_prompt)
  int *out;                   // (batch, n_gen); (batch, n_prompt + n_gen) with rtl_loop
  const double *part_v; const int *part_i;
  int *last;                  // (batch,) argmax of the last head evaluation
  int rtl_loop;               // loop policy of the FPGA driver instead of the simulator's
};

struct EmbedArgs {
  int D, batch, VOCAB;
  const float *embed;
  const int *state;           // tokens at state[1 + b]
  int16_t *h_m; int8_t *h_e;
};

}  // namespace bfp
