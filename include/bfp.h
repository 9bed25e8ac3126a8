/*
 * libbfp -- MI355X (gfx950) block-floating-point decode datapath, C ABI.
 *
 * The reference has no native API for this path: its interface is the
 * numpy-in/numpy-out function set of its model-level simulator,
 * rtl/vc707/host/gen_smollm_blockfp_full.py (below: full.py).  Each entry
 * point names the function(s) it replaces.  The Python package
 * (tinyllm-fpga_amd/bfp) binds these with ctypes and re-exposes the
 * reference's names.
 *
 * BFP format: a tile is 16 int16 mantissas sharing one int8 exponent;
 * value = m * 2^(e-15)  (rtl/vc707/src/smollm/bfp_format.svh:1-27).
 * "Reference layout": mantissas (rows, in/16, 16) int16 row-major and
 * exponents (rows, in/16) int8, i.e. what full.py:110-119 quantize_W returns.
 *
 * Conventions: every function returns 0 (BFP_OK) or a negative errno-style
 * code; no exception crosses the ABI.  *_d functions take device pointers
 * and a hipStream_t passed as void* (NULL = default stream) and are
 * stream-ordered (asynchronous).  Context functions are synchronous, and a
 * context must not be used from two threads at once.
 * bfp_last_error() returns the message of the calling thread's last error.
 */
#ifndef BFP_H
#define BFP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BFP_OK 0
#define BFP_EINVAL (-22) /* bad argument / shape */
#define BFP_ENOMEM (-12) /* device allocation failed */
#define BFP_EIO (-5)     /* HIP runtime error */
#define BFP_ERANGE (-34) /* position / token beyond the configured capacity */

#define BFP_TILE 16

/* Model dimensions (full.py:54-60 reads them from env vars). */
typedef struct bfp_dims {
  int D, H_Q, H_KV, HD, FFN, NL, MAX_CTX, VOCAB;
} bfp_dims;

/* Weight slots of a layer (full.py:312-318), plus the model-level tables. */
enum bfp_which {
  BFP_WQ = 0, BFP_WK = 1, BFP_WV = 2, BFP_WO = 3, BFP_WG = 4, BFP_WU = 5, BFP_WD = 6,
  BFP_G1 = 7, BFP_G2 = 8,       /* per-layer RMSNorm gammas (D,)           */
  BFP_EMBED = 9,                /* tied embedding (VOCAB, D), layer ignored */
  BFP_NORM_W = 10               /* final norm weight (D,), layer ignored    */
};

const char *bfp_last_error(void);
const char *bfp_version(void);

/* ---------------------------------------------------------------- layout */
/* Bytes of one matrix in the device layout (16-row chunks, tile-major). */
size_t bfp_packed_bytes_m(int n_out, int n_in);
size_t bfp_packed_bytes_e(int n_out, int n_in);

/* Reference layout -> device layout.  Replaces the wide packing of
 * full.py:131-161 / gen_smollm_blockfp_ddr.py:88-119 with this build's HBM
 * layout. */
int bfp_pack_d(const int16_t *W_m, const int8_t *W_e, int n_out, int n_in,
               void *P_m, void *P_e, void *stream);

/* The reference's wide layout -> device layout.  wide_m: (n_out/16, n_in, 16)
 * int16, one 32-byte entry per (16-row chunk, input column) with row
 * chunk*16 + lane at lane; wide_e: (n_out/16, n_in/16, 16) int8, one
 * 16-byte entry per (chunk, tile).  This is the format of the FPGA's DDR3
 * weight image (gen_smollm_blockfp_ddr.py:88-119, read by
 * weight_streamer_bfp_mt.sv at the lbfp_ddr3.svh offsets) and of the
 * per-matrix hex sets (gen_smollm_blockfp_full.py:131-161), one layer of one
 * matrix at a time. */
int bfp_pack_wide_d(const void *wide_m, const void *wide_e, int n_out, int n_in, void *P_m,
                    void *P_e, void *stream);

/* Device layout -> reference layout (inverse of bfp_pack_d). */
int bfp_unpack_d(const void *P_m, const void *P_e, int n_out, int n_in,
                 int16_t *W_m, int8_t *W_e, void *stream);

/* ----------------------------------------------------------- quantisation */
/* tile_quantize (full.py:90-97) of n float64 values (n % 16 == 0):
 * m (n) int16, e (n/16) int8. */
int bfp_tile_quantize_f64_d(const double *v, size_t n, int16_t *m, int8_t *e, void *stream);
/* Same for float32 input (widened exactly, as full.py:319 does). */
int bfp_tile_quantize_f32_d(const float *v, size_t n, int16_t *m, int8_t *e, void *stream);
/* quantize_W (full.py:110-119) of a float32 (n_out, n_in) matrix straight
 * into the device layout. */
int bfp_quantize_pack_f32_d(const float *W, int n_out, int n_in, void *P_m, void *P_e,
                            void *stream);
/* tile_decode (full.py:100-102): (m, e) -> float64, exact. */
int bfp_tile_decode_d(const int16_t *m, const int8_t *e, size_t n, double *v, void *stream);
/* The encoding of values that are already BFP, as the reference's float64
 * arrays hold them (full.py:105-107: every stage keeps decoded tiles):
 * tile_quantize's tile, except where that tile would round a value -- the
 * raw form of a tile whose largest magnitude is the mantissa -32768, which
 * tile_quantize maps to exponent e+1, halving odd mantissas -- in which case
 * the tile one exponent lower that holds every value exactly.  Decoding the
 * result gives v back whenever v is BFP-exact; other tiles are quantised as
 * tile_quantize does, and set *inexact = 1 (inexact: optional device int,
 * left alone otherwise).  The inverse of bfp_tile_decode_d on decoded
 * tiles. */
int bfp_tile_encode_f64_d(const double *v, size_t n, int16_t *m, int8_t *e, int *inexact,
                          void *stream);

/* ------------------------------------------------------- float64 leaf ops */
/* The reference simulator's float64 leaf ops (full.py:236-258), float64 in
 * and out (device pointers), stream-ordered.  Sums use numpy's pairwise
 * order, every product and quotient is rounded separately. */
/* rmsnorm_fp (full.py:236-238) of batch rows of n (n % 16 == 0, n <= 4096),
 * gamma shared: y = fp_quantize_vec((x*gamma) / sqrt(mean(x*x) + eps)). */
int bfp_rmsnorm_fp_d(const double *x, const double *gamma, int n, int batch, double eps,
                     double *y, void *stream);
/* silu_fp (full.py:241-242): y = fp_quantize_vec(x / (1 + exp(-x))), n % 16 == 0. */
int bfp_silu_fp_d(const double *x, size_t n, double *y, void *stream);
/* softmax_fp (full.py:245-247) of batch rows of n (n <= 4096):
 * y = exp(x - max) / sum, float64 (not quantised). */
int bfp_softmax_fp_d(const double *x, int n, int batch, double *y, void *stream);
/* The (cos, sin) pairs rope_fp (full.py:250-258) rotates by at position pos:
 * cs[2j], cs[2j+1] = cos, sin of 1.0 / (base ** (2*j/head_dim)) * pos for
 * j < head_dim/2, with the host's libm as CPython evaluates them.  Host
 * code (no device). */
int bfp_rope_cos_sin(int pos, int head_dim, double base, double *cs);
/* rope_fp of n_heads heads of 64 (x, y: n_heads*64 float64): out[j] =
 * a*c - b*s, out[j+32] = b*c + a*s (a = x[j], b = x[j+32]), fp_quantize_vec
 * per head.  cs: device copy of bfp_rope_cos_sin(pos, 64, base). */
int bfp_rope_fp_d(const double *x, int n_heads, const double *cs, double *y, void *stream);

/* ---------------------------------------------------------------- matvec */
/* matvec_hw_golden (full.py:217-233) for n_mats independent problems in one
 * launch: y_r = W_r x_r, r < n_mats.  W_r is in the device layout at
 * P_m + r*mat_stride_m bytes / P_e + r*mat_stride_e bytes; x_r mantissas at
 * x_m + r*x_stride elements and exponents at x_e + r*(x_stride/16); y_r at
 * y_m + r*y_stride, y_e + r*(y_stride/16).  Output is the BFP (m, e) of
 * fp_quantize_vec over 16-row tiles, computed in exact integer arithmetic.
 * n_out % 16 == 0, n_in % 16 == 0.  waves = 0 picks the default workgroup
 * shape; otherwise 1, 2, 3, 4, 6, 8 or 9 waves per 16-row chunk. */
int bfp_matvec_d(const void *P_m, const void *P_e, int n_out, int n_in, int n_mats,
                 long long mat_stride_m, long long mat_stride_e, const int16_t *x_m,
                 const int8_t *x_e, long long x_stride, int16_t *y_m, int8_t *y_e,
                 long long y_stride, int waves, void *stream);

/* Same, but problem r reads matrix (r mod ring) -- a ring of distinct weight
 * copies, so a long batch streams from HBM rather than from cache.  ring = 0
 * means ring = n_mats.  (Benchmark form; no reference counterpart.) */
int bfp_matvec_ring_d(const void *P_m, const void *P_e, int n_out, int n_in, int n_mats,
                      int ring, long long mat_stride_m, long long mat_stride_e,
                      const int16_t *x_m, const int8_t *x_e, long long x_stride, int16_t *y_m,
                      int8_t *y_e, long long y_stride, int waves, void *stream);

/* Measurement probe, no reference counterpart: reads [p, p + bytes) once
 * with 16-byte loads (non-temporal when nt != 0, the matvec's weight-stream
 * policy), each of n_wg workgroups of 256 threads streaming one contiguous
 * range and folding it into one word, stored to out[w] (n_wg words) only
 * when it equals a fixed sentinel, so out is normally left untouched.  Its
 * bytes / time is the practical HBM read ceiling the matvec is compared
 * with (fastest with 16 KB per workgroup).  bytes % 16 == 0, every
 * workgroup gets at least one word and at most 1 GiB. */
int bfp_probe_read_d(const void *p, size_t bytes, uint32_t *out, int n_wg, int nt, void *stream);

/* Host-buffer convenience form of matvec_hw_golden: W in the reference
 * layout, x and y in host memory.  Allocates and frees device memory. */
int bfp_matvec_h(const int16_t *W_m, const int8_t *W_e, int n_out, int n_in,
                 const int16_t *x_m, const int8_t *x_e, int16_t *y_m, int8_t *y_e);

/* ------------------------------------------------------- RTL-exact ops */
/* The FPGA engines' bit-exact leaf ops (rtl/vc707/src/smollm/<op>_bfp.sv as
 * specified by rtl/vc707/host/gen_*_bfp_golden.py).  Not on the
 * model-level simulator's token path; per-op semantics of the hardware. */

/* EXP_LUT[1024] (sim/gen_exp_lut.py:36-42), SILU_LUT[65536] indexed by the
 * int16 code & 0xFFFF (sim/gen_swiglu_lut.py:27-44), FREQ_TURNS_Q31[hd/2]
 * (sim/gen_rope_freq_table.py:31-37), built on the host; NULL skips one. */
int bfp_rtl_tables(uint16_t *exp_lut, int16_t *silu_lut, uint32_t *freq_q31, int head_dim,
                   double base);
/* matvec_bfp_engine.sv (gen_matvec_bfp_golden.py:53-108): sequential
 * tile alignment, 48-bit saturating accumulator, per-row (m, e).  W in the
 * reference layout; y_e has one exponent per row. */
int bfp_rtl_matvec_d(const int16_t *x_m, const int8_t *x_e, const int16_t *W_m, const int8_t *W_e,
                     int n_out, int n_in, int16_t *y_m, int8_t *y_e, void *stream);
/* requant_mant + chunk emax (smollm_layer_bfp.sv:1387-1396,1672-1693):
 * per-lane exponents -> one exponent per 16 lanes. */
int bfp_rtl_requant_d(const int16_t *m, const int8_t *e, int n, int16_t *out_m, int8_t *out_e,
                      void *stream);
/* rmsnorm_bfp.sv (gen_rmsnorm_bfp_golden.py:42-142) of batch vectors of D;
 * gamma shared. */
int bfp_rtl_rmsnorm_d(const int16_t *x_m, const int8_t *x_e, const int16_t *g_m, const int8_t *g_e,
                      int D, int batch, int16_t *y_m, int8_t *y_e, void *stream);
/* rope_bfp.sv + cordic_sincos.sv (gen_rope_bfp_golden.py:37-121) of n_heads
 * 64-wide heads (x_e per 16-tile); y_e has one exponent per element. */
int bfp_rtl_rope_d(const int16_t *x_m, const int8_t *x_e, int pos, int n_heads,
                   const uint32_t *freq_q31, int16_t *y_m, int8_t *y_e, void *stream);
/* softmax_bfp.sv (gen_softmax_bfp_golden.py:33-78): batch problems of n
 * <= 4096 mantissas at x_m + b*stride sharing exponent x_e[b]; y_e[b]. */
int bfp_rtl_softmax_d(const int16_t *x_m, const int8_t *x_e, int n, int batch, int stride,
                      const uint16_t *exp_lut, int16_t *y_m, int8_t *y_e, void *stream);
/* swiglu_bfp.sv (gen_swiglu_bfp_golden.py:43-78). */
int bfp_rtl_swiglu_d(const int16_t *g_m, const int8_t *g_e, const int16_t *u_m, const int8_t *u_e,
                     int n, const int16_t *silu_lut, int16_t *y_m, int8_t *y_e, void *stream);
/* residual_bfp.sv (gen_residual_bfp_golden.py:23-48). */
int bfp_rtl_residual_d(const int16_t *a_m, const int8_t *a_e, const int16_t *b_m,
                       const int8_t *b_e, int n, int16_t *y_m, int8_t *y_e, void *stream);
/* The decode head's bfp_gt running argmax (smollm_decode_head_bfp.sv:
 * 253-274,322-324,399-430) over batch rows of n (m, e) pairs (one exponent
 * per element); work: 3*batch*n/16 int32 of device scratch. */
int bfp_rtl_argmax_d(const int16_t *m, const int8_t *e, int n, int batch, int32_t *work,
                     int32_t *idx, void *stream);
/* No counterpart in the reference: bfp_rtl_argmax_d for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The same kernel and result; its
 * workspace is the library's static device scratch (3 MiB per GPU, held
 * until the process ends), so it calls no allocator.  batch * n/16 must be
 * at most 262144 (e.g. 64 rows of a 65536-entry vocabulary), else
 * BFP_EINVAL.  Calls that overlap on one GPU share the scratch and race. */
int bfp_rtl_argmax_static_d(const int16_t *m, const int8_t *e, int n, int batch, int32_t *idx,
                            void *stream);

/* ------------------------------------------------------------- model */
/* A context owns one GPU's copy of the model (BFP weights in the device
 * layout, float64 gammas, the float32 tied embedding, the RoPE table), the
 * KV cache for max_batch sequences x dims->MAX_CTX positions, and a stream.
 * Replaces the module-level model state of full.py:299-428.  Returns NULL
 * on error (see bfp_last_error). */
typedef struct bfp_ctx bfp_ctx;
bfp_ctx *bfp_create(const bfp_dims *dims, int device, int max_batch);
void bfp_destroy(bfp_ctx *ctx);
int bfp_get_dims(const bfp_ctx *ctx, bfp_dims *out);

/* Load one tensor (which = enum bfp_which).  Matrices (rows x cols as in
 * full.py:312-318) from float32 -- quantize_W on the device (full.py:110-119)
 * -- or from the reference layout (m, e).  BFP_G1/G2/NORM_W: float32
 * (quantised as fp_quantize_vec, full.py:322-323,413) or (m, e).
 * BFP_EMBED: float32 only (the head uses the raw table, full.py:439); a
 * NaN or infinity in it is refused with BFP_EINVAL (the batched head's
 * logit bounds hold for finite values only).
 * layer is ignored for EMBED and NORM_W.  Host buffers are copied. */
int bfp_load_weights(bfp_ctx *ctx, int which, int layer, const float *fp32, const int16_t *m,
                     const int8_t *e);

/* Load one matrix of one layer (which = BFP_WQ .. BFP_WD) from host
 * buffers in the reference's wide layout (see bfp_pack_wide_d): the region
 * slice of a DDR3 weight image or of a *_m.hex/_e.hex set for that layer.
 * Replaces the FPGA's weight streamer reading the image
 * (weight_streamer_bfp_mt.sv, lbfp_ddr3.svh:45-86). */
int bfp_load_weights_wide(bfp_ctx *ctx, int which, int layer, const void *wide_m,
                          const void *wide_e);

/* Zero the KV cache (the reference starts every run from zeros, full.py:426-428). */
int bfp_reset_kv(bfp_ctx *ctx);

/* Copy KV-cache positions [t0, t0+n) of one layer and sequence between the
 * device and host buffers: k_m/v_m are n x H_KV*HD int16 (post-RoPE K, raw
 * V, as full.py:270-272 stores them), k_e/v_e n x H_KV*HD/16 int8.
 * write != 0 uploads (e.g. the preloaded cache of gen_smollm_blockfp_bfp.py
 * :209-216, or a saved cache), write == 0 reads back. */
int bfp_kv_io(bfp_ctx *ctx, int layer, int seq, int t0, int n, int16_t *k_m, int8_t *k_e,
              int16_t *v_m, int8_t *v_e, int write);

/* Per-stage BFP outputs of one layer step, as gen_smollm_blockfp_bfp.py:398-409
 * dumps them (Q and K after RoPE).  Host buffers of batch x len mantissas and
 * batch x len/16 exponents; NULL entries are skipped.  Stage order:
 * N1 Q K V ATTN O H1 N2 G U MLP D HOUT, lengths D D KV KV D D D D FFN FFN FFN D D. */
#define BFP_N_STAGES 13
typedef struct bfp_stage_dump {
  int16_t *m[BFP_N_STAGES];
  int8_t *e[BFP_N_STAGES];
} bfp_stage_dump;

/* fwd_layer (full.py:261-293) at position pos (kv_pos = pos) for batch
 * sequences: h (batch x D BFP, host) -> out; writes the KV cache slot pos of
 * this layer. */
int bfp_layer_step(bfp_ctx *ctx, int layer, int pos, int batch, const int16_t *h_m,
                   const int8_t *h_e, int16_t *out_m, int8_t *out_e, bfp_stage_dump *dump);

/* fwd_layer(h, lw, pos, kv, kv_pos) (full.py:261-293) with pos and kv_pos
 * apart, as the single-layer harness drives them
 * (gen_smollm_blockfp_bfp.py:42-43,332-344): RoPE at position pos (any
 * pos >= 0; positions past MAX_CTX get their cos/sin row computed on the
 * host), K and V written to slot kv_pos (< MAX_CTX) of this layer's cache,
 * attention over slots 0..kv_pos.  bfp_layer_step is this with
 * kv_pos = pos. */
int bfp_layer_step_kv(bfp_ctx *ctx, int layer, int pos, int kv_pos, int batch, const int16_t *h_m,
                      const int8_t *h_e, int16_t *out_m, int8_t *out_e, bfp_stage_dump *dump);

/* bfp_kv_io in the reference's own cache form: k, v are n x H_KV x HD
 * float64 host arrays, rows [t0, t0+n) of kv['k'] / kv['v']
 * (full.py:270-272,426-428).  write != 0 encodes them into the cache with
 * bfp_tile_encode_f64_d (values the reference wrote keep their tiles) and
 * fails with BFP_EINVAL, the cache rows then undefined, when a value is not
 * BFP-exact; write == 0 decodes the cache into them (exact). */
int bfp_kv_io_f64(bfp_ctx *ctx, int layer, int seq, int t0, int n, double *k, double *v,
                  int write);

/* matvec_hw_golden (full.py:217-233) of batch input vectors with one of the
 * context's loaded matrices (which = BFP_WQ .. BFP_WD of layer): x (batch x
 * n_in BFP, host) -> y (batch x n_out BFP, host), the raw (m, e) that
 * fp_quantize_vec forms over 16-row tiles. */
int bfp_matvec(bfp_ctx *ctx, const int16_t *x_m, const int8_t *x_e, int which, int layer,
               int batch, int16_t *y_m, int8_t *y_e);

/* The FPGA's decoder layer (rtl/vc707/src/smollm/smollm_layer_bfp.sv:
 * 1603-2600, the RTL engines of the bfp_rtl_* ops wired in its FSM order) on
 * one sequence, with this context's weights (gammas through tile_quantize,
 * as the gamma ROM holds them) and KV cache: NORM1, Q/K/V matvecs on the
 * engine with a per-chunk re-tile, RoPE-CORDIC at pos (0..2047, the RTL's
 * 11-bit port) and re-tile, KV write at slot kv_pos, per head QK on the
 * engine, pre-aligned softmax, AV over one 16-input tile (positions 0..15
 * only, as :2139-2180 drives it), O, residual, NORM2, G, U, SwiGLU, D,
 * residual.  Stage dumps as bfp_layer_step's (Q and K after RoPE).  The
 * reference's acceptance bound against the float layer is 256 mantissa LSB
 * and 1 exponent step (sim/tb_smollm_layer_bfp.sv:132-175). */
int bfp_rtl_layer_step(bfp_ctx *ctx, int layer, int pos, int kv_pos, const int16_t *h_m,
                       const int8_t *h_e, int16_t *out_m, int8_t *out_e, bfp_stage_dump *dump);

/* The FPGA decode head (rtl/vc707/src/smollm/smollm_decode_head_bfp.sv:
 * 303-430) on one hidden state: the RMSNorm engine with the final norm
 * gamma (through tile_quantize, as its ROM holds it), the lm_head on the
 * matvec engine over the tile-quantised tied embedding (16 rows per chunk,
 * per-row (m, e)), and the bfp_gt running argmax (sentinel (-32768, -128),
 * strict > within and across chunks).  h: D BFP on the host; logit_m /
 * logit_e (VOCAB each, host) may be NULL.  D a multiple of 64, VOCAB of 16. */
int bfp_rtl_head(bfp_ctx *ctx, const int16_t *h_m, const int8_t *h_e, int16_t *logit_m,
                 int8_t *logit_e, int32_t *token);

/* The FPGA's token loop (rtl/vc707/src/smollm/autoregress_bfp_top.sv:357-386)
 * over the composed RTL layer (bfp_rtl_layer_step) and head (bfp_rtl_head),
 * sequence 0: step s embeds prompt[s] while s < n_prompt, else the
 * prediction of step s-1 (tile_quantize of its embedding row), runs every
 * layer at position and KV slot s, and records its prediction in preds[s]
 * (n_prompt + n_gen of them, at most the KV capacity and 2048).  hist_m /
 * hist_e (optional, host): the last layer's output per step. */
int bfp_rtl_decode(bfp_ctx *ctx, const int32_t *prompt, int n_prompt, int n_gen, int32_t *preds,
                   int16_t *hist_m, int8_t *hist_e);

/* Decode head (full.py:438-440): final norm, float64 logits over the raw
 * embedding, first-index argmax.  logits may be NULL: then, from 32
 * sequences on (contexts made with max_batch >= 32), the argmax comes from
 * the bounded head, which forms float64 logits only for the rows that can
 * hold the largest (an exact int16 dot product brackets every logit) and
 * returns the same index; the environment variable BFP_HEAD_BOUNDED=0
 * keeps the full head. */
int bfp_head(bfp_ctx *ctx, int batch, const int16_t *h_m, const int8_t *h_e, double *logits,
             int32_t *argmax);

/* The golden-token loop (full.py:426-443) on the device for batch
 * independent sequences, including the reference's quirk that step
 * n_prompt re-feeds the last prompt token.  prompt: batch x n_prompt;
 * tokens_out: batch x n_gen.  hist_m/hist_e (optional): every layer's
 * output at every step, (batch, n_prompt + n_gen, NL, D) / (..., D/16).
 * The KV cache is overwritten from position 0. */
#define BFP_DECODE_NO_GRAPH 1
#define BFP_DECODE_STEP_TIMES 2   /* record one HIP event per step */
/* Loop policy of the FPGA driver (autoregress_bfp_top.sv:357-386, the
 * tb_full_bfp.cpp auto-feed run) instead of the simulator's: step s feeds
 * prompt[s] while s < n_prompt, else step s-1's argmax (no repeat of the last
 * prompt token); every step's argmax is recorded, so tokens_out holds
 * batch x (n_prompt + n_gen) tokens (the RTL's result_buf / RTL_TOKENS). */
#define BFP_DECODE_RTL_LOOP 4
/* Batch 1 runs the whole decode as one persistent launch (one
 * workgroup per compute unit, stages handing over through device-coherent
 * memory) when the dimensions allow it (D <= 576, FFN <= 1536, NL >= 2, the
 * Q|K|V, O, G/U and D chunks of a layer within the compute units); else, or
 * with this flag or the environment variable BFP_PERSIST=0, each step is a
 * replayed graph of per-stage kernels.  Both give identical outputs. */
#define BFP_DECODE_NO_PERSIST 8
/* Record the device clock (100 MHz) for bfp_decode_trace: on the persistent
 * path as each stage's input becomes ready and as its output is stored, in
 * the first workgroup of each role; on the batched matrix-core path at the
 * phases of every block of the four matvec kernels; on the pipelined step
 * (BFP_DECODE_PIPE) at the start, inputs-in, phases and end of every job of
 * the last step's launch. */
#define BFP_DECODE_TRACE 16
/* Test hook for the bounded waits: the decode's abort word is set after its
 * per-decode clearing and before its first launch, so every wait for
 * hand-off words that does not find them at once gives up through its own
 * bounded loop, the kernels still run to their end, and bfp_decode returns
 * BFP_EIO.  The next decode clears the word again. */
#define BFP_DECODE_ABORT_TEST 32
/* The pipelined batched step: each step's layers as one launch (one
 * workgroup per compute unit; the sequences pass the stages in groups of 16,
 * the stages handing over through device-coherent memory), when the
 * dimensions allow it (HD = 64, D <= 640, FFN <= 1536, D and FFN multiples of
 * 64, NL <= 32, at most 4 query heads per KV group, a KV capacity of at most
 * 256, the Q|K|V, O, G/U and D chunks of a layer within the compute units).  BFP_DECODE_PIPE asks for it at any
 * batch size; without it, batches of at least BFP_PIPE_MIN_BATCH sequences
 * (environment; unset or 0: none) take it; BFP_DECODE_NO_PIPE keeps the
 * per-stage launches.  Both give identical outputs. */
#define BFP_DECODE_NO_PIPE 64
#define BFP_DECODE_PIPE 128
int bfp_decode(bfp_ctx *ctx, const int32_t *prompt, int n_prompt, int n_gen, int batch,
               int32_t *tokens_out, int16_t *hist_m, int8_t *hist_e, int flags);
/* How the last bfp_decode ran: BFP_PATH_PERSIST (one persistent launch),
 * BFP_PATH_GRAPH (a replayed graph per step) or BFP_PATH_EAGER (per-stage
 * launches, BFP_DECODE_NO_GRAPH); -1 before any decode. */
#define BFP_PATH_GRAPH 0
#define BFP_PATH_PERSIST 1
#define BFP_PATH_EAGER 2
int bfp_decode_path(const bfp_ctx *ctx);
/* The launch form of the last bfp_decode's layers (no reference
 * counterpart; for tests and tuning): BFP_FORM_SINGLE (per-sequence stage
 * kernels, batches below 4), BFP_FORM_MULTI (multi-sequence kernels on the
 * vector unit), or BFP_FORM_MX (int8 matrix-core matvecs) with
 * BFP_FORM_QKV_ATTN when Q|K|V and attention ran as one launch (with
 * BFP_FORM_ATT_GROUP when its attention workgroups each took a whole KV
 * group's query heads: contexts of at most 256, the default; the environment
 * variable BFP_ATT_GROUP=0 keeps one head per workgroup) and
 * BFP_FORM_NORM_FUSED when the RMSNorms ran inside the O and D launches;
 * BFP_FORM_PERSIST for the persistent batch-1 decode, BFP_FORM_PIPE for the
 * pipelined batched step; -1 before any decode. */
#define BFP_FORM_SINGLE 0
#define BFP_FORM_MULTI 1
#define BFP_FORM_MX 2
#define BFP_FORM_QKV_ATTN 4
#define BFP_FORM_NORM_FUSED 8
#define BFP_FORM_PERSIST 16
#define BFP_FORM_PIPE 32
#define BFP_FORM_ATT_GROUP 64
int bfp_decode_form(const bfp_ctx *ctx);
/* The stage trace of the last decode run with BFP_DECODE_TRACE on the
 * persistent path: per (step, layer) 20 stamps -- 0/1 Q|K|V input ready /
 * output stored, 2 the first attention job's q|k|v input in, 3 attention
 * output stored, 4/5 O, 6/7 G/U, 8/9 D
 * input ready / output stored, 10/11 Q|K|V norm / matvec done, 12/13 G/U
 * norm / matvecs done, 14 D matvec done, 15 O matvec done, and the first
 * attention job's phases: 16 q|k|v in and RoPE done, 17 scores, 18 softmax,
 * 19 AV chains done -- then per step 3 head stamps (h ready, slice argmax
 * stored, token known; 0 where the step ran no head).  After a batched
 * decode on the matrix cores: per kernel (Q|K|V, O, G/U, D), per block (up to
 * 1024), 6 stamps -- entry, exponents staged, row maxima reduced, tile sums
 * formed, sums reduced, epilogue done -- from the last launch of each kernel
 * (0 for blocks that did not run); in the Q|K|V kernel's rows the grouped
 * attention workgroups of the joined launch follow its matvec blocks, with
 * entry, q|k|v in, RoPE and staged rows, scores, softmax and AV chains.
 * After a pipelined decode: per workgroup
 * 1024 job slots of 8 stamps -- the job code + 1 ((layer << 26) | (stage <<
 * 23) | (group << 16) | index; 0 for an unused slot), start, inputs in,
 * end, then a matvec job's row maxima (5), tile sums (6) and epilogue
 * stored (7), an attention job's RoPE (4), scores (5), softmax (6) and AV
 * chains (7) -- from the last step's launch.
 * Copies up to n values and returns how many were recorded (0 if none). */
int bfp_decode_trace(const bfp_ctx *ctx, uint64_t *out, size_t n);

/* Device time (HIP events) of the last bfp_decode: all steps, and the steps
 * from n_prompt on. */
int bfp_decode_time(const bfp_ctx *ctx, float *total_ms, float *gen_ms);
/* Per-step device times of the last decode run with BFP_DECODE_STEP_TIMES;
 * copies up to n values, returns the number of steps recorded.  (On the
 * persistent path they are read from the device clock at each step's start
 * in workgroup 0, always recorded.) */
int bfp_decode_step_times(const bfp_ctx *ctx, float *ms, int n);

/* ------------------------------------------------------------ vocabulary */
/* Token-id -> text for human-readable output.  The table is the "BFPV" v1
 * file written by rtl/vc707/host/gen_bfp_vocab_bin.py:10-17,69-74 (magic,
 * u32 version, u32 n_tokens, u32 blob_size, n_tokens x {u32 offset, u32
 * length}, blob; little-endian), as read by the reference's native client
 * (rtl/vc707/host/bfp_client.cpp:876-903, struct Vocab::load).  Host code:
 * no device is needed. */
typedef struct bfp_vocab bfp_vocab;
/* Vocab::load (bfp_client.cpp:879-903): bad magic, a version other than 1 or
 * a short file -> BFP_EINVAL; *out = NULL on error. */
int bfp_vocab_open(const char *path, bfp_vocab **out);
/* The same from a buffer of n bytes (copied). */
int bfp_vocab_parse(const void *buf, size_t n, bfp_vocab **out);
void bfp_vocab_close(bfp_vocab *v);
/* n_tokens of the table (0 for NULL). */
int bfp_vocab_size(const bfp_vocab *v);
/* Vocab::bytes_for (bfp_client.cpp:906-911): a token's raw bytes (not
 * NUL-terminated, owned by v); an id outside [0, n_tokens) or an entry
 * reaching past the blob gives len 0. */
int bfp_vocab_token(const bfp_vocab *v, int id, const char **bytes, size_t *len);
/* decode_tokens (bfp_client.cpp:1020-1027): the ids' bytes concatenated,
 * read as lenient UTF-8 and repaired for Windows-1252 mojibake
 * (fix_mojibake, :973-1018).  Writes at most cap-1 bytes and a NUL to out
 * (out may be NULL with cap 0) and returns the full text length, or a
 * negative error code. */
long long bfp_vocab_decode(const bfp_vocab *v, const int32_t *ids, int n, char *out, size_t cap);

/* Narrow embedding rows (m, e) of n token ids from the reference's
 * EMBED_LU table (gen_smollm_blockfp_ddr.py:203-216: mantissa row d int16
 * per token, exponent rows of e_row_bytes >= D/16 int8), as the FPGA's
 * embedding lookup reads them, gathered on the device: out_m (n, D) int16,
 * out_e (n, D/16) int8.  All pointers are device pointers; an id outside
 * [0, vocab) yields the zero tile (m 0, e -127), as tile_quantize maps a
 * zero vector. */
int bfp_embed_gather_d(const void *lu_m, const void *lu_e, int vocab, int D, int e_row_bytes,
                       const int32_t *ids, int n, int16_t *out_m, int8_t *out_e, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* BFP_H */
