// Host-side internals shared by the libbfp translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "bfp.h"

namespace bfp {

int set_err(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
const char *last_error();
int launch_status(const char *what);

#define HIP_TRY(expr)                                                                   \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess)                                                               \
      return ::bfp::set_err(BFP_EIO, "%s: %s (%s:%d)", #expr, hipGetErrorString(_e),    \
                            __FILE__, __LINE__);                                        \
  } while (0)

#define BFP_TRY(expr)          \
  do {                         \
    int _rc = (expr);          \
    if (_rc) return _rc;       \
  } while (0)

// Scoped device allocations for the host-buffer convenience entry points.
struct DevBuf {
  std::vector<void *> ptrs;
  int alloc(void **p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
      *p = nullptr;
      return set_err(BFP_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    ptrs.push_back(*p);
    return BFP_OK;
  }
  ~DevBuf() {
    for (void *p : ptrs) (void)hipFree(p);
  }
};

int default_waves(int nT);
int launch_matvec(const void *P_m, const void *P_e, int n_out, int n_in, int n_mats, int ring,
                  long long smat_m, long long smat_e, const int16_t *x_m, const int8_t *x_e,
                  long long x_stride, int16_t *y_m, int8_t *y_e, long long y_stride, int waves,
                  hipStream_t stream, int cstride = 1);
int pack(const int16_t *W_m, const int8_t *W_e, int n_out, int n_in, void *P_m, void *P_e,
         hipStream_t s, int cstride = 1);
int quantize_pack_f32(const float *W, int n_out, int n_in, void *P_m, void *P_e, hipStream_t s,
                      int cstride = 1);
int pack_wide(const void *wide_m, const void *wide_e, int n_out, int n_in, void *P_m, void *P_e,
              hipStream_t s, int cstride = 1);
int tile_quantize_f64(const double *v, size_t n, int16_t *m, int8_t *e, hipStream_t s);
int tile_encode_f64(const double *v, size_t n, int16_t *m, int8_t *e, int *inexact,
                    hipStream_t s);
void rope_row(double *cs, int pos, int HD, double base);

}  // namespace bfp

namespace bfp {
struct LayerArgs;
struct HeadArgs;
struct HeadQRow;
struct CtlArgs;
struct EmbedArgs;
// mx_traced: the matrix-core matvecs stamp their phases into the buffer
// set_mx_trace names (batched decodes traced with BFP_DECODE_TRACE).
int launch_layer(const LayerArgs &a, hipStream_t s, bool mx_traced = false);
int set_mx_trace(unsigned long long *p);
// The launch form launch_layer takes for a (BFP_FORM_* bits).
int layer_form(const LayerArgs &a);
int prepare_layer_kernels(int max_ctx, int D, int FFN);
int prepare_head_kernels(int D);
// Raise a kernel's dynamic-LDS limit on the current device to at least
// `bytes` (never lowering it: the limit is process-wide per device).
int raise_lds_limit(const void *f, int bytes);
int head_workgroups(int vocab, int D, int rows_single, int batch, bool have64);
int launch_embed(const EmbedArgs &a, hipStream_t s);
int launch_head(const HeadArgs &a, hipStream_t s);
// The bounded head's copy of the embedding (k_embq_build).
int launch_embq_build(const float *embed, int VOCAB, int D, uint4 *q, HeadQRow *meta, hipStream_t s);
int launch_ctl(const CtlArgs &a, hipStream_t s);
// k_ctl + step increment + the next step's k_embed in one launch; the step
// counter's arrival count lives at state[1 + batch] and must be 0 at entry.
int launch_ctl_embed(const CtlArgs &a, const EmbedArgs &e, hipStream_t s);
struct RtlArgs;
// The composed RTL-exact layer step (bfp_rtl.hip).
int launch_rtl_layer(const RtlArgs &a, hipStream_t s);
struct RtlHeadArgs;
int launch_rtl_head(const RtlHeadArgs &a, hipStream_t s);
struct RtlCtlArgs;
int launch_rtl_ctl(const RtlCtlArgs &a, hipStream_t s);
}  // namespace bfp
