// The model-level simulator's float64 leaf ops as standalone kernels: the
// drop-in forms of rmsnorm_fp, silu_fp, softmax_fp and rope_fp
// (rtl/vc707/host/gen_smollm_blockfp_full.py:236-258).  The fused layer
// kernels (bfp_layer.hip) inline the same arithmetic; these entry points
// expose each op on its own, float64 in and float64 out as the reference's
// functions are.  Every sum uses numpy's pairwise order and every product
// and quotient is rounded on its own (-ffp-contract=off).
#include <math.h>

#include "bfp.h"
#include "bfp_device.h"
#include "bfp_f64.h"
#include "bfp_internal.h"

namespace bfp {

constexpr int LEAF_BS = 256;
constexpr int LEAF_MAX_N = 4096;   // pairwise_sum_block's range

// rmsnorm_fp (full.py:236-238) of row blockIdx.x: v = np.mean(x*x) + eps
// (numpy's pairwise sum, then / n), y = fp_quantize_vec((x*gamma)/np.sqrt(v)).
__global__ __launch_bounds__(LEAF_BS) void k_rmsnorm_fp(const double *__restrict__ x,
                                                        const double *__restrict__ g, int n,
                                                        double eps, double *__restrict__ y) {
  __shared__ double leaf[PW_MAX_LEAVES];
  const double *xv = x + (long long)blockIdx.x * n;
  double *yv = y + (long long)blockIdx.x * n;
  const double s = pairwise_sum_block_g(
      [xv](int i) {
        const double v = xv[i];
        return v * v;
      },
      n, leaf);
  const double rt = sqrt(s / (double)n + eps);
  for (int base = 0; base < n; base += LEAF_BS) {   // uniform: all lanes quantise
    const int i = base + threadIdx.x;
    const bool ok = i < n;
    const double v = ok ? (xv[i] * g[i]) / rt : 0.0;
    int e;
    const int m = quantize16_lanes(v, e);
    if (ok) yv[i] = bfp_val(m, e);
  }
}

// silu_fp (full.py:241-242): fp_quantize_vec(x / (1.0 + np.exp(-x))); one
// element per thread, tiles of 16 consecutive lanes.
__global__ __launch_bounds__(LEAF_BS) void k_silu_fp(const double *__restrict__ x, long long n,
                                                     double *__restrict__ y) {
  const long long i = (long long)blockIdx.x * LEAF_BS + threadIdx.x;
  const bool ok = i < n;
  const double v = ok ? x[i] : 0.0;
  int e;
  const int m = quantize16_lanes(v / (1.0 + exp_f64(-v)), e);
  if (ok) y[i] = bfp_val(m, e);
}

// softmax_fp (full.py:245-247) of row blockIdx.x: e = np.exp(x - x.max());
// e / e.sum() (pairwise), float64 probabilities (not quantised).
__global__ __launch_bounds__(LEAF_BS) void k_softmax_fp(const double *__restrict__ x, int n,
                                                        double *__restrict__ y) {
  __shared__ double ex[LEAF_MAX_N];
  __shared__ double leaf[PW_MAX_LEAVES];
  __shared__ double red[LEAF_BS / 64];
  const double *xv = x + (long long)blockIdx.x * n;
  double *yv = y + (long long)blockIdx.x * n;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  double mx = -INFINITY;
  for (int t = tid; t < n; t += LEAF_BS) mx = fmax(mx, xv[t]);
  mx = fmax(mx, peer<32>(mx));
  mx = fmax(mx, peer<16>(mx));
  mx = fmax(mx, peer<8>(mx));
  mx = fmax(mx, peer<4>(mx));
  mx = fmax(mx, peer<2>(mx));
  mx = fmax(mx, peer<1>(mx));
  if (l == 0) red[w] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int i = 1; i < LEAF_BS / 64; ++i) mx = fmax(mx, red[i]);
  for (int t = tid; t < n; t += LEAF_BS) ex[t] = exp_f64(xv[t] - mx);
  __syncthreads();
  const double sum = pairwise_sum_block(ex, n, leaf);
  for (int t = tid; t < n; t += LEAF_BS) yv[t] = ex[t] / sum;
}

// rope_fp (full.py:250-258) of one 64-wide head per wave: out[j] = a*c - b*s,
// out[j+32] = b*c + a*s with (c, s) from cs, then fp_quantize_vec.
__global__ __launch_bounds__(64) void k_rope_fp(const double *__restrict__ x,
                                                const double *__restrict__ cs,
                                                double *__restrict__ y) {
  const long long i = (long long)blockIdx.x * 64 + threadIdx.x;
  int e;
  const int m = rope_lane(x[i], cs, e);
  y[i] = bfp_val(m, e);
}

// theta_j = 1.0 / (base ** (2*j/HD)) * pos, then math.cos / math.sin
// (full.py:253-254): CPython's float ** and math.cos/sin call the C
// library's pow/cos/sin, and 2*j/HD is a correctly rounded int division.
void rope_row(double *cs, int pos, int HD, double base) {
  for (int j = 0; j < HD / 2; ++j) {
    const double theta = 1.0 / pow(base, (double)(2 * j) / (double)HD) * (double)pos;
    cs[2 * j] = cos(theta);
    cs[2 * j + 1] = sin(theta);
  }
}

}  // namespace bfp

using namespace bfp;

extern "C" {

int bfp_rmsnorm_fp_d(const double *x, const double *gamma, int n, int batch, double eps,
                     double *y, void *stream) {
  if (!x || !gamma || !y) return set_err(BFP_EINVAL, "rmsnorm_fp: null pointer");
  if (n <= 0 || n % 16 || n > LEAF_MAX_N || batch < 0)
    return set_err(BFP_EINVAL, "rmsnorm_fp: n=%d must be a multiple of 16 in [16, %d], batch=%d",
                   n, LEAF_MAX_N, batch);
  if (batch == 0) return BFP_OK;
  hipLaunchKernelGGL(k_rmsnorm_fp, dim3(batch), dim3(LEAF_BS), 0, (hipStream_t)stream, x, gamma,
                     n, eps, y);
  return launch_status("rmsnorm_fp");
}

int bfp_silu_fp_d(const double *x, size_t n, double *y, void *stream) {
  if (!x || !y) return set_err(BFP_EINVAL, "silu_fp: null pointer");
  if (n % 16) return set_err(BFP_EINVAL, "silu_fp: n=%zu is not a multiple of 16", n);
  if (n == 0) return BFP_OK;
  const long long nb = ((long long)n + LEAF_BS - 1) / LEAF_BS;
  if (nb > 0x7fffffffLL) return set_err(BFP_EINVAL, "silu_fp: n=%zu too large", n);
  hipLaunchKernelGGL(k_silu_fp, dim3((unsigned)nb), dim3(LEAF_BS), 0, (hipStream_t)stream, x,
                     (long long)n, y);
  return launch_status("silu_fp");
}

int bfp_softmax_fp_d(const double *x, int n, int batch, double *y, void *stream) {
  if (!x || !y) return set_err(BFP_EINVAL, "softmax_fp: null pointer");
  if (n <= 0 || n > LEAF_MAX_N || batch < 0)
    return set_err(BFP_EINVAL, "softmax_fp: n=%d must be in [1, %d], batch=%d", n, LEAF_MAX_N,
                   batch);
  if (batch == 0) return BFP_OK;
  hipLaunchKernelGGL(k_softmax_fp, dim3(batch), dim3(LEAF_BS), 0, (hipStream_t)stream, x, n, y);
  return launch_status("softmax_fp");
}

int bfp_rope_cos_sin(int pos, int head_dim, double base, double *cs) {
  if (!cs || head_dim <= 0 || head_dim % 2)
    return set_err(BFP_EINVAL, "rope_cos_sin: head_dim=%d", head_dim);
  rope_row(cs, pos, head_dim, base);
  return BFP_OK;
}

int bfp_rope_fp_d(const double *x, int n_heads, const double *cs, double *y, void *stream) {
  if (!x || !cs || !y) return set_err(BFP_EINVAL, "rope_fp: null pointer");
  if (n_heads < 0) return set_err(BFP_EINVAL, "rope_fp: n_heads=%d", n_heads);
  if (n_heads == 0) return BFP_OK;
  hipLaunchKernelGGL(k_rope_fp, dim3(n_heads), dim3(64), 0, (hipStream_t)stream, x, cs, y);
  return launch_status("rope_fp");
}

}  // extern "C"
