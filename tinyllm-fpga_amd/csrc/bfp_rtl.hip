// RTL-exact BFP leaf ops (the hardware engines of rtl/vc707/src/smollm/), as
// batched HIP kernels.  Each kernel follows the reference's bit-exact Python
// golden of that engine (rtl/vc707/host/gen_*_bfp_golden.py): truncating
// arithmetic shifts, per-lane / per-element exponents, the engines' own
// sequential fold orders, LUT exp / SiLU and Newton-Raphson reciprocals.
// These ops are not on the model-level simulator's token path; they are the
// per-op semantics of the FPGA datapath.
#include <math.h>
#include <stdint.h>

#include "bfp.h"
#include "bfp_device.h"
#include "bfp_internal.h"

namespace bfp {
namespace rtl {

constexpr int ACC_W = 48;

__device__ __forceinline__ int lead64(long long v) {
  if (v == 0) return 0;
  unsigned long long a = v < 0 ? (unsigned long long)(-v) : (unsigned long long)v;
  return 63 - __clzll(a);
}

// shift = lead - 14; mantissa = low 16 bits of v >> shift (or << -shift)
__device__ __forceinline__ int norm16(long long v, int lead, int &shift) {
  shift = lead - 14;
  long long s = shift >= 0 ? (v >> shift) : v * (1LL << (-shift));
  return (int)(short)(s & 0xFFFF);
}

__device__ __forceinline__ int clamp8(int e) { return e < -128 ? -128 : (e > 127 ? 127 : e); }

__device__ __forceinline__ int max16_lanes(int v) {
  for (int o = 1; o < 16; o <<= 1) {
    int w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

// ------------------------------------------------------------------ matvec
// gen_matvec_bfp_golden.py:53-108: one thread per output row.
__global__ void k_rtl_matvec(const int16_t *__restrict__ xm, const int8_t *__restrict__ xe,
                             const int16_t *__restrict__ Wm, const int8_t *__restrict__ We,
                             int n_out, int nt, int16_t *ym, int8_t *ye) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= n_out) return;
  const long long HI = (1LL << (ACC_W - 1)) - 1, LO = -(1LL << (ACC_W - 1));
  long long acc = 0;
  int acc_e = 0;
  for (int t = 0; t < nt; ++t) {
    long long s = 0;
    const int16_t *w = Wm + ((long long)row * nt + t) * 16;
    for (int k = 0; k < 16; ++k) s += (long long)xm[t * 16 + k] * w[k];
    const int te = (int)xe[t] + (int)We[(long long)row * nt + t];
    if (t == 0) {
      acc = s;
      acc_e = te;
      continue;
    }
    const int d = te - acc_e;
    if (d > 0) {
      acc = d > ACC_W - 1 ? 0 : (acc >> d);
      acc_e = te;
    } else if (d < 0) {
      s = -d > ACC_W - 1 ? 0 : (s >> (-d));
    }
    acc += s;
    acc = acc > HI ? HI : (acc < LO ? LO : acc);
  }
  int sh;
  ym[row] = (int16_t)norm16(acc, lead64(acc), sh);
  ye[row] = (int8_t)clamp8(acc_e + sh - 15);
}

// ----------------------------------------------------------------- requant
// smollm_layer_bfp.sv:1387-1396 (requant_mant) with the chunk emax of
// :1672-1693: 16 lanes per chunk, one thread per lane.
__global__ void k_rtl_requant(const int16_t *__restrict__ m, const int8_t *__restrict__ e, int n,
                              int16_t *om, int8_t *oe) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const bool ok = i < n;
  const int ei = ok ? (int)e[i] : -128;
  const int emax = max16_lanes(ei);
  if (!ok) return;
  const int sh = emax - ei;
  om[i] = (int16_t)(sh >= 16 ? 0 : ((int)m[i] >> sh));
  if ((i & 15) == 0) oe[i >> 4] = (int8_t)emax;
}

// ----------------------------------------------------------------- rmsnorm
__constant__ int c_rms_seed[32] = {
    16777215, 16777215, 16777215, 16777215, 16777215, 16777215, 13698540, 9686330,
    6849270, 4843165, 3424635, 2421583, 1712317, 1210791, 856159, 605396,
    428079, 302698, 214040, 151349, 107020, 75674, 53510, 37837,
    26755, 18919, 13377, 9459, 6689, 4730, 3344, 2365};

// gen_rmsnorm_bfp_golden.py:42-142: one workgroup (64 threads) per vector;
// tile sums in parallel, the cross-tile fold and Newton-Raphson in lane 0,
// the per-tile output normalisation one element per lane.
__global__ __launch_bounds__(64) void k_rtl_rmsnorm(const int16_t *__restrict__ xm,
                                                    const int8_t *__restrict__ xe,
                                                    const int16_t *__restrict__ gm,
                                                    const int8_t *__restrict__ ge, int D,
                                                    int16_t *ym, int8_t *ye) {
  extern __shared__ long long sums[];   // nt tile sums
  __shared__ long long s_inv;
  __shared__ int s_einv;
  const int b = blockIdx.x, tid = threadIdx.x, nt = D / 16;
  const int16_t *x = xm + (long long)b * D;
  const int8_t *xex = xe + (long long)b * nt;
  for (int t = tid; t < nt; t += 64) {
    long long s = 0;
    for (int k = 0; k < 16; ++k) s += (long long)x[t * 16 + k] * x[t * 16 + k];
    sums[t] = s;
  }
  __syncthreads();
  if (tid == 0) {
    long long acc = sums[0];
    int acc_e = 2 * xex[0];
    for (int t = 1; t < nt; ++t) {
      const int te = 2 * xex[t];
      const int d = te - acc_e;
      if (d > 0) {
        acc = d > ACC_W - 1 ? 0 : (acc >> d);
        acc_e = te;
        acc += sums[t];
      } else if (d < 0) {
        acc += (-d <= ACC_W - 1) ? (sums[t] >> (-d)) : 0;
      } else {
        acc += sums[t];
      }
    }
    const unsigned long long inv_d = (1ULL << 32) / (unsigned)D;
    // mean = (acc * inv_d) >> 32, acc >= 0
    const unsigned __int128 prod = (unsigned __int128)(unsigned long long)acc * inv_d;
    const unsigned long long mean = (unsigned long long)(prod >> 32);
    int lead = mean ? 63 - __clzll(mean) : 0;
    if ((acc_e + lead) & 1) lead -= 1;
    long long v = lead >= 30 ? (long long)(mean >> (lead - 30))
                             : (long long)(mean << (30 - lead));
    v += 10737;                                       // EPS_Q30
    const int vmsb = v ? 63 - __clzll((unsigned long long)v) : 0;
    long long inv = vmsb < 32 ? c_rms_seed[vmsb] : 16777215;
    const long long C = (3LL << 30) / 2;
    for (int it = 0; it < 3; ++it) {
      const __int128 vy2 = ((__int128)v * inv * inv) >> 24;
      long long corr;
      if (vy2 >= ((__int128)1 << 32)) {
        corr = 0;
      } else {
        corr = C - ((long long)vy2 >> 1);
        corr = corr < 0 ? 0 : corr;
      }
      long long ni = (inv * corr + (1LL << 29)) >> 30;
      inv = ni < 16777215 ? ni : 16777215;
    }
    s_inv = inv;
    s_einv = (30 - acc_e - lead) >> 1;
  }
  __syncthreads();
  const long long inv = s_inv;
  const int16_t *g = gm + 0;
  for (int base = 0; base < D; base += 64) {
    const int i = base + tid;                         // D % 64 == 0 not required: D % 16 == 0
    const bool ok = i < D;
    const long long p = ok ? (long long)x[i] * g[i] * inv : 0;
    const int ml = max16_lanes(p ? lead64(p) : 0);
    if (ok) {
      int sh;
      ym[(long long)b * D + i] = (int16_t)norm16(p, ml, sh);
      if ((i & 15) == 0)
        ye[(long long)b * nt + (i >> 4)] =
            (int8_t)clamp8((int)xex[i >> 4] + (int)ge[i >> 4] + s_einv + sh - 27);
    }
  }
}

// -------------------------------------------------------------------- rope
constexpr long long PI_HALF_Q27 = 210828714, PI_Q27 = 421657428, PI_OVER_8_Q29 = 210828714,
                    K_Q3_27 = 81504109;
__constant__ long long c_atan[16] = {105414357, 62229729, 32880480, 16690645, 8377711, 4192939,
                                     2096981, 1048555, 524285, 262144, 131072, 65536,
                                     32768, 16384, 8192, 4096};

__device__ __forceinline__ long long wrap31(long long v) {
  v &= (1LL << 31) - 1;
  return (v & (1LL << 30)) ? v - (1LL << 31) : v;
}

// 16-iteration Q3.27 CORDIC of cordic_sincos.sv (gen_rope_bfp_golden.py:37-60).
__device__ void cordic(long long a, int &c, int &s) {
  long long z;
  bool neg;
  if (a > PI_HALF_Q27) {
    z = PI_Q27 - a;
    neg = true;
  } else if (a < -PI_HALF_Q27) {
    z = -PI_Q27 - a;
    neg = true;
  } else {
    z = a;
    neg = false;
  }
  long long x = K_Q3_27, y = 0;
  for (int i = 0; i < 16; ++i) {
    const long long xs = x >> i, ys = y >> i;
    if (z >= 0) {
      x -= ys;
      y += xs;
      z -= c_atan[i];
    } else {
      x += ys;
      y -= xs;
      z += c_atan[i];
    }
  }
  const long long xr = (x + 2048) >> 12, yr = (y + 2048) >> 12;
  if (xr > 32767)
    c = neg ? -32767 : 32767;
  else if (xr < -32768)
    c = neg ? 32767 : -32768;
  else
    c = (int)(neg ? -xr : xr);
  s = (int)(yr > 32767 ? 32767 : (yr < -32768 ? -32768 : yr));
}

// rope_bfp.sv golden (gen_rope_bfp_golden.py:72-121): one 64-thread
// workgroup per head, thread j < 32 rotates pair (j, j+32).
__global__ __launch_bounds__(64) void k_rtl_rope(const int16_t *__restrict__ xm,
                                                 const int8_t *__restrict__ xe, int pos,
                                                 const unsigned *__restrict__ freq, int16_t *ym,
                                                 int8_t *ye) {
  const int h = blockIdx.x, j = threadIdx.x;
  if (j >= 32) return;
  const int16_t *x = xm + h * 64;
  const int8_t *e = xe + h * 4;
  const long long ang = wrap31((wrap31((long long)pos * freq[j]) * PI_OVER_8_Q29) >> 29);
  int c, s;
  cordic(ang, c, s);
  const int a = x[j], bb = x[j + 32];
  const int ea = e[j >> 4], eb = e[(j + 32) >> 4];
  const int em = ea > eb ? ea : eb;
  const long long aa = em - ea < 16 ? (a >> (em - ea)) : 0;
  const long long ba = em - eb < 16 ? (bb >> (em - eb)) : 0;
  const long long lo = aa * c - ba * s, hi = ba * c + aa * s;
  int sh;
  ym[h * 64 + j] = (int16_t)norm16(lo, lead64(lo), sh);
  ye[h * 64 + j] = (int8_t)clamp8(em + sh - 15);
  ym[h * 64 + j + 32] = (int16_t)norm16(hi, lead64(hi), sh);
  ye[h * 64 + j + 32] = (int8_t)clamp8(em + sh - 15);
}

// ----------------------------------------------------------------- softmax
// softmax_bfp.sv golden (gen_softmax_bfp_golden.py:33-78): one 64-thread
// workgroup per problem of n <= 4096 scores sharing one exponent.
__global__ __launch_bounds__(64) void k_rtl_softmax(const int16_t *__restrict__ xm,
                                                    const int8_t *__restrict__ xe, int n,
                                                    int stride,
                                                    const uint16_t *__restrict__ lut,
                                                    int16_t *ym, int8_t *ye) {
  extern __shared__ long long vals[];   // n LUT values
  __shared__ long long s_inv;
  __shared__ int s_red[2];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int16_t *x = xm + (long long)b * stride;
  int mx = -32768;
  for (int i = tid; i < n; i += 64) mx = x[i] > mx ? x[i] : mx;
  for (int o = 1; o < 64; o <<= 1) {
    int w = __shfl_xor(mx, o, 64);
    mx = w > mx ? w : mx;
  }
  const int sh = (int)xe[b] - 8;
  long long part = 0;
  for (int i = tid; i < n; i += 64) {
    const long long d = (long long)x[i] - mx;
    const long long ds = sh >= 0 ? d * (1LL << (sh > 40 ? 40 : sh)) : (d >> (-sh > 62 ? 62 : -sh));
    const int idx = ds >= 0 ? 1023 : (ds <= -1023 ? 0 : (int)(ds + 1023));
    vals[i] = lut[idx];
    part += lut[idx];
  }
  for (int o = 1; o < 64; o <<= 1) part += __shfl_xor(part, o, 64);
  if (tid == 0) {
    const long long tot = part;
    const int msb = tot ? 63 - __clzll((unsigned long long)tot) : 0;
    __int128 y = (__int128)1 << (31 - msb);
    for (int it = 0; it < 4; ++it) y = (y * (((__int128)1 << 33) - (__int128)tot * y)) >> 32;
    s_inv = (long long)y;
  }
  __syncthreads();
  const long long inv = s_inv;
  int ml = 0;
  for (int i = tid; i < n; i += 64) {
    const long long p = vals[i] * inv;
    const int l = p ? lead64(p) : 0;
    ml = l > ml ? l : ml;
  }
  for (int o = 1; o < 64; o <<= 1) {
    int w = __shfl_xor(ml, o, 64);
    ml = w > ml ? w : ml;
  }
  for (int i = tid; i < n; i += 64) {
    int s2;
    ym[(long long)b * stride + i] = (int16_t)norm16(vals[i] * inv, ml, s2);
  }
  if (tid == 0) ye[b] = (int8_t)clamp8(ml - 14 - 17);
  (void)s_red;
}

// ------------------------------------------------------------------ swiglu
// swiglu_bfp.sv golden (gen_swiglu_bfp_golden.py:43-78): one element per
// thread, 16-lane tiles.
__global__ void k_rtl_swiglu(const int16_t *__restrict__ gm, const int8_t *__restrict__ ge,
                             const int16_t *__restrict__ um, const int8_t *__restrict__ ue, int n,
                             const int16_t *__restrict__ lut, int16_t *ym, int8_t *ye) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const bool ok = i < n;
  long long p = 0;
  if (ok) {
    const int sh = (int)ge[i >> 4] - 5;
    const long long mg = gm[i];
    long long idx;
    if (sh >= 0)
      idx = sh >= 16 ? (mg > 0 ? 32767 : (mg < 0 ? -32768 : 0)) : mg * (1LL << sh);
    else
      idx = -sh >= 16 ? (mg < 0 ? -1 : 0) : (mg >> (-sh));
    idx = idx < -32768 ? -32768 : (idx > 32767 ? 32767 : idx);
    p = (long long)lut[idx & 0xFFFF] * um[i];
  }
  const int ml = max16_lanes(p ? lead64(p) : 0);
  if (!ok) return;
  int s;
  ym[i] = (int16_t)norm16(p, ml, s);
  if ((i & 15) == 0) ye[i >> 4] = (int8_t)clamp8((int)ue[i >> 4] + s - 10);
}

// ---------------------------------------------------------------- residual
// residual_bfp.sv golden (gen_residual_bfp_golden.py:23-48).
__global__ void k_rtl_residual(const int16_t *__restrict__ am, const int8_t *__restrict__ ae,
                               const int16_t *__restrict__ bm, const int8_t *__restrict__ be,
                               int n, int16_t *ym, int8_t *ye) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const bool ok = i < n;
  long long sum = 0;
  int em = 0;
  if (ok) {
    const int ea = ae[i >> 4], eb = be[i >> 4];
    em = ea > eb ? ea : eb;
    const long long a = em - ea < 16 ? (am[i] >> (em - ea)) : 0;
    const long long bv = em - eb < 16 ? (bm[i] >> (em - eb)) : 0;
    sum = a + bv;
  }
  const int ml = max16_lanes(sum ? lead64(sum) : 0);
  if (!ok) return;
  int s;
  ym[i] = (int16_t)norm16(sum, ml, s);
  if ((i & 15) == 0) ye[i >> 4] = (int8_t)clamp8(em + s);
}

// ------------------------------------------------------------------ argmax
__device__ __forceinline__ bool bfp_gt(int ma, int ea, int mb, int eb) {
  const int de = ea - eb;
  if (de == 0) return ma > mb;
  if (de > 0) return ma > (de >= 16 ? 0 : (mb >> de));
  return (-de >= 16 ? 0 : (ma >> (-de))) > mb;
}

// The decode head's running argmax (smollm_decode_head_bfp.sv:322-324,
// 399-430): chunk-local bests in parallel, then the ordered fold over chunks
// (bfp_gt is not transitive under truncation, so the fold order is kept).
__global__ __launch_bounds__(256) void k_rtl_argmax(const int16_t *__restrict__ m,
                                                    const int8_t *__restrict__ e, int n,
                                                    int *lm, int *le, int *li, int *out) {
  const int b = blockIdx.x, tid = threadIdx.x, nc = n / 16;
  const int16_t *mb = m + (long long)b * n;
  const int8_t *eb = e + (long long)b * n;
  int *LM = lm + (long long)b * nc, *LE = le + (long long)b * nc, *LI = li + (long long)b * nc;
  for (int c = tid; c < nc; c += blockDim.x) {
    int bm = mb[c * 16], be_ = eb[c * 16], bi = 0;
    for (int k = 1; k < 16; ++k)
      if (bfp_gt(mb[c * 16 + k], eb[c * 16 + k], bm, be_)) {
        bm = mb[c * 16 + k];
        be_ = eb[c * 16 + k];
        bi = k;
      }
    LM[c] = bm;
    LE[c] = be_;
    LI[c] = c * 16 + bi;
  }
  __syncthreads();
  if (tid == 0) {
    int bm = -32768, be_ = -128, bi = 0;
    for (int c = 0; c < nc; ++c)
      if (bfp_gt(LM[c], LE[c], bm, be_)) {
        bm = LM[c];
        be_ = LE[c];
        bi = LI[c];
      }
    out[b] = bi;
  }
}

}  // namespace rtl
}  // namespace bfp

using namespace bfp;

static inline unsigned nb(long long n, int bs) { return (unsigned)((n + bs - 1) / bs); }

extern "C" {

// LUTs and tables of the RTL ops, built on the host from their defining
// formulas with the host libm: EXP_LUT (sim/gen_exp_lut.py:36-42),
// SILU_LUT (sim/gen_swiglu_lut.py:27-44, indexed by the int16 code & 0xFFFF),
// FREQ_TURNS_Q31 (sim/gen_rope_freq_table.py:31-37).  Any pointer may be NULL.
int bfp_rtl_tables(uint16_t *exp_lut, int16_t *silu_lut, uint32_t *freq_q31, int head_dim,
                   double base) {
  if (exp_lut)
    for (int i = 0; i < 1024; ++i) {
      double v = nearbyint(exp((i - 1023) / 128.0) * 32768.0);
      exp_lut[i] = (uint16_t)(v > 65535 ? 65535 : (v < 0 ? 0 : v));
    }
  if (silu_lut)
    for (int c = 0; c < 65536; ++c) {
      const double code = (double)(int16_t)(uint16_t)c;
      const double g = code / 32768.0 * 32.0;
      const double s = g * (1.0 / (1.0 + exp(-g)));
      double q = nearbyint(s * 32768.0 / 32.0);
      q = q > 32767 ? 32767 : (q < -32768 ? -32768 : q);
      silu_lut[c] = (int16_t)q;
    }
  if (freq_q31) {
    if (head_dim <= 0 || head_dim % 2) return set_err(BFP_EINVAL, "head_dim %d", head_dim);
    for (int j = 0; j < head_dim / 2; ++j) {
      const double f = 1.0 / pow(base, 2.0 * j / head_dim);
      freq_q31[j] = (uint32_t)nearbyint(f / (2.0 * M_PI) * (double)(1LL << 31));
    }
  }
  return BFP_OK;
}

int bfp_rtl_matvec_d(const int16_t *x_m, const int8_t *x_e, const int16_t *W_m, const int8_t *W_e,
                     int n_out, int n_in, int16_t *y_m, int8_t *y_e, void *stream) {
  if (n_out <= 0 || n_in <= 0 || n_in % 16) return set_err(BFP_EINVAL, "rtl_matvec: shape");
  hipLaunchKernelGGL(rtl::k_rtl_matvec, dim3(nb(n_out, 64)), dim3(64), 0, (hipStream_t)stream,
                     x_m, x_e, W_m, W_e, n_out, n_in / 16, y_m, y_e);
  return launch_status("rtl_matvec");
}

int bfp_rtl_requant_d(const int16_t *m, const int8_t *e, int n, int16_t *out_m, int8_t *out_e,
                      void *stream) {
  if (n <= 0 || n % 16) return set_err(BFP_EINVAL, "rtl_requant: n=%d", n);
  hipLaunchKernelGGL(rtl::k_rtl_requant, dim3(nb(n, 64)), dim3(64), 0, (hipStream_t)stream, m, e,
                     n, out_m, out_e);
  return launch_status("rtl_requant");
}

int bfp_rtl_rmsnorm_d(const int16_t *x_m, const int8_t *x_e, const int16_t *g_m, const int8_t *g_e,
                      int D, int batch, int16_t *y_m, int8_t *y_e, void *stream) {
  if (D <= 0 || D % 16 || D > 65536 || batch <= 0)
    return set_err(BFP_EINVAL, "rtl_rmsnorm: D=%d batch=%d", D, batch);
  hipLaunchKernelGGL(rtl::k_rtl_rmsnorm, dim3(batch), dim3(64), (size_t)(D / 16) * 8,
                     (hipStream_t)stream, x_m, x_e, g_m, g_e, D, y_m, y_e);
  return launch_status("rtl_rmsnorm");
}

int bfp_rtl_rope_d(const int16_t *x_m, const int8_t *x_e, int pos, int n_heads,
                   const uint32_t *freq_q31, int16_t *y_m, int8_t *y_e, void *stream) {
  if (n_heads <= 0 || pos < 0) return set_err(BFP_EINVAL, "rtl_rope: heads=%d pos=%d", n_heads, pos);
  hipLaunchKernelGGL(rtl::k_rtl_rope, dim3(n_heads), dim3(64), 0, (hipStream_t)stream, x_m, x_e,
                     pos, freq_q31, y_m, y_e);
  return launch_status("rtl_rope");
}

int bfp_rtl_softmax_d(const int16_t *x_m, const int8_t *x_e, int n, int batch, int stride,
                      const uint16_t *exp_lut, int16_t *y_m, int8_t *y_e, void *stream) {
  if (n <= 0 || n > 4096 || batch <= 0 || stride < n)
    return set_err(BFP_EINVAL, "rtl_softmax: n=%d batch=%d stride=%d", n, batch, stride);
  hipLaunchKernelGGL(rtl::k_rtl_softmax, dim3(batch), dim3(64), (size_t)n * 8, (hipStream_t)stream,
                     x_m, x_e, n, stride, exp_lut, y_m, y_e);
  return launch_status("rtl_softmax");
}

int bfp_rtl_swiglu_d(const int16_t *g_m, const int8_t *g_e, const int16_t *u_m, const int8_t *u_e,
                     int n, const int16_t *silu_lut, int16_t *y_m, int8_t *y_e, void *stream) {
  if (n <= 0 || n % 16) return set_err(BFP_EINVAL, "rtl_swiglu: n=%d", n);
  hipLaunchKernelGGL(rtl::k_rtl_swiglu, dim3(nb(n, 64)), dim3(64), 0, (hipStream_t)stream, g_m, g_e,
                     u_m, u_e, n, silu_lut, y_m, y_e);
  return launch_status("rtl_swiglu");
}

int bfp_rtl_residual_d(const int16_t *a_m, const int8_t *a_e, const int16_t *b_m,
                       const int8_t *b_e, int n, int16_t *y_m, int8_t *y_e, void *stream) {
  if (n <= 0 || n % 16) return set_err(BFP_EINVAL, "rtl_residual: n=%d", n);
  hipLaunchKernelGGL(rtl::k_rtl_residual, dim3(nb(n, 64)), dim3(64), 0, (hipStream_t)stream, a_m,
                     a_e, b_m, b_e, n, y_m, y_e);
  return launch_status("rtl_residual");
}

// work: 3 * batch * n/16 ints of device scratch supplied by the caller.
int bfp_rtl_argmax_d(const int16_t *m, const int8_t *e, int n, int batch, int32_t *work,
                     int32_t *idx, void *stream) {
  if (n <= 0 || n % 16 || batch <= 0 || !work) return set_err(BFP_EINVAL, "rtl_argmax: n=%d", n);
  const long long nc = (long long)batch * (n / 16);
  hipLaunchKernelGGL(rtl::k_rtl_argmax, dim3(batch), dim3(256), 0, (hipStream_t)stream, m, e, n,
                     work, work + nc, work + 2 * nc, idx);
  return launch_status("rtl_argmax");
}

}  // extern "C"
