// RTL-exact BFP leaf ops (the hardware engines of rtl/vc707/src/smollm/), as
// batched HIP kernels.  Each kernel follows the reference's bit-exact Python
// golden of that engine (rtl/vc707/host/gen_*_bfp_golden.py): truncating
// arithmetic shifts, per-lane / per-element exponents, the engines' own
// sequential fold orders, LUT exp / SiLU and Newton-Raphson reciprocals.
// These ops are not on the model-level simulator's token path; they are the
// per-op semantics of the FPGA datapath.
#include <math.h>
#include <stdint.h>

#include <mutex>

#include "bfp.h"
#include "bfp_device.h"
#include "bfp_internal.h"
#include "bfp_f64.h"
#include "bfp_layer.h"
#include "bfp_mv.h"

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

// requant_mant (smollm_layer_bfp.sv:1387-1396): the shift e_to - e_from is
// held in `logic signed [7:0]` and wraps; >= 16 gives 0, a negative shift
// leaves m unchanged.  The AV pre-shift of V (:2149-2166) has the same form.
__device__ __forceinline__ int shr8(int m, int e_to, int e_from) {
  const int sh = (int)(signed char)(e_to - e_from);
  return sh >= 16 ? 0 : (sh >= 0 ? (m >> sh) : m);
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
  om[i] = (int16_t)shr8(m[i], emax, ei);
  if ((i & 15) == 0) oe[i >> 4] = (int8_t)emax;
}

// ----------------------------------------------------------------- rmsnorm
__constant__ int c_rms_seed[32] = {
    16777215, 16777215, 16777215, 16777215, 16777215, 16777215, 13698540, 9686330,
    6849270, 4843165, 3424635, 2421583, 1712317, 1210791, 856159, 605396,
    428079, 302698, 214040, 151349, 107020, 75674, 53510, 37837,
    26755, 18919, 13377, 9459, 6689, 4730, 3344, 2365};

// One 64-thread wave normalises the D-vector x: writes ym (D) and ye (D/16).
// sums: D/16 int64 of LDS; s_inv / s_einv: LDS scalars.
__device__ void rmsnorm_wave(const int16_t *__restrict__ x, const int8_t *__restrict__ xex,
                             const int16_t *gm, const int8_t *ge, int D, int16_t *ym, int8_t *ye,
                             long long *sums, long long *s_inv, int *s_einv) {
  const int tid = threadIdx.x, nt = D / 16;
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
    *s_inv = inv;
    *s_einv = (30 - acc_e - lead) >> 1;
  }
  __syncthreads();
  const long long inv = *s_inv;
  const int einv = *s_einv;
  for (int base = 0; base < D; base += 64) {
    const int i = base + tid;                         // D % 64 == 0 not required: D % 16 == 0
    const bool ok = i < D;
    const long long p = ok ? (long long)x[i] * gm[i] * inv : 0;
    const int ml = max16_lanes(p ? lead64(p) : 0);
    if (ok) {
      int sh;
      ym[i] = (int16_t)norm16(p, ml, sh);
      if ((i & 15) == 0)
        ye[i >> 4] = (int8_t)clamp8((int)xex[i >> 4] + (int)ge[i >> 4] + einv + sh - 27);
    }
  }
}

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
  const int b = blockIdx.x, nt = D / 16;
  rmsnorm_wave(xm + (long long)b * D, xe + (long long)b * nt, gm, ge, D, ym + (long long)b * D,
               ye + (long long)b * nt, sums, &s_inv, &s_einv);
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

// ===================================================== composed RTL layer
// smollm_layer_bfp.sv:1603-2600 on one sequence: the engines above wired in
// the FSM's order, with the matvec engine's sequential tile fold over the
// device-layout weights.  Eight launches: NORM1, Q/K/V, RoPE + KV write,
// attention, O + residual 1, NORM2, G/U + SwiGLU, D + residual 2.

__device__ __forceinline__ void st_put(const StageDump *sd, int s, int i, int m) {
  if (sd && sd->m[s]) sd->m[s][i] = (int16_t)m;
}
__device__ __forceinline__ void st_pute(const StageDump *sd, int s, int t, int e) {
  if (sd && sd->e[s]) sd->e[s][t] = (int8_t)e;
}

// residual_bfp.sv on one tile held by 16 lanes (gen_residual_bfp_golden.py:23-48).
__device__ __forceinline__ void residual16(int am, int ea, int bm, int eb, int &ym, int &ye) {
  const int em = ea > eb ? ea : eb;
  const long long av = em - ea < 16 ? (am >> (em - ea)) : 0;
  const long long bv = em - eb < 16 ? (bm >> (em - eb)) : 0;
  const long long sum = av + bv;
  const int ml = max16_lanes(sum ? lead64(sum) : 0);
  int s;
  ym = norm16(sum, ml, s);
  ye = clamp8(em + s);
}

// swiglu_bfp.sv on one tile held by 16 lanes (gen_swiglu_bfp_golden.py:43-78).
__device__ __forceinline__ void swiglu16(int gm, int ge, int um, int ue,
                                         const int16_t *__restrict__ lut, int &ym, int &ye) {
  const int sh = ge - 5;
  long long idx;
  if (sh >= 0)
    idx = sh >= 16 ? (gm > 0 ? 32767 : (gm < 0 ? -32768 : 0)) : (long long)gm * (1LL << sh);
  else
    idx = -sh >= 16 ? (gm < 0 ? -1 : 0) : (gm >> (-sh));
  idx = idx < -32768 ? -32768 : (idx > 32767 ? 32767 : idx);
  const long long p = (long long)lut[idx & 0xFFFF] * um;
  const int ml = max16_lanes(p ? lead64(p) : 0);
  int s;
  ym = norm16(p, ml, s);
  ye = clamp8(ue + s - 10);
}

// One step of the engine's fold (gen_matvec_bfp_golden.py:53-108): the side
// with the smaller exponent is shifted right (zeroed past 47), then the
// 48-bit saturating add.
__device__ __forceinline__ void engine_fold(long long &acc, int &acc_e, long long s, int te) {
  const long long HI = (1LL << (ACC_W - 1)) - 1, LO = -(1LL << (ACC_W - 1));
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

// NORM1 (second == 0: h, G1) or NORM2 (h1, G2) -> xn.  The gamma ROM holds
// tile_quantize of the float gamma; it is formed here.
__global__ __launch_bounds__(64) void k_rl_norm(RtlArgs a, int second) {
  extern __shared__ long long rl_lds[];
  __shared__ long long s_inv;
  __shared__ int s_einv;
  const LayerArgs &L = a.L;
  const int D = L.D, nt = D / 16, tid = threadIdx.x;
  long long *sums = rl_lds;
  int16_t *gm = reinterpret_cast<int16_t *>(rl_lds + nt);
  int8_t *ge = reinterpret_cast<int8_t *>(gm + D);
  const double *g = second ? L.g2 : L.g1;
  for (int base = 0; base < D; base += 64) {   // D % 64 == 0: whole 16-lane tiles
    const int i = base + tid;
    int e;
    const int m = quantize16_lanes(g[i], e);
    gm[i] = (int16_t)m;
    if ((i & 15) == 0) ge[i >> 4] = (int8_t)e;
  }
  __syncthreads();
  rmsnorm_wave(second ? L.h1_m : L.h_m, second ? L.h1_e : L.h_e, gm, ge, D, L.xn_m, L.xn_e, sums,
               &s_inv, &s_einv);
  if (L.dump) {
    __syncthreads();
    const int st = second ? ST_N2 : ST_N1;
    for (int i = tid; i < D; i += 64) st_put(L.dump, st, i, L.xn_m[i]);
    for (int t = tid; t < nt; t += 64) st_pute(L.dump, st, t, L.xn_e[t]);
  }
}

// Exact tile sums S = sum_k x[t,k] W[r,t,k] and exponents E = x_e[t] + W_e[r,t]
// of the tiles this lane owns (the layout of load_chunk), into LDS at
// [t*16 + r].
template <int NW, int TPT>
__device__ __forceinline__ void tile_sums_to_lds(const ChunkRegs<TPT> &R, const int *xs,
                                                 const int *xes, int nT, long long *Sl, int *El) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, tq = lane >> 4;
  typedef short s2 __attribute__((ext_vector_type(2)));
#define RL_DOT2(a, b, acc) \
  __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, (a)), __builtin_bit_cast(s2, (b)), (acc), false)
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const int t = tq + 4 * (w + NW * j);
    if (t < nT) {
      const int4 *xp = reinterpret_cast<const int4 *>(xs + t * 16);
      const int4 h0 = xp[0], h1 = xp[1], l0 = xp[2], l1 = xp[3];
      int ah = 0, al = 0;
      ah = RL_DOT2(R.a[j].x, h0.x, ah);
      al = RL_DOT2(R.a[j].x, l0.x, al);
      ah = RL_DOT2(R.a[j].y, h0.y, ah);
      al = RL_DOT2(R.a[j].y, l0.y, al);
      ah = RL_DOT2(R.a[j].z, h0.z, ah);
      al = RL_DOT2(R.a[j].z, l0.z, al);
      ah = RL_DOT2(R.a[j].w, h0.w, ah);
      al = RL_DOT2(R.a[j].w, l0.w, al);
      ah = RL_DOT2(R.b[j].x, h1.x, ah);
      al = RL_DOT2(R.b[j].x, l1.x, al);
      ah = RL_DOT2(R.b[j].y, h1.y, ah);
      al = RL_DOT2(R.b[j].y, l1.y, al);
      ah = RL_DOT2(R.b[j].z, h1.z, ah);
      al = RL_DOT2(R.b[j].z, l1.z, al);
      ah = RL_DOT2(R.b[j].w, h1.w, ah);
      al = RL_DOT2(R.b[j].w, l1.w, al);
      Sl[t * 16 + r] = (long long)ah * 256 + al;
      El[t * 16 + r] = xes[t] + R.e[j];
    }
  }
#undef RL_DOT2
}

// One 16-row chunk on the engine: sets, in every lane of wave 0, row
// (lane & 15)'s per-lane output (m, e) (the engine's out_mant / out_exp).
// All threads call it; it synchronises.
template <int NW, int TPT>
__device__ void rl_chunk_me(const uint4 *__restrict__ pm, const int8_t *__restrict__ pe, int nT,
                            const int *xs, const int *xes, long long *Sl, int *El, int &m, int &e) {
  ChunkRegs<TPT> R;
  load_chunk_nb<NW, TPT>(R, pm, pe, nT);
  tile_sums_to_lds<NW, TPT>(R, xs, xes, nT, Sl, El);
  __syncthreads();
  m = 0;
  e = 0;
  if (threadIdx.x < 64) {
    const int r = threadIdx.x & 15;
    long long acc = Sl[r];
    int acc_e = El[r];
    for (int t = 1; t < nT; ++t) engine_fold(acc, acc_e, Sl[t * 16 + r], El[t * 16 + r]);
    int sh;
    m = norm16(acc, lead64(acc), sh);
    e = clamp8(acc_e + sh - 15);
  }
  __syncthreads();   // Sl / El free for the next chunk
}

// The same chunk, then the chunk re-tile (S_xMV_DRAIN/REQ): returns, in
// every lane of wave 0, row (lane & 15)'s re-tiled mantissa and sets emax
// to the chunk exponent.
template <int NW, int TPT>
__device__ int rl_chunk(const uint4 *__restrict__ pm, const int8_t *__restrict__ pe, int nT,
                        const int *xs, const int *xes, long long *Sl, int *El, int &emax) {
  int m, e;
  rl_chunk_me<NW, TPT>(pm, pe, nT, xs, xes, Sl, El, m, e);
  int mq = 0;
  emax = 0;
  if (threadIdx.x < 64) {
    emax = max16_lanes(e);
    mq = shr8(m, emax, e);
  }
  return mq;
}

// The layer's matvecs, one 16-row output chunk per workgroup.
//   op 0: Q|K|V from xn            (chunks of qkv, re-tiled per chunk)
//   op 1: O from att, then residual 1 with h -> h1
//   op 2: G chunk c and U chunk c from xn, then SwiGLU -> mlp
//   op 3: D from mlp, then residual 2 with h1 -> h
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_rl_mv(RtlArgs a, int op) {
  constexpr int TPT = 3;
  extern __shared__ long long rl_lds[];
  const LayerArgs &L = a.L;
  const int c = blockIdx.x;
  const int nT = (op == 3 ? L.FFN : L.D) / 16;
  long long *Sl = rl_lds;
  int *El = reinterpret_cast<int *>(Sl + nT * 16);
  int *xs = El + nT * 16;
  int *xes = xs + nT * 16;
  const int16_t *xm = op == 1 ? L.att_m : (op == 3 ? L.mlp_m : L.xn_m);
  const int8_t *xe = op == 1 ? L.att_e : (op == 3 ? L.mlp_e : L.xn_e);
  stage_x_bfp(xs, xes, xm, xe, nT);
  __syncthreads();
  const uint4 *wm;
  const int8_t *we;
  int chunk = c;
  if (op == 0) {
    wm = L.w_qkv_m, we = L.w_qkv_e;
  } else if (op == 1) {
    wm = L.w_o_m, we = L.w_o_e;
  } else if (op == 2) {
    wm = L.w_gu_m, we = L.w_gu_e, chunk = 2 * c;
  } else {
    wm = L.w_d_m, we = L.w_d_e;
  }
  int emax;
  const int mq = rl_chunk<NW, TPT>(wm + (size_t)chunk * nT * 32, we + (size_t)chunk * nT * 16, nT,
                                   xs, xes, Sl, El, emax);
  int mu = 0, eu = 0;
  if (op == 2)
    mu = rl_chunk<NW, TPT>(wm + (size_t)(chunk + 1) * nT * 32, we + (size_t)(chunk + 1) * nT * 16,
                           nT, xs, xes, Sl, El, eu);
  if (threadIdx.x >= 64) return;
  const int r = threadIdx.x & 15, i = c * 16 + r;
  const bool w = threadIdx.x < 16;
  const StageDump *sd = L.dump;
  if (op == 0) {
    if (w) {
      L.qkv_m[i] = (int16_t)mq;
      if (r == 0) L.qkv_e[c] = (int8_t)emax;
    }
    return;
  }
  int ym, ye;
  if (op == 1 || op == 3) {
    const int16_t *bm = op == 1 ? L.h_m : L.h1_m;
    const int8_t *be = op == 1 ? L.h_e : L.h1_e;
    residual16(bm[i], be[c], mq, emax, ym, ye);
    int16_t *om = op == 1 ? L.h1_m : L.h_m;
    int8_t *oe = op == 1 ? L.h1_e : L.h_e;
    const int so = op == 1 ? ST_O : ST_D, sr = op == 1 ? ST_H1 : ST_HOUT;
    if (w) {
      om[i] = (int16_t)ym;
      if (r == 0) oe[c] = (int8_t)ye;
      st_put(sd, so, i, mq);
      st_put(sd, sr, i, ym);
      if (r == 0) {
        st_pute(sd, so, c, emax);
        st_pute(sd, sr, c, ye);
      }
    }
    return;
  }
  swiglu16(mq, emax, mu, eu, a.silu_lut, ym, ye);
  if (w) {
    L.mlp_m[i] = (int16_t)ym;
    if (r == 0) L.mlp_e[c] = (int8_t)ye;
    st_put(sd, ST_G, i, mq);
    st_put(sd, ST_U, i, mu);
    st_put(sd, ST_MLP, i, ym);
    if (r == 0) {
      st_pute(sd, ST_G, c, emax);
      st_pute(sd, ST_U, c, eu);
      st_pute(sd, ST_MLP, c, ye);
    }
  }
}

// RoPE of Q head h (h < H_Q) or K head h - H_Q, then the re-tile of its four
// tiles (S_ROPEx_RQ_A/B); K heads also write the KV slot kv_pos with the
// rotated K and the V head (S_KVWR_M/E).  One 64-thread workgroup per head.
// The step of the RTL layer: a.pos / a.kv_pos, or the device step counter.
__device__ __forceinline__ int rl_pos(const RtlArgs &a) { return a.pos_ptr ? *a.pos_ptr : a.pos; }
__device__ __forceinline__ int rl_kv_pos(const RtlArgs &a) { return a.pos_ptr ? *a.pos_ptr : a.kv_pos; }

__global__ __launch_bounds__(64) void k_rl_rope_kv(RtlArgs a) {
  const LayerArgs &L = a.L;
  const int h = blockIdx.x, j = threadIdx.x & 31, HD = 64;
  const bool is_k = h >= L.H_Q;
  const int kh = h - L.H_Q;
  const int off = is_k ? L.D + kh * HD : h * HD;   // element offset in qkv
  const int16_t *x = L.qkv_m + off;
  const int8_t *e = L.qkv_e + off / 16;
  const long long ang = wrap31((wrap31((long long)rl_pos(a) * a.freq[j]) * PI_OVER_8_Q29) >> 29);
  int cs, sn;
  cordic(ang, cs, sn);
  const int xa = x[j], xb = x[j + 32];
  const int ea = e[j >> 4], eb = e[(j + 32) >> 4];
  const int em = ea > eb ? ea : eb;
  const long long aa = em - ea < 16 ? (xa >> (em - ea)) : 0;
  const long long ba = em - eb < 16 ? (xb >> (em - eb)) : 0;
  const long long lo = aa * cs - ba * sn, hi = ba * cs + aa * sn;
  int sh;
  const int mlo = norm16(lo, lead64(lo), sh);
  const int elo = clamp8(em + sh - 15);
  const int mhi = norm16(hi, lead64(hi), sh);
  const int ehi = clamp8(em + sh - 15);
  // lanes 0-15 hold tiles 0 (lo) and 2 (hi), lanes 16-31 tiles 1 and 3
  const int emlo = max16_lanes(elo), emhi = max16_lanes(ehi);
  const int qlo = shr8(mlo, emlo, elo), qhi = shr8(mhi, emhi, ehi);
  if (threadIdx.x >= 32) return;
  const StageDump *sd = L.dump;
  int16_t *ym = L.qkv_m + off;
  int8_t *ye = L.qkv_e + off / 16;
  ym[j] = (int16_t)qlo;
  ym[j + 32] = (int16_t)qhi;
  if ((j & 15) == 0) {
    ye[j >> 4] = (int8_t)emlo;
    ye[(j + 32) >> 4] = (int8_t)emhi;
  }
  const int st = is_k ? ST_K : ST_Q, so = is_k ? kh * HD : h * HD;
  st_put(sd, st, so + j, qlo);
  st_put(sd, st, so + j + 32, qhi);
  if ((j & 15) == 0) {
    st_pute(sd, st, so / 16 + (j >> 4), emlo);
    st_pute(sd, st, so / 16 + ((j + 32) >> 4), emhi);
  }
  if (!is_k) return;
  const size_t slot = (size_t)rl_kv_pos(a) * L.H_KV + kh;   // sequence 0
  int16_t *km = L.k_m + slot * HD;
  int8_t *ke = L.k_e + slot * (HD / 16);
  km[j] = (int16_t)qlo;
  km[j + 32] = (int16_t)qhi;
  if ((j & 15) == 0) {
    ke[j >> 4] = (int8_t)emlo;
    ke[(j + 32) >> 4] = (int8_t)emhi;
  }
  const int voff = L.D + L.KV + kh * HD;
  int16_t *vm = L.v_m + slot * HD;
  int8_t *ve = L.v_e + slot * (HD / 16);
  const int v0 = L.qkv_m[voff + j], v1 = L.qkv_m[voff + j + 32];
  vm[j] = (int16_t)v0;
  vm[j + 32] = (int16_t)v1;
  st_put(sd, ST_V, kh * HD + j, v0);
  st_put(sd, ST_V, kh * HD + j + 32, v1);
  if (j < 4) {
    const int vt = L.qkv_e[voff / 16 + j];
    ve[j] = (int8_t)vt;
    st_pute(sd, ST_V, kh * 4 + j, vt);
  }
}

constexpr int RL_ATT_T = 256;

__device__ __forceinline__ int block_max_i(int v, int *red) {
  for (int o = 1; o < 64; o <<= 1) {
    const int w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = red[0];
  for (int i = 1; i < RL_ATT_T / 64; ++i) v = red[i] > v ? red[i] : v;
  return v;
}

__device__ __forceinline__ long long block_sum_ll(long long v, long long *red) {
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = 0;
  for (int i = 0; i < RL_ATT_T / 64; ++i) v += red[i];
  return v;
}

// Attention of query head h (S_QK_* .. S_AV_*): scores of t = 0..kv_pos on
// the engine's lane 0 (Q head as x, K[t] as the weight row), pre-align to the
// shared max exponent, softmax with exponent - 3 (1/sqrt(64)), then per
// 16-dim chunk the engine over one 16-input tile of probabilities (t <= 15)
// with V pre-shifted to its largest exponent over t <= kv_pos.
__global__ __launch_bounds__(RL_ATT_T) void k_rl_attn(RtlArgs a) {
  extern __shared__ long long rl_lds[];
  __shared__ int qs[64], qe[4], red_i[RL_ATT_T / 64], s_pe, s_vmax[4];
  __shared__ long long red_l[RL_ATT_T / 64], s_inv;
  __shared__ int pm[16];
  const LayerArgs &L = a.L;
  const int h = blockIdx.x, tid = threadIdx.x, HD = 64;
  const int g = (h * L.H_KV) / L.H_Q;
  const int n = rl_kv_pos(a) + 1;
  int *xs = reinterpret_cast<int *>(rl_lds);   // n aligned scores, then LUT values
  int *se = xs + n;                             // n score exponents
  if (tid < 64) qs[tid] = L.qkv_m[h * HD + tid];
  if (tid < 4) qe[tid] = L.qkv_e[h * 4 + tid];
  __syncthreads();
  for (int t = tid; t < n; t += RL_ATT_T) {
    const size_t slot = (size_t)t * L.H_KV + g;
    const int16_t *k = L.k_m + slot * HD;
    const int8_t *ke = L.k_e + slot * 4;
    long long acc = 0;
    int acc_e = 0;
    for (int c = 0; c < 4; ++c) {
      long long s = 0;
      for (int kk = 0; kk < 16; ++kk) s += (long long)qs[c * 16 + kk] * k[c * 16 + kk];
      const int te = qe[c] + ke[c];
      if (c == 0) {
        acc = s;
        acc_e = te;
      } else {
        engine_fold(acc, acc_e, s, te);
      }
    }
    int sh;
    xs[t] = norm16(acc, lead64(acc), sh);
    se[t] = clamp8(acc_e + sh - 15);
  }
  __syncthreads();
  int lmax = -128;
  for (int t = tid; t < n; t += RL_ATT_T) lmax = se[t] > lmax ? se[t] : lmax;
  const int es = block_max_i(lmax, red_i);
  int xmax = -32768;
  for (int t = tid; t < n; t += RL_ATT_T) {
    const int d = es - se[t];               // 9-bit in the FSM: no wrap
    const int v = d >= 16 ? 0 : (xs[t] >> d);
    xs[t] = v;
    xmax = v > xmax ? v : xmax;
  }
  const int mx = block_max_i(xmax, red_i);
  const int xe = (int)(signed char)(es - 3);
  const int sh = xe - 8;
  long long part = 0;
  for (int t = tid; t < n; t += RL_ATT_T) {
    const long long d = (long long)xs[t] - mx;
    const long long ds = sh >= 0 ? d * (1LL << (sh > 40 ? 40 : sh)) : (d >> (-sh > 62 ? 62 : -sh));
    const int idx = ds >= 0 ? 1023 : (ds <= -1023 ? 0 : (int)(ds + 1023));
    const int v = a.exp_lut[idx];
    xs[t] = v;
    part += v;
  }
  const long long tot = block_sum_ll(part, red_l);
  if (tid == 0) {
    const int msb = tot ? 63 - __clzll((unsigned long long)tot) : 0;
    __int128 y = (__int128)1 << (31 - msb);
    for (int it = 0; it < 4; ++it) y = (y * (((__int128)1 << 33) - (__int128)tot * y)) >> 32;
    s_inv = (long long)y;
  }
  __syncthreads();
  const long long inv = s_inv;
  int ml = 0;
  for (int t = tid; t < n; t += RL_ATT_T) {
    const long long p = (long long)xs[t] * inv;
    const int l = p ? lead64(p) : 0;
    ml = l > ml ? l : ml;
  }
  ml = block_max_i(ml, red_i);
  if (tid < 16) {
    int s2;
    pm[tid] = tid < n ? norm16((long long)xs[tid] * inv, ml, s2) : 0;
  }
  if (tid == 0) s_pe = clamp8(ml - 14 - 17);
  // V exponent max per 16-dim chunk over t <= kv_pos
  int vm4[4] = {-128, -128, -128, -128};
  for (int t = tid; t < n; t += RL_ATT_T) {
    const int8_t *ve = L.v_e + ((size_t)t * L.H_KV + g) * 4;
    for (int c = 0; c < 4; ++c) vm4[c] = ve[c] > vm4[c] ? ve[c] : vm4[c];
  }
  for (int c = 0; c < 4; ++c) {
    const int v = block_max_i(vm4[c], red_i);
    if (tid == 0) s_vmax[c] = v;
  }
  __syncthreads();
  if (tid >= 64) return;
  const int c = tid >> 4, l = tid & 15;
  const int vmax = s_vmax[c];
  const int nav = n < 16 ? n : 16;
  long long s = 0;
  for (int t = 0; t < nav; ++t) {
    const size_t slot = (size_t)t * L.H_KV + g;
    const int vt = L.v_e[slot * 4 + c];
    s += (long long)pm[t] * shr8(L.v_m[slot * HD + c * 16 + l], vmax, vt);
  }
  int sh2;
  const int m = norm16(s, lead64(s), sh2);
  const int e = clamp8(s_pe + vmax + sh2 - 15);
  const int emax = max16_lanes(e);
  const int mq = shr8(m, emax, e);
  const int i = h * HD + c * 16 + l;
  L.att_m[i] = (int16_t)mq;
  if (l == 0) L.att_e[h * 4 + c] = (int8_t)emax;
  st_put(L.dump, ST_ATTN, i, mq);
  if (l == 0) st_pute(L.dump, ST_ATTN, h * 4 + c, emax);
}

// ------------------------------------------------------------- decode head
// smollm_decode_head_bfp.sv: S_NORM (the RMSNorm engine with the final norm
// gamma from its ROM, i.e. tile_quantize'd), then per 16-row chunk of the
// tied embedding the matvec engine (S_MV_*), whose per-lane (m, e) feed the
// bfp_gt running argmax (S_MV_LANE_CMP / S_MV_MERGE, k_rtl_argmax).
__global__ __launch_bounds__(64) void k_rl_head_norm(RtlHeadArgs a) {
  extern __shared__ long long rl_lds[];
  __shared__ long long s_inv;
  __shared__ int s_einv;
  const int D = a.D, nt = D / 16, tid = threadIdx.x;
  long long *sums = rl_lds;
  int16_t *gm = reinterpret_cast<int16_t *>(rl_lds + nt);
  int8_t *ge = reinterpret_cast<int8_t *>(gm + D);
  for (int base = 0; base < D; base += 64) {   // D % 64 == 0: whole 16-lane tiles
    const int i = base + tid;
    int e;
    const int m = quantize16_lanes(a.norm_w[i], e);
    gm[i] = (int16_t)m;
    if ((i & 15) == 0) ge[i >> 4] = (int8_t)e;
  }
  __syncthreads();
  rmsnorm_wave(a.h_m, a.h_e, gm, ge, D, a.xn_m, a.xn_e, sums, &s_inv, &s_einv);
}

// One 16-row chunk of the embedding per workgroup: the engine's per-row
// (m, e) into lg_m / lg_e.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_rl_head_mv(RtlHeadArgs a) {
  constexpr int TPT = 3;
  extern __shared__ long long rl_lds[];
  const int c = blockIdx.x, nT = a.D / 16;
  long long *Sl = rl_lds;
  int *El = reinterpret_cast<int *>(Sl + nT * 16);
  int *xs = El + nT * 16;
  int *xes = xs + nT * 16;
  stage_x_bfp(xs, xes, a.xn_m, a.xn_e, nT);
  __syncthreads();
  int m, e;
  rl_chunk_me<NW, TPT>(a.emb_m + (size_t)c * nT * 32, a.emb_e + (size_t)c * nT * 16, nT, xs, xes,
                       Sl, El, m, e);
  if (threadIdx.x < 16) {
    a.lg_m[c * 16 + threadIdx.x] = (int16_t)m;
    a.lg_e[c * 16 + threadIdx.x] = (int8_t)e;
  }
}

// One step of the FPGA driver's token loop on the device
// (autoregress_bfp_top.sv:357-386): record the head's token as this step's
// prediction (and the last layer's output when a history is kept), then the
// next step's input -- prompt[step + 1] while the prompt lasts, else this
// prediction -- and advance the step.  One 64-thread workgroup.
__global__ __launch_bounds__(64) void k_rtl_ctl(RtlCtlArgs a) {
  const int tid = threadIdx.x;
  const int step = a.state[0], tok = *a.tok;
  if (a.hist_m) {
    for (int i = tid; i < a.D; i += 64) a.hist_m[(size_t)step * a.D + i] = a.h_m[i];
    for (int i = tid; i < a.D / 16; i += 64) a.hist_e[(size_t)step * (a.D / 16) + i] = a.h_e[i];
  }
  __syncthreads();   // every thread has read the step before it changes
  if (tid == 0) {
    a.preds[step] = tok;
    a.state[1] = step + 1 < a.n_prompt ? a.prompt[step + 1] : tok;
    a.state[0] = step + 1;
  }
}

}  // namespace rtl
}  // namespace bfp

// ---------------------------------------------- allocation-free argmax
// Scratch of bfp_rtl_argmax_static_d: the per-chunk bests (mantissa,
// exponent, index) of at most ARGMAX_STATIC_CHUNKS chunks (batch * n/16),
// in one device-global array per GPU: 3 MiB, held until the process ends.
// Host code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): argmax_scratch() looks its address up
// once per device with hipGetSymbolAddress and hands that out.
namespace bfp {
namespace {
constexpr long long ARGMAX_STATIC_CHUNKS = 262144;
static __device__ __align__(256) int scratch[3 * ARGMAX_STATIC_CHUNKS];
constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
int *g_scratch[SCRATCH_MAX_DEVICES] = {};

int argmax_scratch(int **out) {
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
    return set_err(BFP_EINVAL, "rtl_argmax_static: device %d beyond the %d supported", dev,
                   SCRATCH_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return set_err(BFP_EIO, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                     hipGetErrorString(err));
    g_scratch[dev] = static_cast<int *>(p);
  }
  *out = g_scratch[dev];
  return BFP_OK;
}
}  // namespace
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

// bfp_rtl_argmax_d with its workspace in the library's static device
// scratch (no allocation).  The kernel writes every chunk's entry before it
// reads it, so nothing needs clearing between calls; calls that overlap on
// one GPU share the scratch and race.
int bfp_rtl_argmax_static_d(const int16_t *m, const int8_t *e, int n, int batch, int32_t *idx,
                            void *stream) {
  if (n <= 0 || n % 16 || batch <= 0 || !m || !e || !idx)
    return set_err(BFP_EINVAL, "rtl_argmax_static: n=%d batch=%d", n, batch);
  const long long nc = (long long)batch * (n / 16);
  if (nc > bfp::ARGMAX_STATIC_CHUNKS)
    return set_err(BFP_EINVAL,
                   "rtl_argmax_static: batch * n/16 = %lld chunks exceeds the static scratch's "
                   "%lld (use bfp_rtl_argmax_d with a workspace)",
                   nc, bfp::ARGMAX_STATIC_CHUNKS);
  int *w = nullptr;
  BFP_TRY(bfp::argmax_scratch(&w));
  hipLaunchKernelGGL(rtl::k_rtl_argmax, dim3(batch), dim3(256), 0, (hipStream_t)stream, m, e, n, w,
                     w + nc, w + 2 * nc, idx);
  return launch_status("rtl_argmax_static");
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

namespace bfp {

namespace {
typedef void (*rl_mv_fn)(RtlArgs, int);
rl_mv_fn rl_mv_kernel(int nw) {
  static const rl_mv_fn k[9] = {rtl::k_rl_mv<1>, rtl::k_rl_mv<2>, rtl::k_rl_mv<3>,
                                rtl::k_rl_mv<4>, rtl::k_rl_mv<5>, rtl::k_rl_mv<6>,
                                rtl::k_rl_mv<7>, rtl::k_rl_mv<8>, rtl::k_rl_mv<9>};
  return nw >= 1 && nw <= 9 ? k[nw - 1] : nullptr;
}

// One matvec op of the layer: nT input tiles, n_wg output chunks.
int rl_mv(const RtlArgs &a, int op, int nT, int n_wg, hipStream_t s) {
  const int nw = (nT + 11) / 12;   // 3 tiles per lane, 4 tile lanes per wave
  rl_mv_fn f = rl_mv_kernel(nw);
  if (!f) return set_err(BFP_EINVAL, "rtl layer: %d input tiles unsupported", nT);
  hipLaunchKernelGGL(f, dim3(n_wg), dim3(64 * nw), (size_t)nT * 260, s, a, op);
  return launch_status("rtl layer matvec");
}
}  // namespace

int launch_rtl_layer(const RtlArgs &a, hipStream_t s) {
  const LayerArgs &L = a.L;
  const int ntD = L.D / 16, ntF = L.FFN / 16;
  // with pos_ptr the caller keeps the device step inside the capacity
  if (L.batch != 1 || L.HD != 64 ||
      (!a.pos_ptr && (a.kv_pos < 0 || a.kv_pos >= L.max_ctx || a.pos < 0)))
    return set_err(BFP_EINVAL, "rtl layer: batch %d, HD %d, pos %d, kv_pos %d (capacity %d)",
                   L.batch, L.HD, a.pos, a.kv_pos, L.max_ctx);
  const int n_att = a.pos_ptr ? L.max_ctx : a.kv_pos + 1;   // positions the attention's LDS holds
  const size_t lds_norm = (size_t)ntD * 9 + (size_t)L.D * 2;
  hipLaunchKernelGGL(rtl::k_rl_norm, dim3(1), dim3(64), lds_norm, s, a, 0);
  BFP_TRY(launch_status("rtl layer norm1"));
  BFP_TRY(rl_mv(a, 0, ntD, (L.D + 2 * L.KV) / 16, s));
  hipLaunchKernelGGL(rtl::k_rl_rope_kv, dim3(L.H_Q + L.H_KV), dim3(64), 0, s, a);
  BFP_TRY(launch_status("rtl layer rope"));
  hipLaunchKernelGGL(rtl::k_rl_attn, dim3(L.H_Q), dim3(rtl::RL_ATT_T), (size_t)n_att * 8, s, a);
  BFP_TRY(launch_status("rtl layer attention"));
  BFP_TRY(rl_mv(a, 1, ntD, ntD, s));
  hipLaunchKernelGGL(rtl::k_rl_norm, dim3(1), dim3(64), lds_norm, s, a, 1);
  BFP_TRY(launch_status("rtl layer norm2"));
  BFP_TRY(rl_mv(a, 2, ntD, ntF, s));
  return rl_mv(a, 3, ntF, ntD, s);
}

int launch_rtl_ctl(const RtlCtlArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(rtl::k_rtl_ctl, dim3(1), dim3(64), 0, s, a);
  return launch_status("rtl loop control");
}

int launch_rtl_head(const RtlHeadArgs &a, hipStream_t s) {
  const int nT = a.D / 16;
  if (a.D % 64 || a.VOCAB % 16 || a.VOCAB <= 0)
    return set_err(BFP_EINVAL, "rtl head: D %d (multiple of 64), VOCAB %d (multiple of 16)", a.D,
                   a.VOCAB);
  typedef void (*hm_fn)(RtlHeadArgs);
  static const hm_fn k[9] = {rtl::k_rl_head_mv<1>, rtl::k_rl_head_mv<2>, rtl::k_rl_head_mv<3>,
                             rtl::k_rl_head_mv<4>, rtl::k_rl_head_mv<5>, rtl::k_rl_head_mv<6>,
                             rtl::k_rl_head_mv<7>, rtl::k_rl_head_mv<8>, rtl::k_rl_head_mv<9>};
  const int nw = (nT + 11) / 12;   // 3 tiles per lane, 4 tile lanes per wave
  if (nw > 9) return set_err(BFP_EINVAL, "rtl head: %d input tiles unsupported", nT);
  hipLaunchKernelGGL(rtl::k_rl_head_norm, dim3(1), dim3(64), (size_t)nT * 9 + (size_t)a.D * 2, s, a);
  BFP_TRY(launch_status("rtl head norm"));
  hipLaunchKernelGGL(k[nw - 1], dim3(a.VOCAB / 16), dim3(64 * nw), (size_t)nT * 260, s, a);
  BFP_TRY(launch_status("rtl head matvec"));
  const long long nc = a.VOCAB / 16;
  hipLaunchKernelGGL(rtl::k_rtl_argmax, dim3(1), dim3(256), 0, s, a.lg_m, a.lg_e, a.VOCAB, a.work,
                     a.work + nc, a.work + 2 * nc, a.token);
  return launch_status("rtl head argmax");
}

}  // namespace bfp
