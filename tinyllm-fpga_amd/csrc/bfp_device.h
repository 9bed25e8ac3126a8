// Device-side helpers shared by the BFP kernels (gfx950, wave64).
//
// Numerics follow the reference's model-level simulator,
// rtl/vc707/host/gen_smollm_blockfp_full.py (full.py):
//   tile_quantize  full.py:90-97   e = clip(floor(log2 max|v|) + 1, -127, 127)
//                                  m = clip(rne(v * 2^(15-e)), -32768, 32767)
//   matvec         full.py:217-233 exact integer tile sums, max-first floor
//                                  alignment, float64 scale, re-quantise.
// All float64 code in this build is compiled with -ffp-contract=off: every
// product and sum is rounded separately, as numpy does.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bfp {

constexpr int TILE = 16;
constexpr int ALIGN_MAX = 47;
constexpr long long SAT_HI = (1LL << 47) - 1;
constexpr long long SAT_LO = -(1LL << 47);

// floor(np.log2(a)) as numpy computes it.  np.log2 is correctly rounded, so
// for a in [2^(k-1), 2^k) it returns k itself -- not a value below k -- when
// log2(a) = k - d lies within half a double spacing of k, i.e. when
// a >= 2^k (1 - n 2^-53) with n = n_up(k) = floor(2^p ln 2), where p is
// floor(log2 |k|) (less one for a power of two k > 0, whose lower neighbour
// sits in the binade below).  n_up is 0 for |k| <= 2, 1 for k = 3, 4, -2,
// -3, ... 44 for k = 65..128 and -64..-127; the tests check every
// k in [-130, 130] against numpy.  0xB17217F7D1CF79AB is ln 2 in 0.64 fixed
// point: its top p bits are floor(2^p ln 2).
__device__ __forceinline__ int log2_up_ulps(int k) {
  if (k == 0) return 0;
  const int a = k < 0 ? -k : k;
  int p = 31 - __clz(a);
  if (k > 0 && (a & (a - 1)) == 0) --p;
  if (p <= 0) return 0;
  if (p > 10) p = 10;
  return (int)(0xB17217F7D1CF79ABull >> (64 - p));
}

// Shared exponent of a tile from its max |v|: floor(np.log2(amax)) + 1
// clipped to [-127, 127] (full.py:92).  frexp gives amax = f * 2^x with f in
// [0.5, 1), so the exact floor(log2(amax)) + 1 is x; numpy's rounding of
// log2 makes it x + 1 when f >= 1 - n_up(x) 2^-53 (1 - n 2^-53 is exact).
// amax == 0 -> -127 (the reference floors amax at 1e-300, whose exponent
// clips to -127).
__device__ __forceinline__ int tile_exp_of(double amax) {
  if (!(amax > 0.0)) return -127;
  int x;
  const double f = frexp(amax, &x);
  const int n = log2_up_ulps(x);
  if (n > 0 && f >= 1.0 - (double)n * 0x1p-53) ++x;
  return x < -127 ? -127 : (x > 127 ? 127 : x);
}

// Mantissa: rne(v * 2^(15-e)) clipped; ldexp is exact here, rint is
// round-half-even (np.round with 0 decimals).
__device__ __forceinline__ int tile_mant_of(double v, int e) {
  double s = rint(ldexp(v, 15 - e));
  s = fmin(fmax(s, -32768.0), 32767.0);
  return (int)s;
}

// rne(A / 2^s) clipped to int16, for |A| < 2^48; s may be <= 0 (left shift).
__device__ __forceinline__ int rne_shr_clip(long long A, int s) {
  long long v;
  if (A == 0) {
    v = 0;
  } else if (s <= 0) {
    int l = -s;
    v = (l > 20) ? (A > 0 ? 32767 : -32768) : (A * (1LL << l));
  } else if (s >= 62) {
    v = 0;
  } else {
    long long q = A >> s;                  // floor
    long long r = A - q * (1LL << s);      // 0 <= r < 2^s
    long long h = 1LL << (s - 1);
    v = q + ((r > h || (r == h && (q & 1))) ? 1 : 0);
  }
  return v < -32768 ? -32768 : (v > 32767 ? 32767 : (int)v);
}

__device__ __forceinline__ int msb64(unsigned long long a) { return 63 - __clzll(a); }

constexpr int L_NONE = -(1 << 30);

// The chunk exponent's reduction key of one row: 2 L + u, where L =
// floor(log2|y|) and u = 1 when np.log2(|y|) rounds up to L + 1 (|y| within
// n_up(L + 1) double spacings below 2^(L+1), see log2_up_ulps).  With |A| in
// [2^b, 2^(b+1)) that is (2^(b+1) - |A|) 2^(52-b) <= n_up, which needs b >= 44
// (|A| < 2^48 here, n_up <= 709).  The max of the keys over a tile gives the
// largest L and whether its largest |y| rounds up.
__device__ __forceinline__ int row_exp_key(long long A, int M) {
  if (A == 0) return L_NONE;
  const unsigned long long a = A < 0 ? (unsigned long long)(-A) : (unsigned long long)A;
  const int b = msb64(a);
  const int L = b + M - 30;
  int u = 0;
  if (b >= 44) {
    const unsigned long long gap = (2ull << b) - a;            // >= 1
    u = (gap << (52 - b)) <= (unsigned long long)log2_up_ulps(L + 1) ? 1 : 0;
  }
  return 2 * L + u;
}

// Tile exponent from the max of row_exp_key over the tile.
__device__ __forceinline__ int chunk_exp_from_key(int key) {
  if (key == L_NONE) return -127;
  const int e = (key >> 1) + 1 + (key & 1);
  return e < -127 ? -127 : (e > 127 ? 127 : e);
}

// Wave-level reductions (wave64) with cross-lane shuffles.
template <typename T>
__device__ __forceinline__ T xor_max(T v, int mask) {
  T o = __shfl_xor(v, mask, 64);
  return o > v ? o : v;
}
template <typename T>
__device__ __forceinline__ T xor_sum(T v, int mask) {
  return v + __shfl_xor(v, mask, 64);
}

// Register-only cross-lane exchange for gfx950 (no LDS round trip).
// peer<M>(v) returns, for M = 16 or 32, the value of lane i^M (permlane16 /
// permlane32 swap); for M = 1, 2, 4, 8, the value of lane (i - M) mod 16 of
// the same 16-lane row (DPP row rotate).  A row reduction that combines v
// with peer<M>(v) for M = 8, 4, 2, 1 in that order, or with any order for an
// order-free operation (max, or, integer add), gives every lane the same
// result as the xor butterfly: after the steps for the larger masks the
// values are symmetric under them, and rotate and xor partners differ only
// by such masks (float addition is commutative).
// Workgroup barrier over LDS data only: every wave's LDS accesses complete
// before it, but its global loads and stores in flight do not have to (a
// __syncthreads() after a global store waits for all of the wave's memory
// operations, e.g. a weight prefetch issued for a later stage).  No code
// here passes data between the threads of a workgroup through global memory.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Non-temporal loads (the nt cache policy): for data read once per pass,
// such as weight matrices streamed from HBM.  A plain streaming read of
// 4 GiB measured 7.1-7.2 TB/s this way against 6.0-6.4 TB/s with ordinary
// loads.
__device__ __forceinline__ uint4 ld_nt(const uint4 *p) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const u4 t = __builtin_nontemporal_load(reinterpret_cast<const u4 *>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ int ld_nt(const int8_t *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ float4 ld_nt(const float4 *p) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4 t = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(p));
  return make_float4(t.x, t.y, t.z, t.w);
}

template <int M>
__device__ __forceinline__ int peer_u32(int v) {
  if constexpr (M == 16) {
    auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (int)((threadIdx.x & 16) ? p[0] : p[1]);
  } else if constexpr (M == 32) {
    auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (int)((threadIdx.x & 32) ? p[0] : p[1]);
  } else {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8, "row rotate by 1, 2, 4 or 8");
    return __builtin_amdgcn_update_dpp(0, v, 0x120 + M, 0xf, 0xf, false);
  }
}
template <int M>
__device__ __forceinline__ int peer(int v) {
  return peer_u32<M>(v);
}
template <int M>
__device__ __forceinline__ long long peer(long long v) {
  const int lo = peer_u32<M>((int)(v & 0xffffffffLL));
  const int hi = peer_u32<M>((int)(v >> 32));
  return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
template <int M>
__device__ __forceinline__ double peer(double v) {
  const long long b = __double_as_longlong(v);
  return __longlong_as_double(peer<M>(b));
}
template <int M, typename T>
__device__ __forceinline__ T pmax(T v) {
  const T o = peer<M>(v);
  return o > v ? o : v;
}
template <int M, typename T>
__device__ __forceinline__ T psum(T v) {
  return v + peer<M>(v);
}

}  // namespace bfp
