// float64 building blocks of the model-level simulator's leaf ops, in the
// reduction orders numpy/OpenBLAS use (rtl/vc707/host/gen_smollm_blockfp_full.py
// :236-258,274-281).  Compiled with -ffp-contract=off: each + and * rounds.
#pragma once
#include <hip/hip_runtime.h>

#include "bfp_device.h"

namespace bfp {

// ---------------------------------------------------------------- pairwise
// numpy's float64 add-reduce of one contiguous block (n <= 8192): blocks of
// <= 128 are summed with 8 accumulators, longer ranges split at
// n2 = n/2 rounded down to a multiple of 8.  Leaves are numbered in
// left-to-right order.
constexpr int PW_DEPTH = 6;        // n <= 128 * 2^6 = 8192
constexpr int PW_MAX_LEAVES = 64;  // leaf slots: one per 64-element block, n <= 4096

// numpy's combination of the leaves of a range of n elements: split at
// n2 = n/2 rounded down to a multiple of 8 while longer than 128, each node
// the sum left + right; the leaf starting at element lo is leaf[lo / 64]
// (see pairwise_sum_block_g).  Evaluated across the 64 lanes of a wave
// (every lane of the wave calls; every lane returns the root).  Lane i, with
// q = 63 - i, follows the path from the root that the bits of q give, most
// significant first (1 = right part of a split); it starts with the value
// of the leaf it reaches when the remaining bits of q are all 0 (the first
// q of the leaf's span of 64 >> depth), else with none.  Step k adds the
// value at q + 2^k (lane i - 2^k: a row rotate for k < 4, a permlane swap
// for 16 and 32) into q (bits 0..k of q clear): where both hold a value the
// span is an internal node and that addition is numpy's left + right; where
// only the left part holds one it is a leaf covering both halves.  q = 0
// (lane 63) ends with the root.
__device__ __forceinline__ double pw_combine_wave(int n, const double *leaf) {
  const int q = 63 - (int)(threadIdx.x & 63);
  int lo = 0, len = n, span = 64;
#pragma unroll
  for (int d = 0; d < PW_DEPTH; ++d) {
    if (len > 128) {
      int n2 = len / 2;
      n2 -= n2 % 8;
      span >>= 1;
      if (q & span) {
        lo += n2;
        len -= n2;
      } else {
        len = n2;
      }
    }
  }
  int have = (q & (span - 1)) == 0;
  double v = have ? leaf[lo >> 6] : 0.0;
  // the deepest leaves span 2^(6 - depth) lanes: the steps below that span
  // have no pair to add (a range of at most 128 elements is one leaf)
  int depth = 0;
  for (int m = n; m > 128; ++depth) {
    int n2 = m / 2;
    n2 -= n2 % 8;
    m -= n2;   // the right part is the longer one
  }
  const int first = PW_DEPTH - depth;   // wave-uniform
  auto step = [&](double o, int oh, int m) {
    if (!(q & m) && oh) {
      v = have ? v + o : o;
      have = 1;
    }
  };
  if (first <= 0) step(peer<1>(v), peer<1>(have), 1);
  if (first <= 1) step(peer<2>(v), peer<2>(have), 2);
  if (first <= 2) step(peer<4>(v), peer<4>(have), 4);
  if (first <= 3) step(peer<8>(v), peer<8>(have), 8);
  if (first <= 4) step(peer<16>(v), peer<16>(have), 16);
  if (first <= 5) step(peer<32>(v), peer<32>(have), 32);
  const long long b = __double_as_longlong(v);
  const int lo32 = __builtin_amdgcn_readlane((int)(b & 0xffffffffLL), 63);
  const int hi32 = __builtin_amdgcn_readlane((int)(b >> 32), 63);
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi32 << 32) | (unsigned)lo32));
}

// Sum of get(0) .. get(n-1) (1 <= n <= 4096) in numpy order, plus numpy's
// initial 0.0; get(i) is called for the elements of this lane's leaf (and
// for index 0 by lanes that own none), so it may read global memory.
// Called by all threads of a workgroup (uses lds_barrier);
// leafbuf holds PW_MAX_LEAVES doubles of LDS.  Returns the sum in every
// thread; waves may still read leafbuf on return, so it is written again
// only after a later barrier.
//
// numpy splits a range longer than 128 at n/2 rounded down to a multiple of
// 8, so every leaf of a range longer than 128 has at least 64 elements and
// each 64-element block [64g, 64g+64) holds at most one leaf start.  Group
// g of 8 lanes descends to the leaf holding element min(64g+63, n-1) and
// owns it if the leaf starts in its block.  Lane j of the group runs
// numpy's accumulator r_j (elements j, j+8, ... of the leaf, in order); the
// tree ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) is formed with row rotates (lane
// 7 of the group ends with it; float addition is commutative, so the
// rotate partners give the same sums); then the leaf's last n%8 elements
// are added in order.  A leaf of fewer than 8 elements is summed from 0.0
// by one lane, as numpy does.
template <class Get>
__device__ __forceinline__ double pairwise_sum_block_g(Get get, int n, double *leafbuf) {
  const int t = threadIdx.x, bs = blockDim.x;
  const int ng = (n + 63) >> 6;
  for (int base = 0; base < 8 * ng; base += bs) {   // uniform loop
    const int q = base + t, gq = q >> 3, j = q & 7;
    const int e = min(gq * 64 + 63, n - 1);
    int flo = 0, fn = n;
    while (fn > 128) {
      int n2 = fn / 2;
      n2 -= n2 % 8;
      if (e < flo + n2) {
        fn = n2;
      } else {
        flo += n2;
        fn -= n2;
      }
    }
    const bool own = gq < ng && flo >= gq * 64;
    const int top = fn - fn % 8, end = flo + top;
    double x[16];   // a leaf has at most 128 elements: 16 per accumulator
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int idx = flo + j + 8 * i;
      x[i] = get(own && idx < end ? idx : 0);
    }
    double r = x[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) r = flo + j + 8 * i < end ? r + x[i] : r;
    r = r + peer<1>(r);
    r = r + peer<2>(r);
    r = r + peer<4>(r);
    if (own && j == 7) {
      double res;
      if (fn < 8) {
        res = 0.0;
        for (int i = 0; i < fn; ++i) res += get(flo + i);
      } else {
        res = r;
        for (int i = top; i < fn; ++i) res += get(flo + i);
      }
      leafbuf[gq] = res;
    }
  }
  lds_barrier();
  return 0.0 + pw_combine_wave(n, leafbuf);
}

// The same sum of a[0..n) held in LDS.
__device__ __forceinline__ double pairwise_sum_block(const double *a, int n, double *leafbuf) {
  return pairwise_sum_block_g([a](int i) { return a[i]; }, n, leafbuf);
}

// ------------------------------------------------------------------ ddot
// OpenBLAS 0.3.29 x86_64 ddot, SkylakeX micro-kernel, n = 64: four 8-lane
// FMA accumulators over two blocks of 32, each folded 512->256 bit (lane l +
// lane l+4), summed ((a0+a1)+a2)+a3, then 128-bit halves and a horizontal
// add.  This is np.dot's order on SkylakeX/SapphireRapids hosts.
__device__ inline double ddot64_skx(const double *x, const double *y) {
  double acc[4][8];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[r][l] = fma(x[8 * r + l], y[8 * r + l], 0.0);
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[r][l] = fma(x[32 + 8 * r + l], y[32 + 8 * r + l], acc[r][l]);
  double s[4];
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    double f0 = acc[0][l] + acc[0][l + 4];
    double f1 = acc[1][l] + acc[1][l + 4];
    double f2 = acc[2][l] + acc[2][l + 4];
    double f3 = acc[3][l] + acc[3][l + 4];
    s[l] = ((f0 + f1) + f2) + f3;
  }
  return (s[0] + s[2]) + (s[1] + s[3]);
}

// The same dot product with the second operand a BFP 64-vector: mantissas
// km (8 x uint4, 8 int16 each), the 4 tile exponents packed little-endian
// in ke4.  Each element is decoded exactly
// (m * 2^(e-15)) before its FMA, so the result equals ddot64_skx(x, y).
__device__ inline double ddot64_skx_bfp(const double *x, const uint4 *__restrict__ km, int ke4) {
  double acc[4][8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint4 u = km[4 * h + r];
      const int ex = (int)(signed char)((ke4 >> (8 * (2 * h + (r >> 1)))) & 0xff);
      const double s = ldexp(1.0, ex - 15);
      const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const int m = (int)(short)((w[l >> 1] >> (16 * (l & 1))) & 0xffff);
        const double y = (double)m * s;
        acc[r][l] = fma(x[32 * h + 8 * r + l], y, h == 0 ? 0.0 : acc[r][l]);
      }
    }
  }
  double s4[4];
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    double f0 = acc[0][l] + acc[0][l + 4];
    double f1 = acc[1][l] + acc[1][l + 4];
    double f2 = acc[2][l] + acc[2][l + 4];
    double f3 = acc[3][l] + acc[3][l + 4];
    s4[l] = ((f0 + f1) + f2) + f3;
  }
  return (s4[0] + s4[2]) + (s4[1] + s4[3]);
}

// --------------------------------------------------------------- exp
// np.exp is numpy's own SIMD exp (not correctly rounded for ~5% of inputs);
// the device uses the ROCm device library's exp.  The two may differ in the
// last bit; that reaches a BFP mantissa only at a rounding tie of the 16-bit
// re-quantisation (about 2^-36 per element).
__device__ __forceinline__ double exp_f64(double x) { return exp(x); }

// -------------------------------------------------------- tile quantise
// Canonical BFP form.  Each stage of the reference hands float64 values
// (the decoded "raw" quantisation) to the next op.  Where the next op is a
// matvec, those values are quantised again with tile_quantize
// (full.py:264,283,287,291), and so are the stage dumps
// (gen_smollm_blockfp_bfp.py:393-409).  Re-quantising is the identity except
// for a tile whose largest magnitude is the mantissa -32768: it becomes
// e+1 with every mantissa round-half-even(m/2) -- which changes the values of
// odd mantissas.  So the pipeline carries raw tiles between stages and
// forms the canonical tile only for matvec inputs and dumps.  16 lanes (one
// mantissa each) call it.
__device__ __forceinline__ void canon16_lanes(int &m, int &e) {
  int hit = (m == -32768) ? 1 : 0;
  hit |= peer<1>(hit);
  hit |= peer<2>(hit);
  hit |= peer<4>(hit);
  hit |= peer<8>(hit);
  if (hit && e < 127) {
    e += 1;
    int q = m >> 1;                     // floor(m / 2)
    m = (m & 1) ? q + (q & 1) : q;      // ties to even
  }
}

// Quantise the 16 values held by lanes (lane & ~15) .. (lane | 15) of a
// wave (one value per lane): returns this lane's mantissa and sets e to the
// tile exponent (tile_quantize, full.py:90-97; canonical form when
// `canonical`).  All 64 lanes must participate.
__device__ __forceinline__ int quantize16_lanes(double v, int &e, bool canonical = false) {
  double a = fabs(v);
  a = pmax<1>(a);
  a = pmax<2>(a);
  a = pmax<4>(a);
  a = pmax<8>(a);
  e = tile_exp_of(a);
  int m = tile_mant_of(v, e);
  if (canonical) canon16_lanes(m, e);
  return m;
}

__device__ __forceinline__ double bfp_val(int m, int e) { return ldexp((double)m, e - 15); }

// An 8-lane group's maximum / or (lanes 8g .. 8g+7): row half-mirror (lane
// i with 7 - i), then quad swaps i ^ 1 and i ^ 2 -- after the three steps
// every lane has combined all eight.
template <class F>
__device__ __forceinline__ int group8_u32(int v, F op) {
  v = op(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, false));   // row_half_mirror
  v = op(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, false));    // quad_perm 1,0,3,2
  return op(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, false)); // quad_perm 2,3,0,1
}
__device__ __forceinline__ double group8_max(double v) {
  auto dpp = [](double x, int ctrl) {
    const long long b = __double_as_longlong(x);
    int lo = (int)(b & 0xffffffffLL), hi = (int)(b >> 32);
    switch (ctrl) {
      case 0x141:
        lo = __builtin_amdgcn_mov_dpp(lo, 0x141, 0xf, 0xf, false);
        hi = __builtin_amdgcn_mov_dpp(hi, 0x141, 0xf, 0xf, false);
        break;
      case 0xB1:
        lo = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xf, 0xf, false);
        hi = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xf, 0xf, false);
        break;
      default:
        lo = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xf, 0xf, false);
        hi = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xf, 0xf, false);
        break;
    }
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
  };
  v = fmax(v, dpp(v, 0x141));
  v = fmax(v, dpp(v, 0xB1));
  return fmax(v, dpp(v, 0x4E));
}

// numpy's pairwise sum of the squares of D BFP values (hm, he) by one wave
// alone, when numpy's splits give nl <= 8 equal leaves of L <= 128 elements
// with L % 8 == 0 (every D % 64 == 0 up to 1024: 576 = 8 x 72): lane 8f + j
// runs accumulator r_j of leaf f (elements fL + j, fL + j + 8, ... in
// order); the leaf's ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) comes from quad
// swaps i ^ 1, i ^ 2 and the 8-lane half-mirror (after the swaps a quad's
// lanes hold one value, so the mirror partner is the other quad), the
// leaves' ((L0+L1)+(L2+L3))+... from the 16-lane mirror and the 16- and
// 32-lane swaps.  Every lane returns 0.0 + the sum (numpy's initial 0.0).
__device__ __forceinline__ double dpp_f64(double x, int ctrl) {
  const long long b = __double_as_longlong(x);
  int lo = (int)(b & 0xffffffffLL), hi = (int)(b >> 32);
  switch (ctrl) {
    case 0xB1:
      lo = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xf, 0xf, false);
      hi = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xf, 0xf, false);
      break;
    case 0x4E:
      lo = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xf, 0xf, false);
      hi = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xf, 0xf, false);
      break;
    case 0x141:
      lo = __builtin_amdgcn_mov_dpp(lo, 0x141, 0xf, 0xf, false);
      hi = __builtin_amdgcn_mov_dpp(hi, 0x141, 0xf, 0xf, false);
      break;
    default:   // 0x140 row_mirror
      lo = __builtin_amdgcn_mov_dpp(lo, 0x140, 0xf, 0xf, false);
      hi = __builtin_amdgcn_mov_dpp(hi, 0x140, 0xf, 0xf, false);
      break;
  }
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
// Accumulator r_j of this lane's leaf over K = L / 8 elements known at
// compile time: every load is issued before the first add (with L known
// only at run time, each element was its own guarded block, one LDS round
// trip after another).
template <int K>
__device__ __forceinline__ double sum_sq_acc(const int16_t *hm, const int8_t *he, int base) {
  double x[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = base + 8 * k;
    x[k] = bfp_val(hm[i], he[i >> 4]);
  }
  double r = x[0] * x[0];
#pragma unroll
  for (int k = 1; k < K; ++k) r = r + x[k] * x[k];
  return r;
}
__device__ __forceinline__ double sum_sq_wave(const int16_t *hm, const int8_t *he, int nl, int L) {
  const int lane = threadIdx.x & 63;
  const int f = lane >> 3, j = lane & 7;
  const int base = (f < nl ? f : 0) * L + j;
  double r = 0.0;
  if (L == 72) {   // uniform: D = 576 (8 leaves of 72)
    r = sum_sq_acc<9>(hm, he, base);
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (8 * k < L) {
        const int i = base + 8 * k;
        const double x = bfp_val(hm[i], he[i >> 4]);
        r = k == 0 ? x * x : r + x * x;
      }
    }
  }
  r = r + dpp_f64(r, 0xB1);
  r = r + dpp_f64(r, 0x4E);
  r = r + dpp_f64(r, 0x141);
  if (nl >= 2) r = r + dpp_f64(r, 0x140);
  if (nl >= 4) r = r + peer<16>(r);
  if (nl >= 8) r = r + peer<32>(r);
  const long long b = __double_as_longlong(r);
  const int lo32 = __builtin_amdgcn_readlane((int)(b & 0xffffffffLL), 0);
  const int hi32 = __builtin_amdgcn_readlane((int)(b >> 32), 0);
  return 0.0 + __longlong_as_double((long long)(((unsigned long long)(unsigned)hi32 << 32) | (unsigned)lo32));
}
// The leaves of numpy's pairwise sum over n elements when they are nl <= 8
// equal leaves of L elements, L % 8 == 0 (sum_sq_wave's form); false if not.
__host__ __device__ inline bool pw_equal_leaves(int n, int &nl, int &L) {
  nl = 1;
  L = n;
  while (L > 128) {
    int n2 = L / 2;
    n2 -= n2 % 8;
    if (2 * n2 != L) return false;
    L = n2;
    nl *= 2;
  }
  return nl <= 8 && L % 8 == 0 && L >= 8;
}

// numpy's add-reduce of a[0..n) (1 <= n <= 256, in LDS) by one wave, every
// lane returning 0.0 + the sum.  Up to 128 elements are one leaf; above, the
// range splits at n2 = n/2 rounded down to a multiple of 8 and a right part
// longer than 128 splits once more, so there are at most three leaves (each
// of at least 64 elements).  Lane group k = l / 8 sums leaf k: accumulator
// j = l % 8 over elements j, j + 8, ... below the leaf's last multiple of
// 8, the ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) tree from the quad swaps and
// the 8-lane half-mirror (sum_sq_wave's), then the leftover elements in
// order; a leaf of fewer than 8 (n < 8) is 0.0 plus its elements in order.
// The leaves combine as numpy nests them: L0, L0 + L1 or L0 + (L1 + L2).
__device__ __forceinline__ double pairwise_sum_wave256(const double *a, int n) {
  const int l = threadIdx.x & 63, k = l >> 3, j = l & 7;
  int n2 = n, nr = 0, m2 = 0;   // leaves [0, n2), [n2, n2 + m2), [n2 + m2, n)
  if (n > 128) {
    n2 = n / 2;
    n2 -= n2 % 8;
    nr = n - n2;
    m2 = nr;
    if (nr > 128) {
      m2 = nr / 2;
      m2 -= m2 % 8;
    }
  }
  const int flo = k == 0 ? 0 : (k == 1 ? n2 : n2 + m2);
  const int fn = k == 0 ? n2 : (k == 1 ? m2 : (k == 2 ? nr - m2 : 0));
  const int top = fn - fn % 8;
  double r = j < top ? a[flo + j] : 0.0;
  for (int t = flo + 8 + j; t < flo + top; t += 8) r = r + a[t];
  r = r + dpp_f64(r, 0xB1);
  r = r + dpp_f64(r, 0x4E);
  r = r + dpp_f64(r, 0x141);
  double res = r;
  if (fn < 8) {
    res = 0.0;
    for (int t = 0; t < fn; ++t) res += a[flo + t];
  } else {
    for (int t = flo + top; t < flo + fn; ++t) res += a[t];
  }
  auto lane_val = [&](int src) {
    const long long b = __double_as_longlong(res);
    const int lo32 = __builtin_amdgcn_readlane((int)(b & 0xffffffffLL), src);
    const int hi32 = __builtin_amdgcn_readlane((int)(b >> 32), src);
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi32 << 32) | (unsigned)lo32));
  };
  double root = lane_val(0);
  if (n > 128) root = nr > 128 ? root + (lane_val(8) + lane_val(16)) : root + lane_val(8);
  return 0.0 + root;
}

// tile_quantize of the 16 values held two per lane by an 8-lane group
// (elements 2j and 2j+1 in lane j of the group): the tile exponent in e and
// this lane's two mantissas, canonical when `canonical` (the same values as
// quantize16_lanes over the same 16 values).  All 64 lanes participate.
__device__ __forceinline__ void quantize16_pairs(double y0, double y1, int &m0, int &m1, int &e,
                                                 bool canonical) {
  const double a = group8_max(fmax(fabs(y0), fabs(y1)));
  e = tile_exp_of(a);
  m0 = tile_mant_of(y0, e);
  m1 = tile_mant_of(y1, e);
  if (canonical) {
    const int hit = group8_u32((m0 == -32768 || m1 == -32768) ? 1 : 0, [](int x, int y) { return x | y; });
    if (hit && e < 127) {
      e += 1;
      int q = m0 >> 1;
      m0 = (m0 & 1) ? q + (q & 1) : q;
      q = m1 >> 1;
      m1 = (m1 & 1) ? q + (q & 1) : q;
    }
  }
}

// RoPE of one 64-wide head held one value per lane of a wave (lane l holds
// element l, pre-rotation x), re-quantised: returns the lane's mantissa.
// (c, s): the lane's (cos, sin) of pair j = lane % 32.
__device__ __forceinline__ int rope_lane(double x, double c, double s, int &e) {
  const int l = threadIdx.x & 63;
  double other = peer<32>(x);              // the partner element j+32 / j
  double out;
  if (l < 32) {
    out = x * c - other * s;                 // a*c - b*s
  } else {
    out = x * c + other * s;                 // b*c + a*s
  }
  return quantize16_lanes(out, e);
}
__device__ __forceinline__ int rope_lane(double x, const double *cs, int &e) {
  const int j = threadIdx.x & 31;
  return rope_lane(x, cs[2 * j], cs[2 * j + 1], e);
}

}  // namespace bfp
