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

// numpy's leaves combined in its order; the leaf starting at element lo is
// leaf[lo / 64] (see pairwise_sum_block).
template <int DEPTH>
__device__ __forceinline__ double pw_combine_blocks(int lo, int n, const double *leaf) {
  if constexpr (DEPTH > 0) {
    if (n > 128) {
      int n2 = n / 2;
      n2 -= n2 % 8;
      return pw_combine_blocks<DEPTH - 1>(lo, n2, leaf) +
             pw_combine_blocks<DEPTH - 1>(lo + n2, n - n2, leaf);
    }
  }
  return leaf[lo >> 6];
}

// Sum of get(0) .. get(n-1) (1 <= n <= 4096) in numpy order, plus numpy's
// initial 0.0; get(i) is called for the elements of this lane's leaf (and
// for index 0 by lanes that own none), so it may read global memory.
// Called by all threads of a workgroup (uses lds_barrier);
// leafbuf holds PW_MAX_LEAVES doubles of LDS.  Returns the sum in every
// thread.
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
  double s = 0.0 + pw_combine_blocks<PW_DEPTH>(0, n, leafbuf);
  lds_barrier();
  return s;
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

// RoPE of one 64-wide head held one value per lane of a wave (lane l holds
// element l, pre-rotation x), re-quantised: returns the lane's mantissa.
__device__ __forceinline__ int rope_lane(double x, const double *cs, int &e) {
  const int l = threadIdx.x & 63;
  const int j = l & 31;
  double other = peer<32>(x);              // the partner element j+32 / j
  double c = cs[2 * j], s = cs[2 * j + 1];
  double out;
  if (l < 32) {
    out = x * c - other * s;                 // a*c - b*s
  } else {
    out = x * c + other * s;                 // b*c + a*s
  }
  return quantize16_lanes(out, e);
}

}  // namespace bfp
