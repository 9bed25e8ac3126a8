// Exact BFP tile sums of many sequences on the matrix cores (int8 MFMA).
//
// Semantics are the engine's (rtl/vc707/host/gen_smollm_blockfp_full.py
// :217-233): per row o, sequence s and input tile t the exact
// S = sum_k W_m[o,t,k] x_m[s,t,k], E = W_e[o,t] + x_e[s,t], M = max_t E,
// A = sum_t floor(S / 2^(M-E)) for M-E <= 47.
//
// Both int16 operands are split into a signed high byte and an offset low
// byte: v = 256*vh + vl' + 128 with vh = v >> 8 and vl' = (v & 255) - 128,
// both in [-128, 127].  Over one 16-element tile
//   S = 65536*Phh + 256*(Phl + Plh + 128*sum Wh) + (Pll + 128*sum Wl')
//       + 128*sum x
// where Pab = sum_k Wa*xb.  Every product sum is one v_mfma_i32_16x16x32_i8
// whose 32-deep k axis holds the tile twice (k-groups 0-1 and 2-3 of the
// operand layout): Phh and Pll with the second copy of A zeroed, the cross
// term as Wh.xl' over the first copy plus Wl'.xh over the second, and the
// weight sums against a constant 64 operand over both copies (= 128 sum).
// 128 sum x (one value per sequence, from the vector unit) is the initial
// accumulator of the low-byte product sum.  |Phh| <= 2^18
// and the rest fits in 29 bits, so S is formed exactly in 64 bits.  E =
// W_e + x_e of the lane's four output rows comes from one LDS word (the four
// rows' weight exponents, tile-major) and one byte, so every per-output
// quantity is in the lane that owns the output: no lane exchange is needed.
// (E through one more MFMA per tile and chunk, A = [W_e, 1], B = [1, x_e],
// made the max-exponent pass a chain of dependent LDS reads and MFMAs: 1.9
// against 1.0 us for the 576 x 3072 G/U block of 16 sequences.)
//
// A block is NC adjacent 16-row chunks of the device layout by 16
// sequences.  Lane l supplies row / sequence l % 16 and k-group l / 16
// (the tile's 8-element half (l/16) & 1), and owns outputs
// (row 4*(l/16) + v, sequence l % 16), v < 4, of every chunk.  The waves of
// a workgroup split the input tiles; M is reduced with LDS max and A with
// LDS 64-bit adds.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "bfp_device.h"

namespace bfp {

typedef int mx_v4 __attribute__((ext_vector_type(4)));

constexpr int MX_SEQ = 16;    // sequences per block
constexpr int MX_WAVES_MAX = 8;

// High bytes and offset low bytes of the 8 int16 in w (little-endian pairs).
__device__ __forceinline__ void mx_split(const uint4 w, long &hi, long &lo) {
  const unsigned h0 = __builtin_amdgcn_perm(w.y, w.x, 0x07050301u);
  const unsigned h1 = __builtin_amdgcn_perm(w.w, w.z, 0x07050301u);
  const unsigned l0 = __builtin_amdgcn_perm(w.y, w.x, 0x06040200u) ^ 0x80808080u;
  const unsigned l1 = __builtin_amdgcn_perm(w.w, w.z, 0x06040200u) ^ 0x80808080u;
  hi = (long)(((unsigned long)h1 << 32) | h0);
  lo = (long)(((unsigned long)l1 << 32) | l0);
}

__device__ __forceinline__ int mx_sum8(const uint4 w) {
  return (int)(short)(w.x & 0xffffu) + ((int)w.x >> 16) + (int)(short)(w.y & 0xffffu) +
         ((int)w.y >> 16) + (int)(short)(w.z & 0xffffu) + ((int)w.z >> 16) +
         (int)(short)(w.w & 0xffffu) + ((int)w.w >> 16);
}

__device__ __forceinline__ mx_v4 mx_mfma(long a, long b, mx_v4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

// The select-free form of one tile's sums (the pipelined batched step,
// bfp_pipe.hip, whose weights are split once per layer).  Every operand carries the tile
// in both k copies, so each 32-deep product is twice the tile's; only the
// per-lane constant k1 (ones in the first copy, zeros in the second) counts
// once.  With P the 32-deep sum and sum x = 256 sum xh + sum xl' + 2048,
//   2 S = 65536 (P(Wh, xh) + P(Wh, k1) + P(k1, xh) + 8)
//         + 256 (P(Wh, xl') + P(Wl', xh) + P(Wl', k1) + P(k1, xl'))
//         + P(Wl', xl')
// and floor(S / 2^d) = floor(2S / 2^(d+1)).  |hh| < 2^20 and the low part
// lo = 256 cr + ll fits 31 bits (tests/test_mx_split.py).  The two input
// sums P(k1, xh) + 8, P(k1, xl') are one pair per tile (mx_xsum), the
// initial accumulators of every chunk's hh and cr (8 is an inline operand
// of the product; 2^19 as the low sum's start would be a register copy per
// tile).
__device__ __forceinline__ long mx_k1() { return (threadIdx.x & 63) < 32 ? 0x0101010101010101L : 0L; }
__device__ __forceinline__ void mx_xsum(long xh, long xl, long k1, mx_v4 &sh, mx_v4 &sl) {
  const mx_v4 zero = {0, 0, 0, 0}, c8 = {8, 8, 8, 8};
  sh = mx_mfma(k1, xh, c8);
  sl = mx_mfma(k1, xl, zero);
}
__device__ __forceinline__ void mx_tile2(long wh, long wl, long xh, long xl, long k1, const mx_v4 &sh,
                                         const mx_v4 &sl, mx_v4 &hh, mx_v4 &lo) {
  const mx_v4 zero = {0, 0, 0, 0};
  hh = mx_mfma(wh, xh, sh);
  mx_v4 cr = mx_mfma(wh, xl, sl);
  const mx_v4 ll = mx_mfma(wl, xl, zero);
  hh = mx_mfma(wh, k1, hh);
  cr = mx_mfma(wl, xh, cr);
  cr = mx_mfma(wl, k1, cr);
#pragma unroll
  for (int v = 0; v < 4; ++v) lo[v] = (cr[v] << 8) + ll[v];
}
// floor(S / 2^d) of a tile from (hh, lo) of mx_tile2 with q = d + 1; WIN:
// 0 past the engine's 47-bit window (d > ALIGN_MAX), without a branch (a
// wave whose every (tile, output) lies inside the window skips the test).
template <bool WIN>
__device__ __forceinline__ long long mx_align2(int hh, int lo, int q) {
  const long long s2 = ((long long)hh << 16) + lo;
  if constexpr (!WIN) return s2 >> q;
  const long long t = s2 >> (q & 63);
  return q <= ALIGN_MAX + 1 ? t : 0;
}

// (The per-stage launches keep the form above with the second copy zeroed:
// there the blocks are bound by the matrix cores, and the select-free form's
// eight products a tile instead of five made G/U 5.5 -> 6.7 us and D
// 4.0 -> 5.3 us of tile sums at batch 64.)

// Phase stamps of a traced batched decode (100 MHz clock, thread 0 of each
// block): MX_TRACE_STAMPS per block -- 0 entry, 1 exponents staged, 2 M
// reduced, 3 tile sums formed, 4 A reduced, 5 epilogue done (stamped by the
// kernel) -- for at most MX_TRACE_BLOCKS blocks of each of the MX_TRACE_KERNELS
// matvec kernels (MX_K_*), the last launch of each kind overwriting the one
// before.
constexpr int MX_TRACE_STAMPS = 6, MX_TRACE_BLOCKS = 1024, MX_TRACE_KERNELS = 4;
constexpr int MX_K_QKV = 0, MX_K_O = 1, MX_K_GU = 2, MX_K_D = 3;
__device__ __forceinline__ void mx_mark(unsigned long long *tr, int k) {
  const unsigned b = blockIdx.x + blockIdx.y * gridDim.x;
  if (tr && threadIdx.x == 0 && b < (unsigned)MX_TRACE_BLOCKS)
    tr[b * MX_TRACE_STAMPS + k] = __builtin_amdgcn_s_memrealtime();
}

// LDS bytes mx_block<NC> needs beyond its caller's Ao / Mo: the block's
// weight and input exponents, tile-major.
__host__ __device__ constexpr int mx_lds_bytes(int nc, int nT) { return (nc + 1) * 16 * nT; }

// (A, M) of the (row, sequence) pairs of a block: the NC adjacent 16-row
// chunks at pm / pe (device layout, nT tiles each; chunk c is rows
// 16c..16c+15) against sequences s < ns at x_m + s*nT*16, x_e + s*nT.
// Every thread of the workgroup calls it; on return (after a barrier)
// Ao[row*16 + s] and Mo[row*16 + s] (LDS) hold the pair of (row, s).
// ex: mx_lds_bytes(NC, nT) bytes of LDS.
template <int NC>
__device__ __forceinline__ void mx_block(const uint4 *__restrict__ pm, const int8_t *__restrict__ pe, int nT,
                         const int16_t *__restrict__ xm, const int8_t *__restrict__ xe, int ns,
                         long long *Ao, int *Mo, int8_t *ex, unsigned long long *tr = nullptr) {
  mx_mark(tr, 0);
  constexpr int G = 4;           // tiles whose loads are in flight together
  constexpr int RW = NC * 16;    // rows of the block
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int i = lane & 15, kg = lane >> 4, h = kg & 1;
  const bool first = kg < 2;     // first copy of the tile on the k axis
  const int sc = i < ns ? i : ns - 1;
  const uint4 *xr = reinterpret_cast<const uint4 *>(xm);
  const int wo = h * 16 + i, xo = sc * nT * 2 + h;   // + t*32 (+ c*nT*32), + t*2
  int8_t *wex = ex, *xex = ex + RW * nT;             // [t*RW + row], [t*16 + sequence]
  const int tpw = (nT + nw - 1) / nw;
  const int t0 = w * tpw, t1 = t0 + tpw < nT ? t0 + tpw : nT;
  // operand registers of G tiles, loaded together (the last valid tile
  // stands in for those past t1: in range, never used).  Issuing the first
  // group's loads with the exponent loads measured slower for every kernel
  // (G/U 14.4 -> 15.6 us, D 11.0 -> 13.0 at batch 64).
  uint4 xv[G], wv[G][NC];
  auto load_group = [&](int tb) {
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int t = tb + k < t1 ? tb + k : t1 - 1;
      xv[k] = xr[xo + t * 2];
#pragma unroll
      for (int c = 0; c < NC; ++c) wv[k][c] = pm[wo + c * nT * 32 + t * 32];
    }
  };
  // exponents of the whole block into LDS: the weights' as 4-row words, the
  // inputs' as bytes, every load of a thread issued before its stores
  {
    const int nw4 = NC * nT * 4, nx = MX_SEQ * nT, bs = blockDim.x;
    const int *pe4 = reinterpret_cast<const int *>(pe);
    for (int q0 = threadIdx.x; q0 < nw4 + nx; q0 += 4 * bs) {
      int v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int q = q0 + k * bs;
        if (q < nw4) {
          v[k] = pe4[q];
        } else {
          int qx = q - nw4;
          qx = qx < nx ? qx : nx - 1;
          const int t = qx >> 4, ss = qx & 15;
          v[k] = xe[(ss < ns ? ss : ns - 1) * nT + t];
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int q = q0 + k * bs;
        if (q < nw4) {
          // word q: chunk q / (4nT), tile (q / 4) % nT, rows 4*(q%4) .. +3
          const int c = q / (4 * nT), t = (q >> 2) - c * nT;
          *reinterpret_cast<int *>(wex + t * RW + c * 16 + 4 * (q & 3)) = v[k];
        } else if (q < nw4 + nx) {
          xex[q - nw4] = (int8_t)v[k];
        }
      }
    }
  }
  for (int q = threadIdx.x; q < RW * MX_SEQ; q += blockDim.x) {
    Ao[q] = 0;
    Mo[q] = -(1 << 29);
  }
  __syncthreads();
  mx_mark(tr, 1);
  const mx_v4 zero = {0, 0, 0, 0};
  // E = W_e + x_e of chunk c, tile t for this lane's outputs (rows 4 kg + v,
  // sequence i): the four rows' exponents are one 4-byte word of wex
  auto tile_E = [&](int c, int t, int (&E)[4]) {
    const int ww = *reinterpret_cast<const int *>(wex + t * RW + c * 16 + 4 * kg);
    const int xv = xex[t * 16 + i];
#pragma unroll
    for (int v = 0; v < 4; ++v) E[v] = ((ww << (24 - 8 * v)) >> 24) + xv;
  };
  // pass 1: M over all tiles, split across the waves, reduced in LDS
  int M[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int v = 0; v < 4; ++v) M[c][v] = -(1 << 29);
#pragma unroll 4
    for (int t = t0; t < t1; ++t) {
      int E[4];
      tile_E(c, t, E);
#pragma unroll
      for (int v = 0; v < 4; ++v) M[c][v] = E[v] > M[c][v] ? E[v] : M[c][v];
    }
    if (t0 < t1) {
#pragma unroll
      for (int v = 0; v < 4; ++v) atomicMax(&Mo[(c * 16 + 4 * kg + v) * MX_SEQ + i], M[c][v]);
    }
  }
  __syncthreads();
  mx_mark(tr, 2);
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) M[c][v] = Mo[(c * 16 + 4 * kg + v) * MX_SEQ + i];
  // pass 2: aligned tile sums
  long long A[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) A[c][v] = 0;
  const long k64 = 0x4040404040404040L;
  for (int tb = t0; tb < t1; tb += G) {
    load_group(tb);
#pragma unroll
    for (int k = 0; k < G; ++k) {
      if (tb + k >= t1) break;
      long xh, xl;
      mx_split(xv[k], xh, xl);
      int sx = mx_sum8(xv[k]);
      sx += peer<16>(sx);   // the tile's other half (k-group l/16 ^ 1)
      const int cx = 128 * sx;
      // 128 sum x, one value per sequence, starts the low-byte product sum
      const mx_v4 cxv = {cx, cx, cx, cx};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        long wh, wl;
        mx_split(wv[k][c], wh, wl);
        const mx_v4 hh = mx_mfma(first ? wh : 0, xh, zero);
        mx_v4 ll = mx_mfma(first ? wl : 0, xl, cxv);
        mx_v4 cr = mx_mfma(first ? wh : wl, first ? xl : xh, zero);
        cr = mx_mfma(wh, k64, cr);
        ll = mx_mfma(wl, k64, ll);
        int E[4];
        tile_E(c, tb + k, E);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int d = M[c][v] - E[v];
          const int lo = (cr[v] << 8) + ll[v];
          const long long S = ((long long)hh[v] << 16) + lo;
          if (d <= ALIGN_MAX) A[c][v] += S >> d;
        }
      }
    }
  }
  mx_mark(tr, 3);
  if (t0 < t1) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        atomicAdd(reinterpret_cast<unsigned long long *>(&Ao[(c * 16 + 4 * kg + v) * MX_SEQ + i]),
                  (unsigned long long)A[c][v]);
  }
  __syncthreads();
  mx_mark(tr, 4);
}

// A read back for an epilogue, clipped as the engine clips.
__device__ __forceinline__ long long mx_A(const long long *Ao, int q) {
  const long long A = Ao[q];
  return A < SAT_LO ? SAT_LO : (A > SAT_HI ? SAT_HI : A);
}

}  // namespace bfp
