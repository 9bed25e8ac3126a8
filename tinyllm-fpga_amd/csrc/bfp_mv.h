// The exact-integer BFP matvec engine for one 16-row output chunk, shared by
// the standalone matvec and the fused layer kernels.
//
// Semantics: rtl/vc707/host/gen_smollm_blockfp_full.py:217-233.  Per row o
// and input tile t: S = sum_k x_m[t,k] W_m[o,t,k] (exact), E = x_e[t] +
// W_e[o,t]; M = max_t E; A = sum_t floor(S / 2^(M-E)) for M-E <= 47, clipped
// to +-2^47; y_o = A * 2^(M-30), re-quantised over the 16 rows of the chunk.
//
// Work split inside a workgroup of NW waves: lane (w, lane) takes row
// r = lane % 16 and tile lane tq = lane / 16, and owns tiles
// t = tq + 4*(w + NW*j), j < TPT, so each 16-byte-per-lane load of a wave
// covers four full 256-byte half-tile planes of the device layout.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bfp_device.h"

namespace bfp {

template <int TPT>
struct ChunkRegs {
  uint4 a[TPT], b[TPT];
  int e[TPT];
};

// NT: mantissas with the non-temporal cache policy.  Measured on the
// one-chunk-per-workgroup matvec it lifts the weight stream 3-10%; the
// streaming form and the latency-bound decode kernels read faster with
// ordinary loads.
template <int NW, int TPT, bool NT = false>
__device__ __forceinline__ void load_chunk(ChunkRegs<TPT> &R, const uint4 *__restrict__ pm,
                                           const int8_t *__restrict__ pe, int nT) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, tq = lane >> 4;
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    int t = tq + 4 * (w + NW * j);
    if (t < nT) {
      R.a[j] = NT ? ld_nt(pm + t * 32 + r) : pm[t * 32 + r];
      R.b[j] = NT ? ld_nt(pm + t * 32 + 16 + r) : pm[t * 32 + 16 + r];
      R.e[j] = pe[t * 16 + r];
    } else {
      R.a[j] = make_uint4(0, 0, 0, 0);
      R.b[j] = make_uint4(0, 0, 0, 0);
      R.e[j] = 0;
    }
  }
}

// Same through buffer instructions with the nt cache policy (bit 1 of the
// policy operand): every load is unconditional, tiles past nT fall outside
// the buffer's range and read 0.  On the 1536-input chunk (eight waves) this
// streamed 6.95 TB/s against 6.62 for load_chunk; on 576-input chunks
// (three waves) it was slower (6.41 against 6.83).
template <int NW, int TPT>
__device__ __forceinline__ void load_chunk_buf(ChunkRegs<TPT> &R, const uint4 *pm, const int8_t *pe,
                                               int nT) {
  constexpr int POL = 2;
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  const __amdgpu_buffer_rsrc_t rm =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4 *>(pm), (short)0, nT * 512, 0x00020000);
  const __amdgpu_buffer_rsrc_t re =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(pe), (short)0, nT * 16, 0x00020000);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, tq = lane >> 4;
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const int t = tq + 4 * (w + NW * j);
    const v4u a = __builtin_amdgcn_raw_buffer_load_b128(rm, (t * 32 + r) * 16, 0, POL);
    const v4u b = __builtin_amdgcn_raw_buffer_load_b128(rm, (t * 32 + 16 + r) * 16, 0, POL);
    R.a[j] = make_uint4(a.x, a.y, a.z, a.w);
    R.b[j] = make_uint4(b.x, b.y, b.z, b.w);
    R.e[j] = (int)(signed char)__builtin_amdgcn_raw_buffer_load_b8(re, t * 16 + r, 0, POL);
  }
}

// Same, with every load unconditional (tiles past nT re-read tile nT-1; the
// engine ignores those lanes), so the loads of several chunks can be kept in
// flight without the compiler draining them at a branch.
template <int NW, int TPT>
__device__ __forceinline__ void load_chunk_nb(ChunkRegs<TPT> &R, const uint4 *__restrict__ pm,
                                              const int8_t *__restrict__ pe, int nT) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, tq = lane >> 4;
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    int t = tq + 4 * (w + NW * j);
    t = t < nT ? t : nT - 1;
    R.a[j] = pm[t * 32 + r];
    R.b[j] = pm[t * 32 + 16 + r];
    R.e[j] = pe[t * 16 + r];
  }
}

// LDS form of the input vector: per tile 8 dwords of packed (xh, xh) int16
// pairs then 8 dwords of (xl, xl) pairs, with x = 256*xh + xl.
__device__ __forceinline__ void put_x_pair(int *xs, int t, int k, int lo, int hi) {
  xs[t * 16 + k] = ((lo >> 8) & 0xffff) | ((hi >> 8) << 16);
  xs[t * 16 + 8 + k] = (lo & 0xff) | ((hi & 0xff) << 16);
}

// Stage a BFP vector of nT tiles from global memory (all threads; caller
// syncs).  Each thread issues its loads (addresses clamped in range) before
// its first LDS store, so the staging costs one memory round trip when
// nT*8 <= 4*blockDim.
__device__ __forceinline__ void stage_x_bfp(int *xs, int *xes, const int16_t *__restrict__ xm,
                                            const int8_t *__restrict__ xe, int nT) {
  const int *x32 = reinterpret_cast<const int *>(xm);
  const int n = nT * 8, bs = blockDim.x, tid = threadIdx.x;
  const int ex = xe[tid < nT ? tid : 0];
  for (int p0 = tid; p0 < n; p0 += 4 * bs) {
    int v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int p = p0 + k * bs;
      v[k] = x32[p < n ? p : n - 1];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int p = p0 + k * bs;
      if (p < n) put_x_pair(xs, p >> 3, p & 7, (int)(short)(v[k] & 0xffff), v[k] >> 16);
    }
  }
  if (tid < nT) xes[tid] = ex;
  for (int p = tid + bs; p < nT; p += bs) xes[p] = xe[p];
}

// Row (A, M) of the chunk.  Every thread of the workgroup must call it (it
// synchronises when NW > 1).  On return the lanes of wave 0 hold their row
// r's (A, M); other waves hold partial values.
template <int NW, int TPT>
__device__ __forceinline__ void chunk_AM(const ChunkRegs<TPT> &R, const int *xs, const int *xes,
                                         int nT, int *redM, long long *redA, long long &A_out,
                                         int &M_out) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, tq = lane >> 4;
  typedef short s2 __attribute__((ext_vector_type(2)));
#define BFP_DOT2(a, b, acc) \
  __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, (a)), __builtin_bit_cast(s2, (b)), (acc), false)
  long long S[TPT];
  int E[TPT];
  int M = -(1 << 29);
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    int t = tq + 4 * (w + NW * j);
    if (t < nT) {
      const int4 *xp = reinterpret_cast<const int4 *>(xs + t * 16);
      int4 h0 = xp[0], h1 = xp[1], l0 = xp[2], l1 = xp[3];
      int ah = 0, al = 0;
      ah = BFP_DOT2(R.a[j].x, h0.x, ah);
      al = BFP_DOT2(R.a[j].x, l0.x, al);
      ah = BFP_DOT2(R.a[j].y, h0.y, ah);
      al = BFP_DOT2(R.a[j].y, l0.y, al);
      ah = BFP_DOT2(R.a[j].z, h0.z, ah);
      al = BFP_DOT2(R.a[j].z, l0.z, al);
      ah = BFP_DOT2(R.a[j].w, h0.w, ah);
      al = BFP_DOT2(R.a[j].w, l0.w, al);
      ah = BFP_DOT2(R.b[j].x, h1.x, ah);
      al = BFP_DOT2(R.b[j].x, l1.x, al);
      ah = BFP_DOT2(R.b[j].y, h1.y, ah);
      al = BFP_DOT2(R.b[j].y, l1.y, al);
      ah = BFP_DOT2(R.b[j].z, h1.z, ah);
      al = BFP_DOT2(R.b[j].z, l1.z, al);
      ah = BFP_DOT2(R.b[j].w, h1.w, ah);
      al = BFP_DOT2(R.b[j].w, l1.w, al);
      S[j] = (long long)ah * 256 + al;
      E[j] = xes[t] + R.e[j];
      M = E[j] > M ? E[j] : M;
    } else {
      S[j] = 0;
      E[j] = -(1 << 29);
    }
  }
#undef BFP_DOT2
  M = pmax<16>(M);
  M = pmax<32>(M);
  if (NW > 1) {
    if (tq == 0) redM[w * 16 + r] = M;
    lds_barrier();
    M = redM[r];
#pragma unroll
    for (int i = 1; i < NW; ++i) M = redM[i * 16 + r] > M ? redM[i * 16 + r] : M;
  }
  long long A = 0;
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    int sh = M - E[j];
    if (sh <= ALIGN_MAX) A += S[j] >> sh;
  }
  A = psum<16>(A);
  A = psum<32>(A);
  if (NW > 1) {
    if (tq == 0) redA[w * 16 + r] = A;
    lds_barrier();
    if (w == 0) {
      A = redA[r];
#pragma unroll
      for (int i = 1; i < NW; ++i) A += redA[i * 16 + r];
    }
    lds_barrier();   // redM/redA may be reused by a following chunk
  }
  A = A < SAT_LO ? SAT_LO : (A > SAT_HI ? SAT_HI : A);
  A_out = A;
  M_out = M;
}

// chunk_AM of two chunks (R1, R2) over the same input vector in one pass:
// the x reads and the cross-wave reductions (and their barriers) are shared.
// Same results as two chunk_AM calls.
template <int NW, int TPT>
__device__ __forceinline__ void chunk_AM2(const ChunkRegs<TPT> &R1, const ChunkRegs<TPT> &R2,
                                          const int *xs, const int *xes, int nT, int *redM,
                                          long long *redA, long long &A1, int &M1, long long &A2,
                                          int &M2) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, tq = lane >> 4;
  typedef short s2 __attribute__((ext_vector_type(2)));
#define BFP_DOT2(a, b, acc) \
  __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, (a)), __builtin_bit_cast(s2, (b)), (acc), false)
  long long S1[TPT], S2[TPT];
  int E1[TPT], E2[TPT];
  int m1 = -(1 << 29), m2 = -(1 << 29);
  auto dot = [&](const uint4 &a, const uint4 &b, const int4 &h0, const int4 &h1, const int4 &l0,
                 const int4 &l1) {
    int ah = 0, al = 0;
    ah = BFP_DOT2(a.x, h0.x, ah);
    al = BFP_DOT2(a.x, l0.x, al);
    ah = BFP_DOT2(a.y, h0.y, ah);
    al = BFP_DOT2(a.y, l0.y, al);
    ah = BFP_DOT2(a.z, h0.z, ah);
    al = BFP_DOT2(a.z, l0.z, al);
    ah = BFP_DOT2(a.w, h0.w, ah);
    al = BFP_DOT2(a.w, l0.w, al);
    ah = BFP_DOT2(b.x, h1.x, ah);
    al = BFP_DOT2(b.x, l1.x, al);
    ah = BFP_DOT2(b.y, h1.y, ah);
    al = BFP_DOT2(b.y, l1.y, al);
    ah = BFP_DOT2(b.z, h1.z, ah);
    al = BFP_DOT2(b.z, l1.z, al);
    ah = BFP_DOT2(b.w, h1.w, ah);
    al = BFP_DOT2(b.w, l1.w, al);
    return (long long)ah * 256 + al;
  };
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const int t = tq + 4 * (w + NW * j);
    if (t < nT) {
      const int4 *xp = reinterpret_cast<const int4 *>(xs + t * 16);
      const int4 h0 = xp[0], h1 = xp[1], l0 = xp[2], l1 = xp[3];
      S1[j] = dot(R1.a[j], R1.b[j], h0, h1, l0, l1);
      S2[j] = dot(R2.a[j], R2.b[j], h0, h1, l0, l1);
      E1[j] = xes[t] + R1.e[j];
      E2[j] = xes[t] + R2.e[j];
      m1 = E1[j] > m1 ? E1[j] : m1;
      m2 = E2[j] > m2 ? E2[j] : m2;
    } else {
      S1[j] = S2[j] = 0;
      E1[j] = E2[j] = -(1 << 29);
    }
  }
#undef BFP_DOT2
  m1 = pmax<16>(m1);
  m1 = pmax<32>(m1);
  m2 = pmax<16>(m2);
  m2 = pmax<32>(m2);
  if (NW > 1) {
    if (tq == 0) {
      redM[w * 16 + r] = m1;
      redM[(NW + w) * 16 + r] = m2;
    }
    lds_barrier();
    m1 = redM[r];
    m2 = redM[NW * 16 + r];
#pragma unroll
    for (int i = 1; i < NW; ++i) {
      m1 = redM[i * 16 + r] > m1 ? redM[i * 16 + r] : m1;
      m2 = redM[(NW + i) * 16 + r] > m2 ? redM[(NW + i) * 16 + r] : m2;
    }
  }
  long long a1 = 0, a2 = 0;
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const int sh1 = m1 - E1[j], sh2 = m2 - E2[j];
    if (sh1 <= ALIGN_MAX) a1 += S1[j] >> sh1;
    if (sh2 <= ALIGN_MAX) a2 += S2[j] >> sh2;
  }
  a1 = psum<16>(a1);
  a1 = psum<32>(a1);
  a2 = psum<16>(a2);
  a2 = psum<32>(a2);
  if (NW > 1) {
    if (tq == 0) {
      redA[w * 16 + r] = a1;
      redA[(NW + w) * 16 + r] = a2;
    }
    lds_barrier();
    if (w == 0) {
      a1 = redA[r];
      a2 = redA[NW * 16 + r];
#pragma unroll
      for (int i = 1; i < NW; ++i) {
        a1 += redA[i * 16 + r];
        a2 += redA[(NW + i) * 16 + r];
      }
    }
    lds_barrier();   // redM/redA may be reused by a following chunk
  }
  A1 = a1 < SAT_LO ? SAT_LO : (a1 > SAT_HI ? SAT_HI : a1);
  A2 = a2 < SAT_LO ? SAT_LO : (a2 > SAT_HI ? SAT_HI : a2);
  M1 = m1;
  M2 = m2;
}

// chunk_AM for up to S sequences at once: x of sequence s in LDS at
// xs + s*nT*16 / xes + s*nT (ns <= S valid).  One pass over the weight
// registers forms every sequence's tile sums, so the chunk's weights are
// read once for the group.  Every thread must call it.  On return (after a
// barrier) Ao[r*S + s], Mo[r*S + s] (LDS) hold row r's (A, M) for sequence s.
template <int NW, int TPT, int S>
__device__ __forceinline__ void chunk_AM_multi(const ChunkRegs<TPT> &R, const int *xs,
                                               const int *xes, int nT, int ns, int *redM,
                                               long long *redA, long long *Ao, int *Mo) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, tq = lane >> 4;
  typedef short s2 __attribute__((ext_vector_type(2)));
#define BFP_DOT2(a, b, acc) \
  __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, (a)), __builtin_bit_cast(s2, (b)), (acc), false)
  long long Sv[TPT][S];
  int E[TPT][S];
  int M[S];
#pragma unroll
  for (int s = 0; s < S; ++s) M[s] = -(1 << 29);
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const int t = tq + 4 * (w + NW * j);
    const bool ok = t < nT;
    const int tc = ok ? t : 0;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      Sv[j][s] = 0;
      E[j][s] = -(1 << 29);
      if (s < ns) {
        const int4 *xp = reinterpret_cast<const int4 *>(xs + (s * nT + tc) * 16);
        int4 h0 = xp[0], h1 = xp[1], l0 = xp[2], l1 = xp[3];
        int ah = 0, al = 0;
        ah = BFP_DOT2(R.a[j].x, h0.x, ah);
        al = BFP_DOT2(R.a[j].x, l0.x, al);
        ah = BFP_DOT2(R.a[j].y, h0.y, ah);
        al = BFP_DOT2(R.a[j].y, l0.y, al);
        ah = BFP_DOT2(R.a[j].z, h0.z, ah);
        al = BFP_DOT2(R.a[j].z, l0.z, al);
        ah = BFP_DOT2(R.a[j].w, h0.w, ah);
        al = BFP_DOT2(R.a[j].w, l0.w, al);
        ah = BFP_DOT2(R.b[j].x, h1.x, ah);
        al = BFP_DOT2(R.b[j].x, l1.x, al);
        ah = BFP_DOT2(R.b[j].y, h1.y, ah);
        al = BFP_DOT2(R.b[j].y, l1.y, al);
        ah = BFP_DOT2(R.b[j].z, h1.z, ah);
        al = BFP_DOT2(R.b[j].z, l1.z, al);
        ah = BFP_DOT2(R.b[j].w, h1.w, ah);
        al = BFP_DOT2(R.b[j].w, l1.w, al);
        if (ok) {
          Sv[j][s] = (long long)ah * 256 + al;
          E[j][s] = xes[s * nT + tc] + R.e[j];
        }
        M[s] = E[j][s] > M[s] ? E[j][s] : M[s];
      }
    }
  }
#undef BFP_DOT2
#pragma unroll
  for (int s = 0; s < S; ++s) {
    M[s] = pmax<16>(M[s]);
    M[s] = pmax<32>(M[s]);
  }
  if (NW > 1) {
    if (tq == 0)
#pragma unroll
      for (int s = 0; s < S; ++s) redM[(w * 16 + r) * S + s] = M[s];
    lds_barrier();
#pragma unroll
    for (int s = 0; s < S; ++s) {
      int m = redM[r * S + s];
#pragma unroll
      for (int i = 1; i < NW; ++i) m = redM[(i * 16 + r) * S + s] > m ? redM[(i * 16 + r) * S + s] : m;
      M[s] = m;
    }
  }
  long long A[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    long long acc = 0;
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int sh = M[s] - E[j][s];
      if (sh <= ALIGN_MAX) acc += Sv[j][s] >> sh;
    }
    acc = psum<16>(acc);
    acc = psum<32>(acc);
    A[s] = acc;
  }
  if (NW > 1) {
    if (tq == 0)
#pragma unroll
      for (int s = 0; s < S; ++s) redA[(w * 16 + r) * S + s] = A[s];
    lds_barrier();
    if (w == 0)
#pragma unroll
      for (int s = 0; s < S; ++s) {
        long long acc = redA[r * S + s];
#pragma unroll
        for (int i = 1; i < NW; ++i) acc += redA[(i * 16 + r) * S + s];
        A[s] = acc;
      }
  }
  if (w == 0 && tq == 0)
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const long long a = A[s] < SAT_LO ? SAT_LO : (A[s] > SAT_HI ? SAT_HI : A[s]);
      Ao[r * S + s] = a;
      Mo[r * S + s] = M[s];
    }
  lds_barrier();
}

// Quantise the chunk's 16 rows (wave 0; lanes r and r+16k hold row r): the
// raw tile_quantize of the exact outputs, as fp_quantize_vec forms it.
__device__ __forceinline__ void chunk_quant(long long A, int M, int &m, int &e) {
  int key = row_exp_key(A, M);
  key = pmax<1>(key);
  key = pmax<2>(key);
  key = pmax<4>(key);
  key = pmax<8>(key);
  e = chunk_exp_from_key(key);
  m = rne_shr_clip(A, e + 15 - M);
}

}  // namespace bfp
