// Device-coherent access helpers shared by the persistent decode kernels
// (bfp_persist.hip: batch 1; bfp_pipe.hip: batches): buffer-resource
// loads and stores with explicit cache policies, scalar reads of argument
// blocks held in device memory, tagged hand-off words and bounded waits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bfp {

constexpr unsigned long long PT_SPIN_TICKS = 200000000ull;   // 2 s at 100 MHz
constexpr int PT_POLL_STAGGER = 12;   // s_sleep units (64 clocks): ~0.3 us between the first two polls

// --------------------------------------------------------- memory access
// The roles are separate functions (their register allocations stay apart),
// so pointers reaching them are generic.  Generic (FLAT) accesses count
// against both the vector-memory and the LDS wait counters: an LDS wait would
// then also wait for a weight prefetch in flight.  So every hot access names
// its memory: LDS through lds(), global data through buffer instructions
// (vector-memory counter only; out-of-range offsets read 0), the argument
// blocks through the constant address space (scalar loads).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
#if defined(__HIP_DEVICE_COMPILE__)
#define PT_CONST __attribute__((address_space(4)))   // constant: scalar loads
#else
#define PT_CONST
#endif
// A copy of *p read through the constant address space.
template <class T>
__device__ __forceinline__ T cload(const PT_CONST T *p) {
  return *(const T *)p;
}
// A role function receives its arguments in vector registers, so the
// compiler treats them as varying across lanes (per-lane loads, and a loop
// around every buffer access whose descriptor derives from them).  They are
// the same in every lane: take lane 0's value into scalar registers.
template <class T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
  const unsigned long long u = (unsigned long long)p;
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
  return (T *)(((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ int uniform_int(int v) { return __builtin_amdgcn_readfirstlane(v); }
constexpr int CPOL_SC1 = 16;   // buffer-instruction cache policy: SC1 (device scope)
// non-temporal (streamed once per step: the head's 113 MB float32 embedding
// read 1645 -> 1675 tokens/s at config 3 with it)
constexpr int CPOL_NT = 2;

template <class T>
__device__ __forceinline__ T *lds(T *p) {
  return (T *)(__attribute__((address_space(3))) T *)p;
}
__device__ __forceinline__ rsrc_t rsrc(const void *base, int bytes = 0x7fffffff) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, 0x00020000);
}
template <int POL>
__device__ __forceinline__ uint4 ld_b128(rsrc_t r, int off) {
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ unsigned ld_coh(rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL_SC1);
}
__device__ __forceinline__ void st_coh(rsrc_t r, int off, unsigned v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, CPOL_SC1);
}

// Tagged activation word.
__device__ __forceinline__ unsigned tagged(int m, int e, unsigned tag) {
  return ((unsigned)m & 0xffffu) | (((unsigned)e & 0xffu) << 16) | (tag << 24);
}
__device__ __forceinline__ int tw_m(unsigned w) { return (int)(short)(w & 0xffffu); }
__device__ __forceinline__ int tw_e(unsigned w) { return (int)(signed char)((w >> 16) & 0xffu); }
__device__ __forceinline__ unsigned tag_of(int s, int l, int NL) {
  return (unsigned)(((long long)s * NL + l) % 255) + 1u;
}

// Bounded waits.  `aborted` is per thread: once set, waits return at once.
struct Wait {
  rsrc_t flag;
  bool aborted;
  __device__ __forceinline__ bool give_up(unsigned it, unsigned long long t0) {
    if ((it & 63u) != 0u) return false;
    if (ld_coh(flag, 0) != 0u || __builtin_amdgcn_s_memrealtime() - t0 > PT_SPIN_TICKS) {
      st_coh(flag, 0, 1u);
      aborted = true;
      return true;
    }
    return false;
  }
  // Spin until the words carry `tag`: after the first miss two polls stay
  // in flight, about half a round trip apart (the sleep staggers the first
  // two; each later poll is issued before the oldest is checked), so a
  // store is seen about half a round trip sooner than with one poll at a
  // time.
  __device__ __forceinline__ unsigned word(rsrc_t r, int off, unsigned tag) {
    unsigned v = ld_coh(r, off);
    if ((v >> 24) == tag || aborted) return v;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    unsigned prev = ld_coh(r, off);
    __builtin_amdgcn_s_sleep(PT_POLL_STAGGER);
    for (unsigned it = 1;; ++it) {
      const unsigned next = ld_coh(r, off);
      if ((prev >> 24) == tag || give_up(it, t0)) return prev;
      prev = next;
    }
  }
  // four consecutive words (16-byte aligned, byte offset off) in one load
  __device__ __forceinline__ static bool ok4(const uint4 &v, unsigned tag) {
    return (v.x >> 24) == tag && (v.y >> 24) == tag && (v.z >> 24) == tag && (v.w >> 24) == tag;
  }
  __device__ __forceinline__ uint4 quad(rsrc_t r, int off, unsigned tag) {
    uint4 v = ld_b128<CPOL_SC1>(r, off);
    if (ok4(v, tag) || aborted) return v;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    uint4 prev = ld_b128<CPOL_SC1>(r, off);
    __builtin_amdgcn_s_sleep(PT_POLL_STAGGER);
    for (unsigned it = 1;; ++it) {
      const uint4 next = ld_b128<CPOL_SC1>(r, off);
      if (ok4(prev, tag) || give_up(it, t0)) return prev;
      prev = next;
    }
  }
};

}  // namespace bfp
