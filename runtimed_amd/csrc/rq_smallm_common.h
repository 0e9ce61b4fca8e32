// rq_smallm_common.h -- pieces shared by the small-M kernels (rq_smallm.hip,
// rq_smallm_codes.hip): fragment types, LDS access, the staged copy of an
// activation slice, and the split-K meeting of workgroups in the workspace.
#pragma once

#include <hip/hip_runtime.h>

#include "rq_internal.h"

namespace rq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 pick(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1) {
  return __builtin_bit_cast(bf16x8, (uint4){a0, a1, b0, b1});
}

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
__device__ __forceinline__ u32x4 ds_read16(const uint8_t *p) {
  return *reinterpret_cast<const lds_u32x4 *>((const __attribute__((address_space(3))) uint8_t *)p);
}
__device__ __forceinline__ void ds_write16(uint8_t *p, u32x4 v) {
  *reinterpret_cast<lds_u32x4 *>((__attribute__((address_space(3))) uint8_t *)p) = v;
}

// Piece p (16 bytes) of the slice: row p / ppr, piece p % ppr of the row;
// indices past the end repeat the last piece (the same bytes to the same
// place).  The row comes from a float reciprocal: (p + 1/2) / ppr is at
// least 1 / (2 ppr) away from an integer, far above the rounding error for
// p < 2^20.
struct XStage {
  const uint8_t *x;  // the slice's first byte of row 0
  int64_t rb;        // row stride of x in bytes
  int ppr, total, xstr;
  float inv;
  __device__ __forceinline__ void at(int p, int &r, int &c) const {
    p = p < total ? p : total - 1;
    r = (int)(((float)p + 0.5f) * inv);
    c = p - r * ppr;
  }
};

template <int NT, int XR>
__device__ __forceinline__ void xs_load(u32x4 (&v)[XR], const XStage &st, int base) {
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    int r, c;
    st.at(base + i * NT + (int)threadIdx.x, r, c);
    v[i] = *reinterpret_cast<const u32x4 *>(st.x + r * st.rb + 16 * c);
  }
}

__device__ __forceinline__ XStage make_stage(const uint8_t *x, int64_t rb, int64_t m, int64_t slice_bytes, int xstr) {
  XStage st;
  st.x = x;
  st.rb = rb;
  st.ppr = (int)(slice_bytes / 16);
  st.total = (int)m * st.ppr;
  st.xstr = xstr;
  st.inv = 1.0f / (float)st.ppr;
  return st;
}

// Split K: a workgroup's summed partial tile (NSLOT f32x4 slots) to
// wsp[s NSLOT + slot]; the last of the S workgroups of the tile to count
// itself in cnt (left at zero for the next call) adds the S partials in
// order s = 0 .. S - 1 -- the same order whichever arrives last -- and
// stores them.
// Partials, counter and reads are agent-scope relaxed atomics, which the
// XCDs' separate L2 caches keep coherent at the device's memory.  Every
// thread waits for its own partial stores to be acknowledged
// (s_waitcnt vmcnt(0)) before the workgroup barrier, so no store is still in
// flight when thread 0 counts the workgroup in: a barrier alone orders only
// issue, and a workgroup-scope release waits for LDS, not for global stores.
// (Agent-scope fences instead would write back and invalidate whole L2
// caches per workgroup: measured slower than no split.)
__device__ __forceinline__ void store_agent(f32x4 *p, const f32x4 &v) {
  uint64_t *q = reinterpret_cast<uint64_t *>(p);
  __hip_atomic_store(q, __builtin_bit_cast(uint64_t, (float2v){v[0], v[1]}), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, __builtin_bit_cast(uint64_t, (float2v){v[2], v[3]}), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 load_agent(const f32x4 *p) {
  const uint64_t *q = reinterpret_cast<const uint64_t *>(p);
  const float2v a = __builtin_bit_cast(float2v, __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const float2v b =
      __builtin_bit_cast(float2v, __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  return (f32x4){a[0], a[1], b[0], b[1]};
}

// partial(slot) gives this workgroup's value of a slot (after the caller's
// barrier), store(slot, v) writes a finished slot; NT threads.
template <int NSLOT, int NT, class P, class St>
__device__ __forceinline__ void split_finish(P &&partial, St &&store, int S, int s, f32x4 *__restrict__ wsp,
                                             uint32_t *__restrict__ cnt) {
  __shared__ int last;
  for (int slot = threadIdx.x; slot < NSLOT; slot += NT) store_agent(wsp + (int64_t)s * NSLOT + slot, partial(slot));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t before = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = before == (uint32_t)(S - 1);
    if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  for (int slot = threadIdx.x; slot < NSLOT; slot += NT) {
    f32x4 v = load_agent(wsp + slot);
    for (int q = 1; q < S; ++q) v += load_agent(wsp + (int64_t)q * NSLOT + slot);
    store(slot, v);
  }
}

// Order of the workgroups of a split launch: workgroup b runs on XCD b % 8
// (workgroups are dealt to the eight XCDs in turn, each with its own L2), so
// the S workgroups of a row tile, numbered consecutively, would read the
// 32-byte pieces of the same 128-byte lines from eight different L2s, each
// fetching the line: measured 2x the weight bytes from memory on the
// 896 x 4864 down projection.  XCD x takes the x-th eighth of the
// workgroups instead, so the slices of a tile meet in one L2.  Grids that
// are not a multiple of 8 (and unsplit launches) keep b.
__device__ __forceinline__ int split_order(int b, int grid, int S) {
  if (S == 1 || (grid & 7)) return b;
  return (b & 7) * (grid >> 3) + (b >> 3);
}

// Largest LDS copy of the activation slice (beside the reduction buffer of
// at most 32 KB, within the 160 KB of a CU).
constexpr size_t kSmXsMax = 120 * 1024;

// Dynamic LDS of a kernel instantiation above 64 KB is asked for once.
template <auto KERNEL>
bool lds_allow(size_t bytes) {
  if (bytes <= 65536) return true;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(KERNEL), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)kSmXsMax);
  if (attr != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return true;
}

}  // namespace
}  // namespace rq
