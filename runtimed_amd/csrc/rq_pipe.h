// rq_pipe.h -- pieces shared by the pipelined 256 x 256 matrix-core kernels
// (FP8 GEMM, quantized bf16 GEMM): LDS stage geometry, explicit LDS operand
// reads and writes, and wait helpers.
//
// A stage holds 256 A rows then 256 B rows of 64 bytes each (one K-step).
// Rows carry no padding; the four 16-byte chunks of row r are stored
// XOR-swizzled by (r >> 2) & 3, so the 32 lanes that read one operand column
// of 32 rows hit 16 distinct 16-byte bank slots.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rq {
namespace pipe {

constexpr int P_STAGE = 32768, P_B = 16384;

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

template <int VM>
__device__ __forceinline__ void wait_vm() {
  // s_waitcnt vmcnt(VM) with expcnt / lgkmcnt left at their maxima (gfx9 encoding)
  __builtin_amdgcn_s_waitcnt((VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS operand reads (and writes) are issued as explicit ds_read_b128 /
// ds_write_b128; reads are completed by one
// s_waitcnt lgkmcnt(0) that takes every loaded register as an operand, so no
// use can be scheduled before the wait.  (As compiler-visible LDS loads they
// would each be preceded by a wait for all in-flight direct loads, because
// the compiler cannot prove that those target another stage buffer.)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ds_read16(const uint8_t *p) {
  u32x4 v;
  const uint32_t off = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(off));
  return v;
}

__device__ __forceinline__ void ds_write16(uint8_t *p, u32x4 v) {
  const uint32_t off = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)p;
  asm volatile("ds_write_b128 %0, %1" : : "v"(off), "v"(v));
}

// The same at a byte offset known at compile time (the instruction's 16-bit
// offset field): one base register serves every stage and tile at a fixed
// distance from it.
template <int OFF>
__device__ __forceinline__ u32x4 ds_read16_off(uint32_t base) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(base), "i"(OFF));
  return v;
}

template <int OFF>
__device__ __forceinline__ void ds_write16_off(uint32_t base, u32x4 v) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(base), "v"(v), "i"(OFF));
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// Fragment registers of one K-step: 8 x 16 bytes of A rows, 8 of B rows.
struct Frags {
  u32x4 x[16];
};

// Address (LDS byte offset) of fragment f (0..7 A, 8..15 B) of a stage.
__device__ __forceinline__ const uint8_t *frag_addr(const uint8_t *S, int f, int wm, int wn, int lane) {
  const int g = lane >> 5, half = f & 1, t = (f >> 1) & 3;
  const int r = (f < 8 ? 128 * wm : 128 * wn) + 32 * t + (lane & 31);
  return S + (f < 8 ? 0 : P_B) + r * 64 + 16 * ((2 * g + half) ^ swz(r));
}

__device__ __forceinline__ void wait_lds(Frags &F) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(F.x[0]), "+v"(F.x[1]), "+v"(F.x[2]), "+v"(F.x[3]));
  asm volatile("" : "+v"(F.x[4]), "+v"(F.x[5]), "+v"(F.x[6]), "+v"(F.x[7]));
  asm volatile("" : "+v"(F.x[8]), "+v"(F.x[9]), "+v"(F.x[10]), "+v"(F.x[11]));
  asm volatile("" : "+v"(F.x[12]), "+v"(F.x[13]), "+v"(F.x[14]), "+v"(F.x[15]));
}

__device__ __forceinline__ void read_all(const uint8_t *__restrict__ S, Frags &F, int wm, int wn, int lane) {
#pragma unroll
  for (int f = 0; f < 16; ++f) F.x[f] = ds_read16(frag_addr(S, f, wm, wn, lane));
}
}  // namespace pipe
}  // namespace rq
