// rq_e4m3.h -- scalar e4m3 (OCP e4m3fn) encoders and decoder shared by the
// FP8 GEMM and the KV-cache quantizer (gfx950 device code).
#pragma once

#include "rq_internal.h"

namespace rq {

// f32_to_fp8_e4m3 (load_safetensors.rs:53-69), bit-exact, in closed form.
// The reference binary-searches the e4m3 table for the nearest value and
// breaks ties towards the lower magnitude; |f| >= 448 gives 0x7e, NaN 0x7f.
// Below 2^-6 the table is the grid k * 2^-9 (k = 0..8), so the code is
// ceil(|f| * 512 - 0.5) (exact: scaling by 512 is exact and |f| * 512 - 0.5
// is exact wherever it decides a tie); above it the 3-bit mantissa rounds to
// nearest with an exact tie (remainder 0x80000 of 20 bits) kept low.  The
// distance comparisons of the reference are exact here (Sterbenz), so its
// tie rule is the exact one.
__device__ __forceinline__ uint32_t enc_e4m3_ref(float f) {
  if (f != f) return 0x7Fu;
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x43E00000u) return sign | 0x7Eu;  // |f| >= 448
  if (a < 0x3C800000u) {                       // |f| < 2^-6
    const float q = __uint_as_float(a) * 512.0f;
    return sign | (uint32_t)fmaxf(ceilf(q - 0.5f), 0.0f);
  }
  int e = (int)(a >> 23) - 127;
  const uint32_t man = a & 0x7FFFFFu;
  uint32_t r = man >> 20;
  if ((man & 0xFFFFFu) > 0x80000u) r += 1;
  if (r == 8) {
    r = 0;
    e += 1;
  }
  return sign | ((uint32_t)(e + 7) << 3) | r;
}

// Clamp to +-448 then OCP e4m3fn round-to-nearest-even.
__device__ __forceinline__ uint32_t enc_e4m3_rne(float f) {
  if (f != f) return 0x7Fu;
  const uint32_t sign = (__float_as_uint(f) >> 24) & 0x80u;
  float a = fminf(fabsf(f), 448.0f);
  if (a < 0.015625f) return sign | (uint32_t)__builtin_rintf(a * 512.0f);
  const uint32_t u = __float_as_uint(a);
  int e = (int)((u >> 23) & 0xFFu) - 127;
  const uint32_t man = u & 0x7FFFFFu;
  uint32_t r = man >> 20;
  const uint32_t rem = man & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) r += 1;
  if (r == 8) {
    r = 0;
    e += 1;
  }
  return sign | (((uint32_t)(e + 7) << 3) | r);
}

// enc_e4m3_rne without branches, for the vector quantizer: the normal range
// rounds the f32 bits to three mantissa bits (adding 0x7FFFF plus the kept
// lsb carries into bit 20 exactly when round-to-nearest-even rounds up; the
// carry moves into the exponent when the mantissa overflows), the
// subnormal range is rint(a * 512) as above.  Same code as enc_e4m3_rne for
// every one of the 2^32 f32 inputs (compared exhaustively on the host).
__device__ __forceinline__ uint32_t enc_e4m3_rne_bf(float f) {
  const uint32_t sign = (__float_as_uint(f) >> 24) & 0x80u;
  const float a = fminf(fabsf(f), 448.0f);
  const uint32_t u = __float_as_uint(a);
  const uint32_t nrm = ((u + 0x7FFFFu + ((u >> 20) & 1u)) >> 20) - (120u << 3);
  const uint32_t sub = (uint32_t)__builtin_rintf(a * 512.0f);
  const uint32_t c = a < 0.015625f ? sub : nrm;
  return f != f ? 0x7Fu : (sign | c);
}

// e4m3 decode for the scalar path (LUT formula of load_safetensors.rs:14-29).
__device__ __forceinline__ float dec_e4m3(uint32_t b) {
  const int e = (b >> 3) & 0xF, m = b & 7;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;
  else if (e == 15 && m == 7) v = __uint_as_float(0x7FC00000u);
  else v = ldexpf(1.0f + (float)m * 0.125f, e - 7);
  return (b & 0x80u) ? -v : v;
}

// One activation element of type xtype as f32.
__device__ __forceinline__ float load_x1(const void *x, int xtype, int64_t i) {
  if (xtype == RQ_F32) return static_cast<const float *>(x)[i];
  if (xtype == RQ_BF16) return bf16_bits_to_f32(static_cast<const uint16_t *>(x)[i]);
  return (float)static_cast<const _Float16 *>(x)[i];
}

}  // namespace rq
