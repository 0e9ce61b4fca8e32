// rq_formats.h -- per-lane decoders of GGUF block "pieces" for gfx950.
//
// A piece is the part of one weight row that one lane loads with 128-bit
// loads and decodes alone.  The GEMV kernels (rq_gemv.hip) and the MFMA GEMM
// kernels (rq_gemm.hip) share these decoders.  `decode` yields the exact f32
// weights of runtimed-gguf's dequant (dequant.rs:40-47, dequant_k.rs:19-44,
// dequant_k.rs:87-111); `dot` is the M=1 form that keeps activations in
// registers; `decode_bf16` feeds the bf16 MFMA GEMM (one fused multiply-add
// per weight, then the bf16 rounding).  Pieces with PE = 32 and RUNS = 2 all cover the same k
// positions, two runs of 16 at 64*(p/2) + 16*(p%2) and that + 32, so a GEMM
// K-step of 64 is two pieces per row whatever the format.
#pragma once

#include "rq_internal.h"

namespace rq {

__device__ __forceinline__ float h2f(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

__device__ __forceinline__ float ub(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }

// Returns v unchanged but hides how it was computed.  A word of four masked
// codes (e.g. q & 0x0F0F0F0F) fed to ub() should become one
// v_cvt_f32_ubyte{0..3} per code; seeing the mask, the optimizer instead
// folds it into each extraction (a v_bfe_u32 plus a conversion per code).
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

typedef __bf16 fmt_bf16x2 __attribute__((ext_vector_type(2)));
typedef float fmt_f32x2 __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((fmt_f32x2){lo, hi}, fmt_bf16x2));
}

// Two f32 values as two bf16 limbs each: hi = v rounded to bf16, lo =
// (v - hi) rounded to bf16 (v - hi is exact in f32), packed in pairs as
// pk_bf16 packs them.  hi + lo is v to within 2^-17 |v|, so products of
// limbs carry 16 significant bits of each operand.
__device__ __forceinline__ void limbs2(float a, float b, uint32_t &hi, uint32_t &lo) {
  hi = pk_bf16(a, b);
  lo = pk_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

// Load `len` (multiple of 4) activations starting at x[idx] into f32 registers.
template <int LEN>
__device__ __forceinline__ void load_run(const void *x, int xtype, int64_t idx, float *dst) {
#pragma unroll
  for (int j = 0; j < LEN / 4; ++j) {
    const float4 a = load_x4(x, xtype, idx + 4 * j);
    dst[4 * j + 0] = a.x;
    dst[4 * j + 1] = a.y;
    dst[4 * j + 2] = a.z;
    dst[4 * j + 3] = a.w;
  }
}


// Weight loads.  NT = true marks them non-temporal (streamed once: the M = 1
// GEMVs, whose weights are not read again before the whole model has passed
// through the caches); the GEMM tiles re-read a weight tile for each M tile
// and keep plain loads.  On the decode layer set (128 distinct layer copies)
// the non-temporal GEMV loads took 437 -> 478 GB/s: the gate GEMV 2.95 ->
// 2.83 us, the down projection 3.55 -> 3.29.
typedef uint32_t fmt_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t fmt_u32x2 __attribute__((ext_vector_type(2)));

template <bool NT>
__device__ __forceinline__ uint4 ld_w16(const uint8_t *p) {
  if constexpr (NT) {
    const fmt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const fmt_u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4 *>(p);
  }
}

template <bool NT>
__device__ __forceinline__ uint2 ld_w8(const uint8_t *p) {
  if constexpr (NT) {
    const fmt_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const fmt_u32x2 *>(p));
    return make_uint2(v.x, v.y);
  } else {
    return *reinterpret_cast<const uint2 *>(p);
  }
}

template <bool NT, class T>
__device__ __forceinline__ T ld_w(const T *p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

// ---------------------------------------------------------------- formats --

// Q4_K (dequant_k.rs:19-44) on the aligned GGUF stream.
struct FmtQ4K {
  static constexpr int PE = 32;    // elements per piece
  static constexpr int RUNS = 2;   // runs of 16 activations
  __device__ __forceinline__ static int64_t run_off(int p, int r) { return 64 * (p >> 1) + 16 * (p & 1) + 32 * r; }

  struct Piece {
    uint4 hd, qv;
    int c;
  };
  // The piece of the row whose first element is element rk of the flat
  // stream (rk = row * k).
  template <bool NT = false>
  __device__ __forceinline__ static Piece load_e(const uint8_t *w, const uint8_t *, uint64_t rk, int p) {
    const uint64_t e = rk + 64u * (uint64_t)(p >> 1);
    const uint8_t *bp = w + (e >> 8) * 144u;
    Piece pc;
    pc.c = (int)((e >> 6) & 3u);
    pc.hd = ld_w16<NT>(bp);
    pc.qv = ld_w16<NT>(bp + 16 + 32 * pc.c + 16 * (p & 1));
    return pc;
  }
  template <bool NT = false>
  __device__ __forceinline__ static Piece load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int p) {
    return load_e<NT>(w, aux, (uint64_t)row * (uint64_t)k, p);
  }
  // (d*sc, dmin*m) for sub-blocks 2c (low nibbles) and 2c+1 (high nibbles):
  // scale_min_k4 (dequant_k.rs:8-16) on the packed bytes in hd.y/z/w.
  __device__ __forceinline__ static void scales(const Piece &pc, float &a0, float &b0, float &a1, float &b1) {
    // Both sub-blocks at once, one per byte of a 16-bit pair; the two
    // scale_min_k4 cases are computed side by side and selected (lanes of a
    // wave usually hold different chunks c, and a branch would run both).
    const int sh = 16 * (pc.c & 1);
    const uint32_t Y = pc.hd.y >> sh, Z = pc.hd.z >> sh, W = pc.hd.w >> sh;
    // The case is picked by a mask the optimizer cannot see through, so it
    // cannot turn the selection back into a branch.
    const uint32_t low = opaque(pc.c < 2 ? 0xFFFFFFFFu : 0u);
    const uint32_t sc = opaque((Y & 0x3F3Fu & low) | (((W & 0x0F0Fu) | ((Y >> 2) & 0x3030u)) & ~low));
    const uint32_t mn = opaque((Z & 0x3F3Fu & low) | ((((W >> 4) & 0x0F0Fu) | ((Z >> 2) & 0x3030u)) & ~low));
    const float d = h2f(pc.hd.x), dmin = h2f(pc.hd.x >> 16);
    a0 = d * ub(sc, 0);
    b0 = dmin * ub(mn, 0);
    a1 = d * ub(sc, 1);
    b1 = dmin * ub(mn, 1);
  }
  // M=1: sum over the piece of W*x with the activations in registers.
  __device__ __forceinline__ static float dot(const Piece &pc, const float (&xv)[RUNS][16], const float (&sx)[RUNS]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
    const uint32_t q[4] = {pc.qv.x, pc.qv.y, pc.qv.z, pc.qv.w};
    float dl[4], dh[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = opaque(q[j] & 0x0F0F0F0Fu), hi = opaque(q[j] & 0xF0F0F0F0u);
      dl[j] = xv[0][4 * j] * ub(lo, 0);
      dh[j] = xv[1][4 * j] * ub(hi, 0);
#pragma unroll
      for (int b = 1; b < 4; ++b) {
        dl[j] = fmaf(xv[0][4 * j + b], ub(lo, b), dl[j]);
        dh[j] = fmaf(xv[1][4 * j + b], ub(hi, b), dh[j]);
      }
    }
    const float sl = (dl[0] + dl[1]) + (dl[2] + dl[3]);
    const float shh = ((dh[0] + dh[1]) + (dh[2] + dh[3])) * 0.0625f;  // high nibbles were x16
    return (a0 * sl - b0 * sx[0]) + (a1 * shh - b1 * sx[1]);
  }
  // dot() for MR activation rows at once: the codes are converted once and
  // every row's sums run in dot()'s order (row i's result equals dot() on
  // row i).
  template <int MR>
  __device__ __forceinline__ static void dot_rows(const Piece &pc, const float (&xv)[MR][RUNS][16],
                                                  const float (&sx)[MR][RUNS], float (&out)[MR]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
    const uint32_t q[4] = {pc.qv.x, pc.qv.y, pc.qv.z, pc.qv.w};
    float wl[16], wh[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = opaque(q[j] & 0x0F0F0F0Fu), hi = opaque(q[j] & 0xF0F0F0F0u);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        wl[4 * j + b] = ub(lo, b);
        wh[4 * j + b] = ub(hi, b);
      }
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      float dl[4], dh[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dl[j] = xv[i][0][4 * j] * wl[4 * j];
        dh[j] = xv[i][1][4 * j] * wh[4 * j];
#pragma unroll
        for (int b = 1; b < 4; ++b) {
          dl[j] = fmaf(xv[i][0][4 * j + b], wl[4 * j + b], dl[j]);
          dh[j] = fmaf(xv[i][1][4 * j + b], wh[4 * j + b], dh[j]);
        }
      }
      const float sl = (dl[0] + dl[1]) + (dl[2] + dl[3]);
      const float shh = ((dh[0] + dh[1]) + (dh[2] + dh[3])) * 0.0625f;
      out[i] = (a0 * sl - b0 * sx[i][0]) + (a1 * shh - b1 * sx[i][1]);
    }
  }
  // Weights of the piece as bf16 pairs in run order (o[8r + j]: elements
  // 2j, 2j + 1 of run r) for the MFMA GEMM: one fused multiply-add per
  // weight (a single rounding, then the bf16 rounding), not the exact
  // two-rounding value of decode().
  __device__ __forceinline__ static void decode_bf16(const Piece &pc, uint32_t (&o)[16]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
    const uint32_t q[4] = {pc.qv.x, pc.qv.y, pc.qv.z, pc.qv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = opaque(q[j] & 0x0F0F0F0Fu), hi = opaque((q[j] >> 4) & 0x0F0F0F0Fu);
      o[2 * j] = pk_bf16(fmaf(ub(lo, 0), a0, -b0), fmaf(ub(lo, 1), a0, -b0));
      o[2 * j + 1] = pk_bf16(fmaf(ub(lo, 2), a0, -b0), fmaf(ub(lo, 3), a0, -b0));
      o[8 + 2 * j] = pk_bf16(fmaf(ub(hi, 0), a1, -b1), fmaf(ub(hi, 1), a1, -b1));
      o[8 + 2 * j + 1] = pk_bf16(fmaf(ub(hi, 2), a1, -b1), fmaf(ub(hi, 3), a1, -b1));
    }
  }
  // Exact dequantized weights of the piece, in run order.
  __device__ __forceinline__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
    const uint32_t q[4] = {pc.qv.x, pc.qv.y, pc.qv.z, pc.qv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        wv[0][4 * j + b] = a0 * (float)((q[j] >> (8 * b)) & 0xFu) - b0;
        wv[1][4 * j + b] = a1 * (float)((q[j] >> (8 * b + 4)) & 0xFu) - b1;
      }
  }
};

// Q6_K (dequant_k.rs:87-111) on the split layout: 208-byte records + f16 d.
struct FmtQ6K {
  static constexpr int PE = 64;
  static constexpr int RUNS = 4;
  __device__ __forceinline__ static int64_t run_off(int p, int r) { return 128 * (p >> 1) + 16 * (p & 1) + 32 * r; }

  struct Piece {
    uint4 a, b, h;
    uint2 sc;
    uint32_t d;
    int s;
  };
  // The piece of the row whose first element is element rk of the flat
  // stream (rk = row * k).
  template <bool NT = false>
  __device__ __forceinline__ static Piece load_e(const uint8_t *w, const uint8_t *aux, uint64_t rk, int p) {
    const uint64_t e = rk + 128u * (uint64_t)(p >> 1);
    const uint64_t blk = e >> 8;
    const int hf = (int)((e >> 7) & 1u), s = p & 1;
    const uint8_t *rec = w + blk * 208u;
    Piece pc;
    pc.s = s;
    pc.a = ld_w16<NT>(rec + 64 * hf + 16 * s);
    pc.b = ld_w16<NT>(rec + 64 * hf + 32 + 16 * s);
    pc.h = ld_w16<NT>(rec + 128 + 32 * hf + 16 * s);
    pc.sc = ld_w8<NT>(rec + 192 + 8 * hf);
    pc.d = ld_w<NT>(reinterpret_cast<const uint16_t *>(aux) + (blk));
    return pc;
  }
  template <bool NT = false>
  __device__ __forceinline__ static Piece load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int p) {
    return load_e<NT>(w, aux, (uint64_t)row * (uint64_t)k, p);
  }
  // Unsigned 6-bit codes (q + 32) of run r for dword j.
  __device__ __forceinline__ static uint32_t codes(const Piece &pc, int r, int j) {
    const uint32_t a = (&pc.a.x)[j], b = (&pc.b.x)[j], h = (&pc.h.x)[j];
    switch (r) {
      case 0: return (a & 0x0F0F0F0Fu) | ((h & 0x03030303u) << 4);
      case 1: return (b & 0x0F0F0F0Fu) | ((h & 0x0C0C0C0Cu) << 2);
      case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
      default: return ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    }
  }
  // int8 scale of run r: scales[8*hf + s + 2r] (dequant_k.rs:107).
  __device__ __forceinline__ static float scale(const Piece &pc, int r) {
    const int byte = pc.s + 2 * r;
    const uint32_t word = byte < 4 ? pc.sc.x : pc.sc.y;
    return (float)(int8_t)((word >> (8 * (byte & 3))) & 0xFFu);
  }
  __device__ __forceinline__ static float dot(const Piece &pc, const float (&xv)[RUNS][16], const float (&sx)[RUNS]) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < RUNS; ++r) {
      float dd[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t q = opaque(codes(pc, r, j));
        dd[j] = xv[r][4 * j] * ub(q, 0);
#pragma unroll
        for (int b = 1; b < 4; ++b) dd[j] = fmaf(xv[r][4 * j + b], ub(q, b), dd[j]);
      }
      const float dot = (dd[0] + dd[1]) + (dd[2] + dd[3]);
      acc = fmaf(scale(pc, r), dot - 32.0f * sx[r], acc);
    }
    return h2f(pc.d) * acc;
  }
  __device__ __forceinline__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
    const float d = h2f(pc.d);
#pragma unroll
    for (int r = 0; r < RUNS; ++r) {
      const float ds = d * scale(pc, r);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t q = opaque(codes(pc, r, j));
#pragma unroll
        for (int b = 0; b < 4; ++b) wv[r][4 * j + b] = ds * (ub(q, b) - 32.0f);
      }
    }
  }
};

// Q8_0 (dequant.rs:40-47) on the split layout: int8 quants + f16 d.  A piece
// is the same run pattern as Q4_K (16 quants at chunk offset 16h, 16 at
// 32+16h), so its two runs lie in two different 32-quant blocks.
struct FmtQ8 {
  static constexpr int PE = 32;
  static constexpr int RUNS = 2;
  __device__ __forceinline__ static int64_t run_off(int p, int r) { return 64 * (p >> 1) + 16 * (p & 1) + 32 * r; }

  struct Piece {
    uint4 q[2];
    uint32_t d[2];
  };
  // The piece of the row whose first element is element rk of the flat
  // stream (rk = row * k).
  template <bool NT = false>
  __device__ __forceinline__ static Piece load_e(const uint8_t *w, const uint8_t *aux, uint64_t rk, int p) {
    Piece pc;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint64_t e = rk + (uint64_t)run_off(p, r);
      pc.q[r] = ld_w16<NT>(w + e);
      pc.d[r] = ld_w<NT>(reinterpret_cast<const uint16_t *>(aux) + (e >> 5));
    }
    return pc;
  }
  template <bool NT = false>
  __device__ __forceinline__ static Piece load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int p) {
    return load_e<NT>(w, aux, (uint64_t)row * (uint64_t)k, p);
  }
  __device__ __forceinline__ static float dot(const Piece &pc, const float (&xv)[RUNS][16], const float (&sx)[RUNS]) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t q[4] = {pc.q[r].x, pc.q[r].y, pc.q[r].z, pc.q[r].w};
      float dd[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t u = opaque(q[j] ^ 0x80808080u);  // q + 128 as unsigned bytes
        dd[j] = xv[r][4 * j] * ub(u, 0);
#pragma unroll
        for (int b = 1; b < 4; ++b) dd[j] = fmaf(xv[r][4 * j + b], ub(u, b), dd[j]);
      }
      const float dot = (dd[0] + dd[1]) + (dd[2] + dd[3]);
      acc = fmaf(h2f(pc.d[r]), dot - 128.0f * sx[r], acc);
    }
    return acc;
  }
  __device__ __forceinline__ static void decode_bf16(const Piece &pc, uint32_t (&o)[16]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float d = h2f(pc.d[r]);
      const uint32_t q[4] = {pc.q[r].x, pc.q[r].y, pc.q[r].z, pc.q[r].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[8 * r + 2 * j] = pk_bf16(d * (float)(int8_t)(q[j] & 0xFFu), d * (float)(int8_t)((q[j] >> 8) & 0xFFu));
        o[8 * r + 2 * j + 1] = pk_bf16(d * (float)(int8_t)((q[j] >> 16) & 0xFFu), d * (float)(int8_t)(q[j] >> 24));
      }
    }
  }
  __device__ __forceinline__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float d = h2f(pc.d[r]);
      const uint32_t q[4] = {pc.q[r].x, pc.q[r].y, pc.q[r].z, pc.q[r].w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int b = 0; b < 4; ++b) wv[r][4 * j + b] = d * (float)(int8_t)((q[j] >> (8 * b)) & 0xFFu);
    }
  }
};

// Q5_K (dequant_k.rs:51-80) on the aligned GGUF stream (176-byte blocks:
// d, dmin, 12 scale bytes, qh[32], qs[128]).  Same pieces as Q4_K; element
// l of chunk c adds 16 when bit 2c (low nibbles) or 2c + 1 (high nibbles) of
// qh[l] is set.
struct FmtQ5K {
  static constexpr int PE = 32;
  static constexpr int RUNS = 2;
  __device__ __forceinline__ static int64_t run_off(int p, int r) { return 64 * (p >> 1) + 16 * (p & 1) + 32 * r; }

  struct Piece {
    uint4 hd, qv, hv;
    int c;
  };
  // The piece of the row whose first element is element rk of the flat
  // stream (rk = row * k).
  template <bool NT = false>
  __device__ __forceinline__ static Piece load_e(const uint8_t *w, const uint8_t *, uint64_t rk, int p) {
    const uint64_t e = rk + 64u * (uint64_t)(p >> 1);
    const uint8_t *bp = w + (e >> 8) * 176u;
    Piece pc;
    pc.c = (int)((e >> 6) & 3u);
    pc.hd = ld_w16<NT>(bp);
    pc.qv = ld_w16<NT>(bp + 48 + 32 * pc.c + 16 * (p & 1));
    pc.hv = ld_w16<NT>(bp + 16 + 16 * (p & 1));
    return pc;
  }
  template <bool NT = false>
  __device__ __forceinline__ static Piece load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int p) {
    return load_e<NT>(w, aux, (uint64_t)row * (uint64_t)k, p);
  }
  __device__ __forceinline__ static void scales(const Piece &pc, float &a0, float &b0, float &a1, float &b1) {
    FmtQ4K::Piece q4;
    q4.hd = pc.hd;
    q4.c = pc.c;
    FmtQ4K::scales(q4, a0, b0, a1, b1);
  }
  // 5-bit codes of dword j: run 0 (low nibbles | bit 2c), run 1 (high | bit 2c + 1).
  __device__ __forceinline__ static void codes(const Piece &pc, int j, uint32_t &c0, uint32_t &c1) {
    const uint32_t q = (&pc.qv.x)[j], h = (&pc.hv.x)[j] >> (2 * pc.c);
    c0 = (q & 0x0F0F0F0Fu) | ((h << 4) & 0x10101010u);
    c1 = ((q >> 4) & 0x0F0F0F0Fu) | ((h << 3) & 0x10101010u);
  }
  __device__ __forceinline__ static float dot(const Piece &pc, const float (&xv)[RUNS][16], const float (&sx)[RUNS]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
    float dl[4], dh[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t c0, c1;
      codes(pc, j, c0, c1);
      c0 = opaque(c0);
      c1 = opaque(c1);
      dl[j] = xv[0][4 * j] * ub(c0, 0);
      dh[j] = xv[1][4 * j] * ub(c1, 0);
#pragma unroll
      for (int b = 1; b < 4; ++b) {
        dl[j] = fmaf(xv[0][4 * j + b], ub(c0, b), dl[j]);
        dh[j] = fmaf(xv[1][4 * j + b], ub(c1, b), dh[j]);
      }
    }
    const float sl = (dl[0] + dl[1]) + (dl[2] + dl[3]);
    const float shh = (dh[0] + dh[1]) + (dh[2] + dh[3]);
    return (a0 * sl - b0 * sx[0]) + (a1 * shh - b1 * sx[1]);
  }
  __device__ __forceinline__ static void decode_bf16(const Piece &pc, uint32_t (&o)[16]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t c0, c1;
      codes(pc, j, c0, c1);
      c0 = opaque(c0);
      c1 = opaque(c1);
      o[2 * j] = pk_bf16(fmaf(ub(c0, 0), a0, -b0), fmaf(ub(c0, 1), a0, -b0));
      o[2 * j + 1] = pk_bf16(fmaf(ub(c0, 2), a0, -b0), fmaf(ub(c0, 3), a0, -b0));
      o[8 + 2 * j] = pk_bf16(fmaf(ub(c1, 0), a1, -b1), fmaf(ub(c1, 1), a1, -b1));
      o[8 + 2 * j + 1] = pk_bf16(fmaf(ub(c1, 2), a1, -b1), fmaf(ub(c1, 3), a1, -b1));
    }
  }
  // Exact weights: d1 * (q + hi) - m1 (dequant_k.rs:67-73).
  __device__ __forceinline__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t c0, c1;
      codes(pc, j, c0, c1);
      c0 = opaque(c0);
      c1 = opaque(c1);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        wv[0][4 * j + b] = a0 * ub(c0, b) - b0;
        wv[1][4 * j + b] = a1 * ub(c1, b) - b1;
      }
    }
  }
};

// Bits 0..3 of v spread to bit 0 of bytes 0..3.
__device__ __forceinline__ uint32_t spread4(uint32_t v) { return ((v & 0xFu) * 0x00204081u) & 0x01010101u; }

// Q4_0 (dequant.rs:50-61) and Q5_0 (dequant.rs:64-77) on their split
// layouts: 16 quant bytes per 32-element block in block order, then at aux
// one f16 d per block (Q4_0) or one 8-byte record {qh: u32, d: f16, 0} per
// block (Q5_0).  A piece is the Q4_K run pattern: its two runs are elements
// 16h .. 16h + 15 (h = p & 1) of two consecutive blocks -- the low (h = 0)
// or high (h = 1) nibbles of the block's 16 bytes, and for Q5_0 bits
// 16h .. 16h + 15 of its qh.
template <bool Q5>
struct FmtQx0 {
  static constexpr int PE = 32;
  static constexpr int RUNS = 2;
  __device__ __forceinline__ static int64_t run_off(int p, int r) { return 64 * (p >> 1) + 16 * (p & 1) + 32 * r; }

  struct Piece {
    uint4 q[2];
    uint32_t qh[2];
    uint32_t d[2];
    int h;
  };
  // The piece of the row whose first element is element rk of the flat
  // stream (rk = row * k).
  template <bool NT = false>
  __device__ __forceinline__ static Piece load_e(const uint8_t *w, const uint8_t *aux, uint64_t rk, int p) {
    Piece pc;
    pc.h = p & 1;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint64_t blk = (rk + (uint64_t)run_off(p, r)) >> 5;
      pc.q[r] = ld_w16<NT>(w + 16 * blk);
      if (Q5) {
        const uint2 rec = ld_w8<NT>(aux + 8 * (blk));
        pc.qh[r] = rec.x;
        pc.d[r] = rec.y;
      } else {
        pc.qh[r] = 0;
        pc.d[r] = ld_w<NT>(reinterpret_cast<const uint16_t *>(aux) + (blk));
      }
    }
    return pc;
  }
  template <bool NT = false>
  __device__ __forceinline__ static Piece load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int p) {
    return load_e<NT>(w, aux, (uint64_t)row * (uint64_t)k, p);
  }
  // Unsigned codes (q + 8, or q + 16 for Q5_0) of dword j of run r.
  __device__ __forceinline__ static uint32_t codes(const Piece &pc, int r, int j) {
    const uint32_t q = ((&pc.q[r].x)[j] >> (4 * pc.h)) & 0x0F0F0F0Fu;
    if (!Q5) return q;
    return q | (spread4(pc.qh[r] >> (16 * pc.h + 4 * j)) << 4);
  }
  static constexpr float ZERO = Q5 ? 16.0f : 8.0f;
  __device__ __forceinline__ static float dot(const Piece &pc, const float (&xv)[RUNS][16], const float (&sx)[RUNS]) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float dd[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = opaque(codes(pc, r, j));
        dd[j] = xv[r][4 * j] * ub(c, 0);
#pragma unroll
        for (int b = 1; b < 4; ++b) dd[j] = fmaf(xv[r][4 * j + b], ub(c, b), dd[j]);
      }
      const float dot = (dd[0] + dd[1]) + (dd[2] + dd[3]);
      acc = fmaf(h2f(pc.d[r]), dot - ZERO * sx[r], acc);
    }
    return acc;
  }
  __device__ __forceinline__ static void decode_bf16(const Piece &pc, uint32_t (&o)[16]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float d = h2f(pc.d[r]), z = -ZERO * d;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = opaque(codes(pc, r, j));
        o[8 * r + 2 * j] = pk_bf16(fmaf(ub(c, 0), d, z), fmaf(ub(c, 1), d, z));
        o[8 * r + 2 * j + 1] = pk_bf16(fmaf(ub(c, 2), d, z), fmaf(ub(c, 3), d, z));
      }
    }
  }
  // Exact weights d * (q - 8) or d * (q - 16).
  __device__ __forceinline__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float d = h2f(pc.d[r]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = opaque(codes(pc, r, j));
#pragma unroll
        for (int b = 0; b < 4; ++b) wv[r][4 * j + b] = d * (ub(c, b) - ZERO);
      }
    }
  }
};

// Q6_K in 32-element pieces for the GEMM: the 64 elements [64*ch, 64*ch+64)
// of a 128-element half hf are y[l + 32*kk] for kk = 2ch, 2ch+1 (l < 32);
// piece h takes l in [16h, 16h+16), i.e. the same run pattern as Q4_K.  Its
// codes come from nibble ch of ql[16h..) and ql[32+16h..) and from bits
// 4ch..4ch+3 of qh[16h..).
struct FmtQ6KG {
  static constexpr int PE = 32;
  static constexpr int RUNS = 2;
  __device__ __forceinline__ static int64_t run_off(int p, int r) { return 64 * (p >> 1) + 16 * (p & 1) + 32 * r; }

  struct Piece {
    uint4 a, b, h;
    uint32_t sc;  // int8 scales of run 0 (byte 0) and run 1 (byte 2)
    uint32_t d;
    int ch;
  };
  // The piece of the row whose first element is element rk of the flat
  // stream (rk = row * k).
  template <bool NT = false>
  __device__ __forceinline__ static Piece load_e(const uint8_t *w, const uint8_t *aux, uint64_t rk, int p) {
    const uint64_t e = rk + 64u * (uint64_t)(p >> 1);
    const uint64_t blk = e >> 8;
    const int hf = (int)((e >> 7) & 1u), hh = p & 1;
    const uint8_t *rec = w + blk * 208u;
    Piece pc;
    pc.ch = (int)((e >> 6) & 1u);
    pc.a = ld_w16<NT>(rec + 64 * hf + 16 * hh);
    pc.b = ld_w16<NT>(rec + 64 * hf + 32 + 16 * hh);
    pc.h = ld_w16<NT>(rec + 128 + 32 * hf + 16 * hh);
    // scales[8hf + hh + 2kk] for kk = 2ch and 2ch+1: bytes 4ch+hh and 4ch+hh+2
    pc.sc = ld_w<NT>(reinterpret_cast<const uint32_t *>(rec + 192 + 8 * hf + 4 * pc.ch)) >> (8 * hh);
    pc.d = ld_w<NT>(reinterpret_cast<const uint16_t *>(aux) + (blk));
    return pc;
  }
  template <bool NT = false>
  __device__ __forceinline__ static Piece load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int p) {
    return load_e<NT>(w, aux, (uint64_t)row * (uint64_t)k, p);
  }
  __device__ __forceinline__ static void decode_bf16(const Piece &pc, uint32_t (&o)[16]) {
    const float d = h2f(pc.d);
    const float ds0 = d * (float)(int8_t)(pc.sc & 0xFFu);
    const float ds1 = d * (float)(int8_t)((pc.sc >> 16) & 0xFFu);
    const float z0 = -32.0f * ds0, z1 = -32.0f * ds1;
    const int nsh = 4 * pc.ch;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = (&pc.a.x)[j], b = (&pc.b.x)[j], h = (&pc.h.x)[j] >> nsh;
      const uint32_t q0 = opaque(((a >> nsh) & 0x0F0F0F0Fu) | ((h & 0x03030303u) << 4));
      const uint32_t q1 = opaque(((b >> nsh) & 0x0F0F0F0Fu) | ((h & 0x0C0C0C0Cu) << 2));
      o[2 * j] = pk_bf16(fmaf(ub(q0, 0), ds0, z0), fmaf(ub(q0, 1), ds0, z0));
      o[2 * j + 1] = pk_bf16(fmaf(ub(q0, 2), ds0, z0), fmaf(ub(q0, 3), ds0, z0));
      o[8 + 2 * j] = pk_bf16(fmaf(ub(q1, 0), ds1, z1), fmaf(ub(q1, 1), ds1, z1));
      o[8 + 2 * j + 1] = pk_bf16(fmaf(ub(q1, 2), ds1, z1), fmaf(ub(q1, 3), ds1, z1));
    }
  }
  __device__ __forceinline__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
    const float d = h2f(pc.d);
    const float ds0 = d * (float)(int8_t)(pc.sc & 0xFFu);
    const float ds1 = d * (float)(int8_t)((pc.sc >> 16) & 0xFFu);
    const int nsh = 4 * pc.ch, hsh = 4 * pc.ch;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = (&pc.a.x)[j], b = (&pc.b.x)[j], h = (&pc.h.x)[j] >> hsh;
      const uint32_t q0 = opaque(((a >> nsh) & 0x0F0F0F0Fu) | ((h & 0x03030303u) << 4));
      const uint32_t q1 = opaque(((b >> nsh) & 0x0F0F0F0Fu) | ((h & 0x0C0C0C0Cu) << 2));
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        wv[0][4 * j + bb] = ds0 * (ub(q0, bb) - 32.0f);
        wv[1][4 * j + bb] = ds1 * (ub(q1, bb) - 32.0f);
      }
    }
  }
};

}  // namespace rq
