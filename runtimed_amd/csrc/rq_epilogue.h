// rq_epilogue.h -- stores of 32 x 32 MFMA accumulator tiles (gfx950).
//
// A v_mfma_f32_32x32x* accumulator (16 f32 per lane) holds column lane % 32
// and rows 8*(r/4) + 4*(lane/32) + r%4 in element r.  Stored as is, every
// element is its own 2- or 4-byte write and 64 lanes touch two rows per
// instruction; at 1 workgroup per CU the write phase then costs several
// times the MFMA phase of a GEMM tile.  Instead each group of four
// consecutive rows is transposed across the four lanes of a quad (DPP
// quad_perm, no LDS), after which lane 4q+t holds row 4*(lane/32)+t of the
// group at columns 4q..4q+3: one 16-byte (f32) or 8-byte (bf16 / f16) store.
#pragma once

#include "rq_internal.h"

namespace rq {

typedef float rq_f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 rq_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 rq_f16x2 __attribute__((ext_vector_type(2)));
typedef float rq_f32x2 __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16 (low half = lo), round to nearest even
// (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((rq_f32x2){lo, hi}, rq_bf16x2));
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((rq_f32x2){lo, hi}, rq_f16x2));
}

// One f32 as the output type; same rounding as the four-wide store below.
__device__ __forceinline__ void store_one(void *y, int ytype, int64_t idx, float v) {
  if (ytype == RQ_F32) {
    static_cast<float *>(y)[idx] = v;
  } else if (ytype == RQ_BF16) {
    static_cast<uint16_t *>(y)[idx] = (uint16_t)pack_bf16x2(v, 0.0f);
  } else {
    static_cast<uint16_t *>(y)[idx] = (uint16_t)pack_f16x2(v, 0.0f);
  }
}

// Four consecutive outputs y[idx .. idx+3]; idx % 4 == 0 and y 16-aligned.
__device__ __forceinline__ void store_four(void *y, int ytype, int64_t idx, float a, float b, float c,
                                           float d) {
  if (ytype == RQ_F32) {
    *reinterpret_cast<float4 *>(static_cast<float *>(y) + idx) = make_float4(a, b, c, d);
  } else if (ytype == RQ_BF16) {
    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + idx) =
        make_uint2(pack_bf16x2(a, b), pack_bf16x2(c, d));
  } else {
    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + idx) =
        make_uint2(pack_f16x2(a, b), pack_f16x2(c, d));
  }
}

template <int CTRL>
__device__ __forceinline__ float quad_perm(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// 4 x 4 transpose inside each quad of lanes: afterwards lane 4q+t holds in
// v_j what lane 4q+j held in v_t.  Two exchange stages (lane ^ 1, lane ^ 2).
__device__ __forceinline__ void quad_transpose(float &v0, float &v1, float &v2, float &v3, int lane) {
  constexpr int XOR1 = 0xB1;  // quad_perm [1, 0, 3, 2]
  constexpr int XOR2 = 0x4E;  // quad_perm [2, 3, 0, 1]
  const bool odd = lane & 1, upper = lane & 2;
  const float p0 = quad_perm<XOR1>(v0), p1 = quad_perm<XOR1>(v1);
  const float p2 = quad_perm<XOR1>(v2), p3 = quad_perm<XOR1>(v3);
  const float a0 = odd ? p1 : v0, a1 = odd ? v1 : p0;
  const float a2 = odd ? p3 : v2, a3 = odd ? v3 : p2;
  const float q0 = quad_perm<XOR2>(a0), q1 = quad_perm<XOR2>(a1);
  const float q2 = quad_perm<XOR2>(a2), q3 = quad_perm<XOR2>(a3);
  v0 = upper ? q2 : a0;
  v1 = upper ? q3 : a1;
  v2 = upper ? a2 : q0;
  v3 = upper ? a3 : q1;
}

// Scales of a lane's share of the 32 x 32 tile at (row0, col0) after the
// quad transpose: sx[g] for its row in row group g, sw[j] for its columns
// col0 + (lane & 28) + j.  A null array, or a row or column outside y,
// gives 1.  Loaded once before any store: on gfx9 stores count in vmcnt, so
// a load issued between stores would make its wait drain the stores too.
__device__ __forceinline__ void tile_row_scales(const float *xs, int64_t m, int64_t row0, int lane,
                                                float (&sx)[4]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t row = row0 + 8 * g + 4 * (lane >> 5) + (lane & 3);
    sx[g] = (xs && row < m) ? xs[row] : 1.0f;
  }
}

__device__ __forceinline__ void tile_col_scales(const float *ws, int64_t n, int64_t col0, int lane,
                                                float (&sw)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t col = col0 + (lane & 28) + j;
    sw[j] = (ws && col < n) ? ws[col] : 1.0f;
  }
}

// Biases of the same four columns, rounded to the output type (0 where there
// is none), with one branch on the bias type for all four.
__device__ __forceinline__ void tile_col_bias(const Out &o, int64_t n, int64_t col0, int lane, float (&bb)[4]) {
  const int64_t c0 = col0 + (lane & 28);
#pragma unroll
  for (int j = 0; j < 4; ++j) bb[j] = 0.0f;
  if (!o.bias) return;
  if (o.btype == RQ_F32) {
    const float *b = static_cast<const float *>(o.bias);
#pragma unroll
    for (int j = 0; j < 4; ++j) bb[j] = b[c0 + j < n ? c0 + j : n - 1];
  } else {
    const uint16_t *b = static_cast<const uint16_t *>(o.bias);
    const bool bf = o.btype == RQ_BF16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = b[c0 + j < n ? c0 + j : n - 1];
      bb[j] = bf ? __uint_as_float(u << 16) : f16_bits_to_f32(u);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) bb[j] = round_as(o.ytype, bb[j]);
}

// Writes the 32 x 32 tile at (row0, col0) of o.y[m, n] (row stride n) as
// acc * (xs[row] * ws[col]) when SCALED (a null xs or ws counts as 1), else
// as acc, plus the bias of its column (with_bias).  sx, sw, bb: the lane's
// scales and rounded biases from tile_row_scales / tile_col_scales /
// tile_col_bias (scales read only when SCALED; biases 0 when o has none, so
// the add stays one unconditional instruction in the unrolled epilogues).  vec: y is 16-byte aligned
// and n % 4 == 0.  Tiles not wholly inside y, or not vec, take the
// per-element path.
template <bool SCALED>
__device__ __forceinline__ void store_tile32(const rq_f32x16 &acc, const Out &o, int64_t m, int64_t n, int64_t row0,
                                             int64_t col0, const float (&sx)[4], const float (&sw)[4],
                                             const float (&bb)[4], const float *xs, const float *ws, int lane,
                                             bool vec) {
  const int h = lane >> 5;
  const int ytype = o.ytype;
  // with a bias and a 16-bit output, the product is rounded to y's type
  // before the (rounded) bias is added, as with_bias does
  const bool twice = o.bias && ytype != RQ_F32;
  if (vec && row0 + 32 <= m && col0 + 32 <= n) {
    const int t = lane & 3;
    const int64_t col = col0 + (lane & 28);
    static_for<4>([&](auto G) {
      constexpr int g = decltype(G)::value;
      float v0 = acc[4 * g], v1 = acc[4 * g + 1], v2 = acc[4 * g + 2], v3 = acc[4 * g + 3];
      quad_transpose(v0, v1, v2, v3, lane);
      const int64_t row = row0 + 8 * g + 4 * h + t;
      if (SCALED) {
        v0 *= sx[g] * sw[0];
        v1 *= sx[g] * sw[1];
        v2 *= sx[g] * sw[2];
        v3 *= sx[g] * sw[3];
      }
      if (twice) {
        v0 = round_as(ytype, v0);
        v1 = round_as(ytype, v1);
        v2 = round_as(ytype, v2);
        v3 = round_as(ytype, v3);
      }
      v0 += bb[0];
      v1 += bb[1];
      v2 += bb[2];
      v3 += bb[3];
      store_four(o.y, ytype, row * n + col, v0, v1, v2, v3);
    });
  } else {
    const int64_t col = col0 + (lane & 31);
    const float swe = (SCALED && ws && col < n) ? ws[col] : 1.0f;
    const float be = (o.bias && col < n) ? round_as(ytype, load_as_f32(o.bias, o.btype, col)) : 0.0f;
    static_for<16>([&](auto R) {
      constexpr int r = decltype(R)::value;
      const int64_t row = row0 + 8 * (r / 4) + 4 * h + (r % 4);
      if (row < m && col < n) {
        float v = acc[r];
        if (SCALED) v *= (xs ? xs[row] : 1.0f) * swe;
        store_one(o.y, ytype, row * n + col, (twice ? round_as(ytype, v) : v) + be);
      }
    });
  }
}

// ---- LDS-staged epilogue for 256 x 256 tiles of 2-byte outputs ------------
//
// Stored straight from the accumulators, a 2-byte output tile is written in
// 64-byte row pieces (8 bytes per lane, 8 rows per instruction), half cache
// lines scattered over rows n * 2 bytes apart.  Staged row-major
// in LDS (256 rows of 512 bytes; the 16-byte chunk c of row r at
// c ^ 4 (r % 4), so the four rows that one write instruction covers fall in
// disjoint 64-byte groups and a row's reads stay a permutation), the tile
// leaves as whole rows: 32 lanes x 16 bytes per row, two rows per wave
// instruction.

// A wave's MI x NI block of 32 x 32 MFMA tiles (rows rb.., columns cb.. of
// the staged tile) into T; values scaled by sx * sw when SCALED,
// plus the biases bb (rounded as tile_col_bias leaves them; 0 without one).
// twice: a bias is present, so each value is rounded to y's type before its
// bias is added (with_bias).
template <bool SCALED, int MI, int NI>
__device__ __forceinline__ void stage_block_2b(const rq_f32x16 (&acc)[MI][NI], uint8_t *T, int rb, int cb, int ytype,
                                               const float (&sx)[MI][4], const float (&sw)[NI][4],
                                               const float (&bb)[NI][4], bool twice, int lane) {
  const int h = lane >> 5, t = lane & 3;
  static_for<MI>([&](auto I) {
    static_for<NI>([&](auto J) {
      static_for<4>([&](auto G) {
        constexpr int g = decltype(G)::value;
        const rq_f32x16 &a = acc[I][J];
        float v0 = a[4 * g], v1 = a[4 * g + 1], v2 = a[4 * g + 2], v3 = a[4 * g + 3];
        quad_transpose(v0, v1, v2, v3, lane);
        if (SCALED) {
          v0 *= sx[I][g] * sw[J][0];
          v1 *= sx[I][g] * sw[J][1];
          v2 *= sx[I][g] * sw[J][2];
          v3 *= sx[I][g] * sw[J][3];
        }
        if (twice) {
          v0 = round_as(ytype, v0);
          v1 = round_as(ytype, v1);
          v2 = round_as(ytype, v2);
          v3 = round_as(ytype, v3);
        }
        v0 += bb[J][0];
        v1 += bb[J][1];
        v2 += bb[J][2];
        v3 += bb[J][3];
        const int r = rb + 32 * I + 8 * g + 4 * h + t;
        const int c = cb + 32 * J + (lane & 28);  // first of 4 columns
        const uint32_t lo = ytype == RQ_BF16 ? pack_bf16x2(v0, v1) : pack_f16x2(v0, v1);
        const uint32_t hi = ytype == RQ_BF16 ? pack_bf16x2(v2, v3) : pack_f16x2(v2, v3);
        *reinterpret_cast<uint2 *>(T + r * 512 + (((c >> 3) ^ (4 * (r & 3))) << 4) + ((c >> 2) & 1) * 8) =
            make_uint2(lo, hi);
      });
    });
  });
}

// The staged tile to y[m0 .. m0 + 256, n0 .. n0 + 256) (2-byte elements, row
// stride n), NTH threads (256 or 512).
template <int NTH = 256>
__device__ __forceinline__ void store_staged_2b(const uint8_t *T, void *y, int64_t n, int64_t m0, int64_t n0,
                                                int tid) {
  const int c = tid & 31;
  uint8_t *base = static_cast<uint8_t *>(y) + (m0 * n + n0) * 2 + 16 * c;
#pragma unroll 4
  for (int i = 0; i < 256 / (NTH / 32); ++i) {
    const int r = (NTH / 32) * i + (tid >> 5);
    const uint4 v = *reinterpret_cast<const uint4 *>(T + r * 512 + ((c ^ (4 * (r & 3))) << 4));
    *reinterpret_cast<uint4 *>(base + (int64_t)r * n * 2) = v;
  }
}

// vec flag of store_tile32 for an output buffer.
__device__ __forceinline__ bool vec_stores_ok(const void *y, int64_t n) {
  return ((reinterpret_cast<uintptr_t>(y) & 15) == 0) && ((n & 3) == 0);
}

}  // namespace rq
