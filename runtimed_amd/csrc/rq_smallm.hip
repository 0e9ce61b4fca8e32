// rq_smallm.hip -- quantized linear y = x W^T for 2 <= M <= 64 activation
// rows (speculative verify) on the matrix cores: bf16 activations on
// v_mfma_f32_16x16x32_bf16, f32 / f16 activations on v_mfma_f32_16x16x4_f32
// with exact f32 weights (second half of the file).
//
// The weight rows are the MFMA A operand (v_mfma_f32_16x16x32_bf16: lane l
// holds row l % 16 and 8 k-values chosen by l / 16) and the activation rows
// the B operand, so a weight is decoded once, straight into A registers (no
// LDS), and used by all M rows.  The cost per weight is then the decode
// (about 3 VALU instructions) whatever M is, against decode + M FMAs on the
// VALU.
//
// K order inside an MFMA is free as long as A and B agree.  Per 64-wide
// chunk of a weight row, lane group g = l / 16 takes chunk elements
// [8g, 8g + 8) and [32 + 8g, 32 + 8g + 8) -- the two 4-bit halves of 8 qs
// bytes of Q4_K, or the matching Q6_K / Q8_0 bytes -- and MFMA h in {0, 1}
// takes the quarter [8g + 4h, + 4) of each.  The activations are loaded for
// the same positions.
//
// Workgroup: 4 waves on 16 weight rows; wave w takes chunks w, w + 4, ...,
// loading a batch of them at once; the four partial 16 x (16 MT) tiles are
// summed through LDS.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "rq_epilogue.h"
#include "rq_formats.h"
#include "rq_internal.h"
#include "rq_smallm_common.h"

namespace rq {
namespace {


// The 16 weights of lane group g in chunk t of `row` as bf16 pairs:
// o[0..3] = chunk elements 8g .. 8g+7, o[4..7] = 32 + 8g .. 32 + 8g + 7.

// Q4_K (dequant_k.rs:19-44): elements j and 32 + j of chunk c are the low
// and high nibbles of qs[32c + j].
struct SmQ4K {
  static constexpr int CE = 64;  // elements of a row per chunk
  struct Chunk {
    uint4 hd;
    uint2 q;
    int c;
  };
  __device__ static Chunk load(const uint8_t *w, const uint8_t *, int64_t row, int64_t k, int64_t t, int g) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 64u * (uint64_t)t;
    const uint8_t *bp = w + (e >> 8) * 144u;
    Chunk ch;
    ch.c = (int)((e >> 6) & 3u);
    ch.hd = *reinterpret_cast<const uint4 *>(bp);
    ch.q = *reinterpret_cast<const uint2 *>(bp + 16 + 32 * ch.c + 8 * g);
    return ch;
  }
  template <class E>
  __device__ static void decode_with(const Chunk &ch, int, E &&emit) {
    FmtQ4K::Piece pc;
    pc.hd = ch.hd;
    pc.c = ch.c;
    float a0, b0, a1, b1;
    FmtQ4K::scales(pc, a0, b0, a1, b1);
    const uint32_t q[2] = {ch.q.x, ch.q.y};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t lo = q[j] & 0x0F0F0F0Fu, hi = (q[j] >> 4) & 0x0F0F0F0Fu;
      emit(2 * j, fmaf(ub(lo, 0), a0, -b0), fmaf(ub(lo, 1), a0, -b0));
      emit(2 * j + 1, fmaf(ub(lo, 2), a0, -b0), fmaf(ub(lo, 3), a0, -b0));
      emit(4 + 2 * j, fmaf(ub(hi, 0), a1, -b1), fmaf(ub(hi, 1), a1, -b1));
      emit(4 + 2 * j + 1, fmaf(ub(hi, 2), a1, -b1), fmaf(ub(hi, 3), a1, -b1));
    }
  }
};

// Q6_K (dequant_k.rs:87-111) on the split layout (208-byte records, f16 d
// array).  Chunk ch of half hf: element l < 32 is y[l + 64ch] of the half,
// code nibble ch of ql[l] | bits 4ch.. of qh[l]; element 32 + l is
// y[l + 64ch + 32], nibble ch of ql[l + 32] | bits 4ch + 2.. of qh[l];
// scales sc[l / 16 + 4ch] and sc[l / 16 + 4ch + 2].
struct SmQ6K {
  static constexpr int CE = 64;  // elements of a row per chunk
  struct Chunk {
    uint2 a, b, h;
    uint32_t sc, d;
    int ch;
  };
  __device__ static Chunk load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int64_t t,
                               int g) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 64u * (uint64_t)t;
    const uint64_t blk = e >> 8;
    const int hf = (int)((e >> 7) & 1u);
    const uint8_t *rec = w + blk * 208u;
    Chunk c;
    c.ch = (int)((e >> 6) & 1u);
    c.a = *reinterpret_cast<const uint2 *>(rec + 64 * hf + 8 * g);
    c.b = *reinterpret_cast<const uint2 *>(rec + 64 * hf + 32 + 8 * g);
    c.h = *reinterpret_cast<const uint2 *>(rec + 128 + 32 * hf + 8 * g);
    c.sc = *reinterpret_cast<const uint32_t *>(rec + 192 + 8 * hf + 4 * c.ch);
    c.d = reinterpret_cast<const uint16_t *>(aux)[blk];
    return c;
  }
  template <class E>
  __device__ static void decode_with(const Chunk &c, int g, E &&emit) {
    const float d = h2f(c.d);
    // l / 16 = g / 2 for both runs of this lane group
    const int sb = g >> 1;
    const float s0 = d * (float)(int8_t)((c.sc >> (8 * sb)) & 0xFFu);
    const float s1 = d * (float)(int8_t)((c.sc >> (8 * (sb + 2))) & 0xFFu);
    const float z0 = -32.0f * s0, z1 = -32.0f * s1;
    const int sh = 4 * c.ch;
    const uint32_t a[2] = {c.a.x, c.a.y}, b[2] = {c.b.x, c.b.y}, hh[2] = {c.h.x, c.h.y};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t h = hh[j] >> sh;
      const uint32_t q0 = ((a[j] >> sh) & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
      const uint32_t q1 = ((b[j] >> sh) & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
      emit(2 * j, fmaf(ub(q0, 0), s0, z0), fmaf(ub(q0, 1), s0, z0));
      emit(2 * j + 1, fmaf(ub(q0, 2), s0, z0), fmaf(ub(q0, 3), s0, z0));
      emit(4 + 2 * j, fmaf(ub(q1, 0), s1, z1), fmaf(ub(q1, 1), s1, z1));
      emit(4 + 2 * j + 1, fmaf(ub(q1, 2), s1, z1), fmaf(ub(q1, 3), s1, z1));
    }
  }
};

// Q8_0 (dequant.rs:40-47) on the split layout (int8 quants in element
// order, f16 d per 32): the chunk's two blocks are its two runs.
struct SmQ8 {
  static constexpr int CE = 64;  // elements of a row per chunk
  struct Chunk {
    uint2 a, b;
    uint32_t d;
  };
  __device__ static Chunk load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int64_t t, int g) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 64u * (uint64_t)t;
    Chunk c;
    c.a = *reinterpret_cast<const uint2 *>(w + e + 8 * g);
    c.b = *reinterpret_cast<const uint2 *>(w + e + 32 + 8 * g);
    c.d = *reinterpret_cast<const uint32_t *>(aux + 2 * (e >> 5));
    return c;
  }
  template <class E>
  __device__ static void decode_with(const Chunk &c, int, E &&emit) {
    const float d0 = h2f(c.d), d1 = h2f(c.d >> 16);
    const uint32_t a[2] = {c.a.x, c.a.y}, b[2] = {c.b.x, c.b.y};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      emit(2 * j, d0 * (float)(int8_t)(a[j] & 0xFFu), d0 * (float)(int8_t)((a[j] >> 8) & 0xFFu));
      emit(2 * j + 1, d0 * (float)(int8_t)((a[j] >> 16) & 0xFFu), d0 * (float)(int8_t)(a[j] >> 24));
      emit(4 + 2 * j, d1 * (float)(int8_t)(b[j] & 0xFFu), d1 * (float)(int8_t)((b[j] >> 8) & 0xFFu));
      emit(4 + 2 * j + 1, d1 * (float)(int8_t)((b[j] >> 16) & 0xFFu), d1 * (float)(int8_t)(b[j] >> 24));
    }
  }
};

// Q5_K (dequant_k.rs:51-80): as Q4_K, plus bit 2c / 2c + 1 of qh[j] -> 16.
struct SmQ5K {
  static constexpr int CE = 64;  // elements of a row per chunk
  struct Chunk {
    uint4 hd;
    uint2 q, h;
    int c;
  };
  __device__ static Chunk load(const uint8_t *w, const uint8_t *, int64_t row, int64_t k, int64_t t, int g) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 64u * (uint64_t)t;
    const uint8_t *bp = w + (e >> 8) * 176u;
    Chunk ch;
    ch.c = (int)((e >> 6) & 3u);
    ch.hd = *reinterpret_cast<const uint4 *>(bp);
    ch.q = *reinterpret_cast<const uint2 *>(bp + 48 + 32 * ch.c + 8 * g);
    ch.h = *reinterpret_cast<const uint2 *>(bp + 16 + 8 * g);
    return ch;
  }
  template <class E>
  __device__ static void decode_with(const Chunk &ch, int, E &&emit) {
    FmtQ4K::Piece pc;
    pc.hd = ch.hd;
    pc.c = ch.c;
    float a0, b0, a1, b1;
    FmtQ4K::scales(pc, a0, b0, a1, b1);
    const uint32_t q[2] = {ch.q.x, ch.q.y}, hh[2] = {ch.h.x, ch.h.y};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t h = hh[j] >> (2 * ch.c);
      const uint32_t lo = (q[j] & 0x0F0F0F0Fu) | ((h << 4) & 0x10101010u);
      const uint32_t hi = ((q[j] >> 4) & 0x0F0F0F0Fu) | ((h << 3) & 0x10101010u);
      emit(2 * j, fmaf(ub(lo, 0), a0, -b0), fmaf(ub(lo, 1), a0, -b0));
      emit(2 * j + 1, fmaf(ub(lo, 2), a0, -b0), fmaf(ub(lo, 3), a0, -b0));
      emit(4 + 2 * j, fmaf(ub(hi, 0), a1, -b1), fmaf(ub(hi, 1), a1, -b1));
      emit(4 + 2 * j + 1, fmaf(ub(hi, 2), a1, -b1), fmaf(ub(hi, 3), a1, -b1));
    }
  }
};

// Q4_0 / Q5_0 (dequant.rs:50-77) on their split layouts: the chunk's runs
// are its two 32-element blocks; lane group g takes elements 8g .. 8g + 7 of
// each: nibble g / 2 of quant bytes 8 (g % 2) .. + 7, and for Q5_0 bits
// 8g .. 8g + 7 of qh.
template <bool Q5>
struct SmQx0 {
  static constexpr int CE = 64;  // elements of a row per chunk
  struct Chunk {
    uint2 a, b;
    uint32_t ha, hb, da, db;
  };
  __device__ static Chunk load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int64_t t, int g) {
    const uint64_t b0 = ((uint64_t)row * (uint64_t)k + 64u * (uint64_t)t) >> 5;
    Chunk c;
    c.a = *reinterpret_cast<const uint2 *>(w + 16 * b0 + 8 * (g & 1));
    c.b = *reinterpret_cast<const uint2 *>(w + 16 * (b0 + 1) + 8 * (g & 1));
    if (Q5) {
      const uint2 ra = reinterpret_cast<const uint2 *>(aux)[b0], rb = reinterpret_cast<const uint2 *>(aux)[b0 + 1];
      c.ha = (ra.x >> (8 * g)) & 0xFFu;
      c.hb = (rb.x >> (8 * g)) & 0xFFu;
      c.da = ra.y;
      c.db = rb.y;
    } else {
      c.ha = c.hb = 0;
      c.da = reinterpret_cast<const uint16_t *>(aux)[b0];
      c.db = reinterpret_cast<const uint16_t *>(aux)[b0 + 1];
    }
    return c;
  }
  template <class E>
  __device__ static void decode_with(const Chunk &c, int g, E &&emit) {
    const float z = Q5 ? 16.0f : 8.0f;
    const int sh = 4 * (g >> 1);
    const uint32_t qa[2] = {c.a.x, c.a.y}, qb[2] = {c.b.x, c.b.y};
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float d = h2f(r ? c.db : c.da), nz = -z * d;
      const uint32_t hbits = r ? c.hb : c.ha;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        uint32_t v = ((r ? qb[j] : qa[j]) >> sh) & 0x0F0F0F0Fu;
        if (Q5) v |= spread4(hbits >> (4 * j)) << 4;
        emit(4 * r + 2 * j, fmaf(ub(v, 0), d, nz), fmaf(ub(v, 1), d, nz));
        emit(4 * r + 2 * j + 1, fmaf(ub(v, 2), d, nz), fmaf(ub(v, 3), d, nz));
      }
    }
  }
};

// The 16 weights of lane group g as bf16 pairs (o[i]: weights 2i, 2i + 1) or
// as exact f32 values (f[2i], f[2i + 1]); one fused multiply-add each, which
// is the reference's single rounding (the scale times the code is exact).
template <class C>
__device__ __forceinline__ void decode_chunk(const typename C::Chunk &c, uint32_t (&o)[8], int g) {
  C::decode_with(c, g, [&](int i, float a, float b) { o[i] = pk_bf16(a, b); });
}

template <class C>
__device__ __forceinline__ void decode_chunk_f32(const typename C::Chunk &c, float (&f)[16], int g) {
  C::decode_with(c, g, [&](int i, float a, float b) {
    f[2 * i] = a;
    f[2 * i + 1] = b;
  });
}

// x fragments of chunk t for every column tile: elements [8g, 8g + 8) and
// [32 + 8g, 32 + 8g + 8) of the chunk, 16 bytes each (LLVM vector types:
// loads into HIP's uint4 struct become memcpys that keep the fragment in
// scratch memory).
template <int MT>
struct XFrag {
  u32x4 a[MT], b[MT];
};

template <int MT>
__device__ __forceinline__ void load_x(XFrag<MT> &f, const uint16_t *const (&xr)[MT], int64_t t) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    f.a[ct] = *reinterpret_cast<const u32x4 *>(xr[ct] + 64 * t);
    f.b[ct] = *reinterpret_cast<const u32x4 *>(xr[ct] + 64 * t + 32);
  }
}

// Q4_K with half super-blocks as chunks (rows of k % 128 == 0): lane group
// g takes GEMV piece 4h + g of half h -- 16 contiguous qs bytes, the low and
// high nibbles of chunk 2h + g / 2 at positions 16 (g % 2) .. + 16 -- so
// the four lanes of a row read 64 contiguous bytes per load (against 32 in
// 8-byte pieces for the 64-element chunk), and the scales decoded once serve
// 32 weights.  Four MFMAs per column tile: low nibbles 0..7, 8..15, high
// nibbles 0..7, 8..15 of the lane's bytes, with the activations at the same
// positions (element 64 (g / 2) + 16 (g % 2) + 32 r + 8 j of the chunk).
struct SmQ4KH {
  static constexpr int CE = 128;
  typedef FmtQ4K::Piece Chunk;
  __device__ static Chunk load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int64_t t, int g) {
    // pieces are counted from the half's first element: piece g is chunk
    // 2h + g / 2, bytes 16 (g % 2) .. + 16 of its qs
    return FmtQ4K::load_e(w, aux, (uint64_t)row * (uint64_t)k + 128u * (uint64_t)t, g);
  }
  __device__ static int xoff(int g) { return 64 * (g >> 1) + 16 * (g & 1); }
};

template <int MT>
struct XFragH {
  u32x4 v[MT][4];  // [ct][low 0..7, low 8..15, high 0..7, high 8..15]
};

template <int MT>
__device__ __forceinline__ void load_xh(XFragH<MT> &f, const uint16_t *const (&xr)[MT], int64_t t) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const uint16_t *p = xr[ct] + 128 * t;
    f.v[ct][0] = *reinterpret_cast<const u32x4 *>(p);
    f.v[ct][1] = *reinterpret_cast<const u32x4 *>(p + 8);
    f.v[ct][2] = *reinterpret_cast<const u32x4 *>(p + 32);
    f.v[ct][3] = *reinterpret_cast<const u32x4 *>(p + 40);
  }
}

// ---- activations staged in LDS ----
//
// The workgroup's slice of x -- rows 0 .. m - 1, elements [e0, e0 + ke) --
// is copied into LDS once with coalesced 16-byte loads (consecutive threads
// read consecutive 16 bytes of a row) at a row stride of xstr bytes (the
// longest slice of the launch plus 16 bytes, so the 16 rows of one fragment
// read start on different bank groups).  The MFMA B fragments are then LDS
// reads at the positions the global fragment loads use.  Loaded per lane
// from global memory, each fragment instruction gathers 16-byte pieces of
// 16 rows from 32 cache lines, and that, not the decode, set the kernel's
// time (the same kernel without decode and MFMAs ran within 5% of it).

struct XSlice {
  const uint8_t *row[4];  // this lane's LDS row of each column tile, at its lane group's offset
};

template <int MT>
__device__ __forceinline__ void lds_xh(XFragH<MT> &f, const XSlice &xs, int64_t tl) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const uint8_t *p = xs.row[ct] + 256 * tl;
    f.v[ct][0] = ds_read16(p);
    f.v[ct][1] = ds_read16(p + 16);
    f.v[ct][2] = ds_read16(p + 64);
    f.v[ct][3] = ds_read16(p + 80);
  }
}

template <int MT>
__device__ __forceinline__ void lds_x(XFrag<MT> &f, const XSlice &xs, int64_t tl) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const uint8_t *p = xs.row[ct] + 128 * tl;
    f.a[ct] = ds_read16(p);
    f.b[ct] = ds_read16(p + 64);
  }
}

template <int NT, int XR>
__device__ __forceinline__ void xs_store(uint8_t *xs, const u32x4 (&v)[XR], const XStage &st, int base) {
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    int r, c;
    st.at(base + i * NT + (int)threadIdx.x, r, c);
    ds_write16(xs + r * st.xstr + 16 * c, v[i]);
  }
}

// The same pieces of f32 activations (4 a piece) split into bf16 limbs on
// their way to LDS: the hi limbs where a bf16 copy would put them (row
// stride xstr), the lo limbs lo_off bytes further.
template <int NT, int XR>
__device__ __forceinline__ void xs_store_limbs(uint8_t *xs, const u32x4 (&v)[XR], const XStage &st, int base,
                                               int lo_off) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    int r, c;
    st.at(base + i * NT + (int)threadIdx.x, r, c);
    uint32_t h0, l0, h1, l1;
    limbs2(__uint_as_float(v[i].x), __uint_as_float(v[i].y), h0, l0);
    limbs2(__uint_as_float(v[i].z), __uint_as_float(v[i].w), h1, l1);
    uint8_t *d = xs + r * st.xstr + 8 * c;
    *reinterpret_cast<lds_u32x2 *>((lds_u8 *)d) = (u32x2){h0, h1};
    *reinterpret_cast<lds_u32x2 *>((lds_u8 *)(d + lo_off)) = (u32x2){l0, l1};
  }
}

// The rest of the copy after its first round (loaded by the caller ahead of
// other loads), then the workgroup barrier.  XT = RQ_F32: the limb copy.
template <int NT, int XR, int XT = RQ_BF16>
__device__ __forceinline__ void xs_finish(uint8_t *xs, u32x4 (&v)[XR], const XStage &st, int lo_off = 0) {
  auto put = [&](int base) {
    if constexpr (XT == RQ_BF16) xs_store<NT, XR>(xs, v, st, base);
    else xs_store_limbs<NT, XR>(xs, v, st, base, lo_off);
  };
  put(0);
  for (int base = XR * NT; base < st.total; base += XR * NT) {
    xs_load<NT, XR>(v, st, base);
    put(base);
  }
  __syncthreads();
}

template <int MT>
__device__ __forceinline__ void mma_chunk_h(const FmtQ4K::Piece &pc, const XFragH<MT> &xf, f32x4 (&acc)[MT],
                                            uint32_t vm) {
  float a0, b0, a1, b1;
  FmtQ4K::scales(pc, a0, b0, a1, b1);
  const uint32_t q[4] = {pc.qv.x, pc.qv.y, pc.qv.z, pc.qv.w};
  uint32_t lo[8], hi[8];  // bf16 pairs: positions 2i, 2i + 1
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t l = q[j] & 0x0F0F0F0Fu, h = (q[j] >> 4) & 0x0F0F0F0Fu;
    lo[2 * j] = pk_bf16(fmaf(ub(l, 0), a0, -b0), fmaf(ub(l, 1), a0, -b0)) & vm;
    lo[2 * j + 1] = pk_bf16(fmaf(ub(l, 2), a0, -b0), fmaf(ub(l, 3), a0, -b0)) & vm;
    hi[2 * j] = pk_bf16(fmaf(ub(h, 0), a1, -b1), fmaf(ub(h, 1), a1, -b1)) & vm;
    hi[2 * j + 1] = pk_bf16(fmaf(ub(h, 2), a1, -b1), fmaf(ub(h, 3), a1, -b1)) & vm;
  }
  const bf16x8 f[4] = {pick(lo[0], lo[1], lo[2], lo[3]), pick(lo[4], lo[5], lo[6], lo[7]),
                       pick(hi[0], hi[1], hi[2], hi[3]), pick(hi[4], hi[5], hi[6], hi[7])};
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int ct = 0; ct < MT; ++ct)
      acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f[j], __builtin_bit_cast(bf16x8, xf.v[ct][j]), acc[ct], 0, 0,
                                                        0);
}

// Decode chunk c into A fragments and multiply with the activation
// fragments; vm (all ones or zero) masks the decoded weights, so a masked
// chunk adds exact zeros.
template <class C, int MT>
__device__ __forceinline__ void mma_chunk(const typename C::Chunk &c, const XFrag<MT> &xf, f32x4 (&acc)[MT], int g,
                                          uint32_t vm) {
  uint32_t o[8];
  decode_chunk<C>(c, o, g);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] &= vm;
  // MFMA h takes the quarter [8g + 4h, + 4) of both runs: words 2h, 2h + 1
  // of each 16-byte fragment.
  const bf16x8 f0 = pick(o[0], o[1], o[4], o[5]), f1 = pick(o[2], o[3], o[6], o[7]);
#pragma unroll
  for (int ct = 0; ct < MT; ++ct)
    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f0, pick(xf.a[ct].x, xf.a[ct].y, xf.b[ct].x, xf.b[ct].y),
                                                      acc[ct], 0, 0, 0);
#pragma unroll
  for (int ct = 0; ct < MT; ++ct)
    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f1, pick(xf.a[ct].z, xf.a[ct].w, xf.b[ct].z, xf.b[ct].w),
                                                      acc[ct], 0, 0, 0);
}

// ---- f32 activations as two bf16 limbs -----------------------------------
//
// The limb variant (XT = RQ_F32): activations split into hi + lo bf16 limbs
// (limbs2), weights decoded to their exact f32 values (the reference's
// dequantized weights) and split the same way, each product taken as
// lo*hi + hi*lo + hi*hi on the bf16 matrix cores (three MFMAs, f32 sums; the
// dropped lo*lo term and the limbs' rounding leave about 2^-16 of each
// product).  XFragL holds the hi and lo limbs at XFrag's positions; XRaw
// the 16 f32 activations of a fragment as loaded from global memory (four
// 16-byte pieces), split when used.
template <int MT>
struct XFragL {
  u32x4 a[MT], b[MT], al[MT], bl[MT];
};
template <int MT>
struct XRaw {
  u32x4 v[MT][4];
};

// xr: byte address of element 8g of chunk 0 in each column tile's row.
template <int MT>
__device__ __forceinline__ void load_xraw(XRaw<MT> &f, const uint8_t *const (&xr)[MT], int64_t t) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const uint8_t *p = xr[ct] + 256 * t;
    f.v[ct][0] = *reinterpret_cast<const u32x4 *>(p);
    f.v[ct][1] = *reinterpret_cast<const u32x4 *>(p + 16);
    f.v[ct][2] = *reinterpret_cast<const u32x4 *>(p + 128);
    f.v[ct][3] = *reinterpret_cast<const u32x4 *>(p + 144);
  }
}

// Eight f32 activations (two 16-byte pieces) as hi / lo bf16 pairs in
// element order.
__device__ __forceinline__ void split8_f32(const u32x4 &a, const u32x4 &b, u32x4 &h, u32x4 &l) {
  uint32_t hh[4], ll[4];
  limbs2(__uint_as_float(a.x), __uint_as_float(a.y), hh[0], ll[0]);
  limbs2(__uint_as_float(a.z), __uint_as_float(a.w), hh[1], ll[1]);
  limbs2(__uint_as_float(b.x), __uint_as_float(b.y), hh[2], ll[2]);
  limbs2(__uint_as_float(b.z), __uint_as_float(b.w), hh[3], ll[3]);
  h = (u32x4){hh[0], hh[1], hh[2], hh[3]};
  l = (u32x4){ll[0], ll[1], ll[2], ll[3]};
}

template <int MT>
__device__ __forceinline__ void split_raw(const XRaw<MT> &r, XFragL<MT> &f) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    split8_f32(r.v[ct][0], r.v[ct][1], f.a[ct], f.al[ct]);
    split8_f32(r.v[ct][2], r.v[ct][3], f.b[ct], f.bl[ct]);
  }
}

// Limb fragments of chunk tl of the LDS slice: hi limbs where lds_x reads,
// lo limbs lo_off bytes further.
template <int MT>
__device__ __forceinline__ void lds_xl(XFragL<MT> &f, const XSlice &xs, int64_t tl, int lo_off) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const uint8_t *p = xs.row[ct] + 128 * tl;
    f.a[ct] = ds_read16(p);
    f.b[ct] = ds_read16(p + 64);
    f.al[ct] = ds_read16(p + lo_off);
    f.bl[ct] = ds_read16(p + lo_off + 64);
  }
}

// mma_chunk on limbs: the chunk's exact weights split into hi / lo pairs
// (same order as decode_chunk's pairs), three MFMAs per column tile and
// quarter, the small cross terms first.
template <class C, int MT>
__device__ __forceinline__ void mma_chunk_limbs(const typename C::Chunk &c, const XFragL<MT> &xf, f32x4 (&acc)[MT],
                                                int g, uint32_t vm) {
  float f[16];
  decode_chunk_f32<C>(c, f, g);
  uint32_t oh[8], ol[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    limbs2(f[2 * i], f[2 * i + 1], oh[i], ol[i]);
    oh[i] &= vm;
    ol[i] &= vm;
  }
  const bf16x8 h0 = pick(oh[0], oh[1], oh[4], oh[5]), h1 = pick(oh[2], oh[3], oh[6], oh[7]);
  const bf16x8 l0 = pick(ol[0], ol[1], ol[4], ol[5]), l1 = pick(ol[2], ol[3], ol[6], ol[7]);
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const bf16x8 xh = pick(xf.a[ct].x, xf.a[ct].y, xf.b[ct].x, xf.b[ct].y);
    const bf16x8 xl = pick(xf.al[ct].x, xf.al[ct].y, xf.bl[ct].x, xf.bl[ct].y);
    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l0, xh, acc[ct], 0, 0, 0);
    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h0, xl, acc[ct], 0, 0, 0);
    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h0, xh, acc[ct], 0, 0, 0);
  }
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const bf16x8 xh = pick(xf.a[ct].z, xf.a[ct].w, xf.b[ct].z, xf.b[ct].w);
    const bf16x8 xl = pick(xf.al[ct].z, xf.al[ct].w, xf.bl[ct].z, xf.bl[ct].w);
    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l1, xh, acc[ct], 0, 0, 0);
    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h1, xl, acc[ct], 0, 0, 0);
    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h1, xh, acc[ct], 0, 0, 0);
  }
}

// Lane slot l of the (row tile rt, column tile ct) output tile: activation
// row 16 ct + l % 16, weight rows n0 + 16 rt + 4 (l / 16) + i.
template <int MT>
__device__ __forceinline__ void store_slot(const f32x4 &v, int rt, int ct, int l, int64_t m, int64_t n, int64_t n0,
                                           const Out &o) {
  const int64_t mr = 16 * ct + (l & 15);
  if (mr < m) {
    const int64_t nr0 = n0 + 16 * rt + 4 * (l >> 4);
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t nr = nr0 + i < n ? nr0 + i : n - 1;
      r[i] = o.bias ? with_bias(v[i], bias_at(o, nr), o.ytype) : v[i];
    }
    // The lane's four outputs are consecutive columns of one row: one 16-byte
    // (f32) or 8-byte store where the row holds all four and the addresses
    // are aligned (2-byte stores one by one cost ~0.7 us of a 5 us launch).
    if (nr0 + 3 < n && vec_stores_ok(o.y, n)) {
      store_four(o.y, o.ytype, mr * n + nr0, r[0], r[1], r[2], r[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (nr0 + i < n) store_one(o.y, o.ytype, mr * n + nr0 + i, r[i]);
    }
  }
}

// The NW waves' partial (16 RT) x (16 MT) tiles summed through LDS and
// stored.  16 x 16 C layout: lane l holds column (activation row) l % 16 and
// weight rows 4 (l / 16) + i of its row tile.  Thread t sums one lane slot
// of one (row tile, column tile) pair.
template <int MT, int NW, int RT = 1>
__device__ __forceinline__ void reduce_store(f32x4 (&part)[NW][RT][MT][64], const f32x4 (&acc)[RT][MT], int wave,
                                             int lane, int64_t m, int64_t n, int64_t n0, const Out &o) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < MT; ++ct) part[wave][rt][ct][lane] = acc[rt][ct];
  __syncthreads();
  for (int slot = threadIdx.x; slot < RT * MT * 64; slot += 64 * NW) {
    const int rt = slot / (MT * 64), ct = (slot >> 6) % MT, l = slot & 63;
    f32x4 v = part[0][rt][ct][l];
#pragma unroll
    for (int q = 1; q < NW; ++q) v += part[q][rt][ct][l];
    store_slot<MT>(v, rt, ct, l, m, n, n0, o);
  }
}

// Split K (split_finish): the NW waves' partial tiles summed through LDS,
// then the S workgroups of the tile meet in the workspace.
template <int MT, int NW>
__device__ __forceinline__ void reduce_split(f32x4 (&part)[NW][1][MT][64], const f32x4 (&acc)[1][MT], int wave,
                                             int lane, int64_t m, int64_t n, int64_t n0, const Out &o, int S, int s,
                                             f32x4 *__restrict__ wsp, uint32_t *__restrict__ cnt) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) part[wave][0][ct][lane] = acc[0][ct];
  __syncthreads();
  split_finish<MT * 64, 64 * NW>(
      [&](int slot) {
        const int ct = slot >> 6, l = slot & 63;
        f32x4 v = part[0][0][ct][l];
#pragma unroll
        for (int q = 1; q < NW; ++q) v += part[q][0][ct][l];
        return v;
      },
      [&](int slot, const f32x4 &v) { store_slot<MT>(v, 0, slot >> 6, slot & 63, m, n, n0, o); }, S, s, wsp, cnt);
}

// MT column tiles of 16 activation rows (M <= 16 MT) and RT row tiles of 16
// weight rows per workgroup; NW waves split the workgroup's chunks
// [lo, hi) of K, wave w taking chunks lo + w, lo + w + NW, ...  A wave issues
// the loads of B chunks (the weights of every row tile) at once, then
// decodes and multiplies them.  With XL the workgroup's slice of x is first
// copied into LDS (xs, row stride xstr; the loads of the first batch of
// weights are issued right behind the copy's loads, so both are in flight
// together) and the B fragments are LDS reads; without it each wave loads
// its fragments from global memory with the weights (slices too long for
// LDS).  An activation fragment serves RT row tiles.  The loop body has no
// conditional work: a load whose result is used under a branch is sunk into
// the branch and waited for there, and a prefetch carried from one
// iteration to the next is merged back into a load at the loop top.  Chunks
// past the end load a valid chunk again and are masked; so does a wave with
// no chunk in the slice when x is in LDS (it still joins the copy and the
// barrier); without LDS such a wave skips the work.
// XT: the activation type, RQ_BF16 or (the limb variant) RQ_F32;
// with XL and limbs the LDS slice holds the hi limbs at row stride xstr and
// the lo limbs m * xstr bytes further.
template <class C, int MT, int NW, int B, int RT, bool XL, int XT = RQ_BF16>
__device__ __forceinline__ void smallm_tiles(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                             const void *__restrict__ xv, int64_t m, const Out &o, int64_t n,
                                             int64_t k, int64_t tile, int S, int s, f32x4 *__restrict__ wsp,
                                             uint32_t *__restrict__ cnt, f32x4 (&part)[NW][RT][MT][64],
                                             uint8_t *xs, int xstr) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n0 = tile * 16 * RT;
  int64_t row[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int64_t r = n0 + 16 * rt + (lane & 15);
    row[rt] = r < n ? r : n - 1;
  }
  constexpr bool HALF = C::CE == 128;
  constexpr bool LIMBS = XT != RQ_BF16;
  static_assert(XT == RQ_BF16 || XT == RQ_F32, "bf16 activations, or f32 ones on limbs");
  static_assert(!(HALF && LIMBS), "limbs take 64-element chunks");
  constexpr int XB = LIMBS ? 4 : 2;  // bytes of an activation in memory
  // fragments as loaded in a batch: bf16 (XFrag / XFragH), raw f32 (XRaw,
  // limbs from global memory) or limbs read from LDS (XFragL)
  typedef typename std::conditional<
      LIMBS, typename std::conditional<XL, XFragL<MT>, XRaw<MT>>::type,
      typename std::conditional<HALF, XFragH<MT>, XFrag<MT>>::type>::type XF;
  const uint16_t *x = static_cast<const uint16_t *>(xv);
  const int lo_off = LIMBS ? (int)m * xstr : 0;
  const int64_t nk = k / C::CE, cps = (nk + S - 1) / S;
  const int64_t lo = s * cps, hi = lo + cps < nk ? lo + cps : nk;

  f32x4 acc[RT][MT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < MT; ++ct) acc[rt][ct] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  // Activation rows of this lane in each column tile (rows past m read row
  // m - 1; their results are not stored), at its lane group's offset.
  const int xo = HALF ? 64 * (g >> 1) + 16 * (g & 1) : 8 * g;  // elements
  const uint16_t *xr[MT];
  const uint8_t *xrb[MT];  // the same rows as byte addresses (raw f32 / f16 activations)
  XSlice xsl;
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const int64_t mr = 16 * ct + (lane & 15) < m ? 16 * ct + (lane & 15) : m - 1;
    xr[ct] = x + mr * k + xo;
    xrb[ct] = static_cast<const uint8_t *>(xv) + (mr * k + xo) * XB;
    if constexpr (XL) xsl.row[ct] = xs + mr * xstr + 2 * xo;
  }

  auto load_batch = [&](int64_t t, typename C::Chunk (&c)[B][RT], XF (&xf)[B]) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int64_t ti = t + i * NW < hi ? t + i * NW : (t < hi ? t : lo);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) c[i][rt] = C::load(w, aux, row[rt], k, ti, g);
      if constexpr (!XL) {
        if constexpr (LIMBS) load_xraw<MT>(xf[i], xrb, ti);
        else if constexpr (HALF) load_xh<MT>(xf[i], xr, ti);
        else load_x<MT>(xf[i], xr, ti);
      }
    }
  };
  auto run_batch = [&](int64_t t, const typename C::Chunk (&c)[B][RT], XF (&xf)[B]) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int64_t ti = t + i * NW < hi ? t + i * NW : (t < hi ? t : lo);
      if constexpr (XL) {
        if constexpr (LIMBS) lds_xl<MT>(xf[i], xsl, ti - lo, lo_off);
        else if constexpr (HALF) lds_xh<MT>(xf[i], xsl, ti - lo);
        else lds_x<MT>(xf[i], xsl, ti - lo);
      }
      const uint32_t vm = (!XL && i == 0) ? 0xFFFFFFFFu : opaque(t + i * NW < hi ? 0xFFFFFFFFu : 0u);
      if constexpr (LIMBS) {
        XFragL<MT> lf;
        if constexpr (XL) lf = xf[i];
        else split_raw<MT>(xf[i], lf);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) mma_chunk_limbs<C, MT>(c[i][rt], lf, acc[rt], g, vm);
      } else {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          if constexpr (HALF) mma_chunk_h<MT>(c[i][rt], xf[i], acc[rt], vm);
          else mma_chunk<C, MT>(c[i][rt], xf[i], acc[rt], g, vm);
        }
      }
    }
  };

  // (a workgroup whose slice is empty, lo >= hi, still joins the count)
  if (lo < hi) {
    const int64_t t0 = lo + wave;
    if constexpr (XL) {
      constexpr int NT = 64 * NW, XR = 8;
      const XStage st = make_stage(static_cast<const uint8_t *>(xv) + lo * C::CE * XB, XB * k, m,
                                   XB * (hi - lo) * C::CE, xstr);
      u32x4 v[XR];
      xs_load<NT, XR>(v, st, 0);
      __builtin_amdgcn_sched_barrier(0);  // the copy's loads first: its wait then skips the weights
      typename C::Chunk c0[B][RT];
      XF xf0[B];
      load_batch(t0, c0, xf0);
      // the copy's loads and the first weight loads are all in flight here
      __builtin_amdgcn_sched_barrier(0);
      xs_finish<NT, XR, XT>(xs, v, st, lo_off);
      run_batch(t0, c0, xf0);
      for (int64_t t = t0 + B * NW; t < hi; t += B * NW) {
        typename C::Chunk c[B][RT];
        XF xf[B];
        load_batch(t, c, xf);
        __builtin_amdgcn_sched_barrier(0);
        run_batch(t, c, xf);
      }
    } else {
      for (int64_t t = t0; t < hi; t += B * NW) {
        typename C::Chunk c[B][RT];
        XF xf[B];
        load_batch(t, c, xf);
        // Keep every load of the batch ahead of the first use (the scheduler
        // would otherwise trade loads in flight for registers).
        __builtin_amdgcn_sched_barrier(0);
        run_batch(t, c, xf);
      }
    }
  }

  if constexpr (RT == 1) {
    if (S > 1) {
      reduce_split<MT, NW>(part, acc, wave, lane, m, n, n0, o, S, s, wsp, cnt);
      return;
    }
  }
  reduce_store<MT, NW, RT>(part, acc, wave, lane, m, n, n0, o);
}

// One weight: workgroup b takes row tiles [(b / S) RT, + RT), K slice b % S
// (split partials at wsp + (b / S) S MT 64, counters cnt[b / S]).
template <class C, int MT, int NW, int B, int RT, bool XL, int XT = RQ_BF16>
__global__ __launch_bounds__(64 * NW) void k_smallm(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                    const void *__restrict__ x, int64_t m, const Out o,
                                                    int64_t n, int64_t k, int S, f32x4 *__restrict__ wsp,
                                                    uint32_t *__restrict__ cnt, int xstr) {
  __shared__ f32x4 part[NW][RT][MT][64];
  extern __shared__ __attribute__((aligned(16))) uint8_t xs_dyn[];
  const int bid = split_order((int)blockIdx.x, (int)gridDim.x, S);
  const int64_t tile = bid / S;
  smallm_tiles<C, MT, NW, B, RT, XL, XT>(w, aux, x, m, o, n, k, tile, S, bid % S, wsp + tile * S * MT * 64,
                                         cnt + tile, part, xs_dyn, xstr);
}

// A set of weights sharing x (pick_entry chooses this workgroup's weight;
// every entry's workgroups are a multiple of S, so b / S numbers the tiles
// of the whole set).
template <class C, int MT, int NW, int B, int RT, bool XL, int XT = RQ_BF16>
__global__ __launch_bounds__(64 * NW) void k_smallm_set(const WeightSet set, const void *__restrict__ x,
                                                        int64_t m, int64_t k, int S, f32x4 *__restrict__ wsp,
                                                        uint32_t *__restrict__ cnt, int xstr) {
  __shared__ f32x4 part[NW][RT][MT][64];
  extern __shared__ __attribute__((aligned(16))) uint8_t xs_dyn[];
  const int bid = split_order((int)blockIdx.x, (int)gridDim.x, S);
  const SetEntry e = pick_entry(set, bid);
  const int gt = bid / S;
  smallm_tiles<C, MT, NW, B, RT, XL, XT>(e.w, e.aux, x, m, e.o, e.n, k, (bid - e.g0) / S, S, bid % S,
                                         wsp + (int64_t)gt * S * MT * 64, cnt + gt, part, xs_dyn, xstr);
}

// ---- f32 / f16 activations ------------------------------------------------
//
// The reference computes in f32; for f32 (or f16) activation rows the same
// kernel runs on v_mfma_f32_16x16x4_f32 with the weights decoded to exact f32
// (the reference's dequantized values) as the A operand and the activations
// as the B operand, f32 products and accumulation.  A chunk's 16 weights of
// lane group g take 16 MFMAs of K = 4, the four lane groups supplying the
// four K slots: MFMA j pairs weight j of every lane group with the
// activation at the same position (elements 8g + j, or 32 + 8g + j - 8).
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int MT>
struct XFragF {
  f32x4v a[MT][4];  // elements 8g .. 8g + 7, then 32 + 8g .. 32 + 8g + 7
};

template <int MT, int XT>
__device__ __forceinline__ void load_xf(XFragF<MT> &f, const uint8_t *const (&xr)[MT], int64_t t) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    if constexpr (XT == RQ_F32) {
      const float *p = reinterpret_cast<const float *>(xr[ct]) + 64 * t;
      f.a[ct][0] = *reinterpret_cast<const f32x4v *>(p);
      f.a[ct][1] = *reinterpret_cast<const f32x4v *>(p + 4);
      f.a[ct][2] = *reinterpret_cast<const f32x4v *>(p + 32);
      f.a[ct][3] = *reinterpret_cast<const f32x4v *>(p + 36);
    } else {
      typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
      const _Float16 *p = reinterpret_cast<const _Float16 *>(xr[ct]) + 64 * t;
      const f16x8 lo = *reinterpret_cast<const f16x8 *>(p), hi = *reinterpret_cast<const f16x8 *>(p + 32);
      f.a[ct][0] = (f32x4v){(float)lo[0], (float)lo[1], (float)lo[2], (float)lo[3]};
      f.a[ct][1] = (f32x4v){(float)lo[4], (float)lo[5], (float)lo[6], (float)lo[7]};
      f.a[ct][2] = (f32x4v){(float)hi[0], (float)hi[1], (float)hi[2], (float)hi[3]};
      f.a[ct][3] = (f32x4v){(float)hi[4], (float)hi[5], (float)hi[6], (float)hi[7]};
    }
  }
}

template <class C, int MT>
__device__ __forceinline__ void mma_chunk_f32(const typename C::Chunk &c, const XFragF<MT> &xf, f32x4 (&acc)[MT],
                                              int g, uint32_t vm) {
  float f[16];
  decode_chunk_f32<C>(c, f, g);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float wj = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, f[j]) & vm);
#pragma unroll
    for (int ct = 0; ct < MT; ++ct)
      acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(wj, xf.a[ct][j >> 2][j & 3], acc[ct], 0, 0, 0);
  }
}

// Split K (S > 1): workgroup b takes row tile b / S and the (b % S)-th of
// S equal runs of chunks, its partial tile summed as in reduce_split.
template <class C, int MT, int NW, int B, int XT>
__global__ __launch_bounds__(64 * NW) void k_smallm_f32(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                        const uint8_t *__restrict__ x, int64_t m_all, const Out o_all,
                                                        int64_t n, int64_t k, int S, f32x4 *__restrict__ wsp,
                                                        uint32_t *__restrict__ cnt) {
  __shared__ f32x4 part[NW][1][MT][64];
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bid = split_order((int)blockIdx.x, (int)gridDim.x, S);
  const int64_t tile = bid / S;
  const int sl = bid % S;
  // Slice blockIdx.y: activation rows [16 MT y, 16 MT (y + 1)) of m_all, its
  // own outputs, partials and tile counters.
  const int64_t r0 = (int64_t)blockIdx.y * 16 * MT;
  const int64_t m = m_all - r0 < 16 * MT ? m_all - r0 : 16 * MT;
  const int64_t stile = (int64_t)blockIdx.y * (gridDim.x / S) + tile;
  Out o = o_all;
  o.y = static_cast<uint8_t *>(o_all.y) + r0 * n * (o_all.ytype == RQ_F32 ? 4 : 2);
  const int64_t n0 = tile * 16;
  const int64_t row = n0 + (lane & 15) < n ? n0 + (lane & 15) : n - 1;
  const int64_t nka = k / 64, cps = (nka + S - 1) / S;
  const int64_t lo = sl * cps, nk = lo + cps < nka ? lo + cps : nka;
  constexpr int XB = XT == RQ_F32 ? 4 : 2;  // bytes per activation

  const uint8_t *xr[MT];
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const int64_t mr = 16 * ct + (lane & 15);
    xr[ct] = x + ((r0 + (mr < m ? mr : m - 1)) * k + 8 * g) * XB;
  }

  f32x4 acc[1][MT];
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) acc[0][ct] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  for (int64_t t = lo + wave; t < nk; t += B * NW) {
    typename C::Chunk c[B];
    XFragF<MT> xf[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int64_t ti = t + i * NW < nk ? t + i * NW : t;
      c[i] = C::load(w, aux, row, k, ti, g);
      load_xf<MT, XT>(xf[i], xr, ti);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const uint32_t vm = i == 0 ? 0xFFFFFFFFu : opaque(t + i * NW < nk ? 0xFFFFFFFFu : 0u);
      mma_chunk_f32<C, MT>(c[i], xf[i], acc[0], g, vm);
    }
  }

  if (S > 1) {
    reduce_split<MT, NW>(part, acc, wave, lane, m, n, n0, o, S, sl, wsp + stile * S * MT * 64, cnt + stile);
    return;
  }
  reduce_store<MT, NW>(part, acc, wave, lane, m, n, n0, o);
}

// Workgroups along K for the f32 kernel, measured on the Qwen2-0.5B layer
// (Q4_K, HIP graphs over distinct weights): long rows (32 or more 64-element
// chunks) on few row tiles split four ways (down 896 x 4864: M = 4 12.6 ->
// 9.0 us, M = 16 14.8 -> 9.9, M = 64 38.5 -> 15.5); above 32 activation rows
// short rows split too, four ways on few tiles and two on up to 511 (M = 64:
// o 896 x 896 10.8 -> 7.5, k / v 128 x 896 10.6 -> 6.6, gate 4864 x 896 18.1 ->
// 15.3); at 32 rows or fewer they lose (o at M = 16 5.3 -> 6.5 in two).
inline int f32_splits(int64_t tiles, int64_t nk, int64_t m) {
  if (tiles > WsLease::kCounters) return 1;
  int S = 1;
  if (nk >= 32 && tiles < 128) {
    while (S < 4 && tiles * S * 2 <= 512) S *= 2;
  } else if (m > 32) {
    S = tiles < 128 ? 4 : (tiles < 512 ? 2 : 1);
  }
  while (S > 1 && nk < S) S /= 2;
  return S;
}

template <class C, int MT, int XT>
int run_mt_f32(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease *ws,
               int64_t slices = 1) {
  constexpr int B = MT == 1 ? 4 : (MT == 2 ? 2 : 1);
  const int64_t tiles = (wt->n + 15) / 16, nk = wt->k / 64;
  // K split over S workgroups for few row tiles with long rows (the
  // partials and counters in the workspace; without them, one workgroup a
  // tile).  Slices of 16 MT activation rows run side by side (grid y), each
  // with its own row tiles, so the split is planned on all of them.
  int S = f32_splits(tiles * slices, nk, m / slices);
  f32x4 *wsp = nullptr;
  uint32_t *cnt = nullptr;
  if (S > 1) {
    int rc = RQ_OK;
    cnt = ws ? ws->counters() : nullptr;
    wsp = cnt ? static_cast<f32x4 *>(ws->get((size_t)slices * tiles * S * MT * 64 * sizeof(f32x4), &rc, true))
              : nullptr;
    if (!wsp) S = 1;
  }
  const dim3 grid((unsigned)(tiles * S), (unsigned)slices);
  const int64_t ck = (nk + S - 1) / S;  // chunks a workgroup
  const uint8_t *aux = wt->data + wt->aux_off;
  // One and two column tiles with more than one batch a wave: sixteen waves
  // (measured on the 0.5B layer: 896 x 4864 at M = 16 16.9 -> 14.5 us, at
  // M = 32 24.6 -> 20.8; four column tiles and the bf16 kernel were slower).
  // One column tile and at most one batch a wave (the 896-long rows):
  // sixteen waves of one chunk, so each wave's MFMA chain is a quarter as
  // long (verify with f32 activations on the 0.5B layer, 7 launches: M = 4
  // 206 -> 214, M = 8 209 -> 219, M = 16 204 -> 217 GB/s; the same for two
  // column tiles changed nothing, eight waves for four lost 4%).
  if (MT <= 2 && ck > 4 * B)
    hipLaunchKernelGGL((k_smallm_f32<C, MT, 16, (MT == 1 ? 2 : 1), XT>), grid, dim3(1024), 0, s, wt->data, aux,
                       static_cast<const uint8_t *>(x), m, o, wt->n, wt->k, S, wsp, cnt);
  else if (MT == 1)
    hipLaunchKernelGGL((k_smallm_f32<C, 1, 16, 1, XT>), grid, dim3(1024), 0, s, wt->data, aux,
                       static_cast<const uint8_t *>(x), m, o, wt->n, wt->k, S, wsp, cnt);
  else
    hipLaunchKernelGGL((k_smallm_f32<C, MT, 4, B, XT>), grid, dim3(256), 0, s, wt->data, aux,
                       static_cast<const uint8_t *>(x), m, o, wt->n, wt->k, S, wsp, cnt);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "small-M launch failed");
}

template <class C, int XT>
int run_f32(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease *ws) {
  // Above 16 rows: slices of 16 side by side in one launch rather than two
  // or four column tiles a workgroup (verify with f32 activations on the
  // 0.5B layer, 7 launches: M = 32 179 -> 198, M = 64 184 -> 218 GB/s; two
  // slices of 32 rows at M = 64: 181).
  if (m <= 16) return run_mt_f32<C, 1, XT>(wt, x, m, o, s, ws);
  return run_mt_f32<C, 1, XT>(wt, x, m, o, s, ws, (m + 15) / 16);
}

// m = 64 * slices activation rows as slices of 64 in one launch.
template <int XT>
int dispatch_f32_slices(const rq_weight *wt, const void *x, int64_t slices, const Out &o, hipStream_t s,
                        WsLease *ws) {
  const int64_t m = 64 * slices;
  switch (wt->qtype) {
    case RQ_Q4_K: return run_mt_f32<SmQ4K, 4, XT>(wt, x, m, o, s, ws, slices);
    case RQ_Q6_K: return run_mt_f32<SmQ6K, 4, XT>(wt, x, m, o, s, ws, slices);
    case RQ_Q8_0: return run_mt_f32<SmQ8, 4, XT>(wt, x, m, o, s, ws, slices);
    case RQ_Q5_K: return run_mt_f32<SmQ5K, 4, XT>(wt, x, m, o, s, ws, slices);
    case RQ_Q4_0: return run_mt_f32<SmQx0<false>, 4, XT>(wt, x, m, o, s, ws, slices);
    case RQ_Q5_0: return run_mt_f32<SmQx0<true>, 4, XT>(wt, x, m, o, s, ws, slices);
    default: return RQ_E_UNSUPPORTED;
  }
}

template <int XT>
int dispatch_f32(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease *ws) {
  switch (wt->qtype) {
    case RQ_Q4_K: return run_f32<SmQ4K, XT>(wt, x, m, o, s, ws);
    case RQ_Q6_K: return run_f32<SmQ6K, XT>(wt, x, m, o, s, ws);
    case RQ_Q8_0: return run_f32<SmQ8, XT>(wt, x, m, o, s, ws);
    case RQ_Q5_K: return run_f32<SmQ5K, XT>(wt, x, m, o, s, ws);
    case RQ_Q4_0: return run_f32<SmQx0<false>, XT>(wt, x, m, o, s, ws);
    case RQ_Q5_0: return run_f32<SmQx0<true>, XT>(wt, x, m, o, s, ws);
    default: return RQ_E_UNSUPPORTED;
  }
}

// Launch plan: S workgroups per row tile splitting K, NW waves a workgroup,
// batches of B chunks, RT row tiles a workgroup.
//  * Split K when there are few row tiles (k / v / q / o / down of a small
//    layer: 8 - 72 tiles on 256 CUs) and at least 16 activation rows: S up
//    to 4, at most 512 workgroups, at least two chunks a workgroup.  Timed
//    in HIP graphs on the 0.5B layer (7 launches / rq_linear_multi): M = 64
//    160 -> 195 / 223 -> 287 GB/s, M = 16 238 -> 240 / 343 -> 354, but M = 4
//    and 8 lose 6-10% (265 -> 242 at M = 4), so smaller M does not split.
//    Four slices beat eight on 896 x 4864 (M = 16 8.71 -> 7.98 us, M = 64
//    11.25 -> 10.12; two: 8.93 / 13.78).
//  * Waves and batch so that one batch of every wave covers the
//    workgroup's chunks (each batch is a dependent round trip to memory),
//    within the registers: a batch holds B chunks of every row tile and B
//    activation fragments of 16 MT bytes a lane; 16 waves leave 128 VGPRs
//    a lane.
//  * Row tiles: with four waves and no split, as many as keep at least 256
//    workgroups (each workgroup reads its slice of x once).
struct SmPlan {
  int s, nw, b, rt;
};
// Measured on the Qwen2-0.5B layer (Q4_K, bf16, HIP graphs over distinct
// weights): up to 8 rows, chunks of 8 or fewer in batches of one (o 896 x 896
// at M = 8 3.30 -> 3.18 us, gate/up set 5.55 -> 5.04, M = 4 alike); at up to
// 16 rows a K split of two, not four, with eight waves of single chunks
// (down 896 x 4864: M = 16 7.27 -> 6.40 us, M = 8 7.51 -> 5.81, M = 4 7.03
// -> 5.67).
template <int MT>
SmPlan smallm_plan(int64_t tiles, int64_t nk, bool can_split, int64_t m) {
  int S = 1;
  const int smax = MT == 1 ? 2 : 4;
  if (can_split && tiles < 128)
    while (S < smax && tiles * S * 2 <= 512 && nk >= 4 * S) S *= 2;
  const int64_t c = (nk + S - 1) / S;
  SmPlan p{S, 4, 1, 1};
  if (MT == 4) {
    if (c <= 4) p = {S, 4, 1, 1};
    else if (c <= 8) p = {S, 8, 1, 1};
    else p = {S, 16, 1, 1};
  } else {
    if (c <= 4) p = {S, 4, 1, 1};
    else if (c <= 8) p = m <= 8 ? SmPlan{S, 4, 1, 1} : SmPlan{S, 4, 2, 1};
    else if (MT == 1 && S > 1 && c <= 32) p = {S, 8, 1, 1};
    else if (c <= 16) p = {S, 4, 4, 1};
    else if (c <= 32) p = {S, 8, 4, 1};
    else p = {S, 16, MT == 1 ? 5 : 2, 1};
  }
  const bool rt_ok = S == 1 && p.nw == 4 && p.b == (MT == 4 ? 1 : 4);
  if (rt_ok) p.rt = tiles >= 4 * 256 ? 4 : (tiles >= 2 * 256 ? 2 : 1);
  return p;
}

template <class C, int MT, int NW, int B, int RT, bool XL, int XT = RQ_BF16>
int launch_mt(const rq_weight *const *w, int count, bool set, const void *x, int64_t m, const Out *o, int S,
              f32x4 *wsp, uint32_t *cnt, hipStream_t s, int xstr, size_t xbytes) {
  // the reduction buffer and the activation slice share the CU's 160 KB
  if (XL && (size_t)NW * RT * MT * 64 * sizeof(f32x4) + xbytes > 160 * 1024) return RQ_E_UNSUPPORTED;
  if (!set) {
    const rq_weight *wt = w[0];
    const int64_t tiles = ((wt->n + 15) / 16 + RT - 1) / RT;
    if (!lds_allow<&k_smallm<C, MT, NW, B, RT, XL, XT>>(xbytes)) return RQ_E_UNSUPPORTED;
    hipLaunchKernelGGL((k_smallm<C, MT, NW, B, RT, XL, XT>), dim3((unsigned)(tiles * S)), dim3(64 * NW), xbytes, s,
                       wt->data, wt->data + wt->aux_off, x, m, o[0], wt->n, wt->k, S, wsp, cnt, xstr);
  } else {
    WeightSet ws;
    int64_t total = 0;
    const int rc = fill_set(ws, w, count, o, [&](const rq_weight *wj) { return ((wj->n + 15) / 16 + RT - 1) / RT * S; },
                            &total);
    if (rc) return rc;
    if (!lds_allow<&k_smallm_set<C, MT, NW, B, RT, XL, XT>>(xbytes)) return RQ_E_UNSUPPORTED;
    hipLaunchKernelGGL((k_smallm_set<C, MT, NW, B, RT, XL, XT>), dim3((unsigned)total), dim3(64 * NW), xbytes, s, ws,
                       x, m, w[0]->k, S, wsp, cnt, xstr);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "small-M launch failed");
}

// Chunks a wave loads per batch: the planned B, fewer where the fragments
// are large (half-block chunks; limb fragments hold twice the activation
// registers of bf16 ones).
template <class C, int MT, int NW, int B, int XT = RQ_BF16>
constexpr int sm_batch() {
  if constexpr (XT != RQ_BF16) {
    constexpr int cap = MT == 1 ? 2 : 1;
    return B < cap ? B : cap;
  }
  if constexpr (C::CE == 128) {
    constexpr int cap = MT == 1 ? (NW == 16 ? 3 : 4) : (MT == 2 ? (NW == 16 ? 1 : 2) : 1);
    return B < cap ? B : cap;
  }
  return B;
}

// Plans and launches one weight or a set (every weight of format C, one k);
// XT: bf16 activations, or f32 ones on the limb variant (the LDS slice then
// holds a hi and a lo copy).
template <class C, int MT, int XT = RQ_BF16>
int run_plan(const rq_weight *const *w, int count, bool set, const void *x, int64_t m, const Out *o, hipStream_t s,
             WsLease *ws) {
  int64_t tiles = 0;
  for (int j = 0; j < count; ++j) tiles += (w[j]->n + 15) / 16;
  // No K split for rows of up to 1024 elements at m <= 32: the slice copy
  // makes one unsplit batch cheap and the split's last-workgroup sum costs
  // two round trips (896 x 896 at M = 16 4.72 -> 3.98 us, 128 x 896 3.85 ->
  // 3.46, M = 32 4.91 -> 4.52; at M = 64 even, 5.55 vs 5.61).
  // Nor at m <= 64 (o 896 x 896 at M = 64 5.39 -> 5.15 us, q/k/v set 5.66 ->
  // 5.30, one eight-wave workgroup a tile); below 16 rows only long rows
  // (more than 32 chunks) split.
  const bool split_ok = !(w[0]->k <= 1024 && m <= 64);
  const int64_t nkc = w[0]->k / C::CE;
  SmPlan p = smallm_plan<MT>(
      tiles, nkc, split_ok && ws != nullptr && tiles <= WsLease::kCounters && (m >= 16 || nkc > 32), m);
  f32x4 *wsp = nullptr;
  uint32_t *cnt = nullptr;
  if (p.s > 1) {
    int rc = RQ_OK;
    cnt = ws->counters();
    wsp = cnt ? static_cast<f32x4 *>(ws->get((size_t)tiles * p.s * MT * 64 * sizeof(f32x4), &rc, true)) : nullptr;
    if (!wsp) p = smallm_plan<MT>(tiles, nkc, false, m);  // no scratch: one workgroup per tile
  }
  // (a half-block chunk holds twice the weights and activations of a
  // 64-element chunk: smaller batches where registers are short)
  // The activation slice in LDS (the longest slice of the launch, m rows)
  // for 16 or more activation rows in slices of up to 2048 elements, where it fits
  // beside the reduction buffer.  Timed in HIP graphs (Q4_K, bf16, distinct
  // weights): 4864 x 896 M = 16 5.41 -> 4.84 us, M = 64 10.86 -> 9.79,
  // 896 x 896 M = 64 6.32 -> 5.61; slower at M = 4 / 8 (the fragments are
  // few) and on 896 x 4864 at M = 64 (eight K slices of 83 KB each leave one
  // workgroup per CU: 11.3 -> 14.8 us).
  const int64_t cps = (w[0]->k / C::CE + p.s - 1) / p.s;
  const int xstr = (int)(cps * C::CE * 2 + 16);
  const size_t xbytes = (size_t)m * (size_t)xstr * (XT == RQ_BF16 ? 1 : 2);
  // A copy above 80 KB leaves one workgroup per CU: only where the grid is
  // about one round (the 4864 x 896 gate at M = 64, 304 workgroups, gains;
  // gate and up in one launch, 608, lose: 14.0 -> 14.6 us).
  const size_t part = (size_t)(MT == 4 ? 8 : 4) * MT * 64 * sizeof(f32x4);
  const int64_t per_cu = (int64_t)((160 * 1024) / (part + xbytes));
  // (The slice, not the row, decides: the down projection 896 x 4864 in four
  // K slices of 1280 at M = 16 copies 41 KB, 7.80 -> 7.19 us; M = 32
  // 8.25 -> 8.13; from M = 48 the copy no longer fits.)
  const bool xl = m >= 16 && cps * C::CE <= 2048 && xbytes <= kSmXsMax && tiles * p.s <= 320 * (per_cu > 0 ? per_cu : 1);
#define RQ_SM(NW, B, RT)                                                                                     \
  {                                                                                                          \
    if (xl) {                                                                                                \
      const int rc_ = launch_mt<C, MT, NW, sm_batch<C, MT, NW, B, XT>(), RT, true, XT>(                      \
          w, count, set, x, m, o, p.s, wsp, cnt, s, xstr, xbytes);                                           \
      if (rc_ != RQ_E_UNSUPPORTED) return rc_;                                                               \
    }                                                                                                        \
    return launch_mt<C, MT, NW, sm_batch<C, MT, NW, B, XT>(), RT, false, XT>(w, count, set, x, m, o, p.s, wsp, \
                                                                             cnt, s, 0, 0);                  \
  }
  if constexpr (MT == 4) {
    if (p.nw == 16) RQ_SM(16, 1, 1);
    if (p.nw == 8) RQ_SM(8, 1, 1);
    if (p.rt == 4) RQ_SM(4, 1, 4);
    if (p.rt == 2) RQ_SM(4, 1, 2);
    RQ_SM(4, 1, 1);
  } else {
    if (p.nw == 16) RQ_SM(16, (MT == 1 ? 5 : 2), 1);
    if constexpr (MT == 1) {
      if (p.nw == 8 && p.b == 1) RQ_SM(8, 1, 1);
    }
    if (p.nw == 8) RQ_SM(8, 4, 1);
    if (p.b == 4) {
      if (p.rt == 4) RQ_SM(4, 4, 4);
      if (p.rt == 2) RQ_SM(4, 4, 2);
      RQ_SM(4, 4, 1);
    }
    if (p.b == 2) RQ_SM(4, 2, 1);
    RQ_SM(4, 1, 1);
  }
#undef RQ_SM
}

template <class C, int XT = RQ_BF16>
int run(const rq_weight *const *w, int count, bool set, const void *x, int64_t m, const Out *o, hipStream_t s,
        WsLease *ws) {
  if (m <= 16) return run_plan<C, 1, XT>(w, count, set, x, m, o, s, ws);
  if (m <= 32) return run_plan<C, 2, XT>(w, count, set, x, m, o, s, ws);
  return run_plan<C, 4, XT>(w, count, set, x, m, o, s, ws);
}

// f32 activations on the limb variant (64-element chunks for every format).
template <int XT>
int dispatch_limbs(const rq_weight *const *w, int count, bool set, const void *x, int64_t m, const Out *o,
                   hipStream_t s, WsLease *ws) {
  switch (w[0]->qtype) {
    case RQ_Q4_K: return run<SmQ4K, XT>(w, count, set, x, m, o, s, ws);
    case RQ_Q6_K: return run<SmQ6K, XT>(w, count, set, x, m, o, s, ws);
    case RQ_Q8_0: return run<SmQ8, XT>(w, count, set, x, m, o, s, ws);
    case RQ_Q5_K: return run<SmQ5K, XT>(w, count, set, x, m, o, s, ws);
    case RQ_Q4_0: return run<SmQx0<false>, XT>(w, count, set, x, m, o, s, ws);
    case RQ_Q5_0: return run<SmQx0<true>, XT>(w, count, set, x, m, o, s, ws);
    default: return RQ_E_UNSUPPORTED;
  }
}

int dispatch_bf16(const rq_weight *const *w, int count, bool set, const void *x, int64_t m, const Out *o,
                  hipStream_t s, WsLease *ws) {
  switch (w[0]->qtype) {
    case RQ_Q4_K:
      // half super-blocks as chunks where rows hold whole halves
      if (w[0]->k % 128 == 0) return run<SmQ4KH>(w, count, set, x, m, o, s, ws);
      return run<SmQ4K>(w, count, set, x, m, o, s, ws);
    case RQ_Q6_K: return run<SmQ6K>(w, count, set, x, m, o, s, ws);
    case RQ_Q8_0: return run<SmQ8>(w, count, set, x, m, o, s, ws);
    case RQ_Q5_K: return run<SmQ5K>(w, count, set, x, m, o, s, ws);
    case RQ_Q4_0: return run<SmQx0<false>>(w, count, set, x, m, o, s, ws);
    case RQ_Q5_0: return run<SmQx0<true>>(w, count, set, x, m, o, s, ws);
    default: return RQ_E_UNSUPPORTED;
  }
}

}  // namespace

// f32 / f16 activations, 2 <= m <= 64, k % 64 == 0, 16-byte aligned x
// (dispatched from m = 4, and at m = 2..3 for rows the VALU layouts do not
// take).
// One weight runs on the f32 matrix cores (exact weights, 16 MFMAs of K = 4
// a chunk): for a lone weight it beats the two-limb variant, whose weight
// split costs about four VALU instructions a weight (Qwen2-0.5B layer at
// M = 16, rocprof medians: gate 7.96 vs 8.48 us, o 5.75 vs 6.12, down 10.5 vs
// 11.5; 7 launches a layer M = 64: 218 vs 153 GB/s).
int launch_linear_smallm_f32(const rq_weight *wt, const void *x, int xtype, int64_t m, const Out &o,
                             hipStream_t s, WsLease *ws) {
  if (m < 2 || m > 64 || wt->k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  if (xtype == RQ_F32) return dispatch_f32<RQ_F32>(wt, x, m, o, s, ws);
  if (xtype == RQ_F16) return dispatch_f32<RQ_F16>(wt, x, m, o, s, ws);
  return RQ_E_UNSUPPORTED;
}

int launch_linear_smallm_f32_slices(const rq_weight *wt, const void *x, int xtype, int64_t slices, const Out &o,
                                    hipStream_t s, WsLease *ws) {
  if (slices < 1 || slices > 65535 || wt->k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0)
    return RQ_E_UNSUPPORTED;
  if (xtype == RQ_F32) return dispatch_f32_slices<RQ_F32>(wt, x, slices, o, s, ws);
  if (xtype == RQ_F16) return dispatch_f32_slices<RQ_F16>(wt, x, slices, o, s, ws);
  return RQ_E_UNSUPPORTED;
}

// bf16 (or, on the limb variant, f32) activations, 2 <= m <= 64, k % 64 ==
// 0, 16-byte aligned x, weights of one format and k.  A set of f32 weights
// takes the limb variant: one launch for the set beats the f32 kernel's one
// launch a weight (Qwen2-0.5B layer, q/k/v and gate/up as sets, 4 launches a
// layer: M = 4 / 16 / 64 292 / 291 / 224 GB/s against 207 / 211 / 218 with 7
// launches on the f32 kernel).
int launch_linear_smallm_set(const rq_weight *const *w, int count, const void *x, int xtype, int64_t m,
                             const Out *o, hipStream_t s, WsLease *ws) {
  const int64_t k = w[0]->k;
  if (m < 2 || m > 64 || k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  for (int j = 1; j < count; ++j)
    if (w[j]->qtype != w[0]->qtype || w[j]->k != k) return RQ_E_UNSUPPORTED;
  if (xtype == RQ_F32) return dispatch_limbs<RQ_F32>(w, count, true, x, m, o, s, ws);
  if (xtype != RQ_BF16) return RQ_E_UNSUPPORTED;
  return dispatch_bf16(w, count, true, x, m, o, s, ws);
}

// bf16 activations, 2 <= m <= 64, k % 64 == 0, 16-byte aligned x.
int launch_linear_smallm(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease *ws) {
  if (m < 2 || m > 64 || wt->k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  return dispatch_bf16(&wt, 1, false, x, m, &o, s, ws);
}

}  // namespace rq
