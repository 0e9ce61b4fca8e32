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

#include "rq_epilogue.h"
#include "rq_formats.h"
#include "rq_internal.h"

namespace rq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The 16 weights of lane group g in chunk t of `row` as bf16 pairs:
// o[0..3] = chunk elements 8g .. 8g+7, o[4..7] = 32 + 8g .. 32 + 8g + 7.

// Q4_K (dequant_k.rs:19-44): elements j and 32 + j of chunk c are the low
// and high nibbles of qs[32c + j].
struct SmQ4K {
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

__device__ __forceinline__ bf16x8 pick(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1) {
  return __builtin_bit_cast(bf16x8, (uint4){a0, a1, b0, b1});
}

// x fragments of chunk t for every column tile: elements [8g, 8g + 8) and
// [32 + 8g, 32 + 8g + 8) of the chunk, 16 bytes each.
// (LLVM vector types: loads into HIP's uint4 struct become memcpys that
// keep the fragment in scratch memory.)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
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

// The NW waves' partial 16 x (16 MT) tiles summed through LDS and stored.
// 16 x 16 C layout: lane l holds column (activation row) l % 16 and weight
// rows 4 (l / 16) + i.  Thread t sums one lane slot of one column tile.
template <int MT, int NW>
__device__ __forceinline__ void reduce_store(f32x4 (&part)[NW][MT][64], const f32x4 (&acc)[MT], int wave, int lane,
                                             int64_t m, int64_t n, int64_t n0, const Out &o) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) part[wave][ct][lane] = acc[ct];
  __syncthreads();
  for (int slot = threadIdx.x; slot < MT * 64; slot += 64 * NW) {
    const int ct = slot >> 6, l = slot & 63;
    f32x4 v = part[0][ct][l];
#pragma unroll
    for (int q = 1; q < NW; ++q) v += part[q][ct][l];
    const int64_t mr = 16 * ct + (l & 15);
    if (mr < m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t nr = n0 + 4 * (l >> 4) + i;
        if (nr < n) store_one(o.y, o.ytype, mr * n + nr, o.bias ? with_bias(v[i], bias_at(o, nr), o.ytype) : v[i]);
      }
    }
  }
}

// MT column tiles of 16 activation rows (M <= 16 MT); NW waves split K,
// wave w taking chunks w, w + NW, ...  A wave issues the loads of B chunks
// (weights and activations) at once, then decodes and multiplies them.
// The loop body has no conditional work: a load whose result is used under
// a branch is sunk into the branch and waited for there, and a prefetch
// carried from one iteration to the next is merged back into a load at the
// loop top.  Chunks past the end load a valid chunk again and are masked.
template <class C, int MT, int NW, int B>
__global__ __launch_bounds__(64 * NW) void k_smallm(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                    const uint16_t *__restrict__ x, int64_t m, const Out o,
                                                    int64_t n, int64_t k) {
  __shared__ f32x4 part[NW][MT][64];
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t row = n0 + (lane & 15) < n ? n0 + (lane & 15) : n - 1;
  const int64_t nk = k / 64;

  // Activation rows of this lane in each column tile (rows past m read row
  // m - 1; their results are not stored).
  const uint16_t *xr[MT];
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const int64_t mr = 16 * ct + (lane & 15);
    xr[ct] = x + (mr < m ? mr : m - 1) * k + 8 * g;
  }

  f32x4 acc[MT];
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) acc[ct] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  for (int64_t t = wave; t < nk; t += B * NW) {
    typename C::Chunk c[B];
    XFrag<MT> xf[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int64_t ti = t + i * NW < nk ? t + i * NW : t;
      c[i] = C::load(w, aux, row, k, ti, g);
      load_x<MT>(xf[i], xr, ti);
    }
    // Keep every load of the batch ahead of the first use (the scheduler
    // would otherwise trade loads in flight for registers).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const uint32_t vm = i == 0 ? 0xFFFFFFFFu : opaque(t + i * NW < nk ? 0xFFFFFFFFu : 0u);
      mma_chunk<C, MT>(c[i], xf[i], acc, g, vm);
    }
  }

  reduce_store<MT, NW>(part, acc, wave, lane, m, n, n0, o);
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

template <class C, int MT, int NW, int B, int XT>
__global__ __launch_bounds__(64 * NW) void k_smallm_f32(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                        const uint8_t *__restrict__ x, int64_t m, const Out o,
                                                        int64_t n, int64_t k) {
  __shared__ f32x4 part[NW][MT][64];
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t row = n0 + (lane & 15) < n ? n0 + (lane & 15) : n - 1;
  const int64_t nk = k / 64;
  constexpr int XB = XT == RQ_F32 ? 4 : 2;  // bytes per activation

  const uint8_t *xr[MT];
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const int64_t mr = 16 * ct + (lane & 15);
    xr[ct] = x + ((mr < m ? mr : m - 1) * k + 8 * g) * XB;
  }

  f32x4 acc[MT];
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) acc[ct] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  for (int64_t t = wave; t < nk; t += B * NW) {
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
      mma_chunk_f32<C, MT>(c[i], xf[i], acc, g, vm);
    }
  }

  reduce_store<MT, NW>(part, acc, wave, lane, m, n, n0, o);
}

template <class C, int MT, int XT>
int run_mt_f32(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s) {
  constexpr int B = MT == 1 ? 4 : (MT == 2 ? 2 : 1);
  const dim3 grid((unsigned)((wt->n + 15) / 16));
  const uint8_t *aux = wt->data + wt->aux_off;
  // One and two column tiles with more than one batch a wave: sixteen waves
  // (measured on the 0.5B layer: 896 x 4864 at M = 16 16.9 -> 14.5 us, at
  // M = 32 24.6 -> 20.8; four column tiles and the bf16 kernel were slower).
  if (MT <= 2 && wt->k / 64 > 4 * B)
    hipLaunchKernelGGL((k_smallm_f32<C, MT, 16, (MT == 1 ? 2 : 1), XT>), grid, dim3(1024), 0, s, wt->data, aux,
                       static_cast<const uint8_t *>(x), m, o, wt->n, wt->k);
  else
    hipLaunchKernelGGL((k_smallm_f32<C, MT, 4, B, XT>), grid, dim3(256), 0, s, wt->data, aux,
                       static_cast<const uint8_t *>(x), m, o, wt->n, wt->k);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "small-M launch failed");
}

template <class C, int XT>
int run_f32(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s) {
  if (m <= 16) return run_mt_f32<C, 1, XT>(wt, x, m, o, s);
  if (m <= 32) return run_mt_f32<C, 2, XT>(wt, x, m, o, s);
  return run_mt_f32<C, 4, XT>(wt, x, m, o, s);
}

template <int XT>
int dispatch_f32(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s) {
  switch (wt->qtype) {
    case RQ_Q4_K: return run_f32<SmQ4K, XT>(wt, x, m, o, s);
    case RQ_Q6_K: return run_f32<SmQ6K, XT>(wt, x, m, o, s);
    case RQ_Q8_0: return run_f32<SmQ8, XT>(wt, x, m, o, s);
    case RQ_Q5_K: return run_f32<SmQ5K, XT>(wt, x, m, o, s);
    case RQ_Q4_0: return run_f32<SmQx0<false>, XT>(wt, x, m, o, s);
    case RQ_Q5_0: return run_f32<SmQx0<true>, XT>(wt, x, m, o, s);
    default: return RQ_E_UNSUPPORTED;
  }
}

// Four waves per workgroup.  Batch sizes as measured on the 0.5B-model
// layer shapes: 4 chunks for one and two column tiles; one for four (their
// registers leave no room for a batch, and the kernel is decode-bound).
// More waves per workgroup or deeper batches were slower: the masked
// chunks of a partly filled batch cost as much decode as real ones.
template <class C, int MT>
int run_mt(const rq_weight *wt, const uint16_t *x, int64_t m, const Out &o, hipStream_t s) {
  constexpr int B = MT == 4 ? 1 : 4;
  const dim3 grid((unsigned)((wt->n + 15) / 16));
  const uint8_t *aux = wt->data + wt->aux_off;
  hipLaunchKernelGGL((k_smallm<C, MT, 4, B>), grid, dim3(256), 0, s, wt->data, aux, x, m, o, wt->n, wt->k);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "small-M launch failed");
}

template <class C>
int run(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s) {
  const uint16_t *xb = static_cast<const uint16_t *>(x);
  if (m <= 16) return run_mt<C, 1>(wt, xb, m, o, s);
  if (m <= 32) return run_mt<C, 2>(wt, xb, m, o, s);
  return run_mt<C, 4>(wt, xb, m, o, s);
}

}  // namespace

// f32 / f16 activations, 2 <= m <= 64, k % 64 == 0, 16-byte aligned x
// (dispatched from m = 4, and at m = 2..3 for rows the VALU layouts do not
// take).
int launch_linear_smallm_f32(const rq_weight *wt, const void *x, int xtype, int64_t m, const Out &o,
                             hipStream_t s) {
  if (m < 2 || m > 64 || wt->k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  if (xtype == RQ_F32) return dispatch_f32<RQ_F32>(wt, x, m, o, s);
  if (xtype == RQ_F16) return dispatch_f32<RQ_F16>(wt, x, m, o, s);
  return RQ_E_UNSUPPORTED;
}

// bf16 activations, 2 <= m <= 64, k % 64 == 0, 16-byte aligned x.
int launch_linear_smallm(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s) {
  if (m < 2 || m > 64 || wt->k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  switch (wt->qtype) {
    case RQ_Q4_K: return run<SmQ4K>(wt, x, m, o, s);
    case RQ_Q6_K: return run<SmQ6K>(wt, x, m, o, s);
    case RQ_Q8_0: return run<SmQ8>(wt, x, m, o, s);
    case RQ_Q5_K: return run<SmQ5K>(wt, x, m, o, s);
    case RQ_Q4_0: return run<SmQx0<false>>(wt, x, m, o, s);
    case RQ_Q5_0: return run<SmQx0<true>>(wt, x, m, o, s);
    default: return RQ_E_UNSUPPORTED;
  }
}

}  // namespace rq
