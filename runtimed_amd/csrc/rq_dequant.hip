// rq_dequant.hip -- bit-exact block decode to f32 on gfx950.
//
// Semantics: runtimed-gguf's scalar decoders (crates/runtimed-gguf/src/quant/
// dequant.rs:40-77 for Q8_0/Q4_0/Q5_0, dequant_k.rs:19-111 for Q4_K/Q5_K/Q6_K)
// and the flat dispatcher dequant_tensor (dequant.rs:83-146).  Every product
// the decoders form before their last rounding is exact in f32 (at most 22
// significant bits), and each kernel keeps the reference's evaluation order
// for the one rounding that remains, so the result is bit-identical with or
// without FMA contraction.  f16 scales are widened with integer arithmetic so
// that NaN payloads pass through unchanged, as dequant.rs:11-33 does.
//
// Roofline: HBM-bound; per element the algorithmic traffic is the block bytes
// per element read plus 4 bytes of f32 written.
#include "rq_internal.h"

namespace rq {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ uint32_t rd_u16(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

// scale_min_k4 (dequant_k.rs:8-16) on the 12 packed scale bytes.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *s, uint32_t &sc,
                                             uint32_t &m) {
  if (j < 4) {
    sc = s[j] & 63u;
    m = s[j + 4] & 63u;
  } else {
    sc = (s[j + 4] & 0xFu) | ((uint32_t)(s[j - 4] >> 6) << 4);
    m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
  }
}

// The same on the scale bytes held as three words (bytes 0-3, 4-7, 8-11),
// so they stay in registers.
__device__ __forceinline__ void scale_min_k4_w(int j, uint32_t Y, uint32_t Z, uint32_t W, uint32_t &sc,
                                               uint32_t &m) {
  const int sh = 8 * (j & 3);
  const uint32_t y = (Y >> sh) & 0xFFu, z = (Z >> sh) & 0xFFu, w = (W >> sh) & 0xFFu;
  if (j < 4) {
    sc = y & 63u;
    m = z & 63u;
  } else {
    sc = (w & 0xFu) | ((y >> 6) << 4);
    m = (w >> 4) | ((z >> 6) << 4);
  }
}

// One element of one GGUF block from raw bytes (any alignment).
__device__ float decode_raw(int qtype, const uint8_t *b, int i) {
  switch (qtype) {
    case RQ_Q8_0:  // dequant.rs:40-47
      return f16_bits_to_f32(rd_u16(b)) * (float)(int8_t)b[2 + i];
    case RQ_Q4_0: {  // dequant.rs:50-61
      const float d = f16_bits_to_f32(rd_u16(b));
      const int q = i < 16 ? (b[2 + i] & 0x0F) : (b[2 + i - 16] >> 4);
      return d * (float)(q - 8);
    }
    case RQ_Q5_0: {  // dequant.rs:64-77; element j takes qh bit j
      const float d = f16_bits_to_f32(rd_u16(b));
      const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) |
                          ((uint32_t)b[5] << 24);
      const int lo = i < 16 ? (b[6 + i] & 0x0F) : (b[6 + i - 16] >> 4);
      const int q = lo | (int)(((qh >> i) & 1u) << 4);
      return d * (float)(q - 16);
    }
    case RQ_Q4_K: {  // dequant_k.rs:19-44
      const float d = f16_bits_to_f32(rd_u16(b));
      const float mn = f16_bits_to_f32(rd_u16(b + 2));
      const int chunk = i >> 6, r = i & 63, j = 2 * chunk + (r >> 5);
      uint32_t sc, m;
      scale_min_k4(j, b + 4, sc, m);
      const uint8_t byte = b[16 + 32 * chunk + (r & 31)];
      const uint32_t q = (r < 32) ? (byte & 0xFu) : (uint32_t)(byte >> 4);
      const float d1 = d * (float)sc, m1 = mn * (float)m;
      return d1 * (float)q - m1;
    }
    case RQ_Q5_K: {  // dequant_k.rs:51-80
      const float d = f16_bits_to_f32(rd_u16(b));
      const float mn = f16_bits_to_f32(rd_u16(b + 2));
      const int chunk = i >> 6, r = i & 63, l = r & 31, j = 2 * chunk + (r >> 5);
      uint32_t sc, m;
      scale_min_k4(j, b + 4, sc, m);
      const uint8_t byte = b[48 + 32 * chunk + l];
      const uint32_t q = (r < 32) ? (byte & 0xFu) : (uint32_t)(byte >> 4);
      const uint32_t mask = (r < 32 ? 1u : 2u) << (2 * chunk);
      const float hi = (b[16 + l] & mask) ? 16.0f : 0.0f;
      const float d1 = d * (float)sc, m1 = mn * (float)m;
      return d1 * ((float)q + hi) - m1;
    }
    case RQ_Q6_K: {  // dequant_k.rs:87-111
      const int hf = i >> 7, r = i & 127, kk = r >> 5, l = r & 31;
      const uint8_t qlb = b[64 * hf + l + 32 * (kk & 1)];
      const uint8_t qhb = b[128 + 32 * hf + l];
      const uint32_t q = ((uint32_t)(qlb >> (4 * (kk >> 1))) & 0xFu) |
                         ((((uint32_t)qhb >> (2 * kk)) & 3u) << 4);
      const float v = (float)(int8_t)q - 32.0f;
      const float d = f16_bits_to_f32(rd_u16(b + 208));
      return d * (float)(int8_t)b[192 + 8 * hf + (l >> 4) + 2 * kk] * v;
    }
    default:
      return 0.0f;
  }
}

__global__ __launch_bounds__(kThreads) void k_dequant_raw(int qtype, int elems, int bbytes,
                                                         const uint8_t *__restrict__ src,
                                                         uint64_t total, float *__restrict__ out) {
  const uint64_t stride = (uint64_t)gridDim.x * kThreads;
  for (uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x; e < total; e += stride) {
    const uint64_t blk = e / (uint64_t)elems;
    const int i = (int)(e - blk * (uint64_t)elems);
    out[e] = decode_raw(qtype, src + blk * (uint64_t)bbytes, i);
  }
}

// ---- handle layouts: four consecutive outputs (flat quad t) per call ----

// Q4_K (aligned GGUF blocks).
__device__ float4 quad_q4k(const uint8_t *__restrict__ src, uint64_t t) {
  const uint64_t blk = t >> 6;
  const int i0 = (int)(t & 63) * 4;
  const uint8_t *b = src + blk * 144;
  const uint4 hd = *reinterpret_cast<const uint4 *>(b);
  const int chunk = i0 >> 6, r = i0 & 63, j = 2 * chunk + (r >> 5);
  const uint32_t qw = *reinterpret_cast<const uint32_t *>(b + 16 + 32 * chunk + (r & 31));
  uint32_t sc, m;
  scale_min_k4_w(j, hd.y, hd.z, hd.w, sc, m);
  const float d1 = f16_bits_to_f32(hd.x & 0xFFFFu) * (float)sc;
  const float m1 = f16_bits_to_f32(hd.x >> 16) * (float)m;
  const uint32_t q4 = (r < 32) ? (qw & 0x0F0F0F0Fu) : ((qw >> 4) & 0x0F0F0F0Fu);
  float4 o;
  o.x = d1 * (float)(q4 & 0xFFu) - m1;
  o.y = d1 * (float)((q4 >> 8) & 0xFFu) - m1;
  o.z = d1 * (float)((q4 >> 16) & 0xFFu) - m1;
  o.w = d1 * (float)(q4 >> 24) - m1;
  return o;
}

// Q5_K (aligned GGUF blocks): d1 * (q + hi) - m1 (dequant_k.rs:67-73).
__device__ float4 quad_q5k(const uint8_t *__restrict__ src, uint64_t t) {
  const uint64_t blk = t >> 6;
  const int i0 = (int)(t & 63) * 4;
  const uint8_t *b = src + blk * 176;
  const uint4 hd = *reinterpret_cast<const uint4 *>(b);
  const int chunk = i0 >> 6, r = i0 & 63, l = r & 31, j = 2 * chunk + (r >> 5);
  const uint32_t qw = *reinterpret_cast<const uint32_t *>(b + 48 + 32 * chunk + l);
  const uint32_t hw = *reinterpret_cast<const uint32_t *>(b + 16 + l);
  uint32_t sc, m;
  scale_min_k4_w(j, hd.y, hd.z, hd.w, sc, m);
  const float d1 = f16_bits_to_f32(hd.x & 0xFFFFu) * (float)sc;
  const float m1 = f16_bits_to_f32(hd.x >> 16) * (float)m;
  const int bit = 2 * chunk + (r >> 5);
  const uint32_t q = ((r < 32) ? (qw & 0x0F0F0F0Fu) : ((qw >> 4) & 0x0F0F0F0Fu)) |
                     (((hw >> bit) & 0x01010101u) << 4);
  float4 o;
  o.x = d1 * (float)(q & 0xFFu) - m1;
  o.y = d1 * (float)((q >> 8) & 0xFFu) - m1;
  o.z = d1 * (float)((q >> 16) & 0xFFu) - m1;
  o.w = d1 * (float)(q >> 24) - m1;
  return o;
}

// Q8_0 split layout.
__device__ float4 quad_q8(const uint8_t *__restrict__ qs, const uint8_t *__restrict__ aux, uint64_t t) {
  const uint32_t v = reinterpret_cast<const uint32_t *>(qs)[t];
  const float d = f16_bits_to_f32(reinterpret_cast<const uint16_t *>(aux)[t >> 3]);
  float4 o;
  o.x = d * (float)(int8_t)(v & 0xFFu);
  o.y = d * (float)(int8_t)((v >> 8) & 0xFFu);
  o.z = d * (float)(int8_t)((v >> 16) & 0xFFu);
  o.w = d * (float)(int8_t)(v >> 24);
  return o;
}

// Q6_K split layout.
__device__ float4 quad_q6k(const uint8_t *__restrict__ rec, const uint8_t *__restrict__ aux, uint64_t t) {
  const uint64_t blk = t >> 6;
  const int i0 = (int)(t & 63) * 4;
  const int hf = i0 >> 7, r = i0 & 127, kk = r >> 5, l = r & 31;
  const uint8_t *b = rec + blk * 208;
  const uint32_t ql = *reinterpret_cast<const uint32_t *>(b + 64 * hf + 32 * (kk & 1) + l);
  const uint32_t qh = *reinterpret_cast<const uint32_t *>(b + 128 + 32 * hf + l);
  const float ds = f16_bits_to_f32(reinterpret_cast<const uint16_t *>(aux)[blk]) *
                   (float)(int8_t)b[192 + 8 * hf + (l >> 4) + 2 * kk];
  const uint32_t q = ((ql >> (4 * (kk >> 1))) & 0x0F0F0F0Fu) | (((qh >> (2 * kk)) & 0x03030303u) << 4);
  float4 o;
  o.x = ds * ((float)(q & 0xFFu) - 32.0f);
  o.y = ds * ((float)((q >> 8) & 0xFFu) - 32.0f);
  o.z = ds * ((float)((q >> 16) & 0xFFu) - 32.0f);
  o.w = ds * ((float)(q >> 24) - 32.0f);
  return o;
}

// Q4_0 / Q5_0 split layouts: element i of a block is nibble i / 16 of quant
// byte i % 16 (plus qh bit i for Q5_0), value d * (q - 8) or d * (q - 16)
// (dequant.rs:50-77).
template <bool Q5>
__device__ float4 quad_qx0(const uint8_t *__restrict__ qs, const uint8_t *__restrict__ aux, uint64_t t) {
  const uint64_t blk = t >> 3;
  const int i0 = (int)(t & 7) * 4;
  const uint32_t v = *reinterpret_cast<const uint32_t *>(qs + 16 * blk + (i0 & 15));
  uint32_t q = (v >> (4 * (i0 >> 4))) & 0x0F0F0F0Fu;
  uint32_t dbits;
  if (Q5) {
    const uint2 rec = reinterpret_cast<const uint2 *>(aux)[blk];
    const uint32_t hb = (rec.x >> i0) & 0xFu;
    q |= (((hb & 1u) | ((hb & 2u) << 7) | ((hb & 4u) << 14) | ((hb & 8u) << 21)) << 4);
    dbits = rec.y & 0xFFFFu;
  } else {
    dbits = reinterpret_cast<const uint16_t *>(aux)[blk];
  }
  const float d = f16_bits_to_f32(dbits), z = Q5 ? 16.0f : 8.0f;
  float4 o;
  o.x = d * ((float)(q & 0xFFu) - z);
  o.y = d * ((float)((q >> 8) & 0xFFu) - z);
  o.z = d * ((float)((q >> 16) & 0xFFu) - z);
  o.w = d * ((float)(q >> 24) - z);
  return o;
}

template <int QT>
__device__ __forceinline__ float4 quad_handle(const uint8_t *data, const uint8_t *aux, uint64_t t) {
  if constexpr (QT == RQ_Q4_K) return quad_q4k(data, t);
  else if constexpr (QT == RQ_Q5_K) return quad_q5k(data, t);
  else if constexpr (QT == RQ_Q8_0) return quad_q8(data, aux, t);
  else if constexpr (QT == RQ_Q6_K) return quad_q6k(data, aux, t);
  else if constexpr (QT == RQ_Q4_0) return quad_qx0<false>(data, aux, t);
  else return quad_qx0<true>(data, aux, t);
}

// Whole handle: one thread per 4 outputs.
template <int QT>
__global__ __launch_bounds__(kThreads) void k_dequant_handle(const uint8_t *__restrict__ data,
                                                            const uint8_t *__restrict__ aux, uint64_t quads,
                                                            float4 *__restrict__ out) {
  const uint64_t stride = (uint64_t)gridDim.x * kThreads;
  for (uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x; t < quads; t += stride)
    out[t] = quad_handle<QT>(data, aux, t);
}

// Rows ids[0 .. nid) of an [n, k] handle (k % 4 == 0): output quad q of row
// i is flat quad ids[i] * k / 4 + q.
template <int QT>
__global__ __launch_bounds__(kThreads) void k_gather_rows(const uint8_t *__restrict__ data,
                                                         const uint8_t *__restrict__ aux,
                                                         const uint32_t *__restrict__ ids, int64_t nid,
                                                         int64_t kq, float4 *__restrict__ out) {
  const uint64_t total = (uint64_t)nid * (uint64_t)kq, stride = (uint64_t)gridDim.x * kThreads;
  for (uint64_t o = (uint64_t)blockIdx.x * kThreads + threadIdx.x; o < total; o += stride) {
    const uint64_t i = o / (uint64_t)kq, q = o - i * (uint64_t)kq;
    out[o] = quad_handle<QT>(data, aux, (uint64_t)ids[i] * (uint64_t)kq + q);
  }
}

// y[m, n] = x W^T for any shape and alignment (the shapes the fused kernels
// do not take): one wave per weight row, the lanes striding over k, each
// weight decoded exactly from its flat quad (the element picked from the
// four), four activation rows per pass over the row, f32 accumulation.  A
// fallback: every weight is decoded ceil(m / 4) times.
template <int QT>
__global__ __launch_bounds__(kThreads) void k_linear_generic(const uint8_t *__restrict__ data,
                                                            const uint8_t *__restrict__ aux,
                                                            const void *__restrict__ x, int xtype, int64_t m,
                                                            const Out o, int64_t n, int64_t k) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * (kThreads / 64);
  for (int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); row < n; row += nw) {
    for (int64_t m0 = 0; m0 < m; m0 += 4) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int64_t c = lane; c < k; c += 64) {
        const uint64_t e = (uint64_t)row * (uint64_t)k + (uint64_t)c;
        const float4 q = quad_handle<QT>(data, aux, e >> 2);
        const int sub = (int)(e & 3);
        const float wv = sub == 0 ? q.x : sub == 1 ? q.y : sub == 2 ? q.z : q.w;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (m0 + i < m) acc[i] = fmaf(wv, load_as_f32(x, xtype, (m0 + i) * k + c), acc[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = acc[i];
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
        if (lane == 0 && m0 + i < m) store_linear(o, m0 + i, n, row, v);
      }
    }
  }
}

// linear_bias's broadcast add (linear_layer.rs:111-115) on an output that is
// already in y: the bias cast to y's type, the sum rounded to y's type.
__global__ __launch_bounds__(kThreads) void k_bias_add(void *__restrict__ y, int ytype, int64_t mn, int64_t n,
                                                      const void *__restrict__ bias, int btype) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < mn; i += stride)
    store_out(y, ytype, i, load_as_f32(y, ytype, i) + round_as(ytype, load_as_f32(bias, btype, i % n)));
}

unsigned grid_for(uint64_t items) {
  const uint64_t want = (items + kThreads - 1) / kThreads;
  return (unsigned)(want < 65536 ? (want ? want : 1) : 65536);
}

}  // namespace

int launch_dequant_raw(int qtype, const uint8_t *src, uint64_t nblocks, float *out,
                       hipStream_t s) {
  Geometry g;
  if (!geometry(qtype, &g)) return set_error(RQ_E_UNSUPPORTED, "no decoder for qtype %d", qtype);
  const uint64_t total = nblocks * (uint64_t)g.elems;
  if (total == 0) return RQ_OK;
  hipLaunchKernelGGL(k_dequant_raw, dim3(grid_for(total)), dim3(kThreads), 0, s, qtype, g.elems,
                     g.bytes, src, total, out);
  return hipGetLastError() == hipSuccess ? RQ_OK
                                         : set_error(RQ_E_DEVICE, "dequant launch failed");
}

template <template <int> class K, class... Args>
int by_qtype(int qtype, dim3 grid, hipStream_t s, Args... args) {
  switch (qtype) {
    case RQ_Q4_K: hipLaunchKernelGGL(K<RQ_Q4_K>::fn, grid, dim3(kThreads), 0, s, args...); break;
    case RQ_Q5_K: hipLaunchKernelGGL(K<RQ_Q5_K>::fn, grid, dim3(kThreads), 0, s, args...); break;
    case RQ_Q8_0: hipLaunchKernelGGL(K<RQ_Q8_0>::fn, grid, dim3(kThreads), 0, s, args...); break;
    case RQ_Q6_K: hipLaunchKernelGGL(K<RQ_Q6_K>::fn, grid, dim3(kThreads), 0, s, args...); break;
    case RQ_Q4_0: hipLaunchKernelGGL(K<RQ_Q4_0>::fn, grid, dim3(kThreads), 0, s, args...); break;
    case RQ_Q5_0: hipLaunchKernelGGL(K<RQ_Q5_0>::fn, grid, dim3(kThreads), 0, s, args...); break;
    default: return set_error(RQ_E_UNSUPPORTED, "no decoder for qtype %d", qtype);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "dequant launch failed");
}

template <int QT>
struct DequantK {
  static constexpr auto fn = k_dequant_handle<QT>;
};
template <int QT>
struct GatherK {
  static constexpr auto fn = k_gather_rows<QT>;
};

int launch_dequant_weight(const rq_weight *w, float *out, hipStream_t s) {
  const uint64_t quads = (uint64_t)w->n * (uint64_t)w->k / 4;
  if (quads == 0) return RQ_OK;
  return by_qtype<DequantK>(w->qtype, dim3(grid_for(quads)), s, (const uint8_t *)w->data,
                            (const uint8_t *)(w->data + w->aux_off), quads, reinterpret_cast<float4 *>(out));
}

int launch_gather_rows(const rq_weight *w, const uint32_t *dev_ids, int64_t n_ids, float *out, hipStream_t s) {
  if (n_ids == 0) return RQ_OK;
  const int64_t kq = w->k / 4;
  return by_qtype<GatherK>(w->qtype, dim3(grid_for((uint64_t)n_ids * (uint64_t)kq)), s, (const uint8_t *)w->data,
                           (const uint8_t *)(w->data + w->aux_off), dev_ids, n_ids, kq,
                           reinterpret_cast<float4 *>(out));
}

int launch_linear_generic(const rq_weight *w, const void *x, int xtype, int64_t m, const Out &o, hipStream_t s) {
  int64_t blocks = (w->n + 3) / 4;
  if (blocks > 8192) blocks = 8192;
  const dim3 grid((unsigned)blocks), block(kThreads);
  const uint8_t *aux = w->data + w->aux_off;
  switch (w->qtype) {
    case RQ_Q4_K: hipLaunchKernelGGL(k_linear_generic<RQ_Q4_K>, grid, block, 0, s, w->data, aux, x, xtype, m, o, w->n, w->k); break;
    case RQ_Q5_K: hipLaunchKernelGGL(k_linear_generic<RQ_Q5_K>, grid, block, 0, s, w->data, aux, x, xtype, m, o, w->n, w->k); break;
    case RQ_Q8_0: hipLaunchKernelGGL(k_linear_generic<RQ_Q8_0>, grid, block, 0, s, w->data, aux, x, xtype, m, o, w->n, w->k); break;
    case RQ_Q6_K: hipLaunchKernelGGL(k_linear_generic<RQ_Q6_K>, grid, block, 0, s, w->data, aux, x, xtype, m, o, w->n, w->k); break;
    case RQ_Q4_0: hipLaunchKernelGGL(k_linear_generic<RQ_Q4_0>, grid, block, 0, s, w->data, aux, x, xtype, m, o, w->n, w->k); break;
    case RQ_Q5_0: hipLaunchKernelGGL(k_linear_generic<RQ_Q5_0>, grid, block, 0, s, w->data, aux, x, xtype, m, o, w->n, w->k); break;
    default: return set_error(RQ_E_UNSUPPORTED, "no decoder for qtype %d", w->qtype);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "linear launch failed");
}

int launch_bias_add(void *y, int ytype, int64_t m, int64_t n, const void *bias, int btype, hipStream_t s) {
  const uint64_t mn = (uint64_t)m * (uint64_t)n;
  if (mn == 0) return RQ_OK;
  hipLaunchKernelGGL(k_bias_add, dim3(grid_for(mn)), dim3(kThreads), 0, s, y, ytype, (int64_t)mn, n, bias, btype);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "bias add launch failed");
}

}  // namespace rq
