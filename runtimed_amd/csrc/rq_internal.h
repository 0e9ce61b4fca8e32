// rq_internal.h -- shared declarations for librq (gfx950).
//
// Device layouts held by a weight handle (all arrays 256-byte aligned):
//   Q4_K, Q5_K              the GGUF block stream as uploaded.  Blocks are
//                           144 = 9 x 16 and 176 = 11 x 16 bytes, so every
//                           block of a 16-aligned stream is 16-aligned.
//   Q8_0                    quants: n*k int8 in flat element order, then
//                           scales: one f16 per 32-element block.
//   Q4_0                    16 quant bytes per block in block order, then
//                           one f16 d per block.
//   Q5_0                    16 quant bytes per block, then one 8-byte record
//                           {qh u32, d f16, 0} per block.
//   Q6_K                    208-byte records [ql 128 | qh 64 | scales 16] per
//                           block (13 x 16 bytes), then one f16 d per block.
// The split layouts keep every element value and the flat element order of
// GGUF (dequant.rs:83-146); only the byte placement changes so that 16-byte
// vector loads stay aligned.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <utility>

#include "../../include/rq.h"

struct rq_weight {
  int qtype;
  int device;
  int64_t n, k;
  uint64_t gguf_bytes;
  uint64_t nblocks;
  uint8_t *data;       // device base
  uint64_t data_bytes; // device bytes held
  uint64_t aux_off;    // offset of the scale array for Q8_0 / Q6_K
};

namespace rq {

// f(std::integral_constant<int, 0>) ... f(std::integral_constant<int, N-1>):
// indices stay compile-time constants, so register arrays indexed by them
// (MFMA accumulators) are never demoted to scratch memory.
template <int... I, class F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, I...>, F &&f) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

// Block geometry of GgmlDtype::block (dtype.rs:49-64) for the formats with a
// decoder here.
struct Geometry {
  int elems;
  int bytes;
};
bool geometry(int qtype, Geometry *g);

int set_error(int code, const char *fmt, ...);
void clear_error();
hipStream_t as_stream(void *s);
// rq_fp8_gemm's argument rules (types, mode, shape); clears the last error.
int fp8_gemm_checks(int xtype, int64_t m, int64_t n, int64_t k, int ytype, int mode);

// Host-to-device upload of nblocks GGUF blocks into a handle's layout
// (pinned double-buffered DMA; split layouts scattered on the device).
int upload_blocks(int qtype, const uint8_t *src, uint64_t nblocks, int bbytes, uint8_t *dptr, uint64_t aux_off,
                  int device);

// ---- the output side of a linear call ----
//
// y[m, n] (row stride n) of type ytype, plus an optional per-column bias of
// n values of type btype (F32, F16 or BF16): linear_bias's broadcast add
// (linear_layer.rs:107-118) fused into the epilogue of every kernel.
struct Out {
  void *y;
  const void *bias;  // null: no bias
  int ytype;
  int btype;
};

// ---- workspace: device memory that outlives a call ----
//
// One buffer per (device, stream), grown on demand and reused by every later
// call on that stream, so the split-K partials, activation copies and FP8
// scratch of a call cost no allocation.  A lease holds the (device, stream)
// slot for the duration of one entry point's launches (two threads issuing
// to one stream take turns; their kernels still run in stream order).  Under
// stream capture a buffer that is already large enough is used as it is (the
// graph then refers to it, and it is never freed); a larger need is met by a
// stream-ordered allocation that becomes part of the graph.  A replaced
// buffer is freed in stream order when the lease ends, unless a captured
// graph may refer to it.  The slot is taken at the first get().
class WsLease {
 public:
  WsLease(int device, hipStream_t s);
  ~WsLease();
  WsLease(const WsLease &) = delete;
  WsLease &operator=(const WsLease &) = delete;
  // `bytes` of device memory (256-byte aligned) for this call; null with
  // *rc set (and the error message) on failure.  Earlier pointers of the same
  // lease stay valid.
  void *get(size_t bytes, int *rc);

 private:
  void acquire();
  struct Slot *slot_ = nullptr;
  int device_;
  hipStream_t s_;
  bool capturing_ = false;
  size_t used_ = 0;
  void *async_[4] = {nullptr, nullptr, nullptr, nullptr};  // freed in stream order when the lease ends
  int n_async_ = 0;
};

// ---- launchers (each returns RQ_OK or an error code and message) ----
int launch_dequant_weight(const rq_weight *w, float *out, hipStream_t s);
// Rows dev_ids[0 .. n_ids) of a handle (every id < n, k % 4 == 0) as f32.
int launch_gather_rows(const rq_weight *w, const uint32_t *dev_ids, int64_t n_ids, float *out,
                       hipStream_t s);
int launch_dequant_raw(int qtype, const uint8_t *src, uint64_t nblocks, float *out,
                       hipStream_t s);
// Fused matmul on a handle (x 16-byte aligned); returns RQ_E_UNSUPPORTED
// when the handle's shape has no fused kernel (the caller then takes the
// generic kernel).
int launch_linear_fused(const rq_weight *w, const void *x, int xtype, int64_t m, const Out &o, hipStream_t s,
                        WsLease &ws);
// One launch for several weights of one format sharing x (count <= kMultiMax,
// equal k): M = 1 and M = 2 on the segment layout.  RQ_E_UNSUPPORTED when
// the shapes take another layout (the caller then launches them one by one).
constexpr int kMultiMax = 8;
int launch_linear_multi(const rq_weight *const *w, int count, const void *x, int xtype, int64_t m, const Out *o,
                        hipStream_t s);
// MFMA GEMM for bf16 activations and m > 1 (RQ_E_UNSUPPORTED if the shape or
// format has no tiled kernel).
int launch_linear_mfma(const rq_weight *w, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease &ws);
// Matrix-core kernel for bf16 activations and 2 <= m <= 64 (speculative
// verify), RQ_E_UNSUPPORTED outside that or for formats it has no decoder for.
int launch_linear_smallm(const rq_weight *w, const void *x, int64_t m, const Out &o, hipStream_t s);
// The same for f32 / f16 activations on the f32 matrix cores with exact f32
// weights (f32 accumulation).
int launch_linear_smallm_f32(const rq_weight *wt, const void *x, int xtype, int64_t m, const Out &o,
                             hipStream_t s);
// Every shape and alignment: exact f32 weights decoded element by element
// from the handle, f32 accumulation (the shapes the fused kernels do not
// take: rows cut inside a 64-element chunk, rows longer than the GEMV
// layouts hold).
int launch_linear_generic(const rq_weight *w, const void *x, int xtype, int64_t m, const Out &o, hipStream_t s);
// y[m, n] = (y as ytype) + (bias as ytype): linear_bias's broadcast add
// (linear_layer.rs:111-115) on an output that is already there.
int launch_bias_add(void *y, int ytype, int64_t m, int64_t n, const void *bias, int btype, hipStream_t s);
int launch_fp8_quantize(const void *x, int xtype, int64_t m, int64_t k, int mode, uint8_t *xq,
                        float *xs, hipStream_t s);
int launch_fp8_gemm(const uint8_t *xq, const float *xs, int64_t m, const uint8_t *w,
                    const float *ws, int64_t n, int64_t k, void *y, int ytype, hipStream_t s);

// Marlin INT4 weights (arguments validated by the caller).
int launch_marlin_repack(const void *w, int wtype, const float *s, int64_t n, int64_t k, uint32_t *packed,
                         hipStream_t st);
int launch_marlin_dequant(const uint32_t *packed, const float *s, int64_t n, int64_t k, float *out,
                          hipStream_t st);
int launch_marlin_linear(const uint32_t *packed, const float *s, int64_t n, int64_t k, const void *x, int xtype,
                         int64_t m, void *y, int ytype, hipStream_t st);
// Paged-KV block quantizer (arguments validated by the caller).
int launch_kv_quantize(const void *t, int ttype, int64_t b, int64_t h, int64_t sd, int mode, void *q,
                       float *scales, hipStream_t s, WsLease &ws);
int launch_kv_dequantize(const void *q, int mode, const float *scales, int64_t b, int64_t h, int64_t sd, void *out,
                         int otype, hipStream_t s);

// ---- exact scalar conversions shared by device code ----

// f16 bit pattern -> f32 bit pattern, integer-exact including subnormals and
// NaN payloads: the rule of f16_to_f32 (dequant.rs:11-33).
__host__ __device__ __forceinline__ uint32_t f16_bits_to_f32_bits(uint32_t h) {
  const uint32_t sign = (h >> 15) & 1u;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t mant = h & 0x3FFu;
  if (exp == 0) {
    if (mant == 0) return sign << 31;
    // A subnormal m * 2^-24 with its leading one at bit p is 2^(p-24) * 1.f.
    const int p = 31 - __builtin_clz(mant);
    return (sign << 31) | ((uint32_t)(103 + p) << 23) | (((mant << (10 - p)) & 0x3FFu) << 13);
  }
  if (exp == 31) return (sign << 31) | (0xFFu << 23) | (mant << 13);
  return (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
}

__host__ __device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return __uint_as_float(f16_bits_to_f32_bits(h));
}

// f32 -> bf16 bits, round to nearest even, NaN stays NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Store one f32 result as the requested output type.
__device__ __forceinline__ void store_out(void *y, int ytype, int64_t idx, float v) {
  if (ytype == RQ_F32) {
    static_cast<float *>(y)[idx] = v;
  } else if (ytype == RQ_BF16) {
    static_cast<uint16_t *>(y)[idx] = (uint16_t)f32_to_bf16_bits(v);
  } else {
    static_cast<_Float16 *>(y)[idx] = (_Float16)v;
  }
}

// A dense value of type t (F32, F16 or BF16) at index i, as f32.
__device__ __forceinline__ float load_as_f32(const void *p, int t, int64_t i) {
  if (t == RQ_F32) return static_cast<const float *>(p)[i];
  if (t == RQ_BF16) return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  return (float)static_cast<const _Float16 *>(p)[i];
}

// v rounded to the output type and widened back (exact for F32).  Both
// roundings are computed and one is selected: no branches in the unrolled
// epilogues that use it.
__device__ __forceinline__ float round_as(int ytype, float v) {
  const float b = bf16_bits_to_f32(f32_to_bf16_bits(v));
  const float h = (float)(_Float16)v;
  return ytype == RQ_F32 ? v : (ytype == RQ_BF16 ? b : h);
}

// Bias of output column col as f32 (0 without a bias).
__device__ __forceinline__ float bias_at(const Out &o, int64_t col) {
  return o.bias ? load_as_f32(o.bias, o.btype, col) : 0.0f;
}

// linear_bias (linear_layer.rs:107-118) adds the bias cast to y's dtype to
// linear's result cast to y's dtype.  Fused into an epilogue, the f32 sum
// acc + (bias as ytype) is rounded once by the store: for f32 outputs that
// is the reference's acc + b exactly; for bf16 / f16 outputs it can differ
// from the reference's two roundings by one unit in the last place of y
// (and is the nearer of the two to the exact sum).
__device__ __forceinline__ float with_bias(float acc, float b, int ytype) { return acc + round_as(ytype, b); }

// Output (row, col) of a linear call, with its bias.
__device__ __forceinline__ void store_linear(const Out &o, int64_t row, int64_t n, int64_t col, float acc) {
  store_out(o.y, o.ytype, row * n + col, o.bias ? with_bias(acc, load_as_f32(o.bias, o.btype, col), o.ytype) : acc);
}

// Load 4 consecutive activations starting at element idx (idx % 4 == 0) as f32.
__device__ __forceinline__ float4 load_x4(const void *x, int xtype, int64_t idx) {
  if (xtype == RQ_F32) return *reinterpret_cast<const float4 *>(static_cast<const float *>(x) + idx);
  const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(x) + idx);
  if (xtype == RQ_BF16) {
    return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u),
                       __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xFFFF0000u));
  }
  const _Float16 *h = reinterpret_cast<const _Float16 *>(&v);
  return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}

}  // namespace rq
