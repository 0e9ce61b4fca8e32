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
#include <vector>

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

// ---- several weights in one launch ----
//
// Weights that share one activation block x, and one output and bias type:
// entry j covers the workgroups [g_end[j - 1], g_end[j]) of the grid
// (g_end[-1] = 0; entries past count hold g_end = INT32_MAX), with its own
// rows, output and bias.  Kept small: a kernel's arguments are fetched
// before anything else can start.
constexpr int kMultiMax = 4;
struct WeightSet {
  const uint8_t *w[kMultiMax];
  void *y[kMultiMax];
  const void *bias[kMultiMax];
  uint32_t aux_off[kMultiMax];
  int32_t n[kMultiMax];
  int32_t g_end[kMultiMax];
  int count, ytype, btype;
};

// The entry of workgroup bid: its weight, aux array, output, rows and first
// and end workgroup.  Every table value is pinned in a scalar register first
// (an empty asm that takes them all), so the selects work on registers:
// left alone, the compiler selects an address into the table and loads
// through it, one more dependent round of argument fetches before any load
// can be issued.  The selected pointers go back through the global address
// space so that accesses through them stay global (not flat) instructions.
struct SetEntry {
  const uint8_t *w, *aux;
  Out o;
  int n, g0, g1;
};
__device__ __forceinline__ SetEntry pick_entry(const WeightSet &set, int bid) {
  static_assert(kMultiMax == 4, "one asm statement pins the four entries");
  uint64_t tw[4], ty[4], tb[4];
  uint32_t ta[4];
  int tn[4], te[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    tw[t] = reinterpret_cast<uint64_t>(set.w[t]);
    ty[t] = reinterpret_cast<uint64_t>(set.y[t]);
    tb[t] = reinterpret_cast<uint64_t>(set.bias[t]);
    ta[t] = set.aux_off[t];
    tn[t] = set.n[t];
    te[t] = set.g_end[t];
  }
  asm volatile("" : "+s"(tw[0]), "+s"(tw[1]), "+s"(tw[2]), "+s"(tw[3]), "+s"(ty[0]), "+s"(ty[1]), "+s"(ty[2]),
               "+s"(ty[3]), "+s"(tb[0]), "+s"(tb[1]), "+s"(tb[2]), "+s"(tb[3]), "+s"(ta[0]), "+s"(ta[1]),
               "+s"(ta[2]), "+s"(ta[3]), "+s"(tn[0]), "+s"(tn[1]), "+s"(tn[2]), "+s"(tn[3]), "+s"(te[0]),
               "+s"(te[1]), "+s"(te[2]), "+s"(te[3]));
  uint64_t w = tw[0], y = ty[0], bias = tb[0];
  uint32_t aux_off = ta[0];
  int n = tn[0], g0 = 0, g1 = te[0];
#pragma unroll
  for (int t = 1; t < 4; ++t) {
    const bool here = bid >= te[t - 1];
    w = here ? tw[t] : w;
    y = here ? ty[t] : y;
    bias = here ? tb[t] : bias;
    aux_off = here ? ta[t] : aux_off;
    n = here ? tn[t] : n;
    g0 = here ? te[t - 1] : g0;
    g1 = here ? te[t] : g1;
  }
  typedef __attribute__((address_space(1))) uint8_t gbyte;
  SetEntry e;
  e.w = (const uint8_t *)(const gbyte *)w;
  e.aux = e.w + aux_off;
  e.o = Out{(void *)(gbyte *)y, (const void *)(const gbyte *)bias, set.ytype, set.btype};
  e.n = n;
  e.g0 = g0;
  e.g1 = g1;
  return e;
}

// Fills a WeightSet for count weights (workgroups per weight from wg_of),
// or returns RQ_E_UNSUPPORTED (shapes beyond 32-bit fields, or outputs of
// different types).
template <class WG>
__host__ int fill_set(WeightSet &set, const rq_weight *const *w, int count, const Out *o, WG &&wg_of,
                      int64_t *total_out) {
  set = WeightSet{};
  int64_t total = 0;
  bool have_bias = false;
  for (int j = 0; j < count; ++j) {
    if (w[j]->aux_off > 0xFFFFFFFFull || w[j]->n > 0x7FFFFFFF) return RQ_E_UNSUPPORTED;
    if (o[j].ytype != o[0].ytype || (o[j].bias && have_bias && o[j].btype != set.btype)) return RQ_E_UNSUPPORTED;
    set.w[j] = w[j]->data;
    set.aux_off[j] = (uint32_t)w[j]->aux_off;
    set.y[j] = o[j].y;
    set.bias[j] = o[j].bias;
    set.n[j] = (int32_t)w[j]->n;
    total += wg_of(w[j]);
    if (total > 0x7FFFFFFF) return RQ_E_UNSUPPORTED;
    set.g_end[j] = (int32_t)total;
    if (o[j].bias) {
      set.btype = o[j].btype;
      have_bias = true;
    }
  }
  for (int j = count; j < kMultiMax; ++j) set.g_end[j] = 0x7FFFFFFF;
  set.count = count;
  set.ytype = o[0].ytype;
  *total_out = total;
  return RQ_OK;
}

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
  // *rc set on failure, and the thread's error message too unless `quiet`
  // (a caller with a path that needs no scratch passes quiet, so a call that
  // succeeds leaves no stale message).  Earlier pointers of the same lease
  // stay valid.
  void *get(size_t bytes, int *rc, bool quiet = false);
  // kCounters u32 of the slot that are zero between calls: a kernel that
  // counts in them must leave them zero when it ends.  Made (and zeroed)
  // on the first request outside stream capture; null under capture before
  // that, or on failure (the caller then takes a path without counters).
  static constexpr int kCounters = 8192;
  uint32_t *counters();

 private:
  void acquire();
  struct Slot *slot_ = nullptr;
  int device_;
  hipStream_t s_;
  bool capturing_ = false;
  size_t used_ = 0;
  std::vector<void *> async_;  // freed in stream order when the lease ends
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
// M = 1 Q4_K GEMV on the matrix cores (k % 512 == 0, k <= 8192, x 16-byte
// aligned); RQ_E_UNSUPPORTED for other shapes.
int launch_gemv_mx(const rq_weight *w, const void *x, int xtype, const Out &o, hipStream_t s);
// The same for Q6_K (k % 512 == 0, k <= 8192).
int launch_gemv_mx6(const rq_weight *w, const void *x, int xtype, const Out &o, hipStream_t s);
// One launch for several weights of one format sharing x (count <= kMultiMax,
// equal k, one output type): M = 1 and M = 2 on the segment layout, bf16
// activations with 3 <= M <= 64 on the small-M matrix-core kernel.
// RQ_E_UNSUPPORTED when the shapes take another path (the caller then
// launches them one by one).
int launch_linear_multi(const rq_weight *const *w, int count, const void *x, int xtype, int64_t m, const Out *o,
                        hipStream_t s, WsLease &ws);
// MFMA GEMM for bf16 activations and m > 1 (RQ_E_UNSUPPORTED if the shape or
// format has no tiled kernel).
int launch_linear_mfma(const rq_weight *w, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease &ws);
// f32 / f16 activations, m > 64 (k % 64 == 0, x 16-byte aligned): the same
// tiles on two bf16 limbs per operand (exact weights, f32-accurate sums).
int launch_linear_mfma_limbs(const rq_weight *w, const void *x, int xtype, int64_t m, const Out &o, hipStream_t s,
                             WsLease &ws);
// Matrix-core kernel for bf16 activations and 2 <= m <= 64 (speculative
// verify), RQ_E_UNSUPPORTED outside that or for formats it has no decoder for.
// With a workspace (ws not null), few row tiles split K over several
// workgroups (partials and counters in the workspace).
int launch_linear_smallm(const rq_weight *w, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease *ws);
// The same kernel on a set of weights sharing x (equal k); xtype RQ_BF16,
// or RQ_F32 on the two-limb variant.
int launch_linear_smallm_set(const rq_weight *const *w, int count, const void *x, int xtype, int64_t m,
                             const Out *o, hipStream_t s, WsLease *ws);
// The same for f32 / f16 activations on the f32 matrix cores with exact f32
// weights (f32 accumulation).
int launch_linear_smallm_f32(const rq_weight *wt, const void *x, int xtype, int64_t m, const Out &o,
                             hipStream_t s, WsLease *ws);
// f32 activations, 4 <= m <= 16 (and 17..64 rows on the launches its plan
// names), Q4_K / Q6_K / Q8_0: the integer codes on the bf16 matrix cores
// against two bf16 limbs of x, the scales applied per run to the f32 sums;
// one weight (set false) or a set of count weights of one format and k
// sharing x.  RQ_E_UNSUPPORTED for other formats / shapes.
int launch_linear_smallm_codes(const rq_weight *const *w, int count, bool set, const void *x, int64_t m,
                               const Out *o, hipStream_t s, WsLease *ws);
// 64 * slices f32 / f16 activation rows as slices of 64 rows in one launch.
int launch_linear_smallm_f32_slices(const rq_weight *wt, const void *x, int xtype, int64_t slices, const Out &o,
                                    hipStream_t s, WsLease *ws);
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
// scales[0 .. h) = v on the stream (a kernel: safe under graph capture).
int launch_kv_fill_scales(float *scales, int64_t h, float v, hipStream_t s);

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

// The raw bits of bias element i (a uniform branch on the type, no
// conversion: a value converted right after its load would wait for it
// there) and their f32 value.
__device__ __forceinline__ uint32_t bias_bits(const void *b, int btype, int64_t i) {
  return btype == RQ_F32 ? static_cast<const uint32_t *>(b)[i] : (uint32_t) static_cast<const uint16_t *>(b)[i];
}
__device__ __forceinline__ float bias_bits_f32(uint32_t v, int btype) {
  return btype == RQ_F32 ? __uint_as_float(v) : (btype == RQ_BF16 ? __uint_as_float(v << 16) : f16_bits_to_f32(v));
}

// Bias of output column col as f32 (0 without a bias).
__device__ __forceinline__ float bias_at(const Out &o, int64_t col) {
  return o.bias ? load_as_f32(o.bias, o.btype, col) : 0.0f;
}

// linear_bias (linear_layer.rs:107-118) adds the bias cast to y's dtype to
// linear's result cast to y's dtype, and the broadcast add rounds the sum to
// y's dtype again.  Fused into an epilogue the same two roundings happen:
// acc rounded to ytype, plus the bias rounded to ytype, summed in f32 (exact
// for two bf16 / f16 values of one output) and rounded by the store.  For
// f32 outputs both roundings are the identity.
__device__ __forceinline__ float with_bias(float acc, float b, int ytype) {
  return round_as(ytype, acc) + round_as(ytype, b);
}

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
