// rq_api.cpp -- the C ABI of librq (include/rq.h): argument checks, handle
// ownership, device binding and dispatch to the HIP kernels.
//
// Error rules follow the reference: dequant_tensor's Unsupported / Overflow /
// Truncated (crates/runtimed-gguf/src/quant/dequant.rs:84-95) for block
// streams, ModelError::Shape for activation shapes (linear_layer.rs:88-94).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "rq_internal.h"

namespace rq {

static thread_local std::string g_last_error;

int set_error(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

void clear_error() { g_last_error.clear(); }

int fp8_gemm_checks(int xtype, int64_t m, int64_t n, int64_t k, int ytype, int mode) {
  clear_error();
  if (xtype != RQ_F8E4M3 && xtype != RQ_F32 && xtype != RQ_F16 && xtype != RQ_BF16)
    return set_error(RQ_E_ARG, "activation type %d not supported", xtype);
  if (ytype != RQ_F32 && ytype != RQ_F16 && ytype != RQ_BF16)
    return set_error(RQ_E_ARG, "output type %d not supported", ytype);
  if (xtype != RQ_F8E4M3 && mode != RQ_FP8_UNSCALED && mode != RQ_FP8_PER_TOKEN)
    return set_error(RQ_E_ARG, "bad fp8 mode %d", mode);
  if (m < 0 || n <= 0 || k <= 0)
    return set_error(RQ_E_SHAPE, "bad shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  return RQ_OK;
}

bool geometry(int qtype, Geometry *g) {
  switch (qtype) {
    case RQ_Q4_0: *g = {32, 18}; return true;
    case RQ_Q5_0: *g = {32, 22}; return true;
    case RQ_Q8_0: *g = {32, 34}; return true;
    case RQ_Q4_K: *g = {256, 144}; return true;
    case RQ_Q5_K: *g = {256, 176}; return true;
    case RQ_Q6_K: *g = {256, 210}; return true;
    default: return false;
  }
}

static bool valid_ftype(int t) { return t == RQ_F32 || t == RQ_F16 || t == RQ_BF16; }

static int hip_check(hipError_t e, const char *what) {
  if (e == hipSuccess) return RQ_OK;
  return set_error(e == hipErrorOutOfMemory ? RQ_E_NOMEM : RQ_E_DEVICE, "%s: %s", what,
                   hipGetErrorString(e));
}

// Dequant_tensor's checks on a flat stream of n_elements (dequant.rs:83-95).
static int stream_checks(int qtype, uint64_t nbytes, uint64_t n_elements, Geometry *g) {
  if (!geometry(qtype, g)) return set_error(RQ_E_UNSUPPORTED, "decode of qtype %d not implemented", qtype);
  if (n_elements % (uint64_t)g->elems != 0)
    return set_error(RQ_E_OVERFLOW, "%llu not a multiple of %d", (unsigned long long)n_elements, g->elems);
  const uint64_t need = n_elements / (uint64_t)g->elems * (uint64_t)g->bytes;
  if (nbytes < need)
    return set_error(RQ_E_TRUNCATED, "truncated: %llu bytes, need %llu", (unsigned long long)nbytes,
                     (unsigned long long)need);
  return RQ_OK;
}

static uint64_t align256(uint64_t v) { return (v + 255) & ~(uint64_t)255; }

// Device bytes of the split layout (rq_internal.h) for nblocks blocks, and
// the offset of its scale array.
static uint64_t split_size(int qtype, uint64_t nblocks, uint64_t *aux_off) {
  const uint64_t qbytes = qtype == RQ_Q8_0 ? 32 : qtype == RQ_Q6_K ? 208 : 16;
  const uint64_t abytes = qtype == RQ_Q5_0 ? 8 : 2;
  *aux_off = align256(nblocks * qbytes);
  return *aux_off + nblocks * abytes;
}

// Host-side split of Q8_0 / Q6_K streams into the aligned device layout
// described in rq_internal.h (small tensors; large ones split on the device).
static void split_layout(int qtype, const uint8_t *src, uint64_t nblocks, std::vector<uint8_t> &dst,
                         uint64_t &aux_off) {
  if (qtype == RQ_Q8_0) {
    aux_off = align256(nblocks * 32);
    dst.assign(aux_off + nblocks * 2, 0);
    for (uint64_t b = 0; b < nblocks; ++b) {
      const uint8_t *blk = src + b * 34;
      memcpy(&dst[b * 32], blk + 2, 32);
      memcpy(&dst[aux_off + b * 2], blk, 2);
    }
  } else if (qtype == RQ_Q4_0) {
    aux_off = align256(nblocks * 16);
    dst.assign(aux_off + nblocks * 2, 0);
    for (uint64_t b = 0; b < nblocks; ++b) {
      const uint8_t *blk = src + b * 18;
      memcpy(&dst[b * 16], blk + 2, 16);
      memcpy(&dst[aux_off + b * 2], blk, 2);
    }
  } else if (qtype == RQ_Q5_0) {
    aux_off = align256(nblocks * 16);
    dst.assign(aux_off + nblocks * 8, 0);
    for (uint64_t b = 0; b < nblocks; ++b) {
      const uint8_t *blk = src + b * 22;
      memcpy(&dst[b * 16], blk + 6, 16);
      memcpy(&dst[aux_off + b * 8], blk + 2, 4);  // qh
      memcpy(&dst[aux_off + b * 8 + 4], blk, 2);  // d
    }
  } else {  // Q6_K
    aux_off = align256(nblocks * 208);
    dst.assign(aux_off + nblocks * 2, 0);
    for (uint64_t b = 0; b < nblocks; ++b) {
      const uint8_t *blk = src + b * 210;
      memcpy(&dst[b * 208], blk, 208);
      memcpy(&dst[aux_off + b * 2], blk + 208, 2);
    }
  }
}

}  // namespace rq

using namespace rq;

extern "C" {

int rq_abi_version(void) { return RQ_ABI_VERSION; }

const char *rq_last_error(void) { return g_last_error.c_str(); }

int rq_weight_create(int qtype, const void *host_blocks, size_t nbytes, int64_t n, int64_t k,
                     int device, rq_weight **out) {
  g_last_error.clear();
  if (!out) return set_error(RQ_E_ARG, "out is null");
  *out = nullptr;
  if (!host_blocks) return set_error(RQ_E_ARG, "host_blocks is null");
  if (n <= 0 || k <= 0) return set_error(RQ_E_SHAPE, "shape [%lld, %lld] must be positive", (long long)n, (long long)k);
  Geometry g;
  const uint64_t count = (uint64_t)n * (uint64_t)k;
  int rc = stream_checks(qtype, nbytes, count, &g);
  if (rc) return rc;
  rc = hip_check(hipSetDevice(device), "hipSetDevice");
  if (rc) return rc;
  const uint64_t nblocks = count / (uint64_t)g.elems;
  const uint8_t *src = static_cast<const uint8_t *>(host_blocks);
  const bool split = qtype == RQ_Q8_0 || qtype == RQ_Q6_K || qtype == RQ_Q4_0 || qtype == RQ_Q5_0;
  const uint64_t raw_bytes = nblocks * (uint64_t)g.bytes;
  uint64_t aux_off = 0, bytes = raw_bytes;
  uint8_t *dptr = nullptr;
  if (raw_bytes >= (4ull << 20)) {
    // Large tensors: pinned double-buffered DMA, split on the device.
    if (split) bytes = split_size(qtype, nblocks, &aux_off);
    rc = hip_check(hipMalloc(reinterpret_cast<void **>(&dptr), bytes), "hipMalloc");
    if (rc) return rc;
    if (split) rc = hip_check(hipMemset(dptr, 0, bytes), "hipMemset");
    if (!rc) rc = upload_blocks(qtype, src, nblocks, g.bytes, dptr, aux_off, device);
  } else {
    std::vector<uint8_t> staged;
    if (split) {
      split_layout(qtype, src, nblocks, staged, aux_off);
      src = staged.data();
      bytes = staged.size();
    }
    rc = hip_check(hipMalloc(reinterpret_cast<void **>(&dptr), bytes), "hipMalloc");
    if (rc) return rc;
    rc = hip_check(hipMemcpy(dptr, src, bytes, hipMemcpyHostToDevice), "hipMemcpy");
  }
  if (rc) {
    (void)hipFree(dptr);
    return rc;
  }
  rq_weight *w = new rq_weight;
  w->qtype = qtype;
  w->device = device;
  w->n = n;
  w->k = k;
  w->gguf_bytes = nblocks * (uint64_t)g.bytes;
  w->nblocks = nblocks;
  w->data = dptr;
  w->data_bytes = bytes;
  w->aux_off = aux_off;
  *out = w;
  return RQ_OK;
}

void rq_weight_destroy(rq_weight *w) {
  if (!w) return;
  int cur = 0;
  if (hipGetDevice(&cur) == hipSuccess && cur != w->device) (void)hipSetDevice(w->device);
  (void)hipFree(w->data);
  if (cur != w->device) (void)hipSetDevice(cur);
  delete w;
}

int rq_weight_info(const rq_weight *w, rq_weight_desc *out) {
  if (!w || !out) return set_error(RQ_E_ARG, "null argument");
  out->qtype = w->qtype;
  out->device = w->device;
  out->n = w->n;
  out->k = w->k;
  out->gguf_bytes = w->gguf_bytes;
  out->device_bytes = w->data_bytes;
  return RQ_OK;
}

int rq_dequant_f32(const rq_weight *w, float *dev_out, void *stream) {
  g_last_error.clear();
  if (!w || !dev_out) return set_error(RQ_E_ARG, "null argument");
  int rc = hip_check(hipSetDevice(w->device), "hipSetDevice");
  if (rc) return rc;
  return launch_dequant_weight(w, dev_out, as_stream(stream));
}

int rq_embedding(const rq_weight *w, const uint32_t *ids, int64_t n_ids, float *dev_out, void *stream) {
  g_last_error.clear();
  if (!w) return set_error(RQ_E_ARG, "weight is null");
  if (n_ids < 0) return set_error(RQ_E_ARG, "n_ids %lld is negative", (long long)n_ids);
  if (n_ids == 0) return RQ_OK;
  if (!ids || !dev_out) return set_error(RQ_E_ARG, "null argument");
  if (w->k % 4 != 0) return set_error(RQ_E_UNSUPPORTED, "row length %lld is not a multiple of 4", (long long)w->k);
  for (int64_t i = 0; i < n_ids; ++i)
    if ((int64_t)ids[i] >= w->n)
      return set_error(RQ_E_ARG, "id %u at position %lld is out of range for %lld rows", ids[i], (long long)i,
                       (long long)w->n);
  int rc = hip_check(hipSetDevice(w->device), "hipSetDevice");
  if (rc) return rc;
  const hipStream_t s = as_stream(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return set_error(RQ_E_ARG, "rq_embedding reads host ids and cannot be captured into a graph");
  }
  WsLease ws(w->device, s);
  uint32_t *dids = static_cast<uint32_t *>(ws.get((size_t)n_ids * sizeof(uint32_t), &rc));
  if (!dids) return rc;
  // From pageable memory the copy returns once the ids are staged, so the
  // caller's buffer may be reused on return.
  rc = hip_check(hipMemcpyAsync(dids, ids, (size_t)n_ids * sizeof(uint32_t), hipMemcpyHostToDevice, s),
                 "hipMemcpyAsync");
  if (!rc) rc = launch_gather_rows(w, dids, n_ids, dev_out, s);
  return rc;
}

int rq_dequant_tensor(int qtype, const void *dev_bytes, size_t nbytes, size_t n_elements,
                      float *dev_out, void *stream) {
  g_last_error.clear();
  Geometry g;
  int rc = stream_checks(qtype, nbytes, n_elements, &g);
  if (rc) return rc;
  if (n_elements == 0) return RQ_OK;
  if (!dev_bytes || !dev_out) return set_error(RQ_E_ARG, "null argument");
  return launch_dequant_raw(qtype, static_cast<const uint8_t *>(dev_bytes),
                            n_elements / (uint64_t)g.elems, dev_out, as_stream(stream));
}

static size_t ftype_bytes(int t) { return t == RQ_F32 ? 4 : 2; }

// Argument checks shared by the linear entry points (linear_layer.rs:88-96
// for the width rule).
static int linear_checks(const rq_weight *w, int xtype, int64_t m, int64_t k, const void *bias, int btype,
                         int ytype) {
  if (!w) return set_error(RQ_E_ARG, "weight is null");
  if (!valid_ftype(xtype)) return set_error(RQ_E_ARG, "activation type %d not supported", xtype);
  if (!valid_ftype(ytype)) return set_error(RQ_E_ARG, "output type %d not supported", ytype);
  if (bias && !valid_ftype(btype)) return set_error(RQ_E_ARG, "bias type %d not supported", btype);
  if (k != w->k)
    return set_error(RQ_E_SHAPE, "linear: expected last dim %lld, got %lld", (long long)w->k, (long long)k);
  if (m < 0) return set_error(RQ_E_SHAPE, "negative row count %lld", (long long)m);
  return RQ_OK;
}

// x as the fused kernels read it: 16-byte aligned, else an aligned copy of
// its m * k elements in the workspace.
static const void *aligned_x(const void *x, int xtype, int64_t m, int64_t k, hipStream_t s, WsLease &ws, int *rc) {
  if (reinterpret_cast<uintptr_t>(x) % 16 == 0) return x;
  const size_t bytes = (size_t)m * (size_t)k * ftype_bytes(xtype);
  void *p = ws.get(bytes, rc);
  if (!p) return nullptr;
  *rc = hip_check(hipMemcpyAsync(p, x, bytes, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
  return *rc ? nullptr : p;
}

// One weight: the fused kernels, or the generic one for shapes they do not take.
static int linear_one(const rq_weight *w, const void *xa, int xtype, int64_t m, const Out &o, hipStream_t s,
                      WsLease &ws) {
  int rc = launch_linear_fused(w, xa, xtype, m, o, s, ws);
  if (rc == RQ_E_UNSUPPORTED) rc = launch_linear_generic(w, xa, xtype, m, o, s);
  return rc;
}

int rq_linear_bias(const rq_weight *w, const void *x, int xtype, int64_t m, int64_t k, const void *bias, int btype,
                   void *y, int ytype, void *stream) {
  g_last_error.clear();
  int rc = linear_checks(w, xtype, m, k, bias, btype, ytype);
  if (rc) return rc;
  if (m == 0) return RQ_OK;
  if (!x || !y) return set_error(RQ_E_ARG, "null activation or output");
  rc = hip_check(hipSetDevice(w->device), "hipSetDevice");
  if (rc) return rc;
  const hipStream_t s = as_stream(stream);
  WsLease ws(w->device, s);
  const void *xa = aligned_x(x, xtype, m, k, s, ws, &rc);
  if (!xa) return rc;
  return linear_one(w, xa, xtype, m, Out{y, bias, ytype, btype}, s, ws);
}

int rq_linear(const rq_weight *w, const void *x, int xtype, int64_t m, int64_t k, void *y, int ytype,
              void *stream) {
  return rq_linear_bias(w, x, xtype, m, k, nullptr, RQ_F32, y, ytype, stream);
}

int rq_linear_multi(int count, const rq_weight *const *wts, const void *x, int xtype, int64_t m, int64_t k,
                    const void *const *biases, int btype, void *const *ys, int ytype, void *stream) {
  g_last_error.clear();
  if (count < 0) return set_error(RQ_E_ARG, "negative count %d", count);
  if (count == 0) return RQ_OK;
  if (!wts || !ys) return set_error(RQ_E_ARG, "null weight or output array");
  for (int i = 0; i < count; ++i) {
    const void *b = biases ? biases[i] : nullptr;
    const int rc = linear_checks(wts[i], xtype, m, k, b, btype, ytype);
    if (rc) return rc;
    if (wts[i]->device != wts[0]->device) return set_error(RQ_E_ARG, "weights on different devices");
    if (m > 0 && !ys[i]) return set_error(RQ_E_ARG, "null output %d", i);
  }
  if (m == 0) return RQ_OK;
  if (!x) return set_error(RQ_E_ARG, "null activation");
  int rc = hip_check(hipSetDevice(wts[0]->device), "hipSetDevice");
  if (rc) return rc;
  const hipStream_t s = as_stream(stream);
  WsLease ws(wts[0]->device, s);
  const void *xa = aligned_x(x, xtype, m, k, s, ws, &rc);
  if (!xa) return rc;
  Out outs[kMultiMax];
  for (int i = 0; i < count;) {
    // A run of consecutive weights of one format (at most kMultiMax).
    int j = i + 1;
    while (j < count && j - i < kMultiMax && wts[j]->qtype == wts[i]->qtype) ++j;
    for (int t = i; t < j; ++t) outs[t - i] = Out{ys[t], biases ? biases[t] : nullptr, ytype, btype};
    rc = j - i > 1 ? launch_linear_multi(wts + i, j - i, xa, xtype, m, outs, s, ws) : RQ_E_UNSUPPORTED;
    if (rc == RQ_E_UNSUPPORTED) {
      rc = RQ_OK;
      for (int t = i; t < j && !rc; ++t) rc = linear_one(wts[t], xa, xtype, m, outs[t - i], s, ws);
    }
    if (rc) return rc;
    i = j;
  }
  return RQ_OK;
}

int rq_bias_add(void *y, int ytype, int64_t m, int64_t n, const void *bias, int btype, void *stream) {
  g_last_error.clear();
  if (!valid_ftype(ytype)) return set_error(RQ_E_ARG, "output type %d not supported", ytype);
  if (!valid_ftype(btype)) return set_error(RQ_E_ARG, "bias type %d not supported", btype);
  if (m < 0 || n < 0) return set_error(RQ_E_SHAPE, "bad shape [%lld, %lld]", (long long)m, (long long)n);
  if (m == 0 || n == 0) return RQ_OK;
  if (!y || !bias) return set_error(RQ_E_ARG, "null argument");
  return launch_bias_add(y, ytype, m, n, bias, btype, as_stream(stream));
}

int rq_fp8_quantize(const void *x, int xtype, int64_t m, int64_t k, int mode, uint8_t *xq,
                    float *xscale, void *stream) {
  g_last_error.clear();
  if (!valid_ftype(xtype)) return set_error(RQ_E_ARG, "activation type %d not supported", xtype);
  if (mode != RQ_FP8_UNSCALED && mode != RQ_FP8_PER_TOKEN) return set_error(RQ_E_ARG, "bad fp8 mode %d", mode);
  if (m < 0 || k <= 0) return set_error(RQ_E_SHAPE, "bad shape [%lld, %lld]", (long long)m, (long long)k);
  if (m == 0) return RQ_OK;
  if (!x || !xq || !xscale) return set_error(RQ_E_ARG, "null argument");
  return launch_fp8_quantize(x, xtype, m, k, mode, xq, xscale, as_stream(stream));
}

int rq_fp8_gemm_q(const uint8_t *xq, const float *xscale, int64_t m, const uint8_t *w,
                  const float *w_scale, int64_t n, int64_t k, void *y, int ytype, void *stream) {
  g_last_error.clear();
  if (!valid_ftype(ytype)) return set_error(RQ_E_ARG, "output type %d not supported", ytype);
  if (m < 0 || n <= 0 || k <= 0)
    return set_error(RQ_E_SHAPE, "bad shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  if (m == 0) return RQ_OK;
  if (!xq || !w || !y) return set_error(RQ_E_ARG, "null argument");
  return launch_fp8_gemm(xq, xscale, m, w, w_scale, n, k, y, ytype, as_stream(stream));
}

int rq_fp8_gemm(const void *x, int xtype, int64_t m, const uint8_t *w, const float *w_scale,
                int64_t n, int64_t k, void *y, int ytype, int mode, void *stream) {
  g_last_error.clear();
  if (xtype == RQ_F8E4M3)
    return rq_fp8_gemm_q(static_cast<const uint8_t *>(x), nullptr, m, w, w_scale, n, k, y, ytype, stream);
  if (!valid_ftype(xtype)) return set_error(RQ_E_ARG, "activation type %d not supported", xtype);
  if (mode != RQ_FP8_UNSCALED && mode != RQ_FP8_PER_TOKEN) return set_error(RQ_E_ARG, "bad fp8 mode %d", mode);
  if (m < 0 || n <= 0 || k <= 0)
    return set_error(RQ_E_SHAPE, "bad shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  if (m == 0) return RQ_OK;
  if (!x || !w || !y) return set_error(RQ_E_ARG, "null argument");
  hipStream_t s = as_stream(stream);
  int dev = 0;
  int rc = hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  const uint64_t qbytes = ((uint64_t)m * (uint64_t)k + 255) & ~(uint64_t)255;
  WsLease ws(dev, s);
  uint8_t *scratch = static_cast<uint8_t *>(ws.get(qbytes + (uint64_t)m * 4, &rc));
  if (!scratch) return rc;
  float *xs = reinterpret_cast<float *>(scratch + qbytes);
  rc = launch_fp8_quantize(x, xtype, m, k, mode, scratch, xs, s);
  if (!rc) rc = launch_fp8_gemm(scratch, xs, m, w, w_scale, n, k, y, ytype, s);
  return rc;
}

int rq_marlin_repack(const void *w, int wtype, const float *scales, int64_t n, int64_t k, uint32_t *packed,
                     void *stream) {
  g_last_error.clear();
  if (!valid_ftype(wtype)) return set_error(RQ_E_ARG, "weight type %d not supported", wtype);
  if (n < 0 || k <= 0) return set_error(RQ_E_SHAPE, "bad shape [%lld, %lld]", (long long)n, (long long)k);
  if (n == 0) return RQ_OK;
  if (!w || !scales || !packed) return set_error(RQ_E_ARG, "null argument");
  return launch_marlin_repack(w, wtype, scales, n, k, packed, as_stream(stream));
}

int rq_marlin_dequant(const uint32_t *packed, const float *scales, int64_t n, int64_t k, float *dev_out,
                      void *stream) {
  g_last_error.clear();
  if (n < 0 || k <= 0) return set_error(RQ_E_SHAPE, "bad shape [%lld, %lld]", (long long)n, (long long)k);
  if (n == 0) return RQ_OK;
  if (!packed || !scales || !dev_out) return set_error(RQ_E_ARG, "null argument");
  return launch_marlin_dequant(packed, scales, n, k, dev_out, as_stream(stream));
}

int rq_marlin_linear(const uint32_t *packed, const float *scales, int64_t n, int64_t k, const void *x, int xtype,
                     int64_t m, void *y, int ytype, void *stream) {
  g_last_error.clear();
  if (!valid_ftype(xtype)) return set_error(RQ_E_ARG, "activation type %d not supported", xtype);
  if (!valid_ftype(ytype)) return set_error(RQ_E_ARG, "output type %d not supported", ytype);
  if (m < 0 || n < 0 || k <= 0)
    return set_error(RQ_E_SHAPE, "bad shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  if (m == 0 || n == 0) return RQ_OK;
  if (!packed || !scales || !x || !y) return set_error(RQ_E_ARG, "null argument");
  return launch_marlin_linear(packed, scales, n, k, x, xtype, m, y, ytype, as_stream(stream));
}

static bool valid_kv_mode(int mode) { return mode == RQ_KV_F16 || mode == RQ_KV_FP8 || mode == RQ_KV_INT8; }

int rq_kv_quantize(const void *t, int ttype, int64_t b, int64_t h, int64_t sd, int mode, void *q, float *scales,
                   void *stream) {
  g_last_error.clear();
  if (!valid_ftype(ttype)) return set_error(RQ_E_ARG, "input type %d not supported", ttype);
  if (!valid_kv_mode(mode)) return set_error(RQ_E_ARG, "bad kv mode %d", mode);
  if (b < 0 || h < 0 || sd < 0)
    return set_error(RQ_E_SHAPE, "bad shape [%lld, %lld, %lld]", (long long)b, (long long)h, (long long)sd);
  if (h == 0) return RQ_OK;
  if (!scales) return set_error(RQ_E_ARG, "null scales");
  if (b == 0 || sd == 0) {
    // No elements: every head's maximum is 0, so its scale is the floor,
    // written by a kernel (nothing read from host memory at replay time).
    return launch_kv_fill_scales(scales, h, mode == RQ_KV_F16 ? 1.0f : 1e-8f, as_stream(stream));
  }
  if (!t || !q) return set_error(RQ_E_ARG, "null argument");
  int dev = 0;
  const int rc = hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  WsLease ws(dev, as_stream(stream));
  return launch_kv_quantize(t, ttype, b, h, sd, mode, q, scales, as_stream(stream), ws);
}

int rq_kv_dequantize(const void *q, int mode, const float *scales, int64_t b, int64_t h, int64_t sd, void *out,
                     int otype, void *stream) {
  g_last_error.clear();
  if (!valid_ftype(otype)) return set_error(RQ_E_ARG, "output type %d not supported", otype);
  if (!valid_kv_mode(mode)) return set_error(RQ_E_ARG, "bad kv mode %d", mode);
  if (b < 0 || h < 0 || sd < 0)
    return set_error(RQ_E_SHAPE, "bad shape [%lld, %lld, %lld]", (long long)b, (long long)h, (long long)sd);
  if (b == 0 || h == 0 || sd == 0) return RQ_OK;
  if (!q || !out || (mode != RQ_KV_F16 && !scales)) return set_error(RQ_E_ARG, "null argument");
  return launch_kv_dequantize(q, mode, scales, b, h, sd, out, otype, as_stream(stream));
}

}  // extern "C"
