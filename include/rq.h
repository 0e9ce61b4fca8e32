/*
 * rq.h -- C ABI of librq, the MI355X (gfx950) quantized linear-layer library.
 *
 * This is the drop-in boundary for runtimed's quantized linear path.  Each
 * entry point names the reference interface it replaces (paths relative to
 * the runtimed repository root):
 *
 *   rq_weight_create / rq_weight_destroy
 *       candle `qtensor_from_ggml` + `QMatMul::from_arc`, reached from
 *       crates/runtimed-model/src/weights/load_gguf.rs:28-38; the handle is the
 *       value held in `Weights::q_map` (crates/runtimed-model/src/weights/store.rs:18)
 *       behind an Arc and released by its Drop.
 *   rq_weight_info
 *       `QTensor::storage_size_in_bytes` as summed by `Weights::resident_bytes`
 *       (store.rs:57-76), plus the shape candle keeps as [dims1, dims0]
 *       (load_gguf.rs:35).
 *   rq_dequant_f32
 *       `QTensor::dequantize` as called by `Weights::get` (store.rs:88-94),
 *       with runtimed-gguf's bit-exact semantics
 *       (crates/runtimed-gguf/src/quant/dequant.rs:83-146).
 *   rq_embedding
 *       `QMatMul::embedding` as called by `Weights::embed` and
 *       `Weights::candidate_weights` (crates/runtimed-model/src/weights/embed_layer.rs:16-84).
 *   rq_dequant_tensor
 *       `dequant_tensor` (crates/runtimed-gguf/src/quant/dequant.rs:83-146) on
 *       GGUF bytes already in device memory, same error rules.
 *   rq_linear
 *       `QMatMul::forward` as called by `Weights::linear`
 *       (crates/runtimed-model/src/weights/linear_layer.rs:45-52), with the
 *       last-dimension check of linear_layer.rs:88-96 (ModelError::Shape).
 *   rq_linear_bias
 *       `Weights::linear_bias` (linear_layer.rs:107-118) on a quantized
 *       weight: the linear and the bias's broadcast add in one launch.
 *   rq_linear_multi
 *       consecutive `Weights::linear` / `linear_bias` calls on one input, as
 *       the q/k/v and gate/up projections of qwen2.rs:99-125 and
 *       gemma4.rs:118-156 make them: one launch where the shapes allow.
 *   rq_bias_add
 *       the `broadcast_add` of linear_bias (linear_layer.rs:111-115) for an
 *       output that another path produced (FP8, Marlin).
 *   rq_fp8_quantize, rq_fp8_gemm
 *       `SubstratePort::fp8_gemm` (crates/runtimed-model/src/substrate/port.rs:73)
 *       -> `ops::fp8_gemm` (crates/runtimed-model/src/ops/fp8_gemm.rs:77-191),
 *       used by `Fp8Weight::forward` (crates/runtimed-model/src/weights/fp8_weight.rs:95-97)
 *       and by the F8E4M3 branch of `Weights::linear_dense` (linear_layer.rs:78-87).
 *   rq_marlin_repack, rq_marlin_dequant, rq_marlin_linear
 *       `repack_marlin_tiles`, `MarlinWeight::dequantize` and `marlin_gemv`
 *       (crates/runtimed-model/src/ops/marlin_gemv.rs:42-202), reached through
 *       `SubstratePort::marlin_gemv` (substrate/port.rs:76) from the Marlin
 *       branch of `Weights::linear` (linear_layer.rs:53-63).
 *   rq_kv_quantize, rq_kv_dequantize
 *       `quantize_block_kv` / `quantize_fp8` / `quantize_int8` and
 *       `dequantize_fp8` / `dequantize_int8`
 *       (crates/runtimed-model/src/cache/paged/quantize.rs:12-123), called by
 *       `allocate_block_with_offset` (cache/paged/table.rs:44) and
 *       `QuantizedCacheBlock::dequantize_{k,v}` (cache/paged/block.rs:85-140).
 *   rq_last_error
 *       the message carried by `ModelError::{Shape, Config}`
 *       (crates/runtimed-model/src/error.rs:5-27).
 *
 * Conventions
 *   - Every call returns RQ_OK (0) or a negative rq_status; the thread-local
 *     message from rq_last_error() says what was wrong.
 *   - Shapes follow candle: a weight is [n, k] (n output rows, k inputs,
 *     GGUF dims [k, n]); y[m, n] = sum_k x[m, k] * W[n, k].  Rows are cut from
 *     the flat GGUF block stream, so a block may straddle two rows when k is
 *     not a multiple of the block size (dequant.rs:83-91 checks only the total).
 *   - Activation, output and scale pointers are device pointers owned by the
 *     caller; `stream` is a hipStream_t (NULL = the legacy default stream).
 *     All launches are asynchronous on `stream`.
 *   - Calls on different handles and streams may run concurrently from
 *     different threads.  A weight handle is immutable after creation.
 *   - The device is bound per call: every entry point makes the handle's
 *     device current on the calling thread (store.rs:128-145 does the same
 *     with `ensure_current`).
 */
#ifndef RQ_H
#define RQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RQ_ABI_VERSION 2

/* Block formats, numbered as GgmlDtype (crates/runtimed-gguf/src/quant/dtype.rs:6-24). */
typedef enum rq_qtype {
  RQ_Q4_0 = 2,
  RQ_Q5_0 = 6,
  RQ_Q8_0 = 8,
  RQ_Q4_K = 12,
  RQ_Q5_K = 13,
  RQ_Q6_K = 14
} rq_qtype;

/* Dense element types for activations and outputs.  F32/F16/BF16 keep their
 * GgmlDtype ids; F8E4M3 (OCP e4m3fn, as candle's DType::F8E4M3) has none. */
typedef enum rq_ftype {
  RQ_F32 = 0,
  RQ_F16 = 1,
  RQ_BF16 = 30,
  RQ_F8E4M3 = 128
} rq_ftype;

typedef enum rq_status {
  RQ_OK = 0,
  RQ_E_UNSUPPORTED = -1, /* GgufError::Unsupported (dequant.rs:84-86) */
  RQ_E_OVERFLOW = -2,    /* GgufError::Overflow: n % block elems != 0 (dequant.rs:87-91) */
  RQ_E_TRUNCATED = -3,   /* GgufError::Truncated: too few bytes (dequant.rs:92-95) */
  RQ_E_SHAPE = -4,       /* ModelError::Shape (error.rs:13-18) */
  RQ_E_ARG = -5,         /* null pointer, bad enum or negative size */
  RQ_E_DEVICE = -6,      /* a HIP runtime call failed */
  RQ_E_NOMEM = -7        /* device allocation failed */
} rq_status;

/* Activation encodings for the FP8 GEMM. */
typedef enum rq_fp8_mode {
  /* x -> e4m3 with no scale through the reference encoder (nearest, ties to
   * the lower magnitude, saturating at 448): the CUDA path's semantics,
   * fp8_gemm.rs:94-101. */
  RQ_FP8_UNSCALED = 0,
  /* per-row dynamic scale s[m] = max|x[m,:]| / 448, codes
   * e4m3_rne(x * (448 / max|x[m,:]|)); y is multiplied back by s[m]. */
  RQ_FP8_PER_TOKEN = 1
} rq_fp8_mode;

/* KV-cache block precision (CachePrecision, cache/paged/block.rs:23-27). */
typedef enum rq_kv_mode {
  RQ_KV_F16 = 0,  /* attention-sink / Fp16 blocks: a cast, scales 1 */
  RQ_KV_FP8 = 1,  /* e4m3 codes, per-head scale max|t| / 448 */
  RQ_KV_INT8 = 2  /* int8 codes, per-head scale max|t| / 127 */
} rq_kv_mode;

typedef struct rq_weight rq_weight;

typedef struct rq_weight_desc {
  int32_t qtype;          /* rq_qtype */
  int32_t device;         /* HIP device ordinal */
  int64_t n;              /* output rows */
  int64_t k;              /* inputs per row */
  uint64_t gguf_bytes;    /* size of the GGUF block stream: n*k/elems*block_bytes */
  uint64_t device_bytes;  /* device memory held by the handle */
} rq_weight_desc;

/* ABI version of the loaded library (RQ_ABI_VERSION at build time). */
int rq_abi_version(void);

/* Thread-local description of the last error on this thread ("" if none). */
const char *rq_last_error(void);

/* Upload one GGUF tensor of n x k elements in block format `qtype` from host
 * memory to `device`.  nbytes must cover n*k/elems*block_bytes
 * (header.rs:191-205); n*k must be a multiple of the block size.  Q8_0 and
 * Q6_K are split into 16-byte-aligned arrays on the device; the element
 * values are unchanged.  The handle owns its device memory. */
int rq_weight_create(int qtype, const void *host_blocks, size_t nbytes, int64_t n,
                     int64_t k, int device, rq_weight **out);

/* Release a handle and its device memory.  NULL is ignored. */
void rq_weight_destroy(rq_weight *w);

int rq_weight_info(const rq_weight *w, rq_weight_desc *out);

/* Decode the whole weight to f32 (n*k values, row-major [n, k]) into device
 * memory.  Bit-identical to runtimed-gguf's dequant_tensor. */
int rq_dequant_f32(const rq_weight *w, float *dev_out, void *stream);

/* Rows ids[0 .. n_ids) of the weight, decoded bit-identically to
 * rq_dequant_f32, as f32 [n_ids, k] in device memory: the quantized branch
 * of Weights::embed / Weights::candidate_weights (embed_layer.rs:16-84,
 * QMatMul::embedding).  ids are in host memory and may be reused when the
 * call returns; an id >= n gives RQ_E_ARG and nothing is written; n_ids == 0
 * is a no-op.  Requires k % 4 == 0 (RQ_E_UNSUPPORTED otherwise).  Not for
 * stream capture (a captured copy would read the caller's host buffer when
 * the graph runs): a capturing stream gives RQ_E_ARG. */
int rq_embedding(const rq_weight *w, const uint32_t *ids, int64_t n_ids, float *dev_out, void *stream);

/* Decode a flat GGUF block stream that already sits in device memory, with
 * dequant_tensor's rules: RQ_E_UNSUPPORTED for a type without a decoder,
 * RQ_E_OVERFLOW if n_elements is not a block multiple, RQ_E_TRUNCATED if
 * nbytes is short. */
int rq_dequant_tensor(int qtype, const void *dev_bytes, size_t nbytes, size_t n_elements,
                      float *dev_out, void *stream);

/* y[m, n] = sum_k x[m, k] * W[n, k] for an m x k activation (row-major, type
 * xtype in {F32, F16, BF16}) into y (row-major m x n, type ytype in {F32, F16,
 * BF16}).  Accumulation is in f32.  k is the activation's last dimension: a
 * k that differs from the weight's gives RQ_E_SHAPE and launches nothing
 * (linear_layer.rs:88-96).  m = 0 is a no-op.  x may have any alignment (an
 * x that is not 16-byte aligned is first copied, m*k elements, into the
 * stream's workspace).  Scratch comes from a per-(device, stream) workspace
 * that the library keeps between calls: a graph captured from a stream
 * refers to that stream's workspace, so it must not run concurrently with
 * other librq calls on the stream it was captured from. */
int rq_linear(const rq_weight *w, const void *x, int xtype, int64_t m, int64_t k, void *y, int ytype,
              void *stream);

/* rq_linear plus a bias of n values (type btype in {F32, F16, BF16}, device
 * memory) added to every row, as linear_bias does (the bias cast to y's
 * type, then added).  The add happens in the kernels' epilogues with the
 * reference's two roundings: y = ((acc as ytype) + (bias as ytype)) as ytype,
 * the same bits as rq_linear followed by rq_bias_add (for F32 outputs both
 * roundings are the identity).  A null bias is rq_linear. */
int rq_linear_bias(const rq_weight *w, const void *x, int xtype, int64_t m, int64_t k, const void *bias, int btype,
                   void *y, int ytype, void *stream);

/* count linears on one activation x [m, k]: ys[i][m, n_i] = x W_i^T
 * (+ biases[i] when biases and biases[i] are not null, all of type btype).
 * Every weight lives on one device and has k inputs (RQ_E_SHAPE
 * otherwise).  At m = 1 and 2, runs of up to 4 consecutive weights of one
 * format whose rows hold at most 64 pieces (k <= 2048 for Q4_K / Q5_K /
 * Q8_0 / Q4_0 / Q5_0, k <= 4096 for Q6_K) take one launch, and so do bf16 activations
 * with 3 <= m <= 64 and f32 activations with 4 <= m <= 64 (the small-M
 * matrix-core kernels; f32 as two bf16 limbs per activation, against the
 * weights' integer codes for Q4_K / Q6_K / Q8_0 at m <= 16); other weights
 * take the launches rq_linear_bias would make.  At m <= 2 each output equals
 * that call's output bit for bit; in the small-M sets the K split (and, for
 * f32, the kernel) can differ from a single weight's, so sums can differ in
 * their last bits (every result is deterministic: the same call gives the
 * same bits). */
int rq_linear_multi(int count, const rq_weight *const *ws, const void *x, int xtype, int64_t m, int64_t k,
                    const void *const *biases, int btype, void *const *ys, int ytype, void *stream);

/* y[m, n] += bias[n] in y's type (type ytype, device memory, row-major):
 * the bias cast to ytype, the sum rounded to ytype (linear_layer.rs:111-115). */
int rq_bias_add(void *y, int ytype, int64_t m, int64_t n, const void *bias, int btype, void *stream);

/* Encode an m x k activation (F32, F16 or BF16) to e4m3 codes xq (m*k bytes)
 * and per-row scales xscale (m floats) according to `mode` (RQ_FP8_UNSCALED
 * writes scale 1). */
int rq_fp8_quantize(const void *x, int xtype, int64_t m, int64_t k, int mode, uint8_t *xq,
                    float *xscale, void *stream);

/* FP8 e4m3 GEMM: y[m, n] = sx[m] * w_scale[n] * sum_k xq[m, k] * w[n, k] on
 * CDNA4 fp8 matrix cores with f32 accumulation.  w is n x k e4m3 codes,
 * w_scale has n floats (or NULL for all ones, linear_layer.rs:82-85).  If
 * xtype is RQ_F8E4M3, x holds codes used as they are (sx = 1); otherwise x is
 * encoded first according to `mode`, into the stream's workspace.
 * ytype is F32, F16 or BF16. */
int rq_fp8_gemm(const void *x, int xtype, int64_t m, const uint8_t *w, const float *w_scale,
                int64_t n, int64_t k, void *y, int ytype, int mode, void *stream);

/* rq_fp8_gemm that allocates nothing.  NO COUNTERPART IN THE REFERENCE: it
 * is for callers that cannot allocate device memory -- code under HIP graph
 * capture that must not record allocations, tight serving loops, harnesses
 * that forbid hipMalloc.  Same arguments, kernels and results as
 * rq_fp8_gemm; the activation codes and per-row scales go to a fixed
 * scratch array of RQ_NOALLOC_SCRATCH_BYTES in the library, one per GPU,
 * held until the process ends.  Activations that need more
 * (align256(m * k) + 4 m bytes; 2048 x 4096 needs 8 MiB + 8 KiB) give
 * RQ_E_ARG and launch nothing; e4m3 activations need no scratch.  Every call
 * on one GPU shares that GPU's array: calls that overlap on a GPU (other
 * streams, or replays of a graph holding this call beside eager calls) race
 * on it. */
#define RQ_NOALLOC_SCRATCH_BYTES (16u << 20)
int rq_fp8_gemm_noalloc(const void *x, int xtype, int64_t m, const uint8_t *w, const float *w_scale,
                        int64_t n, int64_t k, void *y, int ytype, int mode, void *stream);

/* The GEMM proper on codes already encoded by rq_fp8_quantize (xscale may be
 * NULL for all ones). */
int rq_fp8_gemm_q(const uint8_t *xq, const float *xscale, int64_t m, const uint8_t *w,
                  const float *w_scale, int64_t n, int64_t k, void *y, int ytype,
                  void *stream);

/* ---- Marlin INT4 weights (marlin_gemv.rs) ----
 * packed: u32 [ceil(k/32)][n][4] in device memory; record [c][r] carries row
 * r, inputs 32c .. 32c+31, input 32c + 8j + i in bits 4i .. 4i+3 of word j;
 * weight = (nibble - 8) * scales[r] (scales: n f32 in device memory). */

/* repack_marlin_tiles (marlin_gemv.rs:66-97) on the device: w is [n, k] of
 * type wtype (F32, F16 or BF16); nibble = clamp(round(w / s) + 8, 0, 15)
 * with round half away from zero, computed as w * (1 / s) (1 when
 * |s| <= 1e-12), NaN -> 0; inputs past k in the last record are 8. */
int rq_marlin_repack(const void *w, int wtype, const float *scales, int64_t n, int64_t k,
                     uint32_t *packed, void *stream);

/* MarlinWeight::dequantize (marlin_gemv.rs:42-61): [n, k] f32, bit-exact. */
int rq_marlin_dequant(const uint32_t *packed, const float *scales, int64_t n, int64_t k,
                      float *dev_out, void *stream);

/* marlin_gemv (marlin_gemv.rs:119-202): y[m, n] = scales[n] * sum_k x[m, k] *
 * (q[n, k] - 8), f32 accumulation; x is m x k (F32, F16 or BF16), y is m x n
 * of type ytype.  m = 0 is a no-op (the reference returns an empty tensor). */
int rq_marlin_linear(const uint32_t *packed, const float *scales, int64_t n, int64_t k,
                     const void *x, int xtype, int64_t m, void *y, int ytype, void *stream);

/* ---- paged-KV block quantizer (cache/paged/quantize.rs) ----
 * t is a K or V chunk viewed as [b, h, sd] (sd = tokens * head_dim; a tensor
 * that is not 4-D is [1, 1, numel, 1], quantize.rs:14-18), type ttype in
 * {F32, F16, BF16}.  RQ_KV_FP8 / RQ_KV_INT8: scales[h] =
 * max(max|t[:, h, :]| / (448 | 127), 1e-8) (NaN elements ignored) and
 * q (b*h*sd bytes) = f32_to_fp8_e4m3(t / s) or (i8)clamp(round(t / s),
 * -128, 127) (NaN -> 0).  RQ_KV_F16: q holds b*h*sd f16 (t cast, round to
 * nearest even) and every scale is 1.  The per-head partial maxima live in
 * the stream's workspace.  With b = 0 or sd = 0 (no elements) every scale is
 * the floor (1e-8, or 1 for RQ_KV_F16), written by a kernel; no call reads
 * host memory at launch time, so every shape may be captured in a graph. */
int rq_kv_quantize(const void *t, int ttype, int64_t b, int64_t h, int64_t sd, int mode, void *q,
                   float *scales, void *stream);

/* dequantize_fp8 / dequantize_int8 (quantize.rs:48-57, 98-107): out =
 * decode(q) * scales[h] (f32 product) as otype (F32, F16 or BF16); RQ_KV_F16
 * casts the f16 values (scales unused, may be NULL). */
int rq_kv_dequantize(const void *q, int mode, const float *scales, int64_t b, int64_t h, int64_t sd,
                     void *out, int otype, void *stream);

#ifdef __cplusplus
}
#endif
#endif
