/*
 * rq_oracle.h -- CPU oracle for the quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of runtimed's
 * scalar CPU semantics (crates/runtimed-gguf/src/quant/ and the FP8
 * helpers in crates/runtimed-model/src/weights/load_safetensors.rs and
 * crates/runtimed-model/src/ops/fp8_gemm.rs).  Only tests/, the smoke check
 * in __graft_entry__.py and the CPU-baseline leg of bench.py may load it, and
 * only to check results or as the timed CPU baseline.  The product library
 * (librq.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates.  How each one is
 * pinned (known-answer tests, closed forms, independent restatements) is
 * listed in tests/test_oracle.py; nothing here is "parity unpinned".
 */
#ifndef RQ_ORACLE_H
#define RQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlDtype ids (crates/runtimed-gguf/src/quant/dtype.rs:6-24). */
enum {
  RQO_F32 = 0, RQO_F16 = 1, RQO_Q4_0 = 2, RQO_Q4_1 = 3, RQO_Q5_0 = 6,
  RQO_Q5_1 = 7, RQO_Q8_0 = 8, RQO_Q8_1 = 9, RQO_Q2K = 10, RQO_Q3K = 11,
  RQO_Q4K = 12, RQO_Q5K = 13, RQO_Q6K = 14, RQO_Q8K = 15, RQO_BF16 = 30
};

/* dequant_tensor error kinds (dequant.rs:84-95, dequant.rs:143). */
enum { RQO_OK = 0, RQO_E_UNSUPPORTED = -1, RQO_E_OVERFLOW = -2, RQO_E_TRUNCATED = -3 };

/* GgmlDtype::block (dtype.rs:49-64): 0 and (elems, bytes) if decodable geometry. */
int rqo_block_geometry(uint32_t dtype, size_t *elems, size_t *bytes);

/* f16_to_f32 (dequant.rs:11-33), bit pattern in and out. */
uint32_t rqo_f16_to_f32_bits(uint16_t h);
float rqo_f16_to_f32(uint16_t h);

/* Block decoders. */
void rqo_dequant_q8_0_block(const uint8_t *blk, float *out32);  /* dequant.rs:40-47  */
void rqo_dequant_q4_0_block(const uint8_t *blk, float *out32);  /* dequant.rs:50-61  */
void rqo_dequant_q5_0_block(const uint8_t *blk, float *out32);  /* dequant.rs:64-77  */
void rqo_dequant_q4_k_block(const uint8_t *blk, float *out256); /* dequant_k.rs:19-44 */
void rqo_dequant_q5_k_block(const uint8_t *blk, float *out256); /* dequant_k.rs:51-80 */
void rqo_dequant_q6_k_block(const uint8_t *blk, float *out256); /* dequant_k.rs:87-111 */

/* dequant_tensor (dequant.rs:83-146): flat decode of n_elements values.
 * Returns RQO_OK or one of the error kinds; `out` holds n_elements floats. */
int rqo_dequant_tensor(uint32_t dtype, const uint8_t *bytes, size_t nbytes,
                       size_t n_elements, float *out);
/* Same, split over `threads` OpenMP threads (the all-core CPU baseline). */
int rqo_dequant_tensor_mt(uint32_t dtype, const uint8_t *bytes, size_t nbytes,
                          size_t n_elements, float *out, int threads);

/* FP8_E4M3_LUT entry (load_safetensors.rs:14-29). */
float rqo_fp8_e4m3_to_f32(uint8_t b);
/* f32_to_fp8_e4m3 (load_safetensors.rs:53-69): nearest LUT value, a tie goes
 * to the lower magnitude, |f| >= 448 saturates to 0x7e, NaN -> 0x7f. */
uint8_t rqo_f32_to_fp8_e4m3(float f);
/* The device's activation encoder: clamp to [-448, 448], then OCP e4m3fn
 * round-to-nearest-even (NaN -> 0x7f). */
uint8_t rqo_f32_to_fp8_e4m3_rne(float f);

/* Dense linear y[m,n] = sum_k x[m,k] * w[n,k] (linear_layer.rs:88-104),
 * accumulated in double: the gate reference for every fused matmul. */
void rqo_linear_f64(const float *x, int64_t m, const float *w, int64_t n,
                    int64_t k, double *y);
/* Same product in f32 with a blocked, OpenMP-parallel loop: the stand-in for
 * candle's CPU f32 matmul (gemm 0.19) in the CPU baseline. */
void rqo_linear_f32(const float *x, int64_t m, const float *w, int64_t n,
                    int64_t k, float *y, int threads);

/* cpu_fp8_gemm_fallback (fp8_gemm.rs:55-74): y = x * (decode(w) * scale)^T,
 * x unquantized, f32 arithmetic.  scale has n entries. */
void rqo_fp8_gemm_fallback(const float *x, int64_t m, const uint8_t *w,
                           const float *scale, int64_t n, int64_t k, float *y);
/* Per-token dynamic activation quantization used by the device FP8 GEMM:
 * s[m] = max|x[m,:]| / 448, q = e4m3_rne(x * (448 / max|x[m,:]|)); a zero row
 * gets s = 0 and all-zero codes. */
void rqo_fp8_quantize_rows(const float *x, int64_t m, int64_t k, uint8_t *xq,
                           float *xscale);
/* The reference's unscaled activation encoding on its CUDA path
 * (fp8_gemm.rs:94-101): every element through f32_to_fp8_e4m3. */
void rqo_fp8_encode_unscaled(const float *x, int64_t count, uint8_t *xq);
/* y[m,n] = xs[m] * ws[n] * sum_k dec(xq[m,k]) * dec(w[n,k]) in double. */
void rqo_fp8_gemm_quantized_f64(const uint8_t *xq, const float *xs, int64_t m,
                                const uint8_t *w, const float *ws, int64_t n,
                                int64_t k, double *y);

/* ---- Marlin INT4 weights (crates/runtimed-model/src/ops/marlin_gemv.rs) ----
 * packed holds ceil(k/32) * n records of 4 u32: record [c][r] carries row r,
 * inputs 32c .. 32c+31, input 32c + 8j + i in bits 4i..4i+3 of word j. */
/* repack_marlin_tiles (marlin_gemv.rs:66-97). */
void rqo_marlin_repack(const float *w, const float *s, int64_t n, int64_t k, uint32_t *packed);
/* MarlinWeight::dequantize (marlin_gemv.rs:42-61): [n, k] f32. */
void rqo_marlin_dequant(const uint32_t *packed, const float *s, int64_t n, int64_t k, float *out);
/* cpu_marlin_gemv_fallback (marlin_gemv.rs:100-116) in double. */
void rqo_marlin_gemv_f64(const float *x, int64_t m, const uint32_t *packed, const float *s, int64_t n,
                         int64_t k, double *y);

/* ---- paged-KV quantizer (crates/runtimed-model/src/cache/paged/quantize.rs) ----
 * t is [b, h, sd] f32 (sd = tokens * head_dim); int8 selects quantize_int8. */
void rqo_kv_quantize(const float *t, int64_t b, int64_t h, int64_t sd, int int8, uint8_t *q,
                     float *scales);
void rqo_kv_dequantize(const uint8_t *q, const float *scales, int64_t b, int64_t h, int64_t sd, int int8,
                       float *out);

#ifdef __cplusplus
}
#endif
#endif
