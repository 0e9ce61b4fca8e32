/*
 * rq_oracle_int4_kv.c -- CPU oracle for the Marlin INT4 weights and the
 * paged-KV FP8 / INT8 quantizer.
 *
 * TEST INFRASTRUCTURE ONLY (see rq_oracle.h): a plain-C restatement of
 * crates/runtimed-model/src/ops/marlin_gemv.rs and
 * crates/runtimed-model/src/cache/paged/quantize.rs, used to check the
 * device kernels and never by the product library.
 *
 * Rust semantics restated here: f32::round rounds half away from zero (C
 * roundf); `x.clamp(lo, hi) as u32 / as i8` maps NaN to 0 and saturates
 * infinities; f32::max returns the non-NaN operand.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "rq_oracle.h"

/* marlin_gemv.rs:66-97 (repack_marlin_tiles): nibble k%8 of word (k%32)/8 of
 * record [k/32][row] is clamp(round(w * inv_s) + 8, 0, 15); inv_s = 1/s when
 * |s| > 1e-12, else 1; positions past k hold 8. */
void rqo_marlin_repack(const float *w, const float *s, int64_t n, int64_t k, uint32_t *packed) {
  const int64_t kc = (k + 31) / 32;
  for (int64_t c = 0; c < kc; ++c) {
    for (int64_t r = 0; r < n; ++r) {
      const float inv_s = fabsf(s[r]) > 1e-12f ? 1.0f / s[r] : 1.0f;
      for (int wi = 0; wi < 4; ++wi) {
        uint32_t word = 0;
        for (int nib = 0; nib < 8; ++nib) {
          const int64_t kk = c * 32 + wi * 8 + nib;
          uint32_t q = 8;
          if (kk < k) {
            const float t = roundf(w[r * k + kk] * inv_s) + 8.0f;
            q = isnan(t) ? 0u : (uint32_t)(t < 0.0f ? 0.0f : (t > 15.0f ? 15.0f : t));
          }
          word |= (q & 0xFu) << (nib * 4);
        }
        packed[(c * n + r) * 4 + wi] = word;
      }
    }
  }
}

/* marlin_gemv.rs:42-61 (MarlinWeight::dequantize): out[r, kk] =
 * (nibble - 8) as f32 * s[r]. */
void rqo_marlin_dequant(const uint32_t *packed, const float *s, int64_t n, int64_t k, float *out) {
  const int64_t kc = (k + 31) / 32;
  for (int64_t c = 0; c < kc; ++c)
    for (int64_t r = 0; r < n; ++r)
      for (int wi = 0; wi < 4; ++wi) {
        const uint32_t word = packed[(c * n + r) * 4 + wi];
        for (int nib = 0; nib < 8; ++nib) {
          const int64_t kk = c * 32 + wi * 8 + nib;
          if (kk < k) out[r * k + kk] = (float)((int)((word >> (nib * 4)) & 0xFu) - 8) * s[r];
        }
      }
}

/* cpu_marlin_gemv_fallback (marlin_gemv.rs:100-116): y = x * dequant^T,
 * accumulated in double (the gate reference). */
void rqo_marlin_gemv_f64(const float *x, int64_t m, const uint32_t *packed, const float *s, int64_t n,
                         int64_t k, double *y) {
  const int64_t kc = (k + 31) / 32;
  for (int64_t i = 0; i < m; ++i)
    for (int64_t r = 0; r < n; ++r) {
      double acc = 0.0;
      for (int64_t c = 0; c < kc; ++c)
        for (int wi = 0; wi < 4; ++wi) {
          const uint32_t word = packed[(c * n + r) * 4 + wi];
          for (int nib = 0; nib < 8; ++nib) {
            const int64_t kk = c * 32 + wi * 8 + nib;
            if (kk < k) acc += (double)x[i * k + kk] * (double)((int)((word >> (nib * 4)) & 0xFu) - 8);
          }
        }
      y[i * n + r] = acc * (double)s[r];
    }
}

/* quantize_fp8 / quantize_int8 (quantize.rs:12-46, 62-96) on t viewed as
 * [b, h, sd]: scale[h] = max(max|t[:, h, :]| / (448 or 127), 1e-8) with NaN
 * elements ignored by the `a > max_abs` test; codes f32_to_fp8_e4m3(v / s)
 * or (i8)clamp(round(v / s), -128, 127). */
void rqo_kv_quantize(const float *t, int64_t b, int64_t h, int64_t sd, int int8, uint8_t *q, float *scales) {
  for (int64_t hh = 0; hh < h; ++hh) {
    float max_abs = 0.0f;
    for (int64_t bb = 0; bb < b; ++bb) {
      const float *p = t + (bb * h + hh) * sd;
      for (int64_t i = 0; i < sd; ++i) {
        const float a = fabsf(p[i]);
        if (a > max_abs) max_abs = a;
      }
    }
    const float sc = max_abs / (int8 ? 127.0f : 448.0f);
    scales[hh] = sc > 1e-8f ? sc : 1e-8f;
  }
  for (int64_t bb = 0; bb < b; ++bb)
    for (int64_t hh = 0; hh < h; ++hh) {
      const int64_t off = (bb * h + hh) * sd;
      for (int64_t i = 0; i < sd; ++i) {
        const float v = t[off + i] / scales[hh];
        if (!int8) {
          q[off + i] = rqo_f32_to_fp8_e4m3(v);
        } else {
          const float r = roundf(v);
          const int8_t c = isnan(r) ? 0 : (int8_t)(r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r));
          memcpy(&q[off + i], &c, 1);
        }
      }
    }
}

/* dequantize_fp8 / dequantize_int8 (quantize.rs:48-57, 98-107) in f32:
 * decode(code) * scale[h]. */
void rqo_kv_dequantize(const uint8_t *q, const float *scales, int64_t b, int64_t h, int64_t sd, int int8,
                       float *out) {
  for (int64_t bb = 0; bb < b; ++bb)
    for (int64_t hh = 0; hh < h; ++hh) {
      const int64_t off = (bb * h + hh) * sd;
      for (int64_t i = 0; i < sd; ++i) {
        const float v = int8 ? (float)(int8_t)q[off + i] : rqo_fp8_e4m3_to_f32(q[off + i]);
        out[off + i] = v * scales[hh];
      }
    }
}
