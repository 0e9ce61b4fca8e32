/*
 * rq_oracle.c -- CPU oracle for the quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY (see rq_oracle.h).  A restatement, in plain C, of
 * runtimed's scalar Rust semantics.  Built with -ffp-contract=off so every
 * f32 expression rounds exactly where the Rust source rounds.
 */
#include "rq_oracle.h"

#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* dtype.rs:49-64 */
int rqo_block_geometry(uint32_t dtype, size_t *elems, size_t *bytes) {
  size_t e, b;
  switch (dtype) {
    case RQO_F32: e = 1; b = 4; break;
    case RQO_F16: case RQO_BF16: e = 1; b = 2; break;
    case RQO_Q4_0: e = 32; b = 18; break;
    case RQO_Q5_0: e = 32; b = 22; break;
    case RQO_Q8_0: e = 32; b = 34; break;
    case RQO_Q2K: e = 256; b = 84; break;
    case RQO_Q3K: e = 256; b = 110; break;
    case RQO_Q4K: e = 256; b = 144; break;
    case RQO_Q5K: e = 256; b = 176; break;
    case RQO_Q6K: e = 256; b = 210; break;
    default: return RQO_E_UNSUPPORTED;
  }
  if (elems) *elems = e;
  if (bytes) *bytes = b;
  return RQO_OK;
}

/* dequant.rs:11-33 */
uint32_t rqo_f16_to_f32_bits(uint16_t bits) {
  uint32_t sign = (bits >> 15) & 1u;
  uint32_t exp = (bits >> 10) & 0x1Fu;
  uint32_t mant = bits & 0x3FFu;
  if (exp == 0) {
    if (mant == 0) return sign << 31;
    uint32_t m = mant;
    int32_t e = 127 - 14;
    while ((m & 0x400u) == 0) {
      m <<= 1;
      e -= 1;
    }
    return (sign << 31) | ((uint32_t)e << 23) | ((m & 0x3FFu) << 13);
  }
  if (exp == 31) return (sign << 31) | (0xFFu << 23) | (mant << 13);
  return (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
}

float rqo_f16_to_f32(uint16_t bits) {
  uint32_t u = rqo_f16_to_f32_bits(bits);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* dequant.rs:35-37 */
static float read_f16(const uint8_t *p) {
  return rqo_f16_to_f32((uint16_t)(p[0] | ((uint16_t)p[1] << 8)));
}

/* dequant.rs:40-47 */
void rqo_dequant_q8_0_block(const uint8_t *blk, float *out) {
  float d = read_f16(blk);
  for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)blk[2 + i];
}

/* dequant.rs:50-61 */
void rqo_dequant_q4_0_block(const uint8_t *blk, float *out) {
  float d = read_f16(blk);
  for (int i = 0; i < 16; ++i) {
    uint8_t byte = blk[2 + i];
    int v0 = (int)(byte & 0x0F) - 8;
    int v1 = (int)(byte >> 4) - 8;
    out[i] = d * (float)v0;
    out[i + 16] = d * (float)v1;
  }
}

/* dequant.rs:64-77 */
void rqo_dequant_q5_0_block(const uint8_t *blk, float *out) {
  float d = read_f16(blk);
  uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                ((uint32_t)blk[5] << 24);
  for (int i = 0; i < 16; ++i) {
    uint8_t byte = blk[6 + i];
    uint8_t h0 = (uint8_t)((qh >> i) & 1u);
    uint8_t h1 = (uint8_t)((qh >> (i + 16)) & 1u);
    int v0 = (int)(int8_t)((byte & 0x0F) | (h0 << 4)) - 16;
    int v1 = (int)(int8_t)((byte >> 4) | (h1 << 4)) - 16;
    out[i] = d * (float)v0;
    out[i + 16] = d * (float)v1;
  }
}

/* scale_min_k4, dequant_k.rs:8-16 */
static void scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
    *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

/* dequant_k.rs:19-44 */
void rqo_dequant_q4_k_block(const uint8_t *blk, float *out) {
  float d = read_f16(blk);
  float mn = read_f16(blk + 2);
  const uint8_t *scales = blk + 4;
  const uint8_t *qs = blk + 16;
  int o = 0, is = 0;
  for (int chunk = 0; chunk < 4; ++chunk) {
    const uint8_t *q = qs + chunk * 32;
    uint8_t sc, m;
    scale_min_k4(is, scales, &sc, &m);
    float d1 = d * (float)sc, m1 = mn * (float)m;
    scale_min_k4(is + 1, scales, &sc, &m);
    float d2 = d * (float)sc, m2 = mn * (float)m;
    for (int l = 0; l < 32; ++l) out[o++] = d1 * (float)(q[l] & 0xF) - m1;
    for (int l = 0; l < 32; ++l) out[o++] = d2 * (float)(q[l] >> 4) - m2;
    is += 2;
  }
}

/* dequant_k.rs:51-80 */
void rqo_dequant_q5_k_block(const uint8_t *blk, float *out) {
  float d = read_f16(blk);
  float mn = read_f16(blk + 2);
  const uint8_t *scales = blk + 4;
  const uint8_t *qh = blk + 16;
  const uint8_t *qs = blk + 48;
  int o = 0, is = 0;
  uint8_t u1 = 1, u2 = 2;
  for (int chunk = 0; chunk < 4; ++chunk) {
    const uint8_t *q = qs + chunk * 32;
    uint8_t sc, m;
    scale_min_k4(is, scales, &sc, &m);
    float d1 = d * (float)sc, m1 = mn * (float)m;
    scale_min_k4(is + 1, scales, &sc, &m);
    float d2 = d * (float)sc, m2 = mn * (float)m;
    for (int l = 0; l < 32; ++l) {
      float hi = (qh[l] & u1) ? 16.0f : 0.0f;
      out[o++] = d1 * ((float)(q[l] & 0xF) + hi) - m1;
    }
    for (int l = 0; l < 32; ++l) {
      float hi = (qh[l] & u2) ? 16.0f : 0.0f;
      out[o++] = d2 * ((float)(q[l] >> 4) + hi) - m2;
    }
    is += 2;
    u1 = (uint8_t)(u1 << 2);
    u2 = (uint8_t)(u2 << 2);
  }
}

/* dequant_k.rs:87-111 */
void rqo_dequant_q6_k_block(const uint8_t *blk, float *out) {
  const uint8_t *ql0 = blk, *qh0 = blk + 128, *sc0 = blk + 192;
  float d = read_f16(blk + 208);
  for (int half = 0; half < 2; ++half) {
    const uint8_t *ql = ql0 + half * 64, *qh = qh0 + half * 32, *sc = sc0 + half * 8;
    float *y = out + half * 128;
    for (int l = 0; l < 32; ++l) {
      int is = l / 16;
      float q[4];
      q[0] = (float)(int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32.0f;
      q[1] = (float)(int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32.0f;
      q[2] = (float)(int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32.0f;
      q[3] = (float)(int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32.0f;
      for (int k = 0; k < 4; ++k) y[l + k * 32] = d * (float)(int8_t)sc[is + k * 2] * q[k];
    }
  }
}

typedef void (*block_fn)(const uint8_t *, float *);

static void decode_range(uint32_t dtype, const uint8_t *bytes, size_t b0, size_t b1,
                         size_t elems, size_t bb, float *out) {
  block_fn fn = 0;
  switch (dtype) {
    case RQO_Q4_0: fn = rqo_dequant_q4_0_block; break;
    case RQO_Q5_0: fn = rqo_dequant_q5_0_block; break;
    case RQO_Q8_0: fn = rqo_dequant_q8_0_block; break;
    case RQO_Q4K: fn = rqo_dequant_q4_k_block; break;
    case RQO_Q5K: fn = rqo_dequant_q5_k_block; break;
    case RQO_Q6K: fn = rqo_dequant_q6_k_block; break;
    default: break;
  }
  for (size_t b = b0; b < b1; ++b) {
    const uint8_t *c = bytes + b * bb;
    float *o = out + b * elems;
    if (fn) {
      fn(c, o);
    } else if (dtype == RQO_F32) {
      memcpy(o, c, 4);
    } else if (dtype == RQO_F16) {
      *o = rqo_f16_to_f32((uint16_t)(c[0] | ((uint16_t)c[1] << 8)));
    } else { /* BF16, dequant.rs:113-117 */
      uint32_t u = ((uint32_t)(c[0] | ((uint16_t)c[1] << 8))) << 16;
      memcpy(o, &u, 4);
    }
  }
}

static int tensor_checks(uint32_t dtype, size_t nbytes, size_t n, size_t *elems, size_t *bb) {
  if (rqo_block_geometry(dtype, elems, bb) != RQO_OK) return RQO_E_UNSUPPORTED;
  if (n % *elems != 0) return RQO_E_OVERFLOW;
  if (nbytes < n / *elems * *bb) return RQO_E_TRUNCATED;
  /* Q2K/Q3K have geometry but no decoder (dequant.rs:143). */
  if (dtype == RQO_Q2K || dtype == RQO_Q3K) return RQO_E_UNSUPPORTED;
  return RQO_OK;
}

/* dequant.rs:83-146 */
int rqo_dequant_tensor(uint32_t dtype, const uint8_t *bytes, size_t nbytes, size_t n,
                       float *out) {
  size_t elems, bb;
  int rc = tensor_checks(dtype, nbytes, n, &elems, &bb);
  if (rc != RQO_OK) return rc;
  decode_range(dtype, bytes, 0, n / elems, elems, bb, out);
  return RQO_OK;
}

int rqo_dequant_tensor_mt(uint32_t dtype, const uint8_t *bytes, size_t nbytes, size_t n,
                          float *out, int threads) {
  size_t elems, bb;
  int rc = tensor_checks(dtype, nbytes, n, &elems, &bb);
  if (rc != RQO_OK) return rc;
  long long nb = (long long)(n / elems);
  if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (long long t = 0; t < threads; ++t) {
    size_t b0 = (size_t)(nb * t / threads), b1 = (size_t)(nb * (t + 1) / threads);
    decode_range(dtype, bytes, b0, b1, elems, bb, out);
  }
  return RQO_OK;
}

/* load_safetensors.rs:14-29 */
float rqo_fp8_e4m3_to_f32(uint8_t b) {
  float sign = (b & 0x80) ? -1.0f : 1.0f;
  int exp = (b >> 3) & 0x0F;
  float mant = (float)(b & 0x07);
  if (exp == 0) return sign * ldexpf(1.0f, -6) * (mant / 8.0f);
  if (exp == 15 && (b & 0x07) == 0x07) return NAN;
  return sign * ldexpf(1.0f, exp - 7) * (1.0f + mant / 8.0f);
}

/* load_safetensors.rs:53-69 */
uint8_t rqo_f32_to_fp8_e4m3(float f) {
  if (isnan(f)) return 0x7f;
  uint8_t sign = signbit(f) ? 0x80 : 0;
  float a = fabsf(f);
  if (a <= 0.0f) return sign;
  if (a >= 448.0f) return sign | 0x7e;
  /* binary_search_by over LUT[..127]: first index whose value is >= a. */
  int lo = 0, hi = 127;
  while (lo < hi) {
    int mid = (lo + hi) / 2;
    if (rqo_fp8_e4m3_to_f32((uint8_t)mid) < a) lo = mid + 1;
    else hi = mid;
  }
  int idx = lo;
  if (idx < 127 && rqo_fp8_e4m3_to_f32((uint8_t)idx) == a) return sign | (uint8_t)idx;
  if (idx == 0) return sign;
  if (idx >= 127) return sign | 0x7e;
  float below = rqo_fp8_e4m3_to_f32((uint8_t)(idx - 1));
  float above = rqo_fp8_e4m3_to_f32((uint8_t)idx);
  int pick = (a - below <= above - a) ? idx - 1 : idx;
  return sign | (uint8_t)pick;
}

uint8_t rqo_f32_to_fp8_e4m3_rne(float f) {
  if (isnan(f)) return 0x7f;
  uint8_t sign = signbit(f) ? 0x80 : 0;
  float a = fabsf(f);
  if (a > 448.0f) a = 448.0f;
  if (a < 0.015625f) { /* below 2^-6: multiples of 2^-9 */
    float q = nearbyintf(a * 512.0f);
    return sign | (uint8_t)q;
  }
  uint32_t u;
  memcpy(&u, &a, 4);
  int e = (int)((u >> 23) & 0xFF) - 127;
  uint32_t man = u & 0x7FFFFFu;
  uint32_t r = man >> 20, rem = man & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) r += 1;
  if (r == 8) {
    r = 0;
    e += 1;
  }
  return sign | (uint8_t)(((e + 7) << 3) | (int)r);
}

void rqo_linear_f64(const float *x, int64_t m, const float *w, int64_t n, int64_t k,
                    double *y) {
#pragma omp parallel for schedule(static)
  for (int64_t j = 0; j < n; ++j) {
    const float *wr = w + j * k;
    for (int64_t i = 0; i < m; ++i) {
      const float *xr = x + i * k;
      double acc = 0.0;
      for (int64_t t = 0; t < k; ++t) acc += (double)xr[t] * (double)wr[t];
      y[i * n + j] = acc;
    }
  }
}

void rqo_fp8_gemm_fallback(const float *x, int64_t m, const uint8_t *w, const float *scale,
                           int64_t n, int64_t k, float *y) {
  /* w_scaled = w_f32 * scale (fp8_gemm.rs:60-63), then x * w_scaled^T
   * (fp8_gemm.rs:68).  candle's gemm summation order is not specified, so the
   * dot product is accumulated in double and rounded once. */
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double acc = 0.0;
      for (int64_t t = 0; t < k; ++t) {
        float ws = rqo_fp8_e4m3_to_f32(w[j * k + t]) * scale[j];
        acc += (double)x[i * k + t] * (double)ws;
      }
      y[i * n + j] = (float)acc;
    }
}

void rqo_fp8_quantize_rows(const float *x, int64_t m, int64_t k, uint8_t *xq, float *xscale) {
  for (int64_t i = 0; i < m; ++i) {
    const float *r = x + i * k;
    float amax = 0.0f;
    for (int64_t t = 0; t < k; ++t) amax = fmaxf(amax, fabsf(r[t]));
    if (amax == 0.0f) {
      xscale[i] = 0.0f;
      memset(xq + i * k, 0, (size_t)k);
      continue;
    }
    float inv = 448.0f / amax;
    xscale[i] = amax / 448.0f;
    for (int64_t t = 0; t < k; ++t) xq[i * k + t] = rqo_f32_to_fp8_e4m3_rne(r[t] * inv);
  }
}

void rqo_fp8_encode_unscaled(const float *x, int64_t count, uint8_t *xq) {
  for (int64_t i = 0; i < count; ++i) xq[i] = rqo_f32_to_fp8_e4m3(x[i]);
}

void rqo_fp8_gemm_quantized_f64(const uint8_t *xq, const float *xs, int64_t m,
                                const uint8_t *w, const float *ws, int64_t n, int64_t k,
                                double *y) {
  double lut[256];
  for (int b = 0; b < 256; ++b) lut[b] = (double)rqo_fp8_e4m3_to_f32((uint8_t)b);
#pragma omp parallel for schedule(static)
  for (int64_t j = 0; j < n; ++j)
    for (int64_t i = 0; i < m; ++i) {
      double acc = 0.0;
      for (int64_t t = 0; t < k; ++t) acc += lut[xq[i * k + t]] * lut[w[j * k + t]];
      y[i * n + j] = (double)xs[i] * (double)ws[j] * acc;
    }
}
