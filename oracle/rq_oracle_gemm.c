/*
 * rq_oracle_gemm.c -- the f32 CPU matmul of the CPU baseline.
 *
 * TEST INFRASTRUCTURE ONLY (see rq_oracle.h).  Stands in for candle's CPU f32
 * matmul (gemm 0.19, reached through linear_layer.rs:100 and
 * substrate/candle.rs:40-42), which is not available here.  Compiled apart
 * from rq_oracle.c so that this loop may use FMA and SIMD reassociation while
 * the dequant restatement keeps the Rust rounding points.
 */
#include "rq_oracle.h"

static float dot_f32(const float *a, const float *b, int64_t k) {
  float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
  for (int64_t t = 0; t < k; ++t) acc += a[t] * b[t];
  return acc;
}

void rqo_linear_f32(const float *x, int64_t m, const float *w, int64_t n, int64_t k,
                    float *y, int threads) {
  const int64_t NB = 32, MB = 64;
  int64_t nblocks = (n + NB - 1) / NB;
  if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (int64_t bj = 0; bj < nblocks; ++bj) {
    int64_t j0 = bj * NB, j1 = j0 + NB < n ? j0 + NB : n;
    for (int64_t i0 = 0; i0 < m; i0 += MB) {
      int64_t i1 = i0 + MB < m ? i0 + MB : m;
      for (int64_t j = j0; j < j1; ++j)
        for (int64_t i = i0; i < i1; ++i) y[i * n + j] = dot_f32(x + i * k, w + j * k, k);
    }
  }
}

