// rq_fp8.hip -- FP8 e4m3 activation encoding and GEMM on gfx950 matrix cores.
//
// Replaces ops::fp8_gemm (crates/runtimed-model/src/ops/fp8_gemm.rs:77-191):
//   - the reference encodes activations on the host, per element, with
//     f32_to_fp8_e4m3 (load_safetensors.rs:53-69) and no scale
//     (fp8_gemm.rs:94-101).  RQ_FP8_UNSCALED reproduces that encoder on the
//     device, bit for bit (nearest LUT value, ties to the lower magnitude).
//   - RQ_FP8_PER_TOKEN is the dynamic per-row scaling of the FP8 workload:
//     s = max|x|/448, codes e4m3_rne(x * (448/max|x|)).
//   - the product runs on v_mfma_f32_32x32x64_f8f6f4 (OCP e4m3 x e4m3, f32
//     accumulate) and applies x-scale * w-scale in the epilogue, where the
//     reference applies the per-channel scale as an extra broadcast_mul pass
//     (fp8_gemm.rs:180-186).
//
// GEMM tiling: a 256-thread workgroup computes a 128 x 128 tile of y; the
// four waves own 64 x 64 quadrants (2 x 2 MFMA tiles of 32 x 32).  K advances
// 128 bytes per step through two LDS buffers (double buffering), rows padded
// to 144 bytes so that the 32 lanes reading one MFMA operand column touch
// distinct 16-byte bank groups.
//
// Roofline: MFMA-bound (fp8 dense peak 5.0 PFLOP/s); flops = 2*m*n*k.
#include "rq_internal.h"

namespace rq {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// FP8_E4M3_LUT value of a positive code 0..126 (load_safetensors.rs:14-29).
__device__ __forceinline__ float e4m3_pos_value(int c) {
  const int e = c >> 3, m = c & 7;
  return e == 0 ? (float)m * 0.001953125f : ldexpf(1.0f + (float)m * 0.125f, e - 7);
}

// f32_to_fp8_e4m3 (load_safetensors.rs:53-69), bit-exact.
__device__ uint32_t enc_e4m3_ref(float f) {
  if (f != f) return 0x7Fu;
  const uint32_t sign = (__float_as_uint(f) >> 24) & 0x80u;
  const float a = fabsf(f);
  if (a <= 0.0f) return sign;
  if (a >= 448.0f) return sign | 0x7Eu;
  int lo = 0, hi = 127;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (e4m3_pos_value(mid) < a) lo = mid + 1;
    else hi = mid;
  }
  const float above = e4m3_pos_value(lo);
  if (above == a) return sign | (uint32_t)lo;
  const float below = e4m3_pos_value(lo - 1);
  return sign | (uint32_t)((a - below <= above - a) ? lo - 1 : lo);
}

// Clamp to +-448 then OCP e4m3fn round-to-nearest-even.
__device__ uint32_t enc_e4m3_rne(float f) {
  if (f != f) return 0x7Fu;
  const uint32_t sign = (__float_as_uint(f) >> 24) & 0x80u;
  float a = fminf(fabsf(f), 448.0f);
  if (a < 0.015625f) return sign | (uint32_t)__builtin_rintf(a * 512.0f);
  const uint32_t u = __float_as_uint(a);
  int e = (int)((u >> 23) & 0xFFu) - 127;
  const uint32_t man = u & 0x7FFFFFu;
  uint32_t r = man >> 20;
  const uint32_t rem = man & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) r += 1;
  if (r == 8) {
    r = 0;
    e += 1;
  }
  return sign | (((uint32_t)(e + 7) << 3) | r);
}

__device__ __forceinline__ float load_x1(const void *x, int xtype, int64_t i) {
  if (xtype == RQ_F32) return static_cast<const float *>(x)[i];
  if (xtype == RQ_BF16) return bf16_bits_to_f32(static_cast<const uint16_t *>(x)[i]);
  return (float)static_cast<const _Float16 *>(x)[i];
}

// One workgroup per activation row.
__global__ __launch_bounds__(256) void k_fp8_quant_rows(const void *__restrict__ x, int xtype,
                                                       int64_t k, int mode, uint8_t *__restrict__ xq,
                                                       float *__restrict__ xs) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  if (mode == RQ_FP8_UNSCALED) {
    for (int64_t t = tid; t < k; t += 256) xq[row * k + t] = (uint8_t)enc_e4m3_ref(load_x1(x, xtype, row * k + t));
    if (tid == 0) xs[row] = 1.0f;
    return;
  }
  float amax = 0.0f;
  for (int64_t t = tid; t < k; t += 256) amax = fmaxf(amax, fabsf(load_x1(x, xtype, row * k + t)));
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (amax == 0.0f) {
    for (int64_t t = tid; t < k; t += 256) xq[row * k + t] = 0;
    if (tid == 0) xs[row] = 0.0f;
    return;
  }
  const float inv = 448.0f / amax;
  for (int64_t t = tid; t < k; t += 256) xq[row * k + t] = (uint8_t)enc_e4m3_rne(load_x1(x, xtype, row * k + t) * inv);
  if (tid == 0) xs[row] = amax / 448.0f;
}

// e4m3 decode for the scalar path (LUT formula of load_safetensors.rs:14-29).
__device__ __forceinline__ float dec_e4m3(uint32_t b) {
  const int e = (b >> 3) & 0xF, m = b & 7;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;
  else if (e == 15 && m == 7) v = __uint_as_float(0x7FC00000u);
  else v = ldexpf(1.0f + (float)m * 0.125f, e - 7);
  return (b & 0x80u) ? -v : v;
}

// Scalar fallback for shapes the tiled kernel does not take (k % 128 != 0).
__global__ __launch_bounds__(256) void k_fp8_gemm_scalar(const uint8_t *__restrict__ xq,
                                                        const float *__restrict__ xs, int64_t m,
                                                        const uint8_t *__restrict__ w,
                                                        const float *__restrict__ ws, int64_t n,
                                                        int64_t k, void *__restrict__ y, int ytype) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= m * n) return;
  const int64_t i = idx / n, j = idx - i * n;
  float acc = 0.0f;
  for (int64_t t = 0; t < k; ++t) acc = fmaf(dec_e4m3(xq[i * k + t]), dec_e4m3(w[j * k + t]), acc);
  const float sx = xs ? xs[i] : 1.0f, sw = ws ? ws[j] : 1.0f;
  store_out(y, ytype, idx, acc * (sx * sw));
}

constexpr int BM = 128, BN = 128, BK = 128, LDS_STRIDE = BK + 16;

__global__ __launch_bounds__(256) void k_fp8_gemm_mfma(const uint8_t *__restrict__ a,
                                                      const float *__restrict__ xs, int64_t m,
                                                      const uint8_t *__restrict__ b,
                                                      const float *__restrict__ ws, int64_t n,
                                                      int64_t k, void *__restrict__ y, int ytype) {
  __shared__ __attribute__((aligned(16))) uint8_t As[2][BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN * LDS_STRIDE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

  // Global -> register staging: each thread moves 4 x 16 bytes of A and of B.
  const int lrow = tid >> 3, lcol = (tid & 7) * 16;
  uint4 ra[4], rb[4];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int r = lrow + 32 * it;
      const int64_t gm = m0 + r, gn = n0 + r;
      ra[it] = gm < m ? *reinterpret_cast<const uint4 *>(a + gm * k + k0 + lcol) : make_uint4(0, 0, 0, 0);
      rb[it] = gn < n ? *reinterpret_cast<const uint4 *>(b + gn * k + k0 + lcol) : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int r = lrow + 32 * it;
      *reinterpret_cast<uint4 *>(&As[buf][r * LDS_STRIDE + lcol]) = ra[it];
      *reinterpret_cast<uint4 *>(&Bs[buf][r * LDS_STRIDE + lcol]) = rb[it];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x16){0};

  const int64_t nk = k / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = (int)(kt & 1);
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
      const int kb = ks * 64 + 32 * (lane >> 5);
      i32x8 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int ar = wm * 64 + i * 32 + (lane & 31);
        const uint4 *pa = reinterpret_cast<const uint4 *>(&As[buf][ar * LDS_STRIDE + kb]);
        const uint4 a0 = pa[0], a1 = pa[1];
        fa[i] = (i32x8){(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        const int br = wn * 64 + i * 32 + (lane & 31);
        const uint4 *pb = reinterpret_cast<const uint4 *>(&Bs[buf][br * LDS_STRIDE + kb]);
        const uint4 b0 = pb[0], b1 = pb[1];
        fb[i] = (i32x8){(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb[j], acc[i][j], 0, 0,
                                                                      0, 0, 0, 0);
    }
    if (kt + 1 < nk) {
      sstore(buf ^ 1);
    }
    __syncthreads();
  }

  // Epilogue: C layout of the 32x32 tile: column lane%32, row
  // 8*(r/4) + 4*(lane/32) + r%4 for register r.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= n) continue;
      const float sw = ws ? ws[col] : 1.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < m) {
          const float sx = xs ? xs[row] : 1.0f;
          store_out(y, ytype, row * n + col, acc[i][j][r] * (sx * sw));
        }
      }
    }
}

}  // namespace

int launch_fp8_quantize(const void *x, int xtype, int64_t m, int64_t k, int mode, uint8_t *xq,
                        float *xs, hipStream_t s) {
  if (m == 0) return RQ_OK;
  hipLaunchKernelGGL(k_fp8_quant_rows, dim3((unsigned)m), dim3(256), 0, s, x, xtype, k, mode, xq, xs);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "fp8 quantize launch failed");
}

int launch_fp8_gemm(const uint8_t *xq, const float *xs, int64_t m, const uint8_t *w,
                    const float *ws, int64_t n, int64_t k, void *y, int ytype, hipStream_t s) {
  if (m == 0 || n == 0) return RQ_OK;
  const bool aligned = (reinterpret_cast<uintptr_t>(xq) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(w) % 16 == 0);
  if (k % BK == 0 && aligned) {
    const dim3 grid((unsigned)((n + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
    hipLaunchKernelGGL(k_fp8_gemm_mfma, grid, dim3(256), 0, s, xq, xs, m, w, ws, n, k, y, ytype);
  } else {
    const int64_t total = m * n;
    hipLaunchKernelGGL(k_fp8_gemm_scalar, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, xq,
                       xs, m, w, ws, n, k, y, ytype);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "fp8 gemm launch failed");
}

}  // namespace rq
