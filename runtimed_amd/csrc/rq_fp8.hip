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
// GEMM tiling: a 256-thread workgroup computes a 256 x 256 tile of y with
// 128 x 128 per wave (4 x 4 MFMA tiles of 32 x 32, accumulators in AGPRs) for
// large problems (K-step 64 bytes, LDS rows of 80 bytes), or 128 x 128 with
// 64 x 64 per wave otherwise (K-step 128 bytes, rows of 144 bytes).  Two LDS
// buffers (double buffering); the row padding makes the 32 lanes that read
// one MFMA operand column touch distinct 16-byte bank groups.
//
// Roofline: MFMA-bound (fp8 dense peak 5.0 PFLOP/s); flops = 2*m*n*k.
#include "rq_e4m3.h"
#include "rq_epilogue.h"
#include "rq_internal.h"
#include "rq_pipe.h"

namespace rq {
namespace {

using namespace pipe;

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

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

// The same per-token encode with one wave per activation row (four rows a
// workgroup): the row's maximum from 16-byte loads and a wave reduction,
// then the codes from a second pass over the row (an L2 hit, or the
// registers when the row is at most one batch), 4 (f32) or 8 (f16 / bf16)
// codes per store.  Same codes and scales as k_fp8_quant_rows (the maximum
// is exact in any order, enc_e4m3_rne_bf equals enc_e4m3_rne).  The
// activation type and the mode are template parameters: as run-time values
// the compiler turned each per-element choice into a branch.  One workgroup
// per row with scalar 2-byte loads took 21 us on 2048 x 4096 bf16.
template <int XT, bool SCALED>
__global__ __launch_bounds__(256) void k_fp8_quant_waves(const void *__restrict__ x, int64_t m, int64_t k,
                                                        uint8_t *__restrict__ xq, float *__restrict__ xs) {
  constexpr bool F32X = XT == RQ_F32;
  constexpr int ES = F32X ? 4 : 8;  // elements per 16-byte chunk
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= m) return;
  const int64_t nch = k / ES;
  const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(x) + row * k * (F32X ? 4 : 2));
  auto unpack = [&](const uint4 &v, float (&f)[ES]) {
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (F32X) {
        f[i] = __uint_as_float(u[i]);
      } else if constexpr (XT == RQ_BF16) {
        f[2 * i] = __uint_as_float(u[i] << 16);
        f[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
      } else {
        f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] & 0xFFFFu));
        f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] >> 16));
      }
    }
  };
  // Batches of U chunks a lane, their loads issued together; a row of at
  // most one batch stays in registers between the two passes.
  constexpr int U = 8;
  uint4 buf[U];
  auto load_batch = [&](int64_t c0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + 64 * u;
      buf[u] = src[c < nch ? c : nch - 1];
    }
  };
  const bool resident = SCALED && nch <= 64 * U;
  float amax = 0.0f;
  bool nan = false;
  if constexpr (SCALED) {
    for (int64_t c0 = lane; c0 < nch; c0 += 64 * U) {
      load_batch(c0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float f[ES];
        unpack(buf[u], f);
        const bool live = c0 + 64 * u < nch;
#pragma unroll
        for (int i = 0; i < ES; ++i) {
          amax = fmaxf(amax, live ? fabsf(f[i]) : 0.0f);
          nan |= f[i] != f[i];
        }
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  }
  // A row without NaN is encoded by the hardware conversion: for |v| <= 448
  // v_cvt_pk_fp8_f32 gives enc_e4m3_rne's code for every f32 input (compared
  // over all 2^32 of them on MI355X); v is clamped to +-448 first (the
  // product can exceed 448 by an ulp).  Rows with a NaN or an infinity (whose
  // product with inv = 0 is NaN) keep the software encoder, whose NaN code
  // differs.
  const bool hw = SCALED && !__any(nan) && amax != 0.0f && amax <= 3.4028235e38f;  // no NaN, no infinity
  // amax == 0: every code 0 (inv = 0 would turn NaN or infinite inputs into
  // NaN codes instead).
  const float inv = 448.0f / amax;
  const uint32_t keep = amax == 0.0f ? 0u : 0xFFu;
  uint8_t *dst = xq + row * k;
  for (int64_t c0 = lane; c0 < nch; c0 += 64 * U) {
    if (!resident) load_batch(c0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + 64 * u;
      float f[ES];
      unpack(buf[u], f);
      uint32_t word[ES / 4];
      if (hw) {
#pragma unroll
        for (int j = 0; j < ES / 4; ++j) {
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = __builtin_amdgcn_fmed3f(f[4 * j + i] * inv, -448.0f, 448.0f);
          const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
          word[j] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], lo, true);
        }
      } else {
        uint32_t q[ES];
#pragma unroll
        for (int i = 0; i < ES; ++i) q[i] = SCALED ? enc_e4m3_rne_bf(f[i] * inv) & keep : enc_e4m3_ref(f[i]);
#pragma unroll
        for (int j = 0; j < ES / 4; ++j)
          word[j] = q[4 * j] | (q[4 * j + 1] << 8) | (q[4 * j + 2] << 16) | (q[4 * j + 3] << 24);
      }
      if (c < nch) {
        if constexpr (F32X) {
          *reinterpret_cast<uint32_t *>(dst + 4 * c) = word[0];
        } else {
          *reinterpret_cast<uint2 *>(dst + 8 * c) = make_uint2(word[0], word[1]);
        }
      }
    }
  }
  if (lane == 0) xs[row] = !SCALED ? 1.0f : amax == 0.0f ? 0.0f : amax / 448.0f;
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

// A BM x BN tile of y per 256-thread workgroup of WM x WN waves; each wave
// owns (BM/WM) x (BN/WN) = MI x NI MFMA tiles of 32 x 32.  With 128 x 128 wave
// tiles every 32-byte operand fragment read from LDS feeds four MFMAs.  BK is
// the K-step in bytes (64 or 128); LDS rows are BK + 16 bytes.
template <int BM, int BN, int WM, int WN, int BK>
__global__ __launch_bounds__(256) void k_fp8_gemm_mfma(const uint8_t *__restrict__ a,
                                                      const float *__restrict__ xs, int64_t m,
                                                      const uint8_t *__restrict__ b,
                                                      const float *__restrict__ ws, int64_t n,
                                                      int64_t k, void *__restrict__ y, int ytype) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int LDS_STRIDE = BK + 16;
  constexpr int TPR = BK / 16;              // threads per row in a load round
  constexpr int RPR = 256 / TPR;            // rows per load round
  constexpr int MI = BM / WM / 32, NI = BN / WN / 32;
  constexpr int A_LOADS = BM / RPR, B_LOADS = BN / RPR;  // 16-byte loads per thread per step
  __shared__ __attribute__((aligned(16))) uint8_t As[2][BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN * LDS_STRIDE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

  // Global -> register staging: TPR threads per row, RPR rows per round.
  const int lrow = tid / TPR, lcol = (tid % TPR) * 16;
  uint4 ra[A_LOADS], rb[B_LOADS];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int it = 0; it < A_LOADS; ++it) {
      const int64_t gm = m0 + lrow + RPR * it;
      ra[it] = gm < m ? *reinterpret_cast<const uint4 *>(a + gm * k + k0 + lcol) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int it = 0; it < B_LOADS; ++it) {
      const int64_t gn = n0 + lrow + RPR * it;
      rb[it] = gn < n ? *reinterpret_cast<const uint4 *>(b + gn * k + k0 + lcol) : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int it = 0; it < A_LOADS; ++it)
      *reinterpret_cast<uint4 *>(&As[buf][(lrow + RPR * it) * LDS_STRIDE + lcol]) = ra[it];
#pragma unroll
    for (int it = 0; it < B_LOADS; ++it)
      *reinterpret_cast<uint4 *>(&Bs[buf][(lrow + RPR * it) * LDS_STRIDE + lcol]) = rb[it];
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = (f32x16){0};

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
      i32x8 fa[MI], fb[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int ar = wm * (BM / WM) + i * 32 + (lane & 31);
        const uint4 *pa = reinterpret_cast<const uint4 *>(&As[buf][ar * LDS_STRIDE + kb]);
        const uint4 a0 = pa[0], a1 = pa[1];
        fa[i] = (i32x8){(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int br = wn * (BN / WN) + j * 32 + (lane & 31);
        const uint4 *pb = reinterpret_cast<const uint4 *>(&Bs[buf][br * LDS_STRIDE + kb]);
        const uint4 b0 = pb[0], b1 = pb[1];
        fb[j] = (i32x8){(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb[j], acc[i][j], 0, 0,
                                                                      0, 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  const bool vec = vec_stores_ok(y, n);
  float sx[MI][4], sw[NI][4];
#pragma unroll
  for (int i = 0; i < MI; ++i) tile_row_scales(xs, m, m0 + wm * (BM / WM) + i * 32, lane, sx[i]);
#pragma unroll
  for (int j = 0; j < NI; ++j) tile_col_scales(ws, n, n0 + wn * (BN / WN) + j * 32, lane, sw[j]);
  const Out o{y, nullptr, ytype, 0};
  const float nob[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  static_for<MI>([&](auto I) {
    static_for<NI>([&](auto J) {
      store_tile32<true>(acc[I][J], o, m, n, m0 + wm * (BM / WM) + I * 32, n0 + wn * (BN / WN) + J * 32, sx[I],
                         sw[J], nob, xs, ws, lane, vec);
    });
  });
}

// ---- pipelined 256 x 256 kernel ------------------------------------------
//
// Four waves of 128 x 128 (4 x 4 MFMA tiles, 256 accumulators in AGPRs).  K
// advances 64 bytes per step through four LDS stages of 32 KB (A rows then B
// rows, 64 bytes each), filled by direct global -> LDS loads
// (global_load_lds_dwordx4: lane L of a wave lands at base + 16*L) issued
// three steps ahead, so about three steps of MFMA work cover the load latency
// without staging registers.  Rows carry no padding; instead the four 16-byte
// chunks of row r are stored XOR-swizzled by (r >> 2) & 3, so the 32 lanes
// that read one operand column of 32 rows hit 16 distinct 16-byte bank slots.

// Issue the direct loads of one stage.  The LDS pointer is __restrict__ so
// that, once inlined, the accesses carry scoped alias metadata and the
// compiler's wait insertion can tell the four stage buffers apart instead of
// draining every load before each LDS read.
__device__ __forceinline__ void pipe_issue(uint8_t *__restrict__ S, const uint8_t *const (&ga)[4],
                                           const uint8_t *const (&gb)[4], int64_t k0, int wave) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    __builtin_amdgcn_global_load_lds(ga[j] + k0, (lds_void *)(S + (64 * wave + 16 * j) * 64), 16, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    __builtin_amdgcn_global_load_lds(gb[j] + k0, (lds_void *)(S + P_B + (64 * wave + 16 * j) * 64), 16, 0, 0);
}

__device__ __forceinline__ i32x8 frag_a(const Frags &F, int i) {
  const u32x4 x0 = F.x[2 * i], x1 = F.x[2 * i + 1];
  return (i32x8){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
}

// The 16 MFMAs of one K-step on `cur`, each followed by one LDS read of the
// next step's fragments into `nxt` (nullptr S: no next step), pinned in that
// order so the LDS reads run under the matrix work.
__device__ __forceinline__ void mfma_step(const Frags &cur, Frags &nxt, const uint8_t *__restrict__ S,
                                          f32x16 (&acc)[4][4], int wm, int wn, int lane) {
  static_for<4>([&](auto I) {
    const i32x8 fa = frag_a(cur, I);
    static_for<4>([&](auto J) {
      const i32x8 fb = frag_a(cur, 4 + J);
      acc[I][J] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, acc[I][J], 0, 0, 0, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (S) nxt.x[4 * I + J] = ds_read16(frag_addr(S, 4 * I + J, wm, wn, lane));
      __builtin_amdgcn_sched_barrier(0);
    });
  });
}

__global__ __launch_bounds__(256) void k_fp8_gemm_pipe(const uint8_t *__restrict__ a,
                                                      const float *__restrict__ xs, int64_t m,
                                                      const uint8_t *__restrict__ b,
                                                      const float *__restrict__ ws, int64_t n,
                                                      int64_t k, void *__restrict__ y, int ytype) {
  // four stages, one array: after the loop it holds the staged output tile
  __shared__ __attribute__((aligned(1024))) uint8_t SM[4 * P_STAGE];
  uint8_t *const S0 = SM, *const S1 = SM + P_STAGE, *const S2 = SM + 2 * P_STAGE, *const S3 = SM + 3 * P_STAGE;
  uint8_t *const SB[4] = {S0, S1, S2, S3};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * 256, n0 = (int64_t)blockIdx.x * 256;
  const int64_t nk = k / 64;

  // Load assignment: wave w fills rows 64w .. 64w+63 of the A and B halves of
  // a stage, 16 rows (4 lanes x 16 bytes per row) per instruction.  Rows past
  // m or n re-read the last valid row; their results are never stored.
  const uint8_t *ga[4], *gb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 64 * wave + 16 * j + (lane >> 2);
    const int gc = (lane & 3) ^ swz(r);
    const int64_t gm = m0 + r < m ? m0 + r : m - 1;
    const int64_t gn = n0 + r < n ? n0 + r : n - 1;
    ga[j] = a + gm * k + 16 * gc;
    gb[j] = b + gn * k + 16 * gc;
  }

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x16){0};

  // Stages 0..3 in flight; fragments of step 0 in registers.
#pragma unroll
  for (int s = 0; s < 4; ++s)
    if (s < nk) pipe_issue(SB[s], ga, gb, 64 * s, wave);
  if (nk > 3) wait_vm<24>();
  else if (nk > 2) wait_vm<16>();
  else if (nk > 1) wait_vm<8>();
  else wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  Frags F0, F1;
  read_all(S0, F0, wm, wn, lane);
  wait_lds(F0);

  // Step t: stage t's fragments are in registers.  Make stage t+1 resident
  // (its loads landed in every wave: wait, then a bare barrier -- a release
  // fence would drain the younger stages too), refill buffer t%4 with stage
  // t+4 (everyone finished reading it before this barrier), then run step t's
  // MFMAs with the reads of step t+1 interleaved.
  auto step = [&](const Frags &cur, Frags &nxt, int64_t t, int buf) {
    const uint8_t *next = nullptr;
    if (t + 1 < nk) {
      if (t + 3 < nk) wait_vm<16>();
      else if (t + 2 < nk) wait_vm<8>();
      else wait_vm<0>();
      __builtin_amdgcn_s_barrier();
      if (t + 4 < nk) pipe_issue(SB[buf], ga, gb, 64 * (t + 4), wave);
      next = SB[(buf + 1) & 3];
    }
    mfma_step(cur, nxt, next, acc, wm, wn, lane);
    if (next) wait_lds(nxt);
  };
  for (int64_t t = 0; t < nk; t += 4) {
    step(F0, F1, t, 0);
    if (t + 1 < nk) step(F1, F0, t + 1, 1);
    if (t + 2 < nk) step(F0, F1, t + 2, 2);
    if (t + 3 < nk) step(F1, F0, t + 3, 3);
  }

  const bool vec = vec_stores_ok(y, n);
  float sx[4][4], sw[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) tile_row_scales(xs, m, m0 + 128 * wm + i * 32, lane, sx[i]);
#pragma unroll
  for (int j = 0; j < 4; ++j) tile_col_scales(ws, n, n0 + 128 * wn + j * 32, lane, sw[j]);
  if (ytype != RQ_F32 && vec && n % 8 == 0 && m0 + 256 <= m && n0 + 256 <= n) {
    __syncthreads();  // every wave's stage reads are done
    const float nob[4][4] = {};
    stage_block_2b<true>(acc, SM, 128 * wm, 128 * wn, ytype, sx, sw, nob, false, lane);
    __syncthreads();
    store_staged_2b(SM, y, n, m0, n0, threadIdx.x);
    return;
  }
  const Out o{y, nullptr, ytype, 0};
  const float nob[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  static_for<4>([&](auto I) {
    static_for<4>([&](auto J) {
      store_tile32<true>(acc[I][J], o, m, n, m0 + 128 * wm + I * 32, n0 + 128 * wn + J * 32, sx[I], sw[J], nob, xs,
                         ws, lane, vec);
    });
  });
}

// ---- the same with eight waves (two a SIMD) ------------------------------
//
// Eight waves of 128 (M) x 64 (N) on the 256 x 256 tile (4 x 2 MFMA tiles,
// 128 accumulators), two waves a SIMD: while one wave waits on its LDS reads
// or the step's barrier the other issues MFMAs (2048 x 14336 x 4096: 148-155
// -> 131-134 us against the four-wave kernel).  The four stages keep their A parts
// side by side (16 KB each) and their B parts side by side (64 KB above), so
// that one base register per operand and pass half reaches every stage and
// tile through the ds_read offset field; each wave fills 32 A rows and 32 B
// rows of a stage (two direct loads each), three steps ahead.
constexpr int F8_A = 16384, F8_B = 65536;

struct Frags8 {
  u32x4 x[12];  // A tiles 0..3 (halves 2t, 2t + 1), then B tiles 0..1 (8 + 2t, 9 + 2t)
};

__device__ __forceinline__ void wait_lds8(Frags8 &F) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(F.x[0]), "+v"(F.x[1]), "+v"(F.x[2]), "+v"(F.x[3]));
  asm volatile("" : "+v"(F.x[4]), "+v"(F.x[5]), "+v"(F.x[6]), "+v"(F.x[7]));
  asm volatile("" : "+v"(F.x[8]), "+v"(F.x[9]), "+v"(F.x[10]), "+v"(F.x[11]));
}

// Fragment f of stage ST (f < 8: A tile f / 2, else B tile (f - 8) / 2; half f % 2).
template <int ST, int F>
__device__ __forceinline__ u32x4 frag8(const uint32_t (&rd)[2][2]) {
  constexpr int t = F < 8 ? F / 2 : (F - 8) / 2;
  return ds_read16_off<ST * F8_A + 2048 * t>(rd[F & 1][F < 8 ? 0 : 1]);
}

__device__ __forceinline__ i32x8 frag8_op(const Frags8 &F, int f) {
  const u32x4 x0 = F.x[f], x1 = F.x[f + 1];
  return (i32x8){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
}

// The 8 MFMAs of one K-step on `cur`; after MFMA f < 6, reads 2f and 2f + 1
// of the next step's fragments from stage ST.
template <int ST>
__device__ __forceinline__ void mfma_step8(const Frags8 &cur, Frags8 &nxt, const uint32_t (&rd)[2][2],
                                           f32x16 (&acc)[4][2]) {
  static_for<4>([&](auto I) {
    static_for<2>([&](auto J) {
      constexpr int f = 2 * decltype(I)::value + decltype(J)::value;
      acc[I][J] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(frag8_op(cur, 2 * I), frag8_op(cur, 8 + 2 * J),
                                                                  acc[I][J], 0, 0, 0, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (f < 6) {
        nxt.x[2 * f] = frag8<ST, 2 * f>(rd);
        nxt.x[2 * f + 1] = frag8<ST, 2 * f + 1>(rd);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  });
}

__global__ __launch_bounds__(512) void k_fp8_gemm_pipe8(const uint8_t *__restrict__ a,
                                                       const float *__restrict__ xs, int64_t m,
                                                       const uint8_t *__restrict__ b,
                                                       const float *__restrict__ ws, int64_t n,
                                                       int64_t k, void *__restrict__ y, int ytype) {
  __shared__ __attribute__((aligned(1024))) uint8_t SM[4 * P_STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int64_t m0 = (int64_t)blockIdx.y * 256, n0 = (int64_t)blockIdx.x * 256;
  const int64_t nk = k / 64;

  // Wave w fills rows 32 w .. 32 w + 31 of the A and B parts of a stage, 16
  // rows (4 lanes x 16 bytes a row) an instruction, lane L at byte 16 L of
  // the instruction's kilobyte; rows past m or n re-read the last valid row.
  const uint8_t *ga[2], *gb[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 32 * wave + 16 * j + (lane >> 2);
    const int gc = (lane & 3) ^ swz(r);
    const int64_t gm = m0 + r < m ? m0 + r : m - 1;
    const int64_t gn = n0 + r < n ? n0 + r : n - 1;
    ga[j] = a + gm * k + 16 * gc;
    gb[j] = b + gn * k + 16 * gc;
  }
  uint8_t *const dA = SM + 2048 * wave, *const dB = SM + F8_B + 2048 * wave;
  auto issue = [&](int st, int64_t k0) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_global_load_lds(ga[j] + k0, (lds_void *)(dA + st * F8_A + 1024 * j), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_global_load_lds(gb[j] + k0, (lds_void *)(dB + st * F8_A + 1024 * j), 16, 0, 0);
  };
  uint32_t rd[2][2];  // [half][A, B]
  {
    const uint32_t sa = lds_addr(SM), sb = sa + F8_B;
    const int l = lane & 31, g = lane >> 5, sw = (l >> 2) & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      rd[h][0] = sa + 8192 * wm + 64 * l + 16 * ((2 * g + h) ^ sw);
      rd[h][1] = sb + 4096 * wn + 64 * l + 16 * ((2 * g + h) ^ sw);
    }
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x16){0};

  // Stages 0..3 in flight; fragments of step 0 in registers.
#pragma unroll
  for (int s = 0; s < 4; ++s)
    if (s < nk) issue(s, 64 * s);
  if (nk > 3) wait_vm<12>();
  else if (nk > 2) wait_vm<8>();
  else if (nk > 1) wait_vm<4>();
  else wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  Frags8 F0, F1;
  static_for<12>([&](auto Fc) { F0.x[decltype(Fc)::value] = frag8<0, decltype(Fc)::value>(rd); });
  wait_lds8(F0);

  // Step t (stage t % 4 in registers): make stage t + 1 resident (wait for its
  // loads, then a bare barrier), refill stage t % 4 with K-step t + 4 (every
  // wave has read it), then the MFMAs of step t with the reads of step t + 1.
  // The last step reads a stale stage (in bounds, never used), so that every
  // step has the same straight-line MFMA code (k % 256 == 0: whole groups of
  // four steps).
  auto step = [&](const Frags8 &cur, Frags8 &nxt, int64_t t, auto STc) {
    constexpr int ST = decltype(STc)::value;
    if (t + 3 < nk) wait_vm<8>();
    else if (t + 2 < nk) wait_vm<4>();
    else wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    if (t + 4 < nk) issue(ST, 64 * (t + 4));
    mfma_step8<(ST + 1) & 3>(cur, nxt, rd, acc);
    wait_lds8(nxt);
  };
  for (int64_t t = 0; t < nk; t += 4) {
    step(F0, F1, t, std::integral_constant<int, 0>{});
    step(F1, F0, t + 1, std::integral_constant<int, 1>{});
    step(F0, F1, t + 2, std::integral_constant<int, 2>{});
    step(F1, F0, t + 3, std::integral_constant<int, 3>{});
  }

  const bool vec = vec_stores_ok(y, n);
  float sx[4][4], sw[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) tile_row_scales(xs, m, m0 + 128 * wm + i * 32, lane, sx[i]);
#pragma unroll
  for (int j = 0; j < 2; ++j) tile_col_scales(ws, n, n0 + 64 * wn + j * 32, lane, sw[j]);
  if (ytype != RQ_F32 && vec && n % 8 == 0 && m0 + 256 <= m && n0 + 256 <= n) {
    __syncthreads();  // every wave's stage reads are done
    const float nob[2][4] = {};
    stage_block_2b<true>(acc, SM, 128 * wm, 64 * wn, ytype, sx, sw, nob, false, lane);
    __syncthreads();
    store_staged_2b<512>(SM, y, n, m0, n0, tid);
    return;
  }
  const Out o{y, nullptr, ytype, 0};
  const float nob[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  static_for<4>([&](auto I) {
    static_for<2>([&](auto J) {
      store_tile32<true>(acc[I][J], o, m, n, m0 + 128 * wm + I * 32, n0 + 64 * wn + J * 32, sx[I], sw[J], nob, xs,
                         ws, lane, vec);
    });
  });
}

template <int BM, int BN, int WM, int WN, int BK>
void launch_tiled(const uint8_t *xq, const float *xs, int64_t m, const uint8_t *w, const float *ws,
                  int64_t n, int64_t k, void *y, int ytype, hipStream_t s) {
  const dim3 grid((unsigned)((n + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
  hipLaunchKernelGGL((k_fp8_gemm_mfma<BM, BN, WM, WN, BK>), grid, dim3(256), 0, s, xq, xs, m, w, ws, n, k, y,
                     ytype);
}

}  // namespace

int launch_fp8_quantize(const void *x, int xtype, int64_t m, int64_t k, int mode, uint8_t *xq,
                        float *xs, hipStream_t s) {
  if (m == 0) return RQ_OK;
  const bool f32x = xtype == RQ_F32;
  const int es = f32x ? 4 : 8;
  const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && k % es == 0 && (k * (f32x ? 4 : 2)) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(xq) % es == 0;
  if (vec) {
    const dim3 grid((unsigned)((m + 3) / 4));
    const bool sc = mode != RQ_FP8_UNSCALED;
#define RQ_QW(XT, SC) hipLaunchKernelGGL((k_fp8_quant_waves<XT, SC>), grid, dim3(256), 0, s, x, m, k, xq, xs)
    if (xtype == RQ_F32) {
      if (sc) RQ_QW(RQ_F32, true); else RQ_QW(RQ_F32, false);
    } else if (xtype == RQ_BF16) {
      if (sc) RQ_QW(RQ_BF16, true); else RQ_QW(RQ_BF16, false);
    } else {
      if (sc) RQ_QW(RQ_F16, true); else RQ_QW(RQ_F16, false);
    }
#undef RQ_QW
  } else {
    hipLaunchKernelGGL(k_fp8_quant_rows, dim3((unsigned)m), dim3(256), 0, s, x, xtype, k, mode, xq, xs);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "fp8 quantize launch failed");
}

int launch_fp8_gemm(const uint8_t *xq, const float *xs, int64_t m, const uint8_t *w,
                    const float *ws, int64_t n, int64_t k, void *y, int ytype, hipStream_t s) {
  if (m == 0 || n == 0) return RQ_OK;
  const bool aligned = (reinterpret_cast<uintptr_t>(xq) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(w) % 16 == 0);
  if (k % 128 == 0 && aligned) {
    // 256 x 256 tiles when there are enough of them to cover the CUs (eight
    // waves of 128 x 64 for whole groups of four K-steps, else four of
    // 128 x 128), else 128 x 128.
    const int64_t big = ((m + 255) / 256) * ((n + 255) / 256);
    if (big >= 200) {
      const dim3 grid((unsigned)((n + 255) / 256), (unsigned)((m + 255) / 256));
      if (k % 256 == 0)
        hipLaunchKernelGGL(k_fp8_gemm_pipe8, grid, dim3(512), 0, s, xq, xs, m, w, ws, n, k, y, ytype);
      else
        hipLaunchKernelGGL(k_fp8_gemm_pipe, grid, dim3(256), 0, s, xq, xs, m, w, ws, n, k, y, ytype);
    } else {
      launch_tiled<128, 128, 2, 2, 128>(xq, xs, m, w, ws, n, k, y, ytype, s);
    }
  } else {
    const int64_t total = m * n;
    hipLaunchKernelGGL(k_fp8_gemm_scalar, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, xq,
                       xs, m, w, ws, n, k, y, ytype);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "fp8 gemm launch failed");
}

}  // namespace rq
