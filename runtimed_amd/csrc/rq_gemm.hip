// rq_gemm.hip -- quantized GEMM on gfx950 matrix cores (prefill and verify).
//
// y[m, n] = sum_k x[m, k] * W[n, k] for bf16 activations x and GGUF weights W
// (Q4_K, Q6_K, Q8_0), f32 accumulation, f32/bf16/f16 output.  Semantics of the
// reference's dense path (linear_layer.rs:88-104 after dequant_tensor,
// dequant.rs:83-146) with the weights rounded once to bf16 on their way into
// the matrix cores (north-star tolerance for bf16 operands: 2e-2 normalized).
//
// Tiling.  A workgroup computes a BM x BN tile of y (256 x 256 with 8 waves
// for large problems, 128 x 128 or 64 x 128 with 4 waves otherwise).  Each
// K-step covers 64 inputs: the activation tile (BM x 64 bf16) is copied global
// -> registers -> LDS; the weight tile (BN rows x 64) is read as 2*BN GGUF
// pieces of 32 elements, one per thread, decoded to exact f32 in registers,
// rounded to bf16 (v_cvt_pk_bf16_f32) and written to LDS.  The waves then run
// v_mfma_f32_32x32x16_bf16 from LDS.  LDS is double buffered: the global
// loads of step t+1 are issued before the matrix work of step t and land in
// the other buffer afterwards, so one barrier per step suffices.  LDS rows
// are padded to 72 elements (144 bytes) so the 32 lanes that read one operand
// column hit distinct 16-byte bank groups.
//
// Roofline: MFMA-bound for M >= ~300 (bf16 dense peak 2.5 PFLOP/s,
// flops = 2*m*n*k); HBM-bound below (weight bytes dominate).
#include "rq_epilogue.h"
#include "rq_formats.h"

namespace rq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64, LDS_K = BK + 8;

// A BM x BN tile of y per workgroup of WM x WN waves; each wave owns a
// (BM / WM) x (BN / WN) sub-tile made of MI x NI MFMA tiles of 32 x 32.  Each
// thread decodes exactly one 32-element weight piece per K-step
// (BN * 2 == 64 * WM * WN).
// Split K: workgroup z covers K-steps [z * steps, (z + 1) * steps) and, when
// part is not null, writes its f32 partial tile to part + z * m * n instead
// of y (k_splitk_sum adds the partials).
template <class F, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void k_qgemm(const uint8_t *__restrict__ w,
                                                       const uint8_t *__restrict__ aux,
                                                       const uint16_t *__restrict__ x, int64_t m,
                                                       int64_t n, int64_t k, void *__restrict__ y,
                                                       int ytype, int64_t steps, float *__restrict__ part) {
  constexpr int NT = 64 * WM * WN;
  static_assert(BN * 2 == NT, "one weight piece per thread");
  constexpr int MI = BM / WM / 32, NI = BN / WN / 32;
  constexpr int A_LOADS = BM * BK / 8 / NT;  // 16-byte loads per thread per step
  constexpr int A_ROWS = NT / 8;              // activation rows covered by one load round
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDS_K];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDS_K];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

  // weight piece of this thread: row n0 + (tid >> 1), half h = tid & 1
  const int brow = tid >> 1, bh = tid & 1;
  const int64_t gn = n0 + brow;
  const bool bvalid = gn < n;
  // activation slots: row (tid >> 3) + A_ROWS * i, 8 bf16 at column 8 * (tid & 7)
  const int arow = tid >> 3, acol = 8 * (tid & 7);

  uint4 ra[A_LOADS];
  typename F::Piece pb;
  auto gload = [&](int64_t kt) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int64_t gm = m0 + arow + A_ROWS * i;
      ra[i] = gm < m ? *reinterpret_cast<const uint4 *>(x + gm * k + kt * BK + acol)
                     : make_uint4(0, 0, 0, 0);
    }
    if (bvalid) pb = F::load(w, aux, gn, k, (int)(2 * kt + bh));
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      *reinterpret_cast<uint4 *>(&As[buf][(arow + A_ROWS * i) * LDS_K + acol]) = ra[i];
    uint32_t ob[16];
    if (bvalid) {
      F::decode_bf16(pb, ob);
    } else {
#pragma unroll
      for (int t = 0; t < 16; ++t) ob[t] = 0u;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      uint4 *dst = reinterpret_cast<uint4 *>(&Bs[buf][brow * LDS_K + 16 * bh + 32 * r]);
#pragma unroll
      for (int q = 0; q < 2; ++q)
        dst[q] = make_uint4(ob[8 * r + 4 * q], ob[8 * r + 4 * q + 1], ob[8 * r + 4 * q + 2], ob[8 * r + 4 * q + 3]);
    }
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = (f32x16){0};

  const int64_t kt0 = (int64_t)blockIdx.z * steps;
  const int64_t nk = (k / BK - kt0 < steps ? k / BK - kt0 : steps);
  gload(kt0);
  sstore(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = (int)(kt & 1);
    if (kt + 1 < nk) gload(kt0 + kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kc = ks * 16 + 8 * (lane >> 5);
      bf16x8 fa[MI], fb[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i)
        fa[i] = *reinterpret_cast<const bf16x8 *>(&As[buf][(wm * (BM / WM) + i * 32 + (lane & 31)) * LDS_K + kc]);
#pragma unroll
      for (int j = 0; j < NI; ++j)
        fb[j] = *reinterpret_cast<const bf16x8 *>(&Bs[buf][(wn * (BN / WN) + j * 32 + (lane & 31)) * LDS_K + kc]);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  void *out = part ? static_cast<void *>(part + (int64_t)blockIdx.z * m * n) : y;
  const int otype = part ? (int)RQ_F32 : ytype;
  const bool vec = vec_stores_ok(out, n);
  const float one[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  static_for<MI>([&](auto I) {
    static_for<NI>([&](auto J) {
      store_tile32<false>(acc[I][J], out, otype, m, n, m0 + wm * (BM / WM) + I * 32,
                          n0 + wn * (BN / WN) + J * 32, one, one, nullptr, nullptr, lane, vec);
    });
  });
}

// y = sum over s < splits of part[s] (f32 partials of m * n outputs).
__global__ __launch_bounds__(256) void k_splitk_sum(const float *__restrict__ part, int splits, int64_t mn,
                                                    void *__restrict__ y, int ytype) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < mn; i += (int64_t)gridDim.x * 256) {
    float v = part[i];
    for (int s = 1; s < splits; ++s) v += part[s * mn + i];
    store_one(y, ytype, i, v);
  }
}

// Workgroups per tile along K: enough to give the 256 CUs a workgroup each,
// but only for long K (at least 32 K-steps of 64 per split): the f32
// partials and their sum cost about as much as a 2048-deep tile; at most 8.
int splits_for(int64_t tiles, int64_t nk) {
  int sp = 1;
  while (sp < 8 && tiles * sp < 256 && nk >= 32 * (2 * sp)) sp *= 2;
  return sp;
}

template <class F, int BM, int BN, int WM, int WN>
int launch(const rq_weight *wt, const void *x, int64_t m, void *y, int ytype, hipStream_t s) {
  const int64_t nk = wt->k / BK;
  const int64_t gx = (wt->n + BN - 1) / BN, gy = (m + BM - 1) / BM;
  const int sp = splits_for(gx * gy, nk);
  const int64_t steps = (nk + sp - 1) / sp;
  const int used = (int)((nk + steps - 1) / steps);  // splits that own at least one step
  float *part = nullptr;
  if (used > 1) {
    if (hipMallocAsync(reinterpret_cast<void **>(&part), (size_t)used * m * wt->n * sizeof(float), s) !=
        hipSuccess)
      return set_error(RQ_E_NOMEM, "split-K workspace of %d x %lld x %lld f32", used, (long long)m,
                       (long long)wt->n);
  }
  const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)used);
  hipLaunchKernelGGL((k_qgemm<F, BM, BN, WM, WN>), grid, dim3(64 * WM * WN), 0, s, wt->data,
                     wt->data + wt->aux_off, static_cast<const uint16_t *>(x), m, wt->n, wt->k, y,
                     ytype, steps, part);
  if (part) {
    const int64_t mn = m * wt->n;
    const int64_t blocks = (mn + 255) / 256 < 4096 ? (mn + 255) / 256 : 4096;
    hipLaunchKernelGGL(k_splitk_sum, dim3((unsigned)blocks), dim3(256), 0, s, part, used, mn, y, ytype);
    (void)hipFreeAsync(part, s);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemm launch failed");
}

template <class F>
int by_m(const rq_weight *wt, const void *x, int64_t m, void *y, int ytype, hipStream_t s) {
  if (m <= 64) return launch<F, 64, 128, 2, 2>(wt, x, m, y, ytype, s);
  // 256 x 256 tiles when they still give every CU a workgroup, else 128 x 128.
  const int64_t big_tiles = ((m + 255) / 256) * ((wt->n + 255) / 256);
  if (big_tiles >= 256) return launch<F, 256, 256, 2, 4>(wt, x, m, y, ytype, s);
  return launch<F, 128, 128, 2, 2>(wt, x, m, y, ytype, s);
}

}  // namespace

// bf16 activations, m > 1, k % 64 == 0, 16-byte aligned x.
int launch_linear_mfma(const rq_weight *wt, const void *x, int64_t m, void *y, int ytype,
                       hipStream_t s) {
  if (wt->k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  switch (wt->qtype) {
    case RQ_Q4_K: return by_m<FmtQ4K>(wt, x, m, y, ytype, s);
    case RQ_Q6_K: return by_m<FmtQ6KG>(wt, x, m, y, ytype, s);
    case RQ_Q8_0: return by_m<FmtQ8>(wt, x, m, y, ytype, s);
    case RQ_Q5_K: return by_m<FmtQ5K>(wt, x, m, y, ytype, s);
    case RQ_Q4_0: return by_m<FmtQx0<false>>(wt, x, m, y, ytype, s);
    case RQ_Q5_0: return by_m<FmtQx0<true>>(wt, x, m, y, ytype, s);
    default: return RQ_E_UNSUPPORTED;
  }
}

}  // namespace rq
