// rq_gemv.hip -- quantized GEMV/GEMM on the VALU for gfx950.
//
// Replaces candle's QMatMul::forward as reached from Weights::linear
// (crates/runtimed-model/src/weights/linear_layer.rs:45-52) with the
// semantics of the dense reference: dequant_tensor (dequant.rs:83-146) to f32
// followed by y = x * W^T (linear_layer.rs:88-104), accumulated in f32.
//
// Work split.  A "piece" is the 16-32 bytes of one row that one lane loads
// with 128-bit loads and decodes alone:
//   Q4_K  16 bytes of qs = 32 elements, two runs of 16 (low nibbles at chunk
//         offset 16h, high nibbles at 32+16h) sharing one header.
//   Q6_K  ql[l..l+16), ql[l+32..l+48), qh[l..l+16) of one 128-element half =
//         64 elements in four runs of 16, each with its own int8 scale.
//   Q8_0  the 32 quants of one block, one f16 scale.
// A row of k inputs is P = k / piece_elems pieces.  The pieces of one row sit
// on an aligned segment of SEG = next_pow2(P) lanes (P <= 32: 64/SEG rows per
// wave step), or, when P > 32, on all 64 lanes with PPL = ceil(P/64) pieces
// per lane.  A lane's pieces keep the same k positions from row to row, so in
// the M=1 kernels its activations are loaded once into registers and every
// later step only streams weight bytes.  Rows are cut from the flat block
// stream, so a Q4_K block that straddles two rows (k = 896: 3.5 blocks per
// row) is read by lanes of both rows, each using the header of the block its
// own piece lies in.
//
// Roofline: HBM-bound.  Algorithmic bytes per call = GGUF block bytes of W +
// activation bytes + output bytes.
#include "rq_internal.h"

namespace rq {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float h2f(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

__device__ __forceinline__ float ub(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }

// Load `len` (multiple of 4) activations starting at x[idx] into f32 registers.
template <int LEN>
__device__ __forceinline__ void load_run(const void *x, int xtype, int64_t idx, float *dst) {
#pragma unroll
  for (int j = 0; j < LEN / 4; ++j) {
    const float4 a = load_x4(x, xtype, idx + 4 * j);
    dst[4 * j + 0] = a.x;
    dst[4 * j + 1] = a.y;
    dst[4 * j + 2] = a.z;
    dst[4 * j + 3] = a.w;
  }
}

// ---------------------------------------------------------------- formats --

// Q4_K (dequant_k.rs:19-44) on the aligned GGUF stream.
struct FmtQ4K {
  static constexpr int PE = 32;    // elements per piece
  static constexpr int RUNS = 2;   // runs of 16 activations
  __device__ static int64_t run_off(int p, int r) { return 64 * (p >> 1) + 16 * (p & 1) + 32 * r; }

  struct Piece {
    uint4 hd, qv;
    int c;
  };
  __device__ static Piece load(const uint8_t *w, const uint8_t *, int64_t row, int64_t k, int p) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 64u * (uint64_t)(p >> 1);
    const uint8_t *bp = w + (e >> 8) * 144u;
    Piece pc;
    pc.c = (int)((e >> 6) & 3u);
    pc.hd = *reinterpret_cast<const uint4 *>(bp);
    pc.qv = *reinterpret_cast<const uint4 *>(bp + 16 + 32 * pc.c + 16 * (p & 1));
    return pc;
  }
  // (d*sc, dmin*m) for sub-blocks 2c (low nibbles) and 2c+1 (high nibbles):
  // scale_min_k4 (dequant_k.rs:8-16) on the packed bytes in hd.y/z/w.
  __device__ static void scales(const Piece &pc, float &a0, float &b0, float &a1, float &b1) {
    const int sh = 16 * (pc.c & 1);
    const uint32_t Y = pc.hd.y >> sh, Z = pc.hd.z >> sh, W = pc.hd.w >> sh;
    uint32_t sc0, m0, sc1, m1;
    if (pc.c < 2) {
      sc0 = Y & 63u;
      m0 = Z & 63u;
      sc1 = (Y >> 8) & 63u;
      m1 = (Z >> 8) & 63u;
    } else {
      sc0 = (W & 0xFu) | ((Y >> 2) & 0x30u);
      m0 = ((W >> 4) & 0xFu) | ((Z >> 2) & 0x30u);
      sc1 = ((W >> 8) & 0xFu) | ((Y >> 10) & 0x30u);
      m1 = ((W >> 12) & 0xFu) | ((Z >> 10) & 0x30u);
    }
    const float d = h2f(pc.hd.x), dmin = h2f(pc.hd.x >> 16);
    a0 = d * (float)sc0;
    b0 = dmin * (float)m0;
    a1 = d * (float)sc1;
    b1 = dmin * (float)m1;
  }
  // M=1: sum over the piece of W*x with the activations in registers.
  __device__ static float dot(const Piece &pc, const float (&xv)[RUNS][16], const float (&sx)[RUNS]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
    const uint32_t q[4] = {pc.qv.x, pc.qv.y, pc.qv.z, pc.qv.w};
    float dl[4], dh[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = q[j] & 0x0F0F0F0Fu, hi = q[j] & 0xF0F0F0F0u;
      dl[j] = xv[0][4 * j] * ub(lo, 0);
      dh[j] = xv[1][4 * j] * ub(hi, 0);
#pragma unroll
      for (int b = 1; b < 4; ++b) {
        dl[j] = fmaf(xv[0][4 * j + b], ub(lo, b), dl[j]);
        dh[j] = fmaf(xv[1][4 * j + b], ub(hi, b), dh[j]);
      }
    }
    const float sl = (dl[0] + dl[1]) + (dl[2] + dl[3]);
    const float shh = ((dh[0] + dh[1]) + (dh[2] + dh[3])) * 0.0625f;  // high nibbles were x16
    return (a0 * sl - b0 * sx[0]) + (a1 * shh - b1 * sx[1]);
  }
  // Exact dequantized weights of the piece, in run order.
  __device__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
    float a0, b0, a1, b1;
    scales(pc, a0, b0, a1, b1);
    const uint32_t q[4] = {pc.qv.x, pc.qv.y, pc.qv.z, pc.qv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        wv[0][4 * j + b] = a0 * (float)((q[j] >> (8 * b)) & 0xFu) - b0;
        wv[1][4 * j + b] = a1 * (float)((q[j] >> (8 * b + 4)) & 0xFu) - b1;
      }
  }
};

// Q6_K (dequant_k.rs:87-111) on the split layout: 208-byte records + f16 d.
struct FmtQ6K {
  static constexpr int PE = 64;
  static constexpr int RUNS = 4;
  __device__ static int64_t run_off(int p, int r) { return 128 * (p >> 1) + 16 * (p & 1) + 32 * r; }

  struct Piece {
    uint4 a, b, h;
    uint2 sc;
    uint32_t d;
    int s;
  };
  __device__ static Piece load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int p) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 128u * (uint64_t)(p >> 1);
    const uint64_t blk = e >> 8;
    const int hf = (int)((e >> 7) & 1u), s = p & 1;
    const uint8_t *rec = w + blk * 208u;
    Piece pc;
    pc.s = s;
    pc.a = *reinterpret_cast<const uint4 *>(rec + 64 * hf + 16 * s);
    pc.b = *reinterpret_cast<const uint4 *>(rec + 64 * hf + 32 + 16 * s);
    pc.h = *reinterpret_cast<const uint4 *>(rec + 128 + 32 * hf + 16 * s);
    pc.sc = *reinterpret_cast<const uint2 *>(rec + 192 + 8 * hf);
    pc.d = reinterpret_cast<const uint16_t *>(aux)[blk];
    return pc;
  }
  // Unsigned 6-bit codes (q + 32) of run r for dword j.
  __device__ static uint32_t codes(const Piece &pc, int r, int j) {
    const uint32_t a = (&pc.a.x)[j], b = (&pc.b.x)[j], h = (&pc.h.x)[j];
    switch (r) {
      case 0: return (a & 0x0F0F0F0Fu) | ((h & 0x03030303u) << 4);
      case 1: return (b & 0x0F0F0F0Fu) | ((h & 0x0C0C0C0Cu) << 2);
      case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
      default: return ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    }
  }
  // int8 scale of run r: scales[8*hf + s + 2r] (dequant_k.rs:107).
  __device__ static float scale(const Piece &pc, int r) {
    const int byte = pc.s + 2 * r;
    const uint32_t word = byte < 4 ? pc.sc.x : pc.sc.y;
    return (float)(int8_t)((word >> (8 * (byte & 3))) & 0xFFu);
  }
  __device__ static float dot(const Piece &pc, const float (&xv)[RUNS][16], const float (&sx)[RUNS]) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < RUNS; ++r) {
      float dd[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t q = codes(pc, r, j);
        dd[j] = xv[r][4 * j] * ub(q, 0);
#pragma unroll
        for (int b = 1; b < 4; ++b) dd[j] = fmaf(xv[r][4 * j + b], ub(q, b), dd[j]);
      }
      const float dot = (dd[0] + dd[1]) + (dd[2] + dd[3]);
      acc = fmaf(scale(pc, r), dot - 32.0f * sx[r], acc);
    }
    return h2f(pc.d) * acc;
  }
  __device__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
    const float d = h2f(pc.d);
#pragma unroll
    for (int r = 0; r < RUNS; ++r) {
      const float ds = d * scale(pc, r);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t q = codes(pc, r, j);
#pragma unroll
        for (int b = 0; b < 4; ++b) wv[r][4 * j + b] = ds * (ub(q, b) - 32.0f);
      }
    }
  }
};

// Q8_0 (dequant.rs:40-47) on the split layout: int8 quants + f16 d.
struct FmtQ8 {
  static constexpr int PE = 32;
  static constexpr int RUNS = 2;
  __device__ static int64_t run_off(int p, int r) { return 32 * p + 16 * r; }

  struct Piece {
    uint4 q0, q1;
    uint32_t d;
  };
  __device__ static Piece load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int p) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 32u * (uint64_t)p;
    Piece pc;
    pc.q0 = *reinterpret_cast<const uint4 *>(w + e);
    pc.q1 = *reinterpret_cast<const uint4 *>(w + e + 16);
    pc.d = reinterpret_cast<const uint16_t *>(aux)[e >> 5];
    return pc;
  }
  __device__ static float dot(const Piece &pc, const float (&xv)[RUNS][16], const float (&sx)[RUNS]) {
    const uint32_t q[8] = {pc.q0.x, pc.q0.y, pc.q0.z, pc.q0.w, pc.q1.x, pc.q1.y, pc.q1.z, pc.q1.w};
    float dd[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t u = q[j] ^ 0x80808080u;  // q + 128 as unsigned bytes
      const float *xr = &xv[j >> 2][4 * (j & 3)];
      dd[j] = xr[0] * ub(u, 0);
#pragma unroll
      for (int b = 1; b < 4; ++b) dd[j] = fmaf(xr[b], ub(u, b), dd[j]);
    }
    const float dot = ((dd[0] + dd[1]) + (dd[2] + dd[3])) + ((dd[4] + dd[5]) + (dd[6] + dd[7]));
    return h2f(pc.d) * (dot - 128.0f * (sx[0] + sx[1]));
  }
  __device__ static void decode(const Piece &pc, float (&wv)[RUNS][16]) {
    const float d = h2f(pc.d);
    const uint32_t q[8] = {pc.q0.x, pc.q0.y, pc.q0.z, pc.q0.w, pc.q1.x, pc.q1.y, pc.q1.z, pc.q1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int b = 0; b < 4; ++b) wv[j >> 2][4 * (j & 3) + b] = d * (float)(int8_t)((q[j] >> (8 * b)) & 0xFFu);
  }
};

// --------------------------------------------------------------- kernels --

// M = 1: activations in registers, weights streamed once.
template <class F, int PPL>
__global__ __launch_bounds__(kThreads) void k_gemv_m1(const uint8_t *__restrict__ w,
                                                     const uint8_t *__restrict__ aux,
                                                     const void *__restrict__ x, int xtype,
                                                     void *__restrict__ y, int ytype, int64_t n,
                                                     int64_t k, int seg_log2) {
  const int lane = threadIdx.x & 63;
  const int seg = lane >> seg_log2, sl = lane & ((1 << seg_log2) - 1);
  const int rg = 64 >> seg_log2;
  const int P = (int)(k / F::PE);
  float xv[PPL][F::RUNS][16];
  float sx[PPL][F::RUNS];
  int pc[PPL];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int p = sl + (i << seg_log2);
    pc[i] = p < P ? p : -1;
#pragma unroll
    for (int r = 0; r < F::RUNS; ++r) {
      sx[i][r] = 0.0f;
      if (p < P) {
        load_run<16>(x, xtype, F::run_off(p, r), xv[i][r]);
#pragma unroll
        for (int t = 0; t < 16; ++t) sx[i][r] += xv[i][r][t];
      } else {
#pragma unroll
        for (int t = 0; t < 16; ++t) xv[i][r][t] = 0.0f;
      }
    }
  }
  const int64_t groups = (n + rg - 1) / rg;
  const int64_t nw = (int64_t)gridDim.x * (kThreads / 64);
  for (int64_t g = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); g < groups; g += nw) {
    const int64_t row = g * rg + seg;
    float acc = 0.0f;
    if (row < n) {
      typename F::Piece pcs[PPL];
#pragma unroll
      for (int i = 0; i < PPL; ++i)
        if (pc[i] >= 0) pcs[i] = F::load(w, aux, row, k, pc[i]);
#pragma unroll
      for (int i = 0; i < PPL; ++i)
        if (pc[i] >= 0) acc += F::dot(pcs[i], xv[i], sx[i]);
    }
    for (int off = 32 >> (6 - seg_log2); off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (sl == 0 && row < n) store_out(y, ytype, row, acc);
  }
}

// M > 1 (interim path): each piece is decoded once to exact f32 weights and
// then dotted with every activation row, read from memory.
template <class F, int PPL>
__global__ __launch_bounds__(kThreads) void k_gemv_multi(const uint8_t *__restrict__ w,
                                                        const uint8_t *__restrict__ aux,
                                                        const void *__restrict__ x, int xtype,
                                                        int64_t m, void *__restrict__ y, int ytype,
                                                        int64_t n, int64_t k, int seg_log2) {
  const int lane = threadIdx.x & 63;
  const int seg = lane >> seg_log2, sl = lane & ((1 << seg_log2) - 1);
  const int rg = 64 >> seg_log2;
  const int P = (int)(k / F::PE);
  const int64_t groups = (n + rg - 1) / rg;
  const int64_t nw = (int64_t)gridDim.x * (kThreads / 64);
  for (int64_t g = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); g < groups; g += nw) {
    const int64_t row = g * rg + seg;
    float wv[PPL][F::RUNS][16];
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int p = sl + (i << seg_log2);
      if (row < n && p < P) {
        F::decode(F::load(w, aux, row, k, p), wv[i]);
      } else {
#pragma unroll
        for (int r = 0; r < F::RUNS; ++r)
#pragma unroll
          for (int t = 0; t < 16; ++t) wv[i][r][t] = 0.0f;
      }
    }
    for (int64_t mi = 0; mi < m; ++mi) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < PPL; ++i) {
        const int p = sl + (i << seg_log2);
        if (row < n && p < P) {
#pragma unroll
          for (int r = 0; r < F::RUNS; ++r) {
            float xr[16];
            load_run<16>(x, xtype, mi * k + F::run_off(p, r), xr);
#pragma unroll
            for (int t = 0; t < 16; ++t) acc = fmaf(wv[i][r][t], xr[t], acc);
          }
        }
      }
      for (int off = 32 >> (6 - seg_log2); off > 0; off >>= 1) acc += __shfl_xor(acc, off);
      if (sl == 0 && row < n) store_out(y, ytype, mi * n + row, acc);
    }
  }
}

// Dense f32 weights (the decode-then-multiply path for shapes without a fused
// kernel): one wave per output row, lanes stride over k.
__global__ __launch_bounds__(kThreads) void k_dense_f32(const float *__restrict__ w, int64_t n,
                                                       int64_t k, const void *__restrict__ x,
                                                       int xtype, int64_t m, void *__restrict__ y,
                                                       int ytype) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * (kThreads / 64);
  for (int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); row < n; row += nw) {
    const float *wr = w + row * k;
    for (int64_t mi = 0; mi < m; ++mi) {
      float acc = 0.0f;
      for (int64_t t = lane; t < k; t += 64) {
        float xv;
        if (xtype == RQ_F32) xv = static_cast<const float *>(x)[mi * k + t];
        else if (xtype == RQ_BF16) xv = bf16_bits_to_f32(static_cast<const uint16_t *>(x)[mi * k + t]);
        else xv = (float)static_cast<const _Float16 *>(x)[mi * k + t];
        acc = fmaf(wr[t], xv, acc);
      }
      for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
      if (lane == 0) store_out(y, ytype, mi * n + row, acc);
    }
  }
}

int ceil_log2(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

template <class F, int PPL>
int run_fused(const rq_weight *wt, const void *x, int xtype, int64_t m, void *y, int ytype,
              int seg_log2, hipStream_t s) {
  const int rg = 64 >> seg_log2;
  const int64_t groups = (wt->n + rg - 1) / rg;
  const int64_t waves_per_block = kThreads / 64;
  int64_t blocks = (groups + waves_per_block - 1) / waves_per_block;
  if (blocks > 8192) blocks = 8192;
  const uint8_t *aux = wt->data + wt->aux_off;
  if (m == 1) {
    hipLaunchKernelGGL((k_gemv_m1<F, PPL>), dim3((unsigned)blocks), dim3(kThreads), 0, s, wt->data,
                       aux, x, xtype, y, ytype, wt->n, wt->k, seg_log2);
  } else {
    hipLaunchKernelGGL((k_gemv_multi<F, PPL>), dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       wt->data, aux, x, xtype, m, y, ytype, wt->n, wt->k, seg_log2);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
}

template <class F>
int dispatch_fmt(const rq_weight *wt, const void *x, int xtype, int64_t m, void *y, int ytype,
                 int max_ppl, hipStream_t s) {
  if (wt->k % F::PE != 0) return RQ_E_UNSUPPORTED;
  const int P = (int)(wt->k / F::PE);
  if (P <= 32) return run_fused<F, 1>(wt, x, xtype, m, y, ytype, ceil_log2(P), s);
  const int ppl = (P + 63) / 64;
  if (ppl > max_ppl) return RQ_E_UNSUPPORTED;
  switch (ppl) {
    case 1: return run_fused<F, 1>(wt, x, xtype, m, y, ytype, 6, s);
    case 2: return run_fused<F, 2>(wt, x, xtype, m, y, ytype, 6, s);
    case 3: return run_fused<F, 3>(wt, x, xtype, m, y, ytype, 6, s);
    case 4: return run_fused<F, 4>(wt, x, xtype, m, y, ytype, 6, s);
    default: return RQ_E_UNSUPPORTED;
  }
}

}  // namespace

int launch_linear_fused(const rq_weight *wt, const void *x, int xtype, int64_t m, void *y,
                        int ytype, hipStream_t s) {
  switch (wt->qtype) {
    case RQ_Q4_K:
      // Pieces must not straddle rows: rows start on 64-element chunk bounds.
      if (wt->k % 64 != 0) return RQ_E_UNSUPPORTED;
      return dispatch_fmt<FmtQ4K>(wt, x, xtype, m, y, ytype, 4, s);
    case RQ_Q6_K:
      if (wt->k % 128 != 0) return RQ_E_UNSUPPORTED;
      return dispatch_fmt<FmtQ6K>(wt, x, xtype, m, y, ytype, 2, s);
    case RQ_Q8_0:
      return dispatch_fmt<FmtQ8>(wt, x, xtype, m, y, ytype, 4, s);
    default:
      return RQ_E_UNSUPPORTED;
  }
}

int launch_linear_dense_f32(const float *w, int64_t n, int64_t k, const void *x, int xtype,
                            int64_t m, void *y, int ytype, hipStream_t s) {
  int64_t blocks = (n + 3) / 4;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_dense_f32, dim3((unsigned)blocks), dim3(kThreads), 0, s, w, n, k, x, xtype,
                     m, y, ytype);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "dense launch failed");
}

}  // namespace rq
