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
// A row of k inputs is P = k / piece_elems pieces.  Three layouts:
//   segment  P <= 64: a row on an aligned segment of max(16, next_pow2(P))
//            lanes, 64 / segment rows per wave (k_gemv_m1);
//   team     P > 64 on n < 4096 (or more than 256 pieces): a row on a team of
//            ceil(P / 64) waves, one piece per lane (k_gemv_team);
//   long     P in 65..256 on n >= 4096: a row on one wave, PPL = ceil(P / 64)
//            pieces per lane (k_gemv_long).
// A lane's pieces keep the same k positions from row to row, so its
// activations (one row, or two / four row slots for M = 2 / 3) are loaded
// once into registers and every later row only streams weight bytes.  Rows
// are cut from the flat block
// stream, so a Q4_K block that straddles two rows (k = 896: 3.5 blocks per
// row) is read by lanes of both rows, each using the header of the block its
// own piece lies in.
//
// Roofline: HBM-bound.  Algorithmic bytes per call = GGUF block bytes of W +
// activation bytes + output bytes.
#include <type_traits>

#include "rq_formats.h"

namespace rq {
namespace {

constexpr int kThreads = 256;

// Formats with a multi-row dot product (F::dot_rows<MR>).
template <class F, class = void>
struct has_dot_rows : std::false_type {};
template <class F>
struct has_dot_rows<F, std::void_t<decltype(&F::template dot_rows<2>)>> : std::true_type {};

// --------------------------------------------------------------- kernels --

// Sum over aligned lane segments of 16, 32 or 64 lanes with DPP: row_ror
// 8/4/2/1 inside each 16-lane row, then row_bcast15 / row_bcast31 across rows.
// The segment total lands in the segment's last lane.
#define RQ_DPP(v, ctrl, rows) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), (rows), 0xF, false))

__device__ __forceinline__ float seg_sum(float v, int seg) {
  v += RQ_DPP(v, 0x128, 0xF);  // row_ror:8
  v += RQ_DPP(v, 0x124, 0xF);  // row_ror:4
  v += RQ_DPP(v, 0x122, 0xF);  // row_ror:2
  v += RQ_DPP(v, 0x121, 0xF);  // row_ror:1
  if (seg >= 32) v += RQ_DPP(v, 0x142, 0xA);  // row_bcast:15 into rows 1 and 3
  if (seg >= 64) v += RQ_DPP(v, 0x143, 0xC);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Activations of an M = 1 call, staged once per workgroup in LDS as f32.
// Loading each lane's 32-64 activations straight from global memory made
// every wave pull a full copy of x through the L1/TA path (x is small, but it
// is read 8-16x more often than the weights): on a 4864 x 896 GEMV that cost
// 1.6 of 4.7 us.  Layout: 16 bytes of padding after every 256 bytes, so the
// 8 lanes served by one ds_read_b128 (pieces 64 floats apart) hit distinct
// banks.  A run of 16 activations never crosses a padding gap.
constexpr int64_t kXldsMaxK = 12288;
__device__ __forceinline__ int xpad(int e) { return e + 4 * (e >> 6); }
__host__ __device__ inline size_t xlds_bytes(int64_t k) { return k <= kXldsMaxK ? (size_t)(k + 4 * (k >> 6) + 4) * sizeof(float) : 0; }

__device__ __forceinline__ void stage_x(const void *x, int xtype, int k, float *xs) {
  for (int e = 4 * (int)threadIdx.x; e < k; e += 4 * (int)blockDim.x)
    *reinterpret_cast<float4 *>(xs + xpad(e)) = load_x4(x, xtype, e);
  __syncthreads();
}

// The same staging split in two, for kernels that issue x's loads before
// their weight loads: the load counter retires loads in issue order, so a
// wait for x loads issued after the weights would hold the staging until the
// (HBM) weights had landed too.  Thread t loads the 16-byte chunks t,
// t + blockDim, ... of x (4 f32 or 8 f16/bf16 elements each) with one
// unconditional load form for every type (clamped to the last chunk); the
// conversion and the LDS stores follow the weight loads.  XR = chunks per
// thread, >= ceil(k / (elements per chunk) / blockDim).
typedef uint32_t chunk16 __attribute__((ext_vector_type(4)));

__host__ __device__ inline int x_chunks(int64_t k, int xtype) { return (int)(k >> (xtype == RQ_F32 ? 2 : 3)); }

template <int XR>
__device__ __forceinline__ void load_x_chunks(const void *x, int xtype, int k, chunk16 (&v)[XR]) {
  const int nc = x_chunks(k, xtype);
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const int c = (int)threadIdx.x + i * (int)blockDim.x;
    v[i] = reinterpret_cast<const chunk16 *>(x)[c < nc ? c : nc - 1];
  }
}

// Every thread stores all XR chunks, threads past the end the (clamped) last
// chunk again: identical bytes to the same place.  A store under "c < nc"
// would let the compiler sink the load into that branch, behind the weights.
template <int XR>
__device__ __forceinline__ void store_x_chunks(int xtype, int k, const chunk16 (&v)[XR], float *xs) {
  const int nc = x_chunks(k, xtype);
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const int c0 = (int)threadIdx.x + i * (int)blockDim.x;
    const int c = c0 < nc ? c0 : nc - 1;
    const chunk16 u = v[i];
    if (xtype == RQ_F32) {
      *reinterpret_cast<float4 *>(xs + xpad(4 * c)) =
          make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
    } else {
      float f[8];
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (xtype == RQ_BF16) {
          f[2 * j] = __uint_as_float(wd[j] << 16);
          f[2 * j + 1] = __uint_as_float(wd[j] & 0xFFFF0000u);
        } else {
          f[2 * j] = h2f(wd[j]);
          f[2 * j + 1] = h2f(wd[j] >> 16);
        }
      }
      *reinterpret_cast<float4 *>(xs + xpad(8 * c)) = make_float4(f[0], f[1], f[2], f[3]);
      *reinterpret_cast<float4 *>(xs + xpad(8 * c + 4)) = make_float4(f[4], f[5], f[6], f[7]);
    }
  }
  __syncthreads();
}

// store_x_chunks for MR activation rows loaded as one run of chunks: chunk
// c holds elements [c e, (c + 1) e) of the flattened [MR][k] block (e = 4
// or 8 values; k is a multiple of e), stored in row c e / k at xstride.
template <int XR>
__device__ __forceinline__ void store_x_chunks_rows(int xtype, int k, int mr, int xstride, const chunk16 (&v)[XR],
                                                    float *xs) {
  const int epc = xtype == RQ_F32 ? 4 : 8;
  const int nc = mr * k / epc;
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const int c0 = (int)threadIdx.x + i * (int)blockDim.x;
    const int c = c0 < nc ? c0 : nc - 1;
    int e = c * epc, row = 0;
    while (e >= k) {  // mr <= 4: at most three steps
      e -= k;
      ++row;
    }
    float *dst = xs + row * xstride;
    const chunk16 u = v[i];
    if (xtype == RQ_F32) {
      *reinterpret_cast<float4 *>(dst + xpad(e)) =
          make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
    } else {
      float f[8];
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (xtype == RQ_BF16) {
          f[2 * j] = __uint_as_float(wd[j] << 16);
          f[2 * j + 1] = __uint_as_float(wd[j] & 0xFFFF0000u);
        } else {
          f[2 * j] = h2f(wd[j]);
          f[2 * j + 1] = h2f(wd[j] >> 16);
        }
      }
      *reinterpret_cast<float4 *>(dst + xpad(e)) = make_float4(f[0], f[1], f[2], f[3]);
      *reinterpret_cast<float4 *>(dst + xpad(e + 4)) = make_float4(f[4], f[5], f[6], f[7]);
    }
  }
  __syncthreads();
}

template <int LEN>
__device__ __forceinline__ void load_run_lds(const float *xs, int e0, float *dst) {
  const float4 *src = reinterpret_cast<const float4 *>(xs + xpad(e0));
#pragma unroll
  for (int j = 0; j < LEN / 4; ++j) {
    const float4 a = src[j];
    dst[4 * j + 0] = a.x;
    dst[4 * j + 1] = a.y;
    dst[4 * j + 2] = a.z;
    dst[4 * j + 3] = a.w;
  }
}

// Loads run r of piece p: from the LDS copy when there is one (xs != null).
template <class F>
__device__ __forceinline__ void load_piece_x(const void *x, int xtype, const float *xs, int p, int r, float *dst) {
  if (xs) load_run_lds<16>(xs, (int)F::run_off(p, r), dst);
  else load_run<16>(x, xtype, F::run_off(p, r), dst);
}

// M = MR (1 or 2), rows of at most 64 pieces: every lane owns one piece
// position; its activations (MR rows) are loaded once into registers, and a
// piece's weights are converted once for the MR dot products.  A row sits on an aligned
// segment of seg = max(16, next_pow2(P)) lanes (64/seg rows per wave).  The
// loads of x (XR 16-byte chunks per thread, L2-resident) are issued first,
// then the bias of the lane's row, and the first row's weight loads right
// behind them, so x is staged in LDS while the weights are still in flight.
// A workgroup walking several row groups (g0 + blockIdx.x, + gridDim.x, ...
// up to groups) issues the next group's loads before it computes the
// current one.
// PLAIN: f32 activations and outputs without a bias (the reference's decode
// call), known at compile time, so the activation-type, output-type and bias
// branches fold away: 931 -> 562 instructions on the Q4_K segment kernel,
// 62 -> 14 branches, decode layer set 414.8 -> 426.6 GB/s (gate 2.99 -> 2.94
// us).
template <class F, int XR, int MR, bool PLAIN = false>
__device__ __forceinline__ void gemv_seg(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                         const void *__restrict__ x, int xtype_arg, const Out &o_arg, int64_t n,
                                         int64_t k, int seg_log2, int rows_per_wg, int64_t g, int64_t groups,
                                         int mrows, bool one_group) {
  const int xtype = PLAIN ? RQ_F32 : xtype_arg;
  const Out o = PLAIN ? Out{o_arg.y, nullptr, RQ_F32, 0} : o_arg;
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int P = (int)(k / F::PE);
  const int row_in_wg = wv * (64 >> seg_log2) + (lane >> seg_log2);
  const int p = lane & ((1 << seg_log2) - 1);
  const bool live = p < P;
  // Loads use a piece and row clamped into the matrix, unconditionally:
  // a load under a branch makes the compiler drain every outstanding load
  // (the prefetched row too) before the next use.  Dead lanes and rows past
  // n contribute nothing (the dot product is selected away).
  const int pl = live ? p : P - 1;
  int64_t row = g * rows_per_wg + row_in_wg;
  extern __shared__ __attribute__((aligned(16))) float xs_dyn[];
  // MR activation rows (x is [MR][k], contiguous) as one run of chunks; row
  // i of the LDS copy starts at i * xstride.
  const int xstride = (int)(xlds_bytes(k) / sizeof(float));
  chunk16 xc[XR];
  // mrows <= MR rows of x exist; loads clamp to them, and rows mrows .. MR - 1
  // of the LDS copy are neither written nor their results stored.
  load_x_chunks<XR>(x, xtype, mrows * (int)k, xc);
  // The bias's bits (a uniform branch) behind x: a wait for x covers them.
  uint32_t bv = 0;
  if (o.bias) bv = bias_bits(o.bias, o.btype, row < n ? row : n - 1);
  __builtin_amdgcn_sched_barrier(0);
  typename F::Piece cur = F::template load<true>(w, aux, row < n ? row : n - 1, k, pl);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (MR == 1) store_x_chunks<XR>(xtype, (int)k, xc, xs_dyn);
  else store_x_chunks_rows<XR>(xtype, (int)k, mrows, xstride, xc, xs_dyn);
  float xv[MR][F::RUNS][16];
  float sx[MR][F::RUNS];
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < F::RUNS; ++r) {
      sx[i][r] = 0.0f;
      if (live) {
        load_run_lds<16>(xs_dyn + i * xstride, (int)F::run_off(p, r), xv[i][r]);
#pragma unroll
        for (int t = 0; t < 16; ++t) sx[i][r] += xv[i][r][t];
      } else {
#pragma unroll
        for (int t = 0; t < 16; ++t) xv[i][r][t] = 0.0f;
      }
    }

  // Dot products, segment totals and stores of one row group.
  auto emit = [&](const typename F::Piece &pc, int64_t r, uint32_t b) {
    float dr[MR];
    if constexpr (MR > 1 && has_dot_rows<F>::value) {
      F::template dot_rows<MR>(pc, xv, sx, dr);
    } else {
#pragma unroll
      for (int i = 0; i < MR; ++i) dr[i] = F::dot(pc, xv[i], sx[i]);
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      const float d = dr[i];
      float acc = (live && r < n) ? d : 0.0f;
      const int seg = 1 << seg_log2;
      acc = seg_sum(acc, seg);
      if (o.bias) acc = with_bias(acc, bias_bits_f32(b, o.btype), o.ytype);
      if ((lane & (seg - 1)) == seg - 1 && r < n && i < mrows) store_out(o.y, o.ytype, i * n + r, acc);
    }
  };
  // One row group per workgroup (every decode-sized matrix): no prefetch.
  // A next-row load in the last pass is never used, and the wave still has
  // to wait for it before it can end.
  if (one_group) {
    emit(cur, row, bv);
    return;
  }
  for (; g < groups; g += gridDim.x) {
    const int64_t gn = g + gridDim.x;
    const int64_t row_n = gn * rows_per_wg + row_in_wg;
    const typename F::Piece nxt = F::template load<true>(w, aux, (gn < groups && row_n < n) ? row_n : (row < n ? row : n - 1), k, pl);
    emit(cur, row, bv);
    cur = nxt;
    row = row_n;
    if (o.bias) bv = bias_bits(o.bias, o.btype, row < n ? row : n - 1);
  }
}

// One weight: groups row groups over the grid.
template <class F, int XR, int MR, bool PLAIN = false>
__global__ __launch_bounds__(256) void k_gemv_m1(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                const void *__restrict__ x, int xtype, const Out o, int64_t n,
                                                int64_t k, int seg_log2, int rows_per_wg, int64_t groups,
                                                int mrows) {
  gemv_seg<F, XR, MR, PLAIN>(w, aux, x, xtype, o, n, k, seg_log2, rows_per_wg, blockIdx.x, groups, mrows,
                             groups <= (int64_t)gridDim.x);
}

// A set of weights sharing x: one row group per workgroup, the grid covering
// every weight's groups (pick_entry chooses this workgroup's weight).
template <class F, int XR, int MR, bool PLAIN = false>
__global__ __launch_bounds__(256) void k_gemv_set(const WeightSet set, const void *__restrict__ x, int xtype,
                                                 int64_t k, int seg_log2, int rows_per_wg, int mrows) {
  const int bid = (int)blockIdx.x;
  const SetEntry e = pick_entry(set, bid);
  gemv_seg<F, XR, MR, PLAIN>(e.w, e.aux, x, xtype, e.o, e.n, k, seg_log2, rows_per_wg, bid - e.g0, e.g1 - e.g0,
                             mrows, true);
}

// M = 1, long rows (P > 64 pieces): one wave per row, PPL pieces per lane
// (piece lane + 64 i), activations in registers; the wave walks the rows
// row0, row0 + nw, row0 + 2 nw, ... (nw = waves in the grid) with the loads
// of D of them in flight: D slots of pieces, refilled with the row D strides
// ahead as soon as a slot's row is computed.  Slot indices are static and
// every load is unconditional (rows past n clamp to the slot's own row, just
// read), so the compiler's waits are exact counts; the last group of D rows
// refills nothing.  No barriers in the loop: the row total is a DPP sum over
// the wave.  WPG waves per workgroup share one LDS copy of x.  With XR > 0
// (XR = 16-byte chunks of x per thread, enough for any k this instance
// takes) x's loads go out first and the first D rows' weight loads right
// behind them, so x is staged while the weights are in flight.
template <class F, int PPL, int WPG>
constexpr int long_xr() {
  constexpr int need = (PPL * F::PE + 4 * WPG - 1) / (4 * WPG);  // f32 chunks per thread at k = 64 PPL PE
  return need <= 4 ? need : 0;
}

template <class F, int PPL, int WPG, int D>
__global__ __launch_bounds__(64 * WPG) void k_gemv_long(const uint8_t *__restrict__ w,
                                                        const uint8_t *__restrict__ aux, const void *__restrict__ x,
                                                        int xtype, const Out o, int64_t n, int64_t k, bool xlds) {
  constexpr int XR = long_xr<F, PPL, WPG>();
  const int lane = threadIdx.x & 63;
  const int P = (int)(k / F::PE);
  const int64_t nw = (int64_t)gridDim.x * WPG;
  const int64_t row0 = (int64_t)blockIdx.x * WPG + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  int pc[PPL];
#pragma unroll
  for (int i = 0; i < PPL; ++i) pc[i] = lane + 64 * i < P ? lane + 64 * i : P - 1;
  typename F::Piece sl[D][PPL];
  auto fill = [&](int j, int64_t r, int64_t fallback) {
    const int64_t rr = r < n ? r : fallback;
#pragma unroll
    for (int i = 0; i < PPL; ++i) sl[j][i] = F::template load<true>(w, aux, rr, k, pc[i]);
  };
  const int64_t first = row0 < n ? row0 : n - 1;

  extern __shared__ __attribute__((aligned(16))) float xs_dyn[];
  if constexpr (XR > 0) {  // launched only with the LDS copy of x
    chunk16 xc[XR];
    load_x_chunks<XR>(x, xtype, (int)k, xc);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < D; ++j) fill(j, row0 + j * nw, first);
    __builtin_amdgcn_sched_barrier(0);
    store_x_chunks<XR>(xtype, (int)k, xc, xs_dyn);
  } else {
#pragma unroll
    for (int j = 0; j < D; ++j) fill(j, row0 + j * nw, first);
    if (xlds) stage_x(x, xtype, (int)k, xs_dyn);  // uniform: the whole workgroup stages x once
  }
  float xv[PPL][F::RUNS][16];
  float sx[PPL][F::RUNS];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int p = lane + 64 * i;
#pragma unroll
    for (int r = 0; r < F::RUNS; ++r) {
      sx[i][r] = 0.0f;
      if (p < P) {
        if constexpr (XR > 0) load_run_lds<16>(xs_dyn, (int)F::run_off(p, r), xv[i][r]);
        else load_piece_x<F>(x, xtype, xlds ? xs_dyn : nullptr, p, r, xv[i][r]);
#pragma unroll
        for (int t = 0; t < 16; ++t) sx[i][r] += xv[i][r][t];
      } else {
#pragma unroll
        for (int t = 0; t < 16; ++t) xv[i][r][t] = 0.0f;
      }
    }
  }

  auto emit = [&](int j, int64_t r) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const float d = F::dot(sl[j][i], xv[i], sx[i]);
      acc += lane + 64 * i < P ? d : 0.0f;
    }
    acc = seg_sum(acc, 64);
    if (lane == 63 && r < n) store_linear(o, 0, n, r, acc);
  };
  // Groups of D rows: every group but the last refills its slots.
  const int64_t rows = row0 < n ? (n - row0 + nw - 1) / nw : 0;  // rows of this wave
  const int64_t groups = (rows + D - 1) / D;
  int64_t base = row0;
  for (int64_t g = 1; g < groups; ++g, base += D * nw) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int64_t r = base + j * nw;
      emit(j, r);
      fill(j, r + D * nw, r < n ? r : n - 1);
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) emit(j, base + j * nw);
}

// A run of 16 activations at element e0 (a multiple of 16) straight from
// global memory: four 16-byte chunks, clamped to the last chunk of x, in one
// unconditional load form for every type (f32 uses all four, f16 / bf16 the
// first two), converted after the loads.
__device__ __forceinline__ void load_run_raw(const void *x, int xtype, int k, int e0, chunk16 (&v)[4]) {
  const int nc = x_chunks(k, xtype);
  const int c0 = e0 >> (xtype == RQ_F32 ? 2 : 3);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = reinterpret_cast<const chunk16 *>(x)[c0 + j < nc ? c0 + j : nc - 1];
}

__device__ __forceinline__ void convert_run(int xtype, const chunk16 (&v)[4], float *dst) {
  if (xtype == RQ_F32) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dst[4 * j + 0] = __uint_as_float(v[j].x);
      dst[4 * j + 1] = __uint_as_float(v[j].y);
      dst[4 * j + 2] = __uint_as_float(v[j].z);
      dst[4 * j + 3] = __uint_as_float(v[j].w);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t wd[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        dst[8 * j + 2 * q] = xtype == RQ_BF16 ? __uint_as_float(wd[q] << 16) : h2f(wd[q]);
        dst[8 * j + 2 * q + 1] = xtype == RQ_BF16 ? __uint_as_float(wd[q] & 0xFFFF0000u) : h2f(wd[q] >> 16);
      }
    }
  }
}

// M = 1, long rows on fewer rows (P > 64 pieces, n < 4096): a workgroup is
// one team of T = blockDim / 64 waves covering a row's pieces (piece
// 64 tm + lane), walking the rows blockIdx.x, blockIdx.x + gridDim.x, ...
// with D rows of weight loads in flight (static slots, unconditional loads,
// as in k_gemv_long).  The team's lanes hold disjoint pieces, so each lane
// loads its own activations straight from global memory, once: x is read
// once per workgroup and needs no LDS copy or barrier.  Those loads go out
// before the first weight loads (the load counter retires in order).  Each
// row's wave sums go to LDS; after the last row one barrier, then one thread
// per row adds the T partial sums.  At most kTeamRows rows per workgroup.
constexpr int kTeamRows = 64;
constexpr int kTeamMax = 16;

template <class F, int D, int MR, bool PLAIN = false>
__global__ __launch_bounds__(1024) void k_gemv_team(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                   const void *__restrict__ x, int xtype_arg, const Out o_arg,
                                                   int64_t n, int64_t k) {
  // PLAIN as in gemv_seg: f32 activations and outputs, no bias, folded
  const int xtype = PLAIN ? RQ_F32 : xtype_arg;
  const Out o = PLAIN ? Out{o_arg.y, nullptr, RQ_F32, 0} : o_arg;
  __shared__ float red[MR][kTeamRows][kTeamMax];
  const int lane = threadIdx.x & 63, tm = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int team = (int)(blockDim.x >> 6);
  const int P = (int)(k / F::PE);
  const int p = 64 * tm + lane;
  const bool live = p < P;
  const int pl = live ? p : P - 1;
  const int64_t r0 = blockIdx.x, stride = gridDim.x;
  const int rows = r0 < n ? (int)((n - r0 + stride - 1) / stride) : 0;  // rows of this workgroup

  // MR activation rows (x is [MR][k], contiguous): row i of x starts at
  // element i k, i.e. chunk i k / (4 or 8) of the whole block.
  chunk16 xc[MR][F::RUNS][4];
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < F::RUNS; ++r) load_run_raw(x, xtype, MR * (int)k, i * (int)k + (int)F::run_off(pl, r), xc[i][r]);
  __builtin_amdgcn_sched_barrier(0);
  typename F::Piece sl[D];
  const int64_t first = r0 < n ? r0 : n - 1;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int64_t r = r0 + j * stride;
    sl[j] = F::template load<true>(w, aux, r < n ? r : first, k, pl);
  }
  __builtin_amdgcn_sched_barrier(0);
  float xv[MR][F::RUNS][16];
  float sx[MR][F::RUNS];
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < F::RUNS; ++r) {
      convert_run(xtype, xc[i][r], xv[i][r]);
      sx[i][r] = 0.0f;
#pragma unroll
      for (int t = 0; t < 16; ++t) sx[i][r] += xv[i][r][t];
    }

  auto emit = [&](int j, int ir) {  // slot j holds row r0 + ir * stride
    float dr[MR];
    if constexpr (MR > 1 && has_dot_rows<F>::value) {
      F::template dot_rows<MR>(sl[j], xv, sx, dr);
    } else {
#pragma unroll
      for (int i = 0; i < MR; ++i) dr[i] = F::dot(sl[j], xv[i], sx[i]);
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      float acc = (live && ir < rows) ? dr[i] : 0.0f;
      acc = seg_sum(acc, 64);
      if (lane == 63 && ir < rows) red[i][ir][tm] = acc;
    }
  };
  const int groups = (rows + D - 1) / D;
  int base = 0;
  for (int g = 1; g < groups; ++g, base += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int ir = base + j;
      emit(j, ir);
      const int64_t r = r0 + (int64_t)ir * stride, rn = r + D * stride;
      sl[j] = F::template load<true>(w, aux, rn < n ? rn : r, k, pl);
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) emit(j, base + j);
  __syncthreads();
  for (int t = (int)threadIdx.x; t < MR * rows; t += (int)blockDim.x) {
    const int i = t / rows, ir = t - i * rows;
    float tot = red[i][ir][0];
    for (int q = 1; q < team; ++q) tot += red[i][ir][q];
    store_linear(o, i, n, r0 + (int64_t)ir * stride, tot);
  }
}

// M = 1, long rows, two rows a workgroup on two teams: team j (waves
// j T .. j T + T - 1) takes row blockIdx.x + j gridDim.x, one piece a lane.
// x is staged once in LDS for both teams (its loads issued before the weight
// loads), so each wave decodes and dots one row: with one team walking both
// rows a SIMD held about one wave, which issues its VALU work at half the
// SIMD's rate.  The teams' wave sums meet in LDS; one thread a row adds them
// in wave order.
template <class F, int XR, bool PLAIN = false>
__global__ __launch_bounds__(1024) void k_gemv_team2(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                    const void *__restrict__ x, int xtype_arg, const Out o_arg,
                                                    int64_t n, int64_t k) {
  const int xtype = PLAIN ? RQ_F32 : xtype_arg;
  const Out o = PLAIN ? Out{o_arg.y, nullptr, RQ_F32, 0} : o_arg;
  __shared__ float red[2][kTeamMax];
  extern __shared__ __attribute__((aligned(16))) float xs_dyn[];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int team = (int)(blockDim.x >> 7);  // waves a team
  const int j = wv >= team ? 1 : 0, tm = wv - j * team;
  const int P = (int)(k / F::PE);
  const int p = 64 * tm + lane;
  const bool live = p < P;
  const int pl = live ? p : P - 1;
  const int64_t row = (int64_t)blockIdx.x + j * (int64_t)gridDim.x;

  chunk16 xc[XR];
  load_x_chunks<XR>(x, xtype, (int)k, xc);
  __builtin_amdgcn_sched_barrier(0);
  const typename F::Piece pc = F::template load<true>(w, aux, row < n ? row : n - 1, k, pl);
  __builtin_amdgcn_sched_barrier(0);
  store_x_chunks<XR>(xtype, (int)k, xc, xs_dyn);  // ends with a barrier
  float xv[F::RUNS][16], sx[F::RUNS];
#pragma unroll
  for (int r = 0; r < F::RUNS; ++r) {
    load_run_lds<16>(xs_dyn, (int)F::run_off(pl, r), xv[r]);
    sx[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < 16; ++t) sx[r] += xv[r][t];
  }
  float acc = live ? F::dot(pc, xv, sx) : 0.0f;
  acc = seg_sum(acc, 64);
  if (lane == 63) red[j][tm] = acc;
  __syncthreads();
  if (threadIdx.x < 2) {
    const int jj = (int)threadIdx.x;
    const int64_t r = (int64_t)blockIdx.x + jj * (int64_t)gridDim.x;
    if (r < n) {
      float tot = red[jj][0];
      for (int q = 1; q < team; ++q) tot += red[jj][q];
      store_linear(o, 0, n, r, tot);
    }
  }
}

// M > 1 (interim path): each piece is decoded once to exact f32 weights and
// then dotted with every activation row, read from memory.
template <class F, int PPL>
__global__ __launch_bounds__(kThreads) void k_gemv_multi(const uint8_t *__restrict__ w,
                                                        const uint8_t *__restrict__ aux,
                                                        const void *__restrict__ x, int xtype,
                                                        int64_t m, const Out o, int64_t n, int64_t k,
                                                        int seg_log2) {
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
        F::decode(F::template load<true>(w, aux, row, k, p), wv[i]);
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
      if (sl == 0 && row < n) store_linear(o, mi, n, row, acc);
    }
  }
}

int ceil_log2(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

template <class F, int PPL>
int run_multi(const rq_weight *wt, const void *x, int xtype, int64_t m, const Out &o, int seg_log2, hipStream_t s) {
  const int rg = 64 >> seg_log2;
  const int64_t groups = (wt->n + rg - 1) / rg;
  const int64_t waves_per_block = kThreads / 64;
  int64_t blocks = (groups + waves_per_block - 1) / waves_per_block;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL((k_gemv_multi<F, PPL>), dim3((unsigned)blocks), dim3(kThreads), 0, s, wt->data,
                     wt->data + wt->aux_off, x, xtype, m, o, wt->n, wt->k, seg_log2);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
}

template <class F, int PPL>
int run_long(const rq_weight *wt, const void *x, int xtype, const Out &o, hipStream_t s) {
  // 16 waves per CU walking rows, each with two rows of weight loads in
  // flight (measured best of 8 / 16 / 24 / 32 waves per CU).
  const int64_t waves = wt->n < 256 * 16 ? wt->n : 256 * 16;
  const size_t xb = xlds_bytes(wt->k);
  // Eight waves per workgroup (measured best of 4 / 8 / 16 on 14336 x 4096)
  // for PPL <= 2; longer rows keep four (the Q6_K decode at PPL = 3 would
  // not fit eight waves' registers).
  if constexpr (PPL <= 2) {
    const unsigned blocks = (unsigned)((waves + 7) / 8);
    if (long_xr<F, PPL, 8>() > 0 && !xb) return RQ_E_UNSUPPORTED;  // k <= 64 PPL PE always fits the LDS copy
    // Two rows in flight per wave: on Q4_K 14336 x 4096, 10.5 us against
    // 11.9 (three rows) and 13.4 (four), whose registers leave room for one
    // eight-wave workgroup per CU instead of two.
    hipLaunchKernelGGL((k_gemv_long<F, PPL, 8, 2>), dim3(blocks), dim3(512), xb, s, wt->data, wt->data + wt->aux_off,
                       x, xtype, o, wt->n, wt->k, xb != 0);
  } else {
    const unsigned blocks = (unsigned)((waves + 3) / 4);
    if (long_xr<F, PPL, 4>() > 0 && !xb) return RQ_E_UNSUPPORTED;
    hipLaunchKernelGGL((k_gemv_long<F, PPL, 4, 2>), dim3(blocks), dim3(256), xb, s, wt->data, wt->data + wt->aux_off,
                       x, xtype, o, wt->n, wt->k, xb != 0);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
}

// Rows of more than 64 pieces, MR activation rows: a team of waves per row,
// each workgroup walking up to kTeamRows rows; about 512 workgroups
// (measured best of 128-2048 on 896 x 4864, 2048 x 8192 and 4096 x 14336).
// Workgroups of four or more rows keep four rows' loads in flight at M = 1
// for two-run pieces (Q4_K 2048 x 8192: 6.8 -> 5.9 us, 4096 x 14336 13.5 ->
// 12.8 against two; Q6_K's four-run pieces lose, 2048 x 8192 7.1 -> 11.7;
// on 896 x 4864, two rows a workgroup, four rows a workgroup were slower,
// 4.09 -> 4.17 us).
template <class F, int MR>
int run_team(const rq_weight *wt, const void *x, int xtype, const Out &o, hipStream_t s) {
  const int P = (int)(wt->k / F::PE);
  const int team = (P + 63) / 64;
  if (team > kTeamMax) return RQ_E_UNSUPPORTED;
  int64_t per = (wt->n + 511) / 512;
  if (per > kTeamRows) per = kTeamRows;
  const int64_t grid = (wt->n + per - 1) / per;
  if (grid > 0x7FFFFFFF) return RQ_E_UNSUPPORTED;
  const bool plain = xtype == RQ_F32 && o.ytype == RQ_F32 && !o.bias;
  if constexpr (MR == 1) {
    const size_t xb = xlds_bytes(wt->k);
    const int xr = (x_chunks(wt->k, xtype) + 128 * team - 1) / (128 * team);
    if (per == 2 && team <= 8 && xb && xr <= 4 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && wt->k % 8 == 0) {
      const unsigned g2 = (unsigned)((wt->n + 1) / 2);
#define RQ_TEAM2(XRV, PL)                                                                                     \
  hipLaunchKernelGGL((k_gemv_team2<F, XRV, PL>), dim3(g2), dim3(128 * team), xb, s, wt->data,               \
                     wt->data + wt->aux_off, x, xtype, o, wt->n, wt->k)
      if (plain) {
        if (xr <= 1) RQ_TEAM2(1, true); else if (xr <= 2) RQ_TEAM2(2, true); else RQ_TEAM2(4, true);
      } else {
        if (xr <= 1) RQ_TEAM2(1, false); else if (xr <= 2) RQ_TEAM2(2, false); else RQ_TEAM2(4, false);
      }
#undef RQ_TEAM2
      return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
    }
  }
  auto go = [&](auto Dc) {
    constexpr int D = decltype(Dc)::value;
    if constexpr (MR == 1) {
      if (plain) {
        hipLaunchKernelGGL((k_gemv_team<F, D, MR, true>), dim3((unsigned)grid), dim3(64 * team), 0, s, wt->data,
                           wt->data + wt->aux_off, x, xtype, o, wt->n, wt->k);
        return;
      }
    }
    hipLaunchKernelGGL((k_gemv_team<F, D, MR>), dim3((unsigned)grid), dim3(64 * team), 0, s, wt->data,
                       wt->data + wt->aux_off, x, xtype, o, wt->n, wt->k);
  };
  if (MR == 1 && F::RUNS == 2 && per >= 4) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, 2>{});
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
}

// Segment layout of a row of P <= 64 pieces: seg = max(16, next_pow2(P))
// lanes a row, four waves a workgroup.
struct SegGeo {
  int seg_log2, rows_per_wg;
};
SegGeo seg_geo(int P) {
  const int l = ceil_log2(P < 16 ? 16 : P);
  return {l, 4 * (64 >> l)};
}

// The segment kernel (x 16-byte aligned; k <= 64 pieces always fits the LDS
// copy of x).  Chunks of x per thread: at most MR 64 PE / 4 / 256 = 4 MR.
template <class F, int MR>
int xr_for(int64_t k, int xtype, int mrows) {
  const int per = (x_chunks(mrows * k, xtype) + 255) / 256;
  if (per <= 1) return 1;
  if (per <= 2) return 2;
  if (MR == 1 || per <= 4) return 4;
  return 8;  // two rows, or four slots of two-run formats: k <= 2048, at most 8 chunks a thread
}

#define RQ_SEG_DISPATCH_PL(KERN, PL, XRV, ...)                              \
  switch (XRV) {                                                            \
    case 1: hipLaunchKernelGGL((KERN<F, 1, MR, PL>), __VA_ARGS__); break;     \
    case 2: hipLaunchKernelGGL((KERN<F, 2, MR, PL>), __VA_ARGS__); break;     \
    case 4: hipLaunchKernelGGL((KERN<F, 4, MR, PL>), __VA_ARGS__); break;     \
    default:                                                                \
      if constexpr (MR > 1) hipLaunchKernelGGL((KERN<F, 8, MR, PL>), __VA_ARGS__); \
      break;                                                                \
  }
// The plain form (f32 activations and outputs, no bias) for one activation
// row, the general one otherwise.
#define RQ_SEG_DISPATCH(KERN, PLAIN, XRV, ...)                                     \
  if constexpr (MR == 1) {                                                         \
    if (PLAIN) {                                                                   \
      RQ_SEG_DISPATCH_PL(KERN, true, XRV, __VA_ARGS__)                             \
    } else {                                                                       \
      RQ_SEG_DISPATCH_PL(KERN, false, XRV, __VA_ARGS__)                            \
    }                                                                              \
  } else {                                                                         \
    RQ_SEG_DISPATCH_PL(KERN, false, XRV, __VA_ARGS__)                              \
  }

// Rows of at most 64 pieces, MR activation rows: the segment kernel.
template <class F, int MR>
int run_seg(const rq_weight *wt, const void *x, int xtype, const Out &o, hipStream_t s, int mrows = MR) {
  const SegGeo geo = seg_geo((int)(wt->k / F::PE));
  const int64_t groups = (wt->n + geo.rows_per_wg - 1) / geo.rows_per_wg;
  const unsigned blocks = (unsigned)(groups < 16384 ? groups : 16384);
  const size_t xb = MR * xlds_bytes(wt->k);
  const bool plain = xtype == RQ_F32 && o.ytype == RQ_F32 && !o.bias;
  RQ_SEG_DISPATCH(k_gemv_m1, plain, (xr_for<F, MR>(wt->k, xtype, mrows)), dim3(blocks), dim3(256), xb, s, wt->data,
                  wt->data + wt->aux_off, x, xtype, o, wt->n, wt->k, geo.seg_log2, geo.rows_per_wg, groups, mrows)
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
}

template <class F>
int run_m1(const rq_weight *wt, const void *x, int xtype, const Out &o, hipStream_t s) {
  const int P = (int)(wt->k / F::PE);
  // Q4_K long rows on many rows: the matrix-core GEMV where it applies; rows
  // of 32 and 64 pieces too where n k >= 2^24 (against the segment kernel:
  // 262144 x 2048 98.8 -> 58.2 us, 151936 x 1024 33.9 -> 20.9, 16384 x 2048
  // 9.46 -> 7.21, 8192 x 2048 5.87 -> 5.22; smaller grids lose: 4096 x 2048
  // 3.71 -> 4.86, 4096 x 1024 2.97 -> 3.81).
  if constexpr (std::is_same_v<F, FmtQ4K>) {
    if ((P > 64 || (P >= 32 && wt->n * wt->k >= (int64_t)1 << 24)) && wt->n >= 4096) {
      const int rc = launch_gemv_mx(wt, x, xtype, o, s);
      if (rc != RQ_E_UNSUPPORTED) return rc;
    }
  }
  // Q6_K the same way (rows of 1024 or more elements, 64-element pieces)
  // where n k >= 2^26: against the segment / long-row kernels 262144 x 2048
  // 98.8 -> 82.3 us, 151936 x 1024 29.9 -> 28.3, 32768 x 2048 17.1 -> 16.0;
  // smaller grids lose or tie (16384 x 2048 9.6 -> 10.3 us, 32768 x 1024 8.6
  // -> 10.5, 8192 x 2048 5.4 -> 7.5, 14336 x 4096 16.2 -> 16.0).
  if constexpr (std::is_same_v<F, FmtQ6K>) {
    if (P >= 16 && wt->n >= 4096 && wt->n * wt->k >= (int64_t)1 << 26) {
      const int rc = launch_gemv_mx6(wt, x, xtype, o, s);
      if (rc != RQ_E_UNSUPPORTED) return rc;
    }
  }
  // Long rows on many rows: one wave per row walking the rows.
  if (P > 64 && wt->n >= 4096) {
    switch ((P + 63) / 64) {
      case 2: return run_long<F, 2>(wt, x, xtype, o, s);
      case 3: return run_long<F, 3>(wt, x, xtype, o, s);
      case 4: return run_long<F, 4>(wt, x, xtype, o, s);
      default: break;
    }
  }
  // Other long rows: a team of waves per row.
  if (P > 64) return run_team<F, 1>(wt, x, xtype, o, s);
  return run_seg<F, 1>(wt, x, xtype, o, s);
}

template <class F, int MAXPPL>
int dispatch_fmt(const rq_weight *wt, const void *x, int xtype, int64_t m, const Out &o, hipStream_t s) {
  if (wt->k % F::PE != 0) return RQ_E_UNSUPPORTED;
  if (m == 1) return run_m1<F>(wt, x, xtype, o, s);
  const int P = (int)(wt->k / F::PE);
  // Two activation rows on the segment kernel: each weight decoded once,
  // one FMA per weight and row.
  if (m == 2 && P <= 64 && wt->k % 8 == 0) return run_seg<F, 2>(wt, x, xtype, o, s);
  // Three f32 / f16 rows: four row slots (two-run formats; Q6_K's four runs
  // a piece would not fit four rows of activations in registers).
  if constexpr (F::RUNS == 2) {
    if ((m == 3 || m == 4) && P <= 64 && wt->k % 8 == 0) return run_seg<F, 4>(wt, x, xtype, o, s, (int)m);
  }
  // (Q6_K's four runs a piece leave no registers for a second row in a
  // sixteen-wave team.)
  if constexpr (F::RUNS == 2) {
    if (m == 2 && P > 64 && wt->n < 4096 && (P + 63) / 64 <= kTeamMax && wt->k % 8 == 0)
      return run_team<F, 2>(wt, x, xtype, o, s);
  }
  if (P <= 32) return run_multi<F, 1>(wt, x, xtype, m, o, ceil_log2(P), s);
  const int ppl = (P + 63) / 64;
  if (ppl > MAXPPL) return RQ_E_UNSUPPORTED;
  switch (ppl) {
    case 1: return run_multi<F, 1>(wt, x, xtype, m, o, 6, s);
    case 2: return run_multi<F, (MAXPPL >= 2 ? 2 : 1)>(wt, x, xtype, m, o, 6, s);
    case 3: return run_multi<F, (MAXPPL >= 3 ? 3 : 1)>(wt, x, xtype, m, o, 6, s);
    case 4: return run_multi<F, (MAXPPL >= 4 ? 4 : 1)>(wt, x, xtype, m, o, 6, s);
    default: return RQ_E_UNSUPPORTED;
  }
}

// Several weights of format F sharing x (equal k, rows of at most 64
// pieces, M = 1 or 2, one output and bias type): the row groups of all of
// them in one grid.
template <class F>
int run_seg_set(const rq_weight *const *w, int count, const void *x, int xtype, int64_t m, const Out *o,
                hipStream_t s) {
  const int64_t k = w[0]->k;
  if (k % F::PE != 0) return RQ_E_UNSUPPORTED;
  const int P = (int)(k / F::PE);
  if (P > 64 || (m == 2 && k % 8 != 0)) return RQ_E_UNSUPPORTED;
  const SegGeo geo = seg_geo(P);
  WeightSet set;
  int64_t total = 0;
  const int rc = fill_set(set, w, count, o, [&](const rq_weight *wj) {
    return (wj->n + geo.rows_per_wg - 1) / geo.rows_per_wg;
  }, &total);
  if (rc) return rc;
  const size_t xb = (m == 1 ? 1 : 2) * xlds_bytes(k);
  bool plain = xtype == RQ_F32 && o[0].ytype == RQ_F32;
  for (int j = 0; j < count; ++j) plain = plain && !o[j].bias;
  if (m == 1) {
    constexpr int MR = 1;
    RQ_SEG_DISPATCH(k_gemv_set, plain, (xr_for<F, 1>(k, xtype, 1)), dim3((unsigned)total), dim3(256), xb, s, set, x,
                    xtype, k, geo.seg_log2, geo.rows_per_wg, 1)
  } else {
    constexpr int MR = 2;
    RQ_SEG_DISPATCH(k_gemv_set, plain, (xr_for<F, 2>(k, xtype, 2)), dim3((unsigned)total), dim3(256), xb, s, set, x,
                    xtype, k, geo.seg_log2, geo.rows_per_wg, 2)
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
}

}  // namespace

int launch_linear_fused(const rq_weight *wt, const void *x, int xtype, int64_t m, const Out &o, hipStream_t s,
                        WsLease &ws) {
  // The fused kernels read activations with 8- or 16-byte vector loads.
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  // bf16 activations with m > 1 run on the matrix cores: up to 64 rows with
  // the weights as the A operand decoded straight into registers, beyond
  // that the LDS-tiled GEMM -- except two rows (segment and team layouts;
  // n < 4096 for long rows), which stay on the VALU GEMVs: a weight decoded
  // once, one FMA per weight and row, exact f32 weights.  (Three and four
  // bf16 rows on the VALU were slower than the matrix cores: 259 -> 201 GB/s
  // on the 0.5B verify layer at m = 3.)
  const int seg_pe = wt->qtype == RQ_Q6_K ? 64 : 32;
  const int64_t seg_p = wt->k / seg_pe;
  const bool two_rows_seg = m == 2 && wt->k % (2 * seg_pe) == 0 &&
                            (seg_p <= 64 ||
                             (wt->n < 4096 && (seg_p + 63) / 64 <= kTeamMax && wt->qtype != RQ_Q6_K)) &&
                            (wt->qtype == RQ_Q4_K || wt->qtype == RQ_Q6_K || wt->qtype == RQ_Q8_0 ||
                             wt->qtype == RQ_Q5_K || wt->qtype == RQ_Q4_0 || wt->qtype == RQ_Q5_0);
  if (m > 1 && xtype == RQ_BF16 && !two_rows_seg) {
    int rc = m <= 64 ? launch_linear_smallm(wt, x, m, o, s, &ws) : RQ_E_UNSUPPORTED;
    if (rc == RQ_E_UNSUPPORTED) rc = launch_linear_mfma(wt, x, m, o, s, ws);
    if (rc != RQ_E_UNSUPPORTED) return rc;
  }
  // f32 / f16 activations with 4 <= m <= 64: exact-f32 weights on the f32
  // matrix cores (16 MFMAs of K = 4 per 64-element chunk; at m = 2..3 the
  // VALU kernels' few FMAs per weight are cheaper: 37 vs 47 us per 0.5B
  // layer at m = 2, 150 vs 54 us at m = 16).
  const bool f32x = xtype == RQ_F32 || xtype == RQ_F16;
  // f32 rows of Q4_K / Q6_K / Q8_0: the integer codes on the bf16 matrix
  // cores against two bf16 limbs of x, scales applied per run of 16 or 32.
  if (m >= 4 && m <= 64 && xtype == RQ_F32) {
    const int rc = launch_linear_smallm_codes(&wt, 1, false, x, m, &o, s, &ws);
    if (rc != RQ_E_UNSUPPORTED) return rc;
  }
  if (m >= 4 && m <= 64 && f32x) {
    const int rc = launch_linear_smallm_f32(wt, x, xtype, m, o, s, &ws);
    if (rc != RQ_E_UNSUPPORTED) return rc;
  }
  // More rows (prefill with f32 activations, the reference's compute type):
  // the tiled GEMM on two bf16 limbs per operand.
  if (m > 64 && f32x) {
    const int rc = launch_linear_mfma_limbs(wt, x, xtype, m, o, s, ws);
    if (rc != RQ_E_UNSUPPORTED) return rc;
  }
  // Otherwise the small-M f32 kernel on slices of 64 activation rows (the
  // weights are read once per slice, mostly from cache), a last slice of 2
  // or 3 rows on the VALU kernel and a single row on the GEMV.
  if (m > 64 && f32x && wt->k % 64 == 0) {
    const size_t xb = xtype == RQ_F32 ? 4 : 2, yb = o.ytype == RQ_F32 ? 4 : 2;
    // The whole slices in one launch (side by side, the weight tiles shared
    // through the cache while they run), then the rest.  Against one launch
    // a slice, M = 512 with f32 activations: q/k/o 2048 x 2048 39 -> 59, v
    // 37 -> 53, gate/up 8192 x 2048 58 -> 67, down 51 -> 57 TFLOP/s.
    int64_t r0 = 0;
    if (m / 64 <= 65535) {
      const int rc = launch_linear_smallm_f32_slices(wt, x, xtype, m / 64, o, s, &ws);
      if (rc != RQ_E_UNSUPPORTED && rc != RQ_OK) return rc;
      if (rc == RQ_OK) r0 = m / 64 * 64;
    }
    for (; r0 < m; r0 += 64) {
      const int64_t mm = m - r0 < 64 ? m - r0 : 64;
      const void *xs = static_cast<const uint8_t *>(x) + (size_t)r0 * (size_t)wt->k * xb;
      Out os = o;
      os.y = static_cast<uint8_t *>(o.y) + (size_t)r0 * (size_t)wt->n * yb;
      const int rc = mm >= 4 ? launch_linear_smallm_f32(wt, xs, xtype, mm, os, s, &ws)
                             : launch_linear_fused(wt, xs, xtype, mm, os, s, ws);
      if (rc) return rc;
    }
    return RQ_OK;
  }
  int rc;
  switch (wt->qtype) {
    case RQ_Q4_K:
      // Pieces must not straddle rows: rows start on 64-element chunk bounds.
      rc = wt->k % 64 ? RQ_E_UNSUPPORTED : dispatch_fmt<FmtQ4K, 4>(wt, x, xtype, m, o, s);
      break;
    case RQ_Q6_K:
      rc = wt->k % 128 ? RQ_E_UNSUPPORTED : dispatch_fmt<FmtQ6K, 2>(wt, x, xtype, m, o, s);
      break;
    case RQ_Q8_0:
      rc = wt->k % 64 ? RQ_E_UNSUPPORTED : dispatch_fmt<FmtQ8, 4>(wt, x, xtype, m, o, s);
      break;
    case RQ_Q5_K:
      rc = wt->k % 64 ? RQ_E_UNSUPPORTED : dispatch_fmt<FmtQ5K, 4>(wt, x, xtype, m, o, s);
      break;
    case RQ_Q4_0:
      rc = wt->k % 64 ? RQ_E_UNSUPPORTED : dispatch_fmt<FmtQx0<false>, 4>(wt, x, xtype, m, o, s);
      break;
    case RQ_Q5_0:
      rc = wt->k % 64 ? RQ_E_UNSUPPORTED : dispatch_fmt<FmtQx0<true>, 4>(wt, x, xtype, m, o, s);
      break;
    default:
      return RQ_E_UNSUPPORTED;
  }
  // Two or three f32 / f16 rows on rows too long for the VALU layouts: the
  // f32 matrix-core kernel takes every format and length (k % 64 == 0).
  if (rc == RQ_E_UNSUPPORTED && f32x && m >= 2 && m <= 3) rc = launch_linear_smallm_f32(wt, x, xtype, m, o, s, &ws);
  return rc;
}

int launch_linear_multi(const rq_weight *const *w, int count, const void *x, int xtype, int64_t m, const Out *o,
                        hipStream_t s, WsLease &ws) {
  if (count < 1 || count > kMultiMax || m < 1) return RQ_E_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  const int qt = w[0]->qtype;
  const int64_t k = w[0]->k;
  for (int j = 1; j < count; ++j)
    if (w[j]->qtype != qt || w[j]->k != k) return RQ_E_UNSUPPORTED;
  // bf16 activations beyond two rows, f32 ones from four: the small-M
  // matrix-core kernel (bf16, or two bf16 limbs for f32), as rq_linear takes
  // them (two rows stay on the segment kernel below, f32 three rows one by
  // one where rq_linear gives them other layouts).
  if (xtype == RQ_BF16 && m >= 3 && m <= 64) return launch_linear_smallm_set(w, count, x, xtype, m, o, s, &ws);
  if (xtype == RQ_F32 && m >= 4 && m <= 64) {
    const int rc = launch_linear_smallm_codes(w, count, true, x, m, o, s, &ws);
    return rc != RQ_E_UNSUPPORTED ? rc : launch_linear_smallm_set(w, count, x, xtype, m, o, s, &ws);
  }
  if (m != 1 && m != 2) return RQ_E_UNSUPPORTED;
  switch (qt) {
    case RQ_Q4_K: return k % 64 ? RQ_E_UNSUPPORTED : run_seg_set<FmtQ4K>(w, count, x, xtype, m, o, s);
    case RQ_Q6_K: return k % 128 ? RQ_E_UNSUPPORTED : run_seg_set<FmtQ6K>(w, count, x, xtype, m, o, s);
    case RQ_Q8_0: return k % 64 ? RQ_E_UNSUPPORTED : run_seg_set<FmtQ8>(w, count, x, xtype, m, o, s);
    case RQ_Q5_K: return k % 64 ? RQ_E_UNSUPPORTED : run_seg_set<FmtQ5K>(w, count, x, xtype, m, o, s);
    case RQ_Q4_0: return k % 64 ? RQ_E_UNSUPPORTED : run_seg_set<FmtQx0<false>>(w, count, x, xtype, m, o, s);
    case RQ_Q5_0: return k % 64 ? RQ_E_UNSUPPORTED : run_seg_set<FmtQx0<true>>(w, count, x, xtype, m, o, s);
    default: return RQ_E_UNSUPPORTED;
  }
}

}  // namespace rq
