// rq_marlin.hip -- Marlin INT4 weights on gfx950: repack, dequant and the
// fused GEMV (crates/runtimed-model/src/ops/marlin_gemv.rs).
//
// Layout (the reference's, marlin_gemv.rs:66-97): u32 packed[ceil(k/32)][n][4];
// record [c][r] holds row r, inputs 32c .. 32c+31, input 32c + 8j + i in bits
// 4i .. 4i+3 of word j; value (nibble - 8) * scale[r].  Records of one chunk
// are contiguous over rows, so lanes on consecutive rows read one contiguous
// run with 128-bit loads.
//
// GEMV (marlin_gemv.rs:119-202 launches one thread per output over all of
// k): here a 512-thread workgroup owns R rows and splits the k chunks over
// 8 waves x (64 / R) lane groups, so a decode-sized matrix still spreads
// over the whole chip; partial sums meet through lane exchanges and LDS,
// scale[r] is applied once at the end as in the reference (acc * scale).
// Bound: HBM, 0.5 byte per weight + 4 bytes of scale per row.
#include "rq_e4m3.h"
#include "rq_formats.h"
#include "rq_internal.h"

namespace rq {
namespace {

// repack_marlin_tiles (marlin_gemv.rs:66-97): one thread per (row, chunk),
// chunk fastest so that a wave reads one row's inputs contiguously.
__global__ __launch_bounds__(256) void k_marlin_repack(const void *__restrict__ w, int wtype,
                                                       const float *__restrict__ s, int64_t n,
                                                       int64_t k, int64_t kc, uint4 *__restrict__ packed) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= n * kc) return;
  const int64_t r = idx / kc, c = idx - r * kc;
  const float sr = s[r];
  const float inv_s = fabsf(sr) > 1e-12f ? 1.0f / sr : 1.0f;
  uint32_t words[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t kk = c * 32 + 8 * j + i;
      uint32_t q = 8;
      if (kk < k) {
        const float t = roundf(load_x1(w, wtype, r * k + kk) * inv_s) + 8.0f;
        q = (t != t) ? 0u : (uint32_t)fminf(fmaxf(t, 0.0f), 15.0f);
      }
      word |= q << (4 * i);
    }
    words[j] = word;
  }
  packed[c * n + r] = make_uint4(words[0], words[1], words[2], words[3]);
}

// MarlinWeight::dequantize (marlin_gemv.rs:42-61): one thread per (row, chunk).
__global__ __launch_bounds__(256) void k_marlin_dequant(const uint4 *__restrict__ packed,
                                                        const float *__restrict__ s, int64_t n, int64_t k,
                                                        int64_t kc, float *__restrict__ out, bool vec) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= n * kc) return;
  const int64_t r = idx / kc, c = idx - r * kc;
  const uint4 q = packed[c * n + r];
  const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
  const float sr = s[r];
  float *o = out + r * k + c * 32;
  if (vec && c * 32 + 32 <= k) {
#pragma unroll
    for (int j4 = 0; j4 < 8; ++j4) {
      const uint32_t v = wd[j4 >> 1] >> (16 * (j4 & 1));
      reinterpret_cast<float4 *>(o)[j4] =
          make_float4((float)((int)(v & 15u) - 8) * sr, (float)((int)((v >> 4) & 15u) - 8) * sr,
                      (float)((int)((v >> 8) & 15u) - 8) * sr, (float)((int)((v >> 12) & 15u) - 8) * sr);
    }
  } else {
    for (int e = 0; e < 32 && c * 32 + e < k; ++e)
      o[e] = (float)((int)((wd[e >> 3] >> (4 * (e & 7))) & 15u) - 8) * sr;
  }
}

// Sum over the 32 inputs of one record of x[base .. base+32) * (q - 8).
// xs: the activation rows of this workgroup staged in LDS as f32 (base is
// then an offset into xs), or null to read x from global memory.
__device__ __forceinline__ float record_dot(const uint32_t (&wd)[4], const void *x, int xtype, const float *xs,
                                            int64_t base, int valid, bool vec) {
  float a = 0.0f;
  if (vec && valid == 32) {
#pragma unroll
    for (int j4 = 0; j4 < 8; ++j4) {
      const float4 xv = xs ? *reinterpret_cast<const float4 *>(xs + base + 4 * j4) : load_x4(x, xtype, base + 4 * j4);
      const uint32_t v = wd[j4 >> 1] >> (16 * (j4 & 1));
      a = fmaf(xv.x, (float)(v & 15u) - 8.0f, a);
      a = fmaf(xv.y, (float)((v >> 4) & 15u) - 8.0f, a);
      a = fmaf(xv.z, (float)((v >> 8) & 15u) - 8.0f, a);
      a = fmaf(xv.w, (float)((v >> 12) & 15u) - 8.0f, a);
    }
  } else {
    for (int e = 0; e < valid; ++e)
      a = fmaf(xs ? xs[base + e] : load_x1(x, xtype, base + e), (float)((wd[e >> 3] >> (4 * (e & 7))) & 15u) - 8.0f,
               a);
  }
  return a;
}

// y[m0 .. m0+MT) x [R rows of this workgroup].
template <int R, int MT>
__global__ __launch_bounds__(512) void k_marlin_gemv(const uint4 *__restrict__ packed, const float *__restrict__ s,
                                                     const void *__restrict__ x, int xtype, int64_t m, int64_t n,
                                                     int64_t k, int64_t kc, void *__restrict__ y, int ytype,
                                                     bool vec, bool xlds) {
  constexpr int GROUPS = 64 / R;      // lane groups per wave
  constexpr int SLOTS = 8 * GROUPS;   // chunk slots per workgroup
  __shared__ float red[8][MT][R];
  extern __shared__ __attribute__((aligned(16))) float xs_dyn[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rl = lane % R;
  const int64_t row = (int64_t)blockIdx.x * R + rl;
  const int slot = wave * GROUPS + lane / R;
  const int64_t m0 = (int64_t)blockIdx.y * MT;
  // The MT activation rows are read by every lane group of the workgroup:
  // staged once in LDS (lane groups on one chunk then read the same address,
  // an LDS broadcast) instead of once per lane from global memory.
  const float *xs = nullptr;
  if (xlds) {
    const int64_t rows = m - m0 < MT ? m - m0 : MT;
    for (int64_t e = threadIdx.x; e < rows * k; e += 512) xs_dyn[e] = load_x1(x, xtype, m0 * k + e);
    __syncthreads();
    xs = xs_dyn;
  }
  float acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
  if (row < n) {
    // Batches of 4 records per lane, all loads issued before the first use.
    for (int64_t c0 = slot; c0 < kc; c0 += 4 * SLOTS) {
      uint4 q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t c = c0 + j * SLOTS;
        q[j] = c < kc ? packed[c * n + row] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t c = c0 + j * SLOTS;
        if (c < kc) {
          const uint32_t wd[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
          const int64_t kb = c * 32;
          const int valid = (int)(k - kb < 32 ? k - kb : 32);
#pragma unroll
          for (int t = 0; t < MT; ++t)
            if (m0 + t < m)
          acc[t] += record_dot(wd, x, xtype, xs, (xs ? t * k : (m0 + t) * k) + kb, valid, vec);
        }
      }
    }
  }
#pragma unroll
  for (int off = R; off < 64; off <<= 1)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] += __shfl_xor(acc[t], off);
  if (lane < R) {
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave][t][rl] = acc[t];
  }
  __syncthreads();
  if (threadIdx.x < R * MT) {
    const int t = threadIdx.x / R, l = threadIdx.x % R;
    const int64_t orow = (int64_t)blockIdx.x * R + l, xr = m0 + t;
    if (orow < n && xr < m) {
      float v = 0.0f;
#pragma unroll
      for (int wv = 0; wv < 8; ++wv) v += red[wv][t][l];
      store_out(y, ytype, xr * n + orow, v * s[orow]);
    }
  }
}

// M = 1, 16-byte aligned x, k % 32 == 0, x in 64 KB of LDS: x is loaded first as
// raw 16-byte chunks (XR a thread; 4 f32 or 8 f16/bf16 values each, one
// unconditional load form), the first batch of records right behind it, and
// x is staged in LDS -- with the sum of each 32-input chunk -- while the
// records are in flight (the load counter retires in issue order: loads of
// x issued after the records would hold the staging until the records had
// landed).  Record loads (B a lane per batch) are unconditional on clamped chunks and rows;
// records past kc are selected away, not branched around (a load whose
// result is used under a branch is sunk into it).  A record's dot product is
// sum x q - 8 sum x, with q converted from masked bytes (low nibbles 0x0F0F0F0F
// of a word are inputs 0, 2, 4, 6; the high ones 1, 3, 5, 7).
typedef uint32_t mchunk __attribute__((ext_vector_type(4)));

template <int R, int XR, int B>
__global__ __launch_bounds__(512) void k_marlin_gemv_x(const mchunk *__restrict__ packed, const float *__restrict__ s,
                                                       const void *__restrict__ x, int xtype, int64_t n, int64_t k,
                                                       int64_t kc, void *__restrict__ y, int ytype) {
  constexpr int GROUPS = 64 / R;      // lane groups per wave
  constexpr int SLOTS = 8 * GROUPS;   // chunk slots per workgroup
  __shared__ float red[8][R];
  extern __shared__ __attribute__((aligned(16))) float xs[];  // k activations, then kc chunk sums
  float *const xsum = xs + k;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rl = lane % R;
  const int64_t row = (int64_t)blockIdx.x * R + rl;
  const int64_t rowc = row < n ? row : n - 1;
  const int slot = wave * GROUPS + lane / R;

  const int epc = xtype == RQ_F32 ? 4 : 8;
  const int nc = (int)(k / epc);
  const mchunk *xc0 = static_cast<const mchunk *>(x);
  mchunk xr[XR];
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const int c = (int)threadIdx.x + 512 * i;
    xr[i] = xc0[c < nc ? c : nc - 1];
  }
  __builtin_amdgcn_sched_barrier(0);
  mchunk q[B];
  auto fetch = [&](int64_t c0) {
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int64_t c = c0 + j * SLOTS;
      // non-temporal: the packed weights are streamed once (4864 x 896 3.73 -> 3.17 us)
      q[j] = __builtin_nontemporal_load(&packed[(c < kc ? c : kc - 1) * n + rowc]);
    }
  };
  fetch(slot);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const int c0 = (int)threadIdx.x + 512 * i;
    const int c = c0 < nc ? c0 : nc - 1;
    const mchunk u = xr[i];
    if (xtype == RQ_F32) {
      *reinterpret_cast<float4 *>(xs + 4 * c) =
          make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
    } else {
      float f[8];
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = wd[j] & 0xFFFFu, hi = wd[j] >> 16;
        f[2 * j] = xtype == RQ_BF16 ? __uint_as_float(lo << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)lo);
        f[2 * j + 1] =
            xtype == RQ_BF16 ? __uint_as_float(hi << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)hi);
      }
      *reinterpret_cast<float4 *>(xs + 8 * c) = make_float4(f[0], f[1], f[2], f[3]);
      *reinterpret_cast<float4 *>(xs + 8 * c + 4) = make_float4(f[4], f[5], f[6], f[7]);
    }
  }
  __syncthreads();
  for (int c = (int)threadIdx.x; c < (int)kc; c += 512) {
    float t = 0.0f;
#pragma unroll
    for (int j4 = 0; j4 < 8; ++j4) {
      const float4 v = *reinterpret_cast<const float4 *>(xs + 32 * c + 4 * j4);
      t += (v.x + v.y) + (v.z + v.w);
    }
    xsum[c] = t;
  }
  __syncthreads();

  float acc = 0.0f;
  for (int64_t c0 = slot; c0 < kc; c0 += B * SLOTS) {
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int64_t c = c0 + j * SLOTS;
      const int64_t cc = c < kc ? c : kc - 1;
      const float *xp = xs + 32 * cc;
      const uint32_t wd[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
      float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {  // word w: inputs 8w .. 8w + 7
        const float4 xa = *reinterpret_cast<const float4 *>(xp + 8 * w);
        const float4 xb = *reinterpret_cast<const float4 *>(xp + 8 * w + 4);
        const uint32_t lo = opaque(wd[w] & 0x0F0F0F0Fu), hi = opaque((wd[w] >> 4) & 0x0F0F0F0Fu);
        a0 = fmaf(xa.x, ub(lo, 0), a0);
        a1 = fmaf(xa.y, ub(hi, 0), a1);
        a0 = fmaf(xa.z, ub(lo, 1), a0);
        a1 = fmaf(xa.w, ub(hi, 1), a1);
        a0 = fmaf(xb.x, ub(lo, 2), a0);
        a1 = fmaf(xb.y, ub(hi, 2), a1);
        a0 = fmaf(xb.z, ub(lo, 3), a0);
        a1 = fmaf(xb.w, ub(hi, 3), a1);
      }
      const float d = (a0 + a1) - 8.0f * xsum[cc];
      acc += c < kc ? d : 0.0f;
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c0 + B * SLOTS < kc) fetch(c0 + B * SLOTS);
  }
#pragma unroll
  for (int off = R; off < 64; off <<= 1) acc += __shfl_xor(acc, off);
  if (lane < R) red[wave][rl] = acc;
  __syncthreads();
  if (threadIdx.x < R) {
    const int l = threadIdx.x;
    const int64_t orow = (int64_t)blockIdx.x * R + l;
    if (orow < n) {
      float v = 0.0f;
#pragma unroll
      for (int wv = 0; wv < 8; ++wv) v += red[wv][l];
      store_out(y, ytype, orow, v * s[orow]);
    }
  }
}

// M = 1 on the matrix cores (k % 32 == 0, x 16-byte aligned): a workgroup
// owns 32 rows, wave w takes chunks w, w + W, .. (CPW of them, chunks past kc
// read chunk kc - 1 against zero activations).  Lane (row r = lane % 32, half
// h = lane / 32) loads words 2h, 2h + 1 of row r's record (8 contiguous
// bytes: the wave reads 32 consecutive records, 512 bytes, per chunk).  Word
// j's codes (inputs 8j .. 8j + 7) become the bf16 patterns 0x4300 | q =
// 128 + q in the order of the masked bytes (inputs 0, 2, 4, 6, 1, 3, 5, 7),
// the B operand of one v_mfma_f32_32x32x16_bf16 (column = row, K group =
// h); x is staged in the same order as two bf16 limbs (hi = bf16(x), lo =
// bf16(x - hi)) in A rows 0 and 1 (rows 2..31 read zeros).  With one scale a
// row no per-block scaling is needed: the accumulator runs over all of the
// wave's chunks, and y = s_r (S - 136 X) with S the hi + lo sums of the
// row's waves (added in wave order) and X the sum of hi + lo over k.
template <int CPW>
__global__ __launch_bounds__(1024) void k_marlin_mx(const mchunk *__restrict__ packed, const float *__restrict__ s,
                                                    const void *__restrict__ x, int xtype, int64_t n, int64_t k,
                                                    int64_t kc, void *__restrict__ y, int ytype) {
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // records, zero block, sums
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int W = (int)(blockDim.x >> 6);
  const int wr = lane & 31, h = lane >> 5;
  const int64_t row0 = (int64_t)blockIdx.x * 32;
  const int64_t rowc = row0 + wr < n ? row0 + wr : n - 1;
  const int nrec = W * CPW * 4;  // 8-input records of the staged x
  const int zero_off = 32 * nrec;
  float *red = reinterpret_cast<float *>(lds + zero_off + 1024);  // [W][32] row sums, then [W] x sums

  // x first (the load counter retires in issue order, so the staging below
  // then waits for x only): thread t stages record t (inputs 8t .. 8t + 7,
  // zero past k; every launch has at most one record a thread), loading a
  // valid record when it has none.
  const bool f32x = xtype == RQ_F32, bfx = xtype == RQ_BF16;
  const int e = tid < nrec ? tid : nrec - 1;
  const bool live = tid < nrec && 8 * (int64_t)e < k;
  const int64_t el = live ? e : 0;
  const uint4 *xc = static_cast<const uint4 *>(x);
  const uint4 xa = xc[f32x ? 2 * el : el];
  const uint4 xb = xc[f32x ? 2 * el + 1 : el];
  __builtin_amdgcn_sched_barrier(0);
  // Weight words of this lane.
  uint2 wq[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int64_t c = (int64_t)wave + (int64_t)W * i;
    const int64_t cc = c < kc ? c : kc - 1;
    {  // non-temporal, as in k_marlin_gemv_x (14336 x 4096 10.6 -> 9.9-10.4 us)
      typedef uint32_t mw2 __attribute__((ext_vector_type(2)));
      const mw2 v = __builtin_nontemporal_load(reinterpret_cast<const mw2 *>(reinterpret_cast<const uint8_t *>(packed + cc * n + rowc) + 8 * h));
      wq[i] = make_uint2(v.x, v.y);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // Record e as hi then lo limbs of inputs 0, 2, 4, 6, 1, 3, 5, 7; the
  // thread's sum of hi + lo.
  float sx = 0.0f;
  {
    const uint32_t va[4] = {xa.x, xa.y, xa.z, xa.w}, vb[4] = {xb.x, xb.y, xb.z, xb.w};
    float xf[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float e0 = bfx ? __uint_as_float(va[j] << 16) : h2f(va[j]);
      const float e1 = bfx ? __uint_as_float(va[j] & 0xFFFF0000u) : h2f(va[j] >> 16);
      const uint32_t f0 = j < 2 ? va[2 * j] : vb[2 * j - 4], f1 = j < 2 ? va[2 * j + 1] : vb[2 * j - 3];
      xf[2 * j] = live ? (f32x ? __uint_as_float(f0) : e0) : 0.0f;
      xf[2 * j + 1] = live ? (f32x ? __uint_as_float(f1) : e1) : 0.0f;
    }
    const float xo[8] = {xf[0], xf[2], xf[4], xf[6], xf[1], xf[3], xf[5], xf[7]};
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hi[j] = pk_bf16(xo[2 * j], xo[2 * j + 1]);
      const float h0 = __uint_as_float(hi[j] << 16), h1 = __uint_as_float(hi[j] & 0xFFFF0000u);
      lo[j] = pk_bf16(xo[2 * j] - h0, xo[2 * j + 1] - h1);
      const float l0 = __uint_as_float(lo[j] << 16), l1 = __uint_as_float(lo[j] & 0xFFFF0000u);
      sx += (h0 + l0) + (h1 + l1);
    }
    if (tid < nrec) {
      *reinterpret_cast<uint4 *>(lds + 32 * e) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
      *reinterpret_cast<uint4 *>(lds + 32 * e + 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
  }
  if (tid < 64) *reinterpret_cast<uint4 *>(lds + zero_off + 16 * tid) = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) sx += __shfl_xor(sx, o);
  if (lane == 0) red[32 * W + wave] = sx;
  __syncthreads();

  // A fragment of word j of chunk c for lane (A row a, half h): record
  // 4c + j, limb a; the MFMA pair of a chunk takes words 2h and 2h + 1.
  const int ar = lane & 31;
  const uint32_t abase = ar < 2 ? (uint32_t)(16 * ar + 64 * h) : (uint32_t)zero_off;
  const uint32_t astride = ar < 2 ? 128u * (uint32_t)W : 0u;  // bytes of records between a wave's chunks
  const uint8_t *ab = lds + abase + (ar < 2 ? 128u * (uint32_t)wave : 0u);
  f32x16 acc = {};
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const uint32_t w0 = wq[i].x, w1 = wq[i].y;
    const uint32_t sel01 = 0x04010400u, sel23 = 0x04030402u, magic = 0x43434343u;
    const uint32_t l0 = w0 & 0x0F0F0F0Fu, h0 = (w0 >> 4) & 0x0F0F0F0Fu;
    const uint32_t l1 = w1 & 0x0F0F0F0Fu, h1 = (w1 >> 4) & 0x0F0F0F0Fu;
    const mchunk b0 = {__builtin_amdgcn_perm(magic, l0, sel01), __builtin_amdgcn_perm(magic, l0, sel23),
                       __builtin_amdgcn_perm(magic, h0, sel01), __builtin_amdgcn_perm(magic, h0, sel23)};
    const mchunk b1 = {__builtin_amdgcn_perm(magic, l1, sel01), __builtin_amdgcn_perm(magic, l1, sel23),
                       __builtin_amdgcn_perm(magic, h1, sel01), __builtin_amdgcn_perm(magic, h1, sel23)};
    const uint8_t *a = ab + astride * (uint32_t)i;
    const bf16x8 a0 = *reinterpret_cast<const bf16x8 *>(a);
    const bf16x8 a1 = *reinterpret_cast<const bf16x8 *>(a + 32);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, __builtin_bit_cast(bf16x8, b0), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, __builtin_bit_cast(bf16x8, b1), acc, 0, 0, 0);
  }
  // Lanes 0..31 hold row wr's hi and lo sums (C rows 0 and 1).
  if (h == 0) red[32 * wave + wr] = acc[0] + acc[1];
  __syncthreads();
  if (tid < 32 && row0 + tid < n) {
    float v = 0.0f, xt = 0.0f;
    for (int i = 0; i < W; ++i) v += red[32 * i + tid];
    for (int i = 0; i < W; ++i) xt += red[32 * W + i];
    store_out(y, ytype, row0 + tid, fmaf(-136.0f, xt, v) * s[row0 + tid]);
  }
}

template <int R, int MT>
void launch_gemv(const uint4 *packed, const float *s, const void *x, int xtype, int64_t m, int64_t n, int64_t k,
                 int64_t kc, void *y, int ytype, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)((n + R - 1) / R), (unsigned)((m + MT - 1) / MT));
  // MT rows of f32 activations in LDS when they fit in 64 KB.
  const size_t xb = (size_t)MT * k * sizeof(float) <= 65536 ? (size_t)MT * k * sizeof(float) : 0;
  // Many weights: the matrix-core GEMV (k <= 8192: at most 16 chunks a wave
  // and 16 waves; x records 4 bytes an input, at most 33 KB of LDS).
  // (A workgroup a 32-row tile: from n >= 8192 the grid fills the chip;
  // 4096 x 8192 ran 7.2 -> 10.2 us on 128 workgroups.)
  if (MT == 1 && m == 1 && vec && k % 32 == 0 && k <= 8192 && n >= 8192 && n * k >= ((int64_t)1 << 24)) {
    const int64_t cpw = kc <= 64 ? 4 : kc <= 128 ? 8 : 16;
    const int64_t waves = (kc + cpw - 1) / cpw;
    const size_t lds = (size_t)waves * cpw * 128 + 1024 + (size_t)(32 * waves + waves) * 4;
    const mchunk *pk = reinterpret_cast<const mchunk *>(packed);
    const dim3 g((unsigned)((n + 31) / 32)), b((unsigned)(64 * waves));
    if (cpw == 4) hipLaunchKernelGGL(k_marlin_mx<4>, g, b, lds, st, pk, s, x, xtype, n, k, kc, y, ytype);
    else if (cpw == 8) hipLaunchKernelGGL(k_marlin_mx<8>, g, b, lds, st, pk, s, x, xtype, n, k, kc, y, ytype);
    else hipLaunchKernelGGL(k_marlin_mx<16>, g, b, lds, st, pk, s, x, xtype, n, k, kc, y, ytype);
    return;
  }
  // x and its chunk sums in at most 64 KB of LDS; x chunks a thread: k / (4 or 8) / 512 <= 8.
  if (MT == 1 && m == 1 && vec && k % 32 == 0 && (k + kc) * (int64_t)sizeof(float) <= 65536) {
    const int64_t per = (k / (xtype == RQ_F32 ? 4 : 8) + 511) / 512;
    const size_t xsb = (size_t)(k + kc) * sizeof(float);
    const mchunk *pk = reinterpret_cast<const mchunk *>(packed);
    // Records a lane loads per batch: one when a lane has at most one
    // (decode-sized rows; the registers of four cost the second workgroup
    // per CU), else four.
    const bool one = kc <= 8 * (64 / R);
#define RQ_MX(XR)                                                                                                    \
  if (one)                                                                                                           \
    hipLaunchKernelGGL((k_marlin_gemv_x<R, XR, 1>), grid, dim3(512), xsb, st, pk, s, x, xtype, n, k, kc, y, ytype); \
  else                                                                                                               \
    hipLaunchKernelGGL((k_marlin_gemv_x<R, XR, 4>), grid, dim3(512), xsb, st, pk, s, x, xtype, n, k, kc, y, ytype)
    if (per <= 1) { RQ_MX(1); }
    else if (per <= 2) { RQ_MX(2); }
    else if (per <= 4) { RQ_MX(4); }
    else { RQ_MX(8); }
#undef RQ_MX
    return;
  }
  hipLaunchKernelGGL((k_marlin_gemv<R, MT>), grid, dim3(512), xb, st, packed, s, x, xtype, m, n, k, kc, y, ytype,
                     vec, xb != 0);
}

template <int R>
void launch_gemv_r(const uint4 *packed, const float *s, const void *x, int xtype, int64_t m, int64_t n, int64_t k,
                   int64_t kc, void *y, int ytype, bool vec, hipStream_t st) {
  if (m == 1) launch_gemv<R, 1>(packed, s, x, xtype, m, n, k, kc, y, ytype, vec, st);
  else if (m == 2) launch_gemv<R, 2>(packed, s, x, xtype, m, n, k, kc, y, ytype, vec, st);
  else launch_gemv<R, 4>(packed, s, x, xtype, m, n, k, kc, y, ytype, vec, st);
}

int last_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "%s launch: %s", what, hipGetErrorString(e));
}

}  // namespace

int launch_marlin_repack(const void *w, int wtype, const float *s, int64_t n, int64_t k, uint32_t *packed,
                         hipStream_t st) {
  const int64_t kc = (k + 31) / 32;
  const int64_t threads = n * kc;
  hipLaunchKernelGGL(k_marlin_repack, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, w, wtype, s, n,
                     k, kc, reinterpret_cast<uint4 *>(packed));
  return last_launch("marlin repack");
}

int launch_marlin_dequant(const uint32_t *packed, const float *s, int64_t n, int64_t k, float *out,
                          hipStream_t st) {
  const int64_t kc = (k + 31) / 32;
  const int64_t threads = n * kc;
  const bool vec = (k % 4 == 0) && (reinterpret_cast<uintptr_t>(out) % 16 == 0);
  hipLaunchKernelGGL(k_marlin_dequant, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<const uint4 *>(packed), s, n, k, kc, out, vec);
  return last_launch("marlin dequant");
}

int launch_marlin_linear(const uint32_t *packed, const float *s, int64_t n, int64_t k, const void *x, int xtype,
                         int64_t m, void *y, int ytype, hipStream_t st) {
  const int64_t kc = (k + 31) / 32;
  const uint4 *p = reinterpret_cast<const uint4 *>(packed);
  const bool vec = (k % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  const int xsize = xtype == RQ_F32 ? 4 : 2, ysize = ytype == RQ_F32 ? 4 : 2;
  // grid.y holds at most 65535 row groups of 4: longer activations go in parts.
  constexpr int64_t PART = 65535 * 4;
  for (int64_t r0 = 0; r0 < m; r0 += PART) {
    const int64_t mp = m - r0 < PART ? m - r0 : PART;
    const void *xp = static_cast<const uint8_t *>(x) + r0 * k * xsize;
    void *yp = static_cast<uint8_t *>(y) + r0 * n * ysize;
    if (n <= 8192) launch_gemv_r<16>(p, s, xp, xtype, mp, n, k, kc, yp, ytype, vec, st);
    else if (n <= 32768) launch_gemv_r<32>(p, s, xp, xtype, mp, n, k, kc, yp, ytype, vec, st);
    else launch_gemv_r<64>(p, s, xp, xtype, mp, n, k, kc, yp, ytype, vec, st);
    const int rc = last_launch("marlin gemv");
    if (rc) return rc;
  }
  return RQ_OK;
}

}  // namespace rq
