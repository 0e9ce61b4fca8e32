// rq_gemv_mx.hip -- M = 1 Q4_K GEMV on the matrix cores, for long rows on
// many rows (k % 512 == 0, k <= 8192, n >= 4096: the streaming shapes).
//
// The VALU GEMVs (rq_gemv.hip) spend about 4.4 VALU instructions per weight
// (code extraction, conversion, one FMA, scales, addressing); on Q4_K
// 14336 x 4096 their VALU time alone is about 8 of the 11.5 us of a launch.
// Here a weight costs about 1.1 in the inner loop:
//  * the codes stay integers: a nibble q (0..15) becomes the bf16 pattern
//    0x4300 | q = 128 + q with one v_perm_b32 per two codes (after the mask);
//  * the activations are split into two bf16 limbs, x = hi + lo (hi = bf16(x),
//    lo = bf16(x - hi); the residual is below 2^-17 |x|), and form rows 0 and
//    1 of the A operand of v_mfma_f32_32x32x16_bf16 (rows 2..31 read zeros);
//    the codes of 32 weight rows are the B operand (column = weight row), so
//    each MFMA returns, per weight row, the hi and the lo sum of x (128 + q)
//    over 16 k positions, with exact products and f32 sums;
//  * per super-block of a row (dequant_k.rs:19-44: w = d sc_t q - dmin m_t on
//    sub-block t): y += d (sum_t sc_t S_t - 128 sum_t sc_t X_t) -
//    dmin sum_t m_t X_t, where S_t is the hi + lo sum of the two MFMAs of
//    sub-block t and X_t the f32 sum of hi + lo over the sub-block, computed
//    once per workgroup; the 6-bit sc_t and m_t enter as exact f32 integers.
//
// Layout: a workgroup owns 32 weight rows and the whole of K; each of its
// k / 512 waves takes two super-blocks (512 k) of those rows, and the waves
// meet in LDS.  The weight bytes are read coalesced: a super-block of seven
// rows is 63 consecutive 16-byte pieces per load (nine a row), consecutive
// lanes reading consecutive bytes of a row (a few cache lines per load
// instead of 32 rows; 9.6 -> 7.6 us on 14336 x 4096 without the arithmetic),
// with non-temporal loads (the bytes are used once; 7.6 -> 7.1 us).  Each
// super-block is then passed through a 4.5 KB LDS region of the wave into
// the MFMA layout: lane l holds weight row l % 32 and 16-byte half h = l / 32
// of each 32-byte chunk of quants; the low nibbles of that half are elements
// 16h .. 16h + 15 of the chunk's even sub-block, the high nibbles the same
// elements of its odd sub-block, one MFMA per 8 of them.  The activations are
// staged once per workgroup in LDS as 16-byte records of 8 bf16 (a hi and a
// lo record per 8 elements), which are exactly A fragments.  Each thread
// loads its x elements first, then the weight bytes of its first and second
// super-block (the load counter retires in issue order), then converts and
// stores x while the weights are in flight; the first super-block is
// computed while the second one's bytes are still arriving.
//
// Roofline: HBM-bound.  Algorithmic bytes per call = GGUF block bytes of W +
// activation bytes + output bytes.
#include "rq_formats.h"

namespace rq {
namespace {

typedef __bf16 mx_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mx_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t mx_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMxSb = 2;            // super-blocks per wave (k / 512 waves)
constexpr int kMxZero = 1024;       // bytes of zeros: the A fragments of rows 2..31
constexpr int kMxMaxK = 8192;       // 16 waves
constexpr int kMxTrans = 32 * 144;  // a wave's LDS region: one super-block of 32 rows
constexpr int kMxLoads = 5;         // loads of one super-block of 32 rows, 7 rows each
constexpr uint32_t kMagic = 0x43434343u;  // bf16 0x43nn = 128 + nn for nn < 128
// v_perm_b32 selectors over {kMagic, codes}: bytes 0 and 1 (2 and 3) of the
// code word into the low bytes of two bf16 halves, 0x43 above each.
constexpr uint32_t kSel01 = 0x04010400u;
constexpr uint32_t kSel23 = 0x04030402u;

// LDS bytes: x records (4 bytes per element), zero block, per-sub-block sums
// of x, per-wave partial sums, per-wave transposition regions.
__host__ __device__ inline size_t mx_lds_bytes(int64_t k) {
  const int64_t waves = k / (256 * kMxSb);
  return (size_t)k * 4 + kMxZero + (size_t)(k / 32) * 4 + (size_t)waves * (32 * 4 + kMxTrans);
}

__device__ __forceinline__ uint32_t code_pair(uint32_t codes, uint32_t sel) {
  return __builtin_amdgcn_perm(kMagic, codes, sel);
}

// B fragment: 8 codes (bytes of c0 then c1, each already masked to 0..15).
__device__ __forceinline__ mx_bf16x8 b_frag(uint32_t c0, uint32_t c1) {
  const mx_u32x4 v = {code_pair(c0, kSel01), code_pair(c0, kSel23), code_pair(c1, kSel01), code_pair(c1, kSel23)};
  return __builtin_bit_cast(mx_bf16x8, v);
}

__global__ __launch_bounds__(1024) void k_gemv_mx(const uint8_t *__restrict__ w, const void *__restrict__ x,
                                                  int xtype, const Out o, int64_t n, int64_t k) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = (int)(blockDim.x >> 6);
  const int wr = lane & 31, h = lane >> 5;
  const uint32_t rstride = (uint32_t)(k >> 8) * 144u;  // bytes a row (the whole matrix is < 2 GB)
  const int64_t row0 = (int64_t)blockIdx.x * 32;
  // Last row of this tile that exists (the last tile may be partial).
  const int rowcap = __builtin_amdgcn_readfirstlane((int)(n - row0 < 32 ? n - row0 - 1 : 31));

  // x: thread t holds elements 8t .. 8t + 7 (blockDim.x = k / 8).  One
  // unconditional load form for every type: f32 takes 16-byte chunks 2t and
  // 2t + 1, 16-bit types chunk t (twice).
  const bool f32x = xtype == RQ_F32;
  const uint4 *xc = static_cast<const uint4 *>(x);
  const uint4 xa = xc[f32x ? 2 * tid : tid];
  const uint4 xb = xc[f32x ? 2 * tid + 1 : tid];
  __builtin_amdgcn_sched_barrier(0);

  // Weight bytes: load i of super-block s covers rows 7i .. 7i + 6 of the
  // tile (lane l: row 7i + l / 9, piece l % 9 of the row's 144 bytes; lane 63
  // repeats a piece of the next load), rows past the tile or the matrix
  // clamped.
  const int l7 = lane / 9, pc = lane - 9 * l7;
  const uint8_t *wt0 = w + (uint64_t)row0 * rstride + (uint64_t)(wv * kMxSb) * 144u;
  mx_u32x4 t[kMxSb][kMxLoads];
#pragma unroll
  for (int s = 0; s < kMxSb; ++s) {
#pragma unroll
    for (int i = 0; i < kMxLoads; ++i) {
      const int r = 7 * i + l7 < rowcap ? 7 * i + l7 : rowcap;
      t[s][i] = __builtin_nontemporal_load(
          reinterpret_cast<const mx_u32x4 *>(wt0 + (uint32_t)r * rstride + 144u * s + 16u * pc));
    }
    __builtin_amdgcn_sched_barrier(0);  // the first super-block's loads first
  }

  // Stage x as hi / lo bf16 records (32 bytes per 8 elements), the zero
  // fragments, and X_t per 32-element sub-block.  Branch-free conversion (a
  // branch on the type would sink the second x load into it, behind the
  // weight loads).
  const bool bfx = xtype == RQ_BF16;
  const int zero_off = (int)(4 * k);
  float *xsum = reinterpret_cast<float *>(lds + zero_off + kMxZero);
  {
    const uint32_t va[4] = {xa.x, xa.y, xa.z, xa.w}, vb[4] = {xb.x, xb.y, xb.z, xb.w};
    float xf[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float e0 = bfx ? __uint_as_float(va[j] << 16) : h2f(va[j]);
      const float e1 = bfx ? __uint_as_float(va[j] & 0xFFFF0000u) : h2f(va[j] >> 16);
      // f32: elements 0..3 from xa, 4..7 from xb
      const uint32_t f0 = j < 2 ? va[2 * j] : vb[2 * j - 4], f1 = j < 2 ? va[2 * j + 1] : vb[2 * j - 3];
      xf[2 * j] = f32x ? __uint_as_float(f0) : e0;
      xf[2 * j + 1] = f32x ? __uint_as_float(f1) : e1;
    }
    uint32_t hi[4], lo[4];
    float sx = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hi[j] = pk_bf16(xf[2 * j], xf[2 * j + 1]);
      const float h0 = __uint_as_float(hi[j] << 16), h1 = __uint_as_float(hi[j] & 0xFFFF0000u);
      lo[j] = pk_bf16(xf[2 * j] - h0, xf[2 * j + 1] - h1);
      const float l0 = __uint_as_float(lo[j] << 16), l1 = __uint_as_float(lo[j] & 0xFFFF0000u);
      sx += (h0 + l0) + (h1 + l1);
    }
    *reinterpret_cast<uint4 *>(lds + 32 * tid) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4 *>(lds + 32 * tid + 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    // X_t: the four threads of a sub-block, in a fixed order.
    sx += __shfl_xor(sx, 1);
    sx += __shfl_xor(sx, 2);
    if ((tid & 3) == 0) xsum[tid >> 2] = sx;
  }
  if (tid < kMxZero / 16) *reinterpret_cast<uint4 *>(lds + zero_off + 16 * tid) = make_uint4(0, 0, 0, 0);
  __syncthreads();

  // A fragment of MFMA (chunk c, half s, part p) for lane (A row r, half h):
  // row r < 2 reads limb r of elements 64c + 32s + 16h + 8p .. + 7 of the
  // super-block, at byte 32 * (element / 8) + 16 r of the records; rows
  // 2..31 read the zero block at the same immediate offset.
  const int ar = lane & 31;
  const uint32_t abase = ar < 2 ? (uint32_t)(16 * ar + 64 * h) : (uint32_t)zero_off;
  const uint32_t astride = ar < 2 ? 1024u : 0u;  // bytes of records per super-block
  const mx_f32x16 zero = {};
  float *red = xsum + k / 32;
  uint8_t *trans = reinterpret_cast<uint8_t *>(red + 32 * waves) + kMxTrans * wv;
  // Row r of the region at byte 144 r: 36 dwords apart, so the 16-byte reads
  // of 16 consecutive rows hit distinct banks.  Load i lands at rows 7i + l7
  // (the last load's rows past 31 on row 31, whose piece they repeat).
  uint8_t *tw = trans + 144 * l7 + 16 * pc;
  uint8_t *tw_last = trans + 144 * (28 + l7 < 31 ? 28 + l7 : 31) + 16 * pc;
  const uint8_t *trd = trans + 144 * wr;
  float yacc = 0.0f;
#pragma unroll
  for (int s = 0; s < kMxSb; ++s) {
    const int sb = wv * kMxSb + s;
    // This super-block's pieces into the region, then each lane's header and
    // quant halves out of it.
#pragma unroll
    for (int i = 0; i < kMxLoads - 1; ++i) *reinterpret_cast<mx_u32x4 *>(tw + 1008 * i) = t[s][i];
    *reinterpret_cast<mx_u32x4 *>(tw_last) = t[s][kMxLoads - 1];
    __builtin_amdgcn_wave_barrier();
    const uint4 hd = *reinterpret_cast<const uint4 *>(trd);
    uint4 qv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) qv[c] = *reinterpret_cast<const uint4 *>(trd + 16 + 32 * c + 16 * h);
    __builtin_amdgcn_wave_barrier();
    const uint8_t *ab = lds + abase + astride * (uint32_t)sb;
    const float4 xs0 = reinterpret_cast<const float4 *>(xsum)[2 * sb];
    const float4 xs1 = reinterpret_cast<const float4 *>(xsum)[2 * sb + 1];
    const float xt[8] = {xs0.x, xs0.y, xs0.z, xs0.w, xs1.x, xs1.y, xs1.z, xs1.w};
    // scale_min_k4 (dequant_k.rs:8-16) for all eight sub-blocks: byte t of
    // sc03 / mn03 (sub-blocks 0..3) and of sc47 / mn47 (4..7).
    const uint32_t sc03 = hd.y & 0x3F3F3F3Fu, mn03 = hd.z & 0x3F3F3F3Fu;
    const uint32_t sc47 = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
    const uint32_t mn47 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    float acc_s = 0.0f, acc_x = 0.0f, acc_m = 0.0f;  // sum sc S, sum sc X, sum m X
    static_for<4>([&](auto Cc) {
      constexpr int c = decltype(Cc)::value;
      const uint32_t q[4] = {qv[c].x, qv[c].y, qv[c].z, qv[c].w};
      uint32_t ql[4], qh[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ql[j] = q[j] & 0x0F0F0F0Fu;
        qh[j] = (q[j] >> 4) & 0x0F0F0F0Fu;
      }
      const mx_bf16x8 al0 = *reinterpret_cast<const mx_bf16x8 *>(ab + 256 * c);
      const mx_bf16x8 al1 = *reinterpret_cast<const mx_bf16x8 *>(ab + 256 * c + 32);
      const mx_bf16x8 ah0 = *reinterpret_cast<const mx_bf16x8 *>(ab + 256 * c + 128);
      const mx_bf16x8 ah1 = *reinterpret_cast<const mx_bf16x8 *>(ab + 256 * c + 160);
      mx_f32x16 cl = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al0, b_frag(ql[0], ql[1]), zero, 0, 0, 0);
      cl = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al1, b_frag(ql[2], ql[3]), cl, 0, 0, 0);
      mx_f32x16 ch = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah0, b_frag(qh[0], qh[1]), zero, 0, 0, 0);
      ch = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah1, b_frag(qh[2], qh[3]), ch, 0, 0, 0);
      // Sub-blocks 2c and 2c + 1: bytes (2c) & 3 and (2c + 1) & 3 of the
      // 0..3 or 4..7 words.
      const uint32_t scw = c < 2 ? sc03 : sc47, mnw = c < 2 ? mn03 : mn47;
      const float sc0 = ub(scw, (2 * c) & 3), sc1 = ub(scw, (2 * c + 1) & 3);
      const float m0 = ub(mnw, (2 * c) & 3), m1 = ub(mnw, (2 * c + 1) & 3);
      acc_s = fmaf(sc0, cl[0] + cl[1], acc_s);
      acc_s = fmaf(sc1, ch[0] + ch[1], acc_s);
      acc_x = fmaf(sc0, xt[2 * c], acc_x);
      acc_x = fmaf(sc1, xt[2 * c + 1], acc_x);
      acc_m = fmaf(m0, xt[2 * c], acc_m);
      acc_m = fmaf(m1, xt[2 * c + 1], acc_m);
    });
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    yacc = fmaf(d, fmaf(-128.0f, acc_x, acc_s), yacc);
    yacc = fmaf(-dmin, acc_m, yacc);
  }

  // Lanes 0..31 hold the rows (A rows 0 and 1 are C rows 0 and 1 of lane
  // half 0); the waves' partial sums meet in LDS, added in wave order.
  if (h == 0) red[32 * wv + wr] = yacc;
  __syncthreads();
  if (tid < 32 && row0 + tid < n) {
    float v = 0.0f;
    for (int i = 0; i < waves; ++i) v += red[32 * i + tid];
    store_linear(o, 0, n, row0 + tid, v);
  }
}

// ---- Q6_K (dequant_k.rs:94-125) ----
//
// The same layout with the device's Q6_K records (208 bytes a super-block:
// ql 128 | qh 64 | int8 scales 16, d in the aux array): a 6-bit code q
// becomes the bf16 pattern 0x4300 | q = 128 + q, and one
// v_mfma_f32_32x32x16_bf16 covers one 16-element sub-block of 32 rows, so
// w . x = d sum_t sc_t (S_t - 160 X_t) with S_t the MFMA's hi + lo sum of
// x (128 + q) and X_t the sum of x over the sub-block.  Sub-block t = 8 hf +
// 2 r + s (half hf, run r, 16-element group s) holds elements 128 hf + 32 r +
// 16 s + j: its low four bits are nibble r / 2 of ql byte 64 hf + 32 (r & 1)
// + 16 s + j, its high two bits bits 2r, 2r + 1 of qh byte 32 hf + 16 s + j.
// Lane (row, half h) takes j = 8h .. 8h + 7.  Records are loaded coalesced
// (13 pieces of 16 bytes a row, 416 a super-block of 32 rows, seven loads)
// through a 6.5 KB LDS region of the wave.
constexpr int kMx6Trans = 32 * 208;  // a wave's LDS region: one super-block of 32 rows
constexpr int kMx6Loads = 7;         // 7 x 64 >= 416 pieces (the rest repeat piece 415)

__host__ __device__ inline size_t mx6_lds_bytes(int64_t k) {
  const int64_t waves = k / (256 * kMxSb);
  return (size_t)k * 4 + kMxZero + (size_t)(k / 16) * 4 + (size_t)waves * (32 * 4 + kMx6Trans);
}

__global__ __launch_bounds__(1024) void k_gemv_mx6(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                   const void *__restrict__ x, int xtype, const Out o, int64_t n,
                                                   int64_t k) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = (int)(blockDim.x >> 6);
  const int wr = lane & 31, h = lane >> 5;
  const int nsb = (int)(k >> 8);
  const uint32_t rstride = (uint32_t)nsb * 208u;  // bytes a row (the whole matrix is < 2 GB)
  const int64_t row0 = (int64_t)blockIdx.x * 32;
  const int rowcap = __builtin_amdgcn_readfirstlane((int)(n - row0 < 32 ? n - row0 - 1 : 31));

  const bool f32x = xtype == RQ_F32;
  const uint4 *xc = static_cast<const uint4 *>(x);
  const uint4 xa = xc[f32x ? 2 * tid : tid];
  const uint4 xb = xc[f32x ? 2 * tid + 1 : tid];
  __builtin_amdgcn_sched_barrier(0);

  // Piece c = lane + 64 i of a super-block: 16-byte piece c % 13 of row
  // c / 13 (c / 13 = (5042 c) >> 16 for c < 448); rows past the matrix
  // clamped.
  int prow[kMx6Loads], ppc[kMx6Loads];
#pragma unroll
  for (int i = 0; i < kMx6Loads; ++i) {
    const int c = lane + 64 * i < 415 ? lane + 64 * i : 415;
    prow[i] = (c * 5042) >> 16;
    ppc[i] = c - 13 * prow[i];
  }
  const uint8_t *wt0 = w + (uint64_t)row0 * rstride + (uint64_t)(wv * kMxSb) * 208u;
  mx_u32x4 t[kMxSb][kMx6Loads];
#pragma unroll
  for (int s = 0; s < kMxSb; ++s) {
#pragma unroll
    for (int i = 0; i < kMx6Loads; ++i) {
      const int r = prow[i] < rowcap ? prow[i] : rowcap;
      t[s][i] = __builtin_nontemporal_load(
          reinterpret_cast<const mx_u32x4 *>(wt0 + (uint32_t)r * rstride + 208u * s + 16u * ppc[i]));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // d of this lane's row for the wave's two super-blocks (nsb and 2 wv are
  // even, so the two halves are one aligned word).
  const int drow = wr < rowcap ? wr : rowcap;
  const uint32_t dd =
      *reinterpret_cast<const uint32_t *>(aux + 2 * ((uint64_t)(row0 + drow) * nsb + (uint64_t)(wv * kMxSb)));

  // x as hi / lo bf16 records (32 bytes per 8 elements), the zero
  // fragments, and X_t per 16-element sub-block (the sum of hi + lo).
  const bool bfx = xtype == RQ_BF16;
  const int zero_off = (int)(4 * k);
  float *xsum = reinterpret_cast<float *>(lds + zero_off + kMxZero);
  {
    const uint32_t va[4] = {xa.x, xa.y, xa.z, xa.w}, vb[4] = {xb.x, xb.y, xb.z, xb.w};
    float xf[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float e0 = bfx ? __uint_as_float(va[j] << 16) : h2f(va[j]);
      const float e1 = bfx ? __uint_as_float(va[j] & 0xFFFF0000u) : h2f(va[j] >> 16);
      const uint32_t f0 = j < 2 ? va[2 * j] : vb[2 * j - 4], f1 = j < 2 ? va[2 * j + 1] : vb[2 * j - 3];
      xf[2 * j] = f32x ? __uint_as_float(f0) : e0;
      xf[2 * j + 1] = f32x ? __uint_as_float(f1) : e1;
    }
    uint32_t hi[4], lo[4];
    float sx = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hi[j] = pk_bf16(xf[2 * j], xf[2 * j + 1]);
      const float h0 = __uint_as_float(hi[j] << 16), h1 = __uint_as_float(hi[j] & 0xFFFF0000u);
      lo[j] = pk_bf16(xf[2 * j] - h0, xf[2 * j + 1] - h1);
      const float l0 = __uint_as_float(lo[j] << 16), l1 = __uint_as_float(lo[j] & 0xFFFF0000u);
      sx += (h0 + l0) + (h1 + l1);
    }
    *reinterpret_cast<uint4 *>(lds + 32 * tid) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4 *>(lds + 32 * tid + 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    sx += __shfl_xor(sx, 1);
    if ((tid & 1) == 0) xsum[tid >> 1] = sx;
  }
  if (tid < kMxZero / 16) *reinterpret_cast<uint4 *>(lds + zero_off + 16 * tid) = make_uint4(0, 0, 0, 0);
  __syncthreads();

  // A fragment of sub-block (hf, r, s) for lane (A row a, half h): element
  // e = 256 sb + 128 hf + 32 r + 16 s + 8 h, record byte 32 (e / 8) + 16 a =
  // 1024 sb + 512 hf + 128 r + 64 s + 32 h + 16 a (rows 2..31 read zeros).
  const int ar = lane & 31;
  const uint32_t abase = ar < 2 ? (uint32_t)(16 * ar + 32 * h) : (uint32_t)zero_off;
  const uint32_t astride = ar < 2 ? 1024u : 0u;
  const mx_f32x16 zero = {};
  float *red = xsum + k / 16;
  uint8_t *trans = reinterpret_cast<uint8_t *>(red + 32 * waves) + kMx6Trans * wv;
  // Row r of the region at byte 208 r (52 dwords apart: 16 consecutive rows
  // start on distinct banks).
  const uint8_t *trd = trans + 208 * wr;
  float yacc = 0.0f;
#pragma unroll
  for (int s = 0; s < kMxSb; ++s) {
    const int sb = wv * kMxSb + s;
#pragma unroll
    for (int i = 0; i < kMx6Loads; ++i)
      *reinterpret_cast<mx_u32x4 *>(trans + 208 * prow[i] + 16 * ppc[i]) = t[s][i];
    __builtin_amdgcn_wave_barrier();
    // ql bytes 64 hf + 16 g + 8 h (g = s16 for r even, 2 + s16 for r odd)
    // and qh bytes 32 hf + 16 s16 + 8 h, for hf, s16 in {0, 1}.
    uint2 qa[2][2], qb[2][2], qq[2][2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int s16 = 0; s16 < 2; ++s16) {
        qa[hf][s16] = *reinterpret_cast<const uint2 *>(trd + 64 * hf + 16 * s16 + 8 * h);
        qb[hf][s16] = *reinterpret_cast<const uint2 *>(trd + 64 * hf + 32 + 16 * s16 + 8 * h);
        qq[hf][s16] = *reinterpret_cast<const uint2 *>(trd + 128 + 32 * hf + 16 * s16 + 8 * h);
      }
    const uint4 scb = *reinterpret_cast<const uint4 *>(trd + 192);
    __builtin_amdgcn_wave_barrier();
    const uint8_t *ab = lds + abase + astride * (uint32_t)sb;
    const float4 *xs4 = reinterpret_cast<const float4 *>(xsum) + 4 * sb;
    const float4 xs[4] = {xs4[0], xs4[1], xs4[2], xs4[3]};
    const uint32_t scw[4] = {scb.x, scb.y, scb.z, scb.w};
    float acc_s = 0.0f, acc_x = 0.0f;  // sum sc S, sum sc X
    static_for<2>([&](auto Hf) {
      constexpr int hf = decltype(Hf)::value;
      static_for<4>([&](auto Rr) {
        constexpr int r = decltype(Rr)::value;
        static_for<2>([&](auto Ss) {
          constexpr int s16 = decltype(Ss)::value;
          constexpr int sub = 8 * hf + 2 * r + s16;
          const uint2 lq = (r & 1) ? qb[hf][s16] : qa[hf][s16];
          const uint2 hq = qq[hf][s16];
          const uint32_t c0 = ((lq.x >> (4 * (r >> 1))) & 0x0F0F0F0Fu) | (((hq.x >> (2 * r)) & 0x03030303u) << 4);
          const uint32_t c1 = ((lq.y >> (4 * (r >> 1))) & 0x0F0F0F0Fu) | (((hq.y >> (2 * r)) & 0x03030303u) << 4);
          const mx_bf16x8 a = *reinterpret_cast<const mx_bf16x8 *>(ab + 512 * hf + 128 * r + 64 * s16);
          const mx_f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b_frag(c0, c1), zero, 0, 0, 0);
          const float sc = (float)(int8_t)((scw[sub >> 2] >> (8 * (sub & 3))) & 0xFFu);
          const float xt = (&xs[sub >> 2].x)[sub & 3];
          acc_s = fmaf(sc, c[0] + c[1], acc_s);
          acc_x = fmaf(sc, xt, acc_x);
        });
      });
    });
    const float d = h2f(s ? dd >> 16 : dd);
    yacc = fmaf(d, fmaf(-160.0f, acc_x, acc_s), yacc);
  }

  if (h == 0) red[32 * wv + wr] = yacc;
  __syncthreads();
  if (tid < 32 && row0 + tid < n) {
    float v = 0.0f;
    for (int i = 0; i < waves; ++i) v += red[32 * i + tid];
    store_linear(o, 0, n, row0 + tid, v);
  }
}

}  // namespace

int launch_gemv_mx(const rq_weight *wt, const void *x, int xtype, const Out &o, hipStream_t s) {
  const int64_t n = wt->n, k = wt->k;
  if (wt->qtype != RQ_Q4_K || k % (256 * kMxSb) != 0 || k > kMxMaxK || n < 32) return RQ_E_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  // 32-bit byte offsets inside the matrix.
  if ((uint64_t)n * (uint64_t)(k / 256) * 144u >= (1ull << 31)) return RQ_E_UNSUPPORTED;
  const int64_t grid = (n + 31) / 32;
  const size_t lds = mx_lds_bytes(k);
  if (lds > 65536) {
    // Above 64 KB of dynamic LDS (k > 4096) the kernel asks for it once.
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_mx),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       (int)mx_lds_bytes(kMxMaxK));
    if (attr != hipSuccess) {
      (void)hipGetLastError();
      return RQ_E_UNSUPPORTED;
    }
  }
  hipLaunchKernelGGL(k_gemv_mx, dim3((unsigned)grid), dim3((unsigned)(k / 8)), lds, s, wt->data, x, xtype, o, n,
                     k);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
}

int launch_gemv_mx6(const rq_weight *wt, const void *x, int xtype, const Out &o, hipStream_t s) {
  const int64_t n = wt->n, k = wt->k;
  if (wt->qtype != RQ_Q6_K || k % (256 * kMxSb) != 0 || k > kMxMaxK || n < 32) return RQ_E_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  if ((uint64_t)n * (uint64_t)(k / 256) * 208u >= (1ull << 31)) return RQ_E_UNSUPPORTED;
  const size_t lds = mx6_lds_bytes(k);
  if (lds > 65536) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_mx6),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       (int)mx6_lds_bytes(kMxMaxK));
    if (attr != hipSuccess) {
      (void)hipGetLastError();
      return RQ_E_UNSUPPORTED;
    }
  }
  hipLaunchKernelGGL(k_gemv_mx6, dim3((unsigned)((n + 31) / 32)), dim3((unsigned)(k / 8)), lds, s, wt->data,
                     wt->data + wt->aux_off, x, xtype, o, n, k);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemv launch failed");
}

}  // namespace rq
