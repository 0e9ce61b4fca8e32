// rq_gemm.hip -- quantized GEMM on gfx950 matrix cores (prefill and verify).
//
// y[m, n] = sum_k x[m, k] * W[n, k] for bf16 activations x and GGUF weights W
// (Q4_K, Q6_K, Q8_0), f32 accumulation, f32/bf16/f16 output.  Semantics of the
// reference's dense path (linear_layer.rs:88-104 after dequant_tensor,
// dequant.rs:83-146) with the weights rounded once to bf16 on their way into
// the matrix cores (the tolerance for bf16 operands: 2e-2 normalized).
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
#include <type_traits>

#include "rq_epilogue.h"
#include "rq_formats.h"
#include "rq_pipe.h"

namespace rq {
namespace {

using namespace pipe;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64, LDS_K = BK + 8;

// A BM x BN tile of y per workgroup of KG groups of WM x WN waves; each
// wave owns a (BM / WM) x (BN / WN) sub-tile made of MI x NI MFMA tiles of
// 32 x 32.  Each thread decodes exactly one 32-element weight piece per K-step
// (BN * 2 == 64 * WM * WN).
// Split K: workgroup z covers K-steps [z * steps, (z + 1) * steps) and, when
// part is not null, writes its f32 partial tile to part + z * m * n instead
// of y (k_splitk_sum adds the partials).  Inside a workgroup, K-group g
// (waves g * WM * WN ..) takes the g-th of KG equal parts of those steps with
// LDS buffers of its own (the host makes steps a multiple of KG); the groups
// meet in LDS at the end (added in group order) and group 0 stores.  More
// waves per tile then keep more loads in flight where a tile's K loop is
// latency-bound (the 2048-wide layers at M = 512: 256 tiles of 64 x 64).
//
// XT is the activation type: RQ_BF16 as above, or RQ_F32 / RQ_F16 (the
// reference computes in f32, store.rs:3-4), which run on the same bf16
// matrix cores as two bf16 limbs per operand: the activations split as they
// go to LDS, the weights decoded to their exact f32 values (the reference's
// dequantized weights) and split the same way, and each product taken as
// hi*hi + hi*lo + lo*hi (three MFMAs, f32 accumulation).  The dropped lo*lo
// term and the limbs' own rounding leave about 2^-16 of each product, far
// inside the 1e-3 gate of f32 paths; LDS holds a hi and a lo tile of each
// operand.
template <class F, int BM, int BN, int WM, int WN, int D, int KG = 1, int XT = RQ_BF16, int NB = 2>
__global__ __launch_bounds__(64 * WM * WN * KG) void k_qgemm(const uint8_t *__restrict__ w,
                                                            const uint8_t *__restrict__ aux,
                                                            const void *__restrict__ xv, int64_t m,
                                                            int64_t n, int64_t k, const Out o, int64_t steps,
                                                            float *__restrict__ part) {
  constexpr bool LIMBS = XT != RQ_BF16;
  constexpr int NL = LIMBS ? 2 : 1;           // LDS tiles of each operand (hi, lo)
  constexpr int XB = XT == RQ_F32 ? 4 : 2;    // bytes of an activation in memory
  constexpr int EPL = 16 / XB;                // activations per 16-byte load
  constexpr int LPR = BK / EPL;               // loads per activation row and step
  constexpr int NT = 64 * WM * WN;  // threads of a K-group
  static_assert(BN * 2 == NT, "one weight piece per thread");
  constexpr int MI = BM / WM / 32, NI = BN / WN / 32;
  constexpr int A_LOADS = BM * LPR / NT;      // 16-byte loads per thread per step
  constexpr int A_ROWS = NT / LPR;            // activation rows covered by one load round
  constexpr int A_BYTES = BM * LDS_K * 2, B_BYTES = BN * LDS_K * 2;
  constexpr int G_BYTES = NB * NL * (A_BYTES + B_BYTES);  // a group's NB buffers of tiles
  static_assert(KG == 1 || BM * BN * 4 <= G_BYTES, "the partial tile of a group fits its buffers");
  __shared__ __attribute__((aligned(16))) uint8_t SM[KG * G_BYTES];

  const int grp = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / NT));
  const int tid = threadIdx.x % NT, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  uint8_t *const G = SM + grp * G_BYTES;
  // tile l (0 = hi, 1 = lo) of buffer buf
  auto As = [&](int buf, int l = 0) { return reinterpret_cast<uint16_t *>(G + (NL * buf + l) * A_BYTES); };
  auto Bs = [&](int buf, int l = 0) {
    return reinterpret_cast<uint16_t *>(G + NB * NL * A_BYTES + (NL * buf + l) * B_BYTES);
  };

  // Weight piece of this thread: row n0 + (tid >> 1), half h = tid & 1;
  // activation slots: row tid / LPR + A_ROWS * i, EPL activations at column
  // EPL * (tid % LPR).  Rows past n or m re-read the last row (unconditional
  // loads); their products land in outputs that are never stored.
  const int brow = tid >> 1, bh = tid & 1;
  const int64_t gn = n0 + brow < n ? n0 + brow : n - 1;
  const int arow = tid / LPR, acol = EPL * (tid % LPR);
  const uint8_t *xa[A_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int64_t gm = m0 + arow + A_ROWS * i;
    xa[i] = static_cast<const uint8_t *>(xv) + ((gm < m ? gm : m - 1) * k + acol) * XB;
  }

  // Loads run D K-steps ahead in D register slots (LLVM vector types: a
  // HIP uint4 array would be copied through private memory).
  const int64_t gsteps = steps / KG;
  const int64_t kt0 = (int64_t)blockIdx.z * steps + grp * gsteps;
  const int64_t nk = (k / BK - kt0 < gsteps ? k / BK - kt0 : gsteps);
  u32x4 ra[D][A_LOADS];
  typename F::Piece pb[D];
  auto gload = [&](int slot, int64_t s) {  // local step s, clamped to the group's steps
    const int64_t kt = kt0 + (s < nk ? s : nk - 1);
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) ra[slot][i] = *reinterpret_cast<const u32x4 *>(xa[i] + kt * BK * XB);
    pb[slot] = F::load(w, aux, gn, k, (int)(2 * kt + bh));
  };
  // The 16 weights of run r, pairs q (8 weights each) of limb l to the LDS tile.
  auto store_b = [&](uint16_t *B, const uint32_t (&ob)[16]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      u32x4 *dst = reinterpret_cast<u32x4 *>(&B[brow * LDS_K + 16 * bh + 32 * r]);
#pragma unroll
      for (int q = 0; q < 2; ++q)
        dst[q] = (u32x4){ob[8 * r + 4 * q], ob[8 * r + 4 * q + 1], ob[8 * r + 4 * q + 2], ob[8 * r + 4 * q + 3]};
    }
  };
  auto sstore = [&](int slot, int buf) {
    if constexpr (!LIMBS) {
      uint16_t *A = As(buf);
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i)
        *reinterpret_cast<u32x4 *>(&A[(arow + A_ROWS * i) * LDS_K + acol]) = ra[slot][i];
      uint32_t ob[16];
      F::decode_bf16(pb[slot], ob);
      store_b(Bs(buf), ob);
    } else {
      uint16_t *Ah = As(buf, 0), *Al = As(buf, 1);
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) {
        const u32x4 v = ra[slot][i];
        const int off = (arow + A_ROWS * i) * LDS_K + acol;
        if constexpr (XT == RQ_F32) {  // 4 activations: 8 bytes of each limb
          uint32_t h0, l0, h1, l1;
          limbs2(__uint_as_float(v.x), __uint_as_float(v.y), h0, l0);
          limbs2(__uint_as_float(v.z), __uint_as_float(v.w), h1, l1);
          *reinterpret_cast<uint2 *>(&Ah[off]) = make_uint2(h0, h1);
          *reinterpret_cast<uint2 *>(&Al[off]) = make_uint2(l0, l1);
        } else {  // 8 f16 activations: 16 bytes of each limb
          const _Float16 *hv = reinterpret_cast<const _Float16 *>(&v);
          uint32_t h[4], l[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) limbs2((float)hv[2 * q], (float)hv[2 * q + 1], h[q], l[q]);
          *reinterpret_cast<u32x4 *>(&Ah[off]) = (u32x4){h[0], h[1], h[2], h[3]};
          *reinterpret_cast<u32x4 *>(&Al[off]) = (u32x4){l[0], l[1], l[2], l[3]};
        }
      }
      float wv[2][16];
      F::decode(pb[slot], wv);
      uint32_t oh[16], ol[16];
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) limbs2(wv[r][2 * j], wv[r][2 * j + 1], oh[8 * r + j], ol[8 * r + j]);
      store_b(Bs(buf, 0), oh);
      store_b(Bs(buf, 1), ol);
    }
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = (f32x16){0};

  auto mfma_step = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kc = ks * 16 + 8 * (lane >> 5);
      bf16x8 fa[NL][MI], fb[NL][NI];
#pragma unroll
      for (int l = 0; l < NL; ++l) {
        const uint16_t *A = As(buf, l), *B = Bs(buf, l);
#pragma unroll
        for (int i = 0; i < MI; ++i)
          fa[l][i] = *reinterpret_cast<const bf16x8 *>(&A[(wm * (BM / WM) + i * 32 + (lane & 31)) * LDS_K + kc]);
#pragma unroll
        for (int j = 0; j < NI; ++j)
          fb[l][j] = *reinterpret_cast<const bf16x8 *>(&B[(wn * (BN / WN) + j * 32 + (lane & 31)) * LDS_K + kc]);
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          if constexpr (LIMBS) {  // the small cross terms first
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[1][i], fb[0][j], acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[0][i], fb[1][j], acc[i][j], 0, 0, 0);
          }
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[0][i], fb[0][j], acc[i][j], 0, 0, 0);
        }
    }
  };

  // Slot (s % D) holds step s once loaded.  Step s: the matrix work on LDS
  // buffer s % 2; step s + 1 (loaded D - 1 steps ago) is written to the other
  // buffer and its slot refilled with step s + 1 + D; one barrier.  With one
  // buffer (NB = 1: half the LDS, so twice the K-groups fit) step s + 1 is
  // written to the same buffer after a second barrier.  The
  // stores of steps past the end are made anyway (clamped data into a buffer
  // that is never read) and only their matrix work is skipped, so no load is
  // made under a branch.  Every group runs the same number of steps.
#pragma unroll
  for (int j = 0; j < D; ++j) gload(j, j);
  sstore(0, 0);
  gload(0, D);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; kt += D) {
    static_for<D>([&](auto J) {
      constexpr int j = decltype(J)::value;
      const int64_t s = kt + j;
      const int buf = NB == 2 ? (int)(s & 1) : 0;
      if (s < nk) mfma_step(buf);
      if constexpr (NB == 1) __syncthreads();  // every wave's reads of the one buffer are done
      sstore((j + 1) % D, NB == 2 ? buf ^ 1 : 0);
      gload((j + 1) % D, s + 1 + D);
      __syncthreads();
    });
  }

  if constexpr (KG > 1) {
    // Groups 1 .. KG - 1 leave their accumulators in their own buffers
    // (free after the last barrier); group 0 adds them in group order.
    float *red = reinterpret_cast<float *>(G);
    auto idx = [&](int i, int j, int r) { return (((wave * MI + i) * NI + j) * 16 + r) * 64 + lane; };
    if (grp > 0) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) red[idx(i, j, r)] = acc[i][j][r];
    }
    __syncthreads();
    if (grp > 0) return;
    for (int g = 1; g < KG; ++g) {
      const float *rg = reinterpret_cast<const float *>(SM + g * G_BYTES);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += rg[idx(i, j, r)];
    }
  }

  // Split K: f32 partials without the bias (k_splitk_sum adds it).
  const Out out = part ? Out{part + (int64_t)blockIdx.z * m * n, nullptr, RQ_F32, 0} : o;
  const bool vec = vec_stores_ok(out.y, n);
  const float one[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  float bb[NI][4];  // loaded before the first store
#pragma unroll
  for (int j = 0; j < NI; ++j) tile_col_bias(out, n, n0 + wn * (BN / WN) + j * 32, lane, bb[j]);
  static_for<MI>([&](auto I) {
    static_for<NI>([&](auto J) {
      store_tile32<false>(acc[I][J], out, m, n, m0 + wm * (BM / WM) + I * 32, n0 + wn * (BN / WN) + J * 32, one,
                          one, bb[J], nullptr, nullptr, lane, vec);
    });
  });
}

// ---- pipelined 256 x 256 kernels ------------------------------------------
//
// Eight waves (two a SIMD) of 128 (M) x 64 (N): 4 x 2 MFMA tiles of 32 x 32,
// 128 accumulators a wave.  K-steps of 32 inputs (64 bytes of bf16 a row)
// pass through four LDS stages: the activation parts of the stages side by
// side (256 rows x 64 bytes, 16 KB each), the weight parts 64 KB above,
// rows unpadded with the 16-byte chunk index XOR-ed with (row / 4) % 4, so
// that one base register per role reaches every stage through the 16-bit
// ds offset field.  Every global load goes to registers (the compiler then
// counts its waits exactly; mixed with direct-to-LDS loads it would wait for
// all of them) and every LDS access is explicit (ordered against the bare
// barriers).  With one wave a SIMD (four waves of 128 x 128, 256
// accumulators) a wave issued its decode and address VALU work at about half
// the SIMD's rate between its MFMAs; two waves a SIMD hide one another's
// waits: the Q6_K head 262144 x 2048 at M = 512 704 -> 634 us, Q4_K
// 2048 x 14336 x 4096 308 -> 283 us, Q8_0 512 x 151936 x 1024 289 -> 222 us
// (outputs bit-identical).
//
// Step s: each thread writes its two 16-byte activation chunks of step s + 2
// (loaded at step s - 2; 4 lanes a row, 16 rows a load instruction) into
// their stage and loads those of step s + 4, and writes the weight runs it
// decoded for the stages of steps s + 2 (and s + 3).  The MFMAs run in two
// passes (pass H takes 16-byte chunk 2g + H of every row, g = lane / 32, for
// A and B alike); the fragments of pass 1 are read from LDS during pass 0
// and those of the next step's pass 0 during pass 1, so a stage is read
// during steps s - 1 and s and written during s - 2 or s - 3.

__device__ __forceinline__ bf16x8 as_bf16(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ void wait_lds_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// ---- pipelined 256 x 256 kernel, Q6_K in chunk pairs ------------------
//
// The two 64-element chunks 2j and 2j + 1 of a row (a half super-block,
// dequant_k.rs:87-111) share their quant bytes: ql byte l holds the low four
// bits of element l of chunk 2j (nibble 0) and of chunk 2j + 1 (nibble 1),
// qh byte l the high two bits of both (bits 0-1 / 2-3 for chunk 2j, 4-5 / 6-7
// for 2j + 1).  The generic kernel (k_qgemm_pipe8 with FmtQ6KG) loads a
// piece's 48 quant bytes once per chunk; here a thread loads them once per
// pair (ql runs [16 hh, + 16) and
// [32 + 16 hh, + 16), qh run [16 hh, + 16), the half's eight scales and d)
// and decodes one 16-weight run of it per K-step: the pair of K-steps
// 4j .. 4j + 3 is decoded during steps 4j - 2 .. 4j + 1 into the stage of
// step s + 2, with the decoded values bit-identical to FmtQ6KG's.  Half the
// load instructions and quant bytes of the per-chunk pieces, and a quarter
// of the decode work per step instead of half of it on every other step.
// Pairs alternate between two register slots, so the loop is unrolled by
// eight steps (k % 256 == 0).
struct Q6Pair {
  u32x4 a, b, h;
  uint32_t sc0, sc1;  // the half's int8 scales: bytes 0..3 (chunk 2j), 4..7 (chunk 2j + 1)
  uint32_t d;
};

__device__ __forceinline__ Q6Pair load_q6_pair(const uint8_t *w, const uint8_t *aux, uint64_t rk, int64_t j,
                                               int hh) {
  const uint64_t e = rk + 128u * (uint64_t)j;
  const uint64_t blk = e >> 8;
  const int hf = (int)((e >> 7) & 1u);
  const uint8_t *rec = w + blk * 208u;
  Q6Pair p;
  p.a = *reinterpret_cast<const u32x4 *>(rec + 64 * hf + 16 * hh);
  p.b = *reinterpret_cast<const u32x4 *>(rec + 64 * hf + 32 + 16 * hh);
  p.h = *reinterpret_cast<const u32x4 *>(rec + 128 + 32 * hf + 16 * hh);
  const uint2 sc = *reinterpret_cast<const uint2 *>(rec + 192 + 8 * hf);
  p.sc0 = sc.x;
  p.sc1 = sc.y;
  p.d = reinterpret_cast<const uint16_t *>(aux)[blk];
  return p;
}

// Run RR of chunk 2j + CC of piece hh: positions 16 hh .. 16 hh + 15 of
// K-step 4j + 2 CC + RR, as eight bf16 pairs (FmtQ6KG::decode_bf16's words
// 8 RR .. 8 RR + 7 of that chunk's piece).
template <int CC, int RR>
__device__ __forceinline__ void q6_pair_run(const Q6Pair &p, int hh, uint32_t (&o)[8]) {
  const float d = h2f(p.d);
  const uint32_t scw = CC ? p.sc1 : p.sc0;
  const float ds = d * (float)(int8_t)((scw >> (8 * (2 * RR + hh))) & 0xFFu);
  const float z = -32.0f * ds;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t src = RR ? p.b[j] : p.a[j];
    const uint32_t hb = p.h[j] >> (4 * CC);
    const uint32_t q = opaque(((src >> (4 * CC)) & 0x0F0F0F0Fu) |
                              (RR ? ((hb & 0x0C0C0C0Cu) << 2) : ((hb & 0x03030303u) << 4)));
    o[2 * j] = pk_bf16(fmaf(ub(q, 0), ds, z), fmaf(ub(q, 1), ds, z));
    o[2 * j + 1] = pk_bf16(fmaf(ub(q, 2), ds, z), fmaf(ub(q, 3), ds, z));
  }
}

// Q6_K in chunk pairs on eight waves (two a SIMD): a 256 x 256 output tile,
// each wave 128 (M) x 64 (N) of it (4 x 2 MFMA tiles of 32 x 32, 128
// accumulators), so that a SIMD interleaves two waves' decode and MFMAs.  A
// single wave a SIMD issues VALU instructions at about half the SIMD's rate
// (a probe of 28 independent FMAs per four 32x32x16 MFMAs: one wave 128-138
// ns an iteration against 72-77 for the MFMAs alone; two waves, twice the
// work, 163-168 ns), and the decode costs about six VALU instructions per
// MFMA.  Each thread decodes one weight row a step (row t / 2, piece t % 2)
// and loads two 16-byte activation chunks; the tile rows' activations of
// step s + 4 are loaded during step s, the chunk pair of steps 4j .. 4j + 3
// during step 4j - 7, and both are written into LDS stage (s + 2) % 4 during
// step s.  Four stages, one barrier every two steps (before even steps:
// the pair of steps reads stages s and s + 1 and writes s + 2 and s + 3, so
// the first pass's fragments of an even step are read after its barrier;
// head 660 -> 649-657 us against a barrier a step), LDS rows of 64 bytes with
// the 16-byte chunk index XOR-ed with (row / 4) % 4.  Workgroups take tiles
// XCD by XCD (XCD x the x-th eighth of the tiles, M fastest) so that the
// workgroups sharing a weight tile share an L2.
struct Pass8 {
  u32x4 x[6];  // A of tiles 0..3, then B of tiles 0..1
};

__device__ __forceinline__ void wait_pass8(Pass8 &P) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(P.x[0]), "+v"(P.x[1]), "+v"(P.x[2]));
  asm volatile("" : "+v"(P.x[3]), "+v"(P.x[4]), "+v"(P.x[5]));
}

// q6_pair_run in pieces, to be placed between MFMAs: the run's scale, then
// words 2J, 2J + 1 (part J < 4).  Same arithmetic, same bits.
struct RunScale {
  float ds, z;
};

template <int CC, int RR>
__device__ __forceinline__ RunScale q6_run_scale(const Q6Pair &p, int hh) {
  const float d = h2f(p.d);
  const uint32_t scw = CC ? p.sc1 : p.sc0;
  const float ds = d * (float)(int8_t)((scw >> (8 * (2 * RR + hh))) & 0xFFu);
  return {ds, -32.0f * ds};
}

template <int CC, int RR, int J>
__device__ __forceinline__ void q6_run_part(const Q6Pair &p, const RunScale &sc, uint32_t (&o)[8]) {
  const uint32_t src = RR ? p.b[J] : p.a[J];
  const uint32_t hb = p.h[J] >> (4 * CC);
  const uint32_t q = opaque(((src >> (4 * CC)) & 0x0F0F0F0Fu) |
                            (RR ? ((hb & 0x0C0C0C0Cu) << 2) : ((hb & 0x03030303u) << 4)));
  o[2 * J] = pk_bf16(fmaf(ub(q, 0), sc.ds, sc.z), fmaf(ub(q, 1), sc.ds, sc.z));
  o[2 * J + 1] = pk_bf16(fmaf(ub(q, 2), sc.ds, sc.z), fmaf(ub(q, 3), sc.ds, sc.z));
  asm volatile("" : "+v"(o[2 * J]), "+v"(o[2 * J + 1]));  // computed here, not next to its use
}

// LDS of the eight-wave kernel: the A (activation) parts of the four stages
// side by side (16 KB each), then the four B (weight-run) parts, so one base
// register per role reaches every stage through the 16-bit offset field.
constexpr int P8_A = 16384, P8_B = 65536;

struct PipeBases8 {
  uint32_t rd[2][2];  // [pass H][A, B]: fragment reads
  uint32_t wa;        // activation writes
  uint32_t wr[2];     // [16-byte chunk q]: weight-run writes
};

// The 8 MFMAs of one pass on `cur`, reading pass H of stage ST into `nxt`
// (one read after each of the first six) and running hook(f) after MFMA f:
// the order is fixed (nothing is moved across the scheduling barriers), so
// the hook's VALU work issues while the MFMAs before it run.
template <int ST, int H, class Hook, bool READ = true>
__device__ __forceinline__ void mfma_pass8(const Pass8 &cur, Pass8 &nxt, const PipeBases8 &pb, f32x16 (&acc)[4][2],
                                           Hook &&hook, std::integral_constant<bool, READ> = {}) {
  static_for<4>([&](auto I) {
    static_for<2>([&](auto J) {
      acc[I][J] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16(cur.x[I]), as_bf16(cur.x[4 + J]), acc[I][J], 0, 0,
                                                          0);
      constexpr int f = 2 * decltype(I)::value + decltype(J)::value;
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (READ && f < 6) nxt.x[f] = ds_read16_off<ST * P8_A + 2048 * (f < 4 ? f : f - 4)>(pb.rd[H][f < 4 ? 0 : 1]);
      hook(std::integral_constant<int, f>{});
      __builtin_amdgcn_sched_barrier(0);
    });
  });
}

template <int ST>
__device__ __forceinline__ void write_a8(const PipeBases8 &pb, const u32x4 (&a)[2]) {
  ds_write16_off<ST * P8_A>(pb.wa, a[0]);
  ds_write16_off<ST * P8_A + 1024>(pb.wa, a[1]);
}

template <int ST>
__device__ __forceinline__ void write_run8(const PipeBases8 &pb, const uint32_t (&o)[8]) {
  ds_write16_off<ST * P8_A>(pb.wr[0], (u32x4){o[0], o[1], o[2], o[3]});
  ds_write16_off<ST * P8_A>(pb.wr[1], (u32x4){o[4], o[5], o[6], o[7]});
}

__device__ __forceinline__ void load_a8(const uint8_t *const (&src)[2], int64_t s, u32x4 (&a)[2]) {
  a[0] = *reinterpret_cast<const u32x4 *>(src[0] + 64 * s);
  a[1] = *reinterpret_cast<const u32x4 *>(src[1] + 64 * s);
}

__global__ __launch_bounds__(512) void k_q6_pipe8(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                  const uint16_t *__restrict__ x, int64_t m, int64_t n, int64_t k,
                                                  const Out o) {
  __shared__ __attribute__((aligned(1024))) uint8_t SM[4 * P_STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int64_t gm = gridDim.y, tiles = (int64_t)gridDim.x * gridDim.y;
  const int64_t b = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
  const int64_t lin = tiles % 8 == 0 ? (b % 8) * (tiles / 8) + b / 8 : b;
  const int64_t m0 = (lin % gm) * 256, n0 = (lin / gm) * 256;
  const int64_t nk = k / 32, np = nk / 4;  // K-steps, chunk pairs
  const int last = (int)nk - 1;

  // Activation rows 32 wave + 16 j + lane / 4 (j < 2), chunk lane % 4.
  const uint8_t *asrc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t gr = m0 + 32 * wave + 16 * j + (lane >> 2);
    asrc[j] = reinterpret_cast<const uint8_t *>(x + (gr < m ? gr : m - 1) * k) + 16 * (lane & 3);
  }
  const int hh = tid & 1, br = tid >> 1;
  const uint64_t rk0 = (uint64_t)(n0 + br < n ? n0 + br : n - 1) * (uint64_t)k;

  PipeBases8 pb;
  {
    const uint32_t sa = lds_addr(SM), sb = sa + P8_B;
    const int l = lane & 31, g = lane >> 5, sw = (l >> 2) & 3;
#pragma unroll
    for (int H = 0; H < 2; ++H) {
      pb.rd[H][0] = sa + 8192 * wm + 64 * l + 16 * ((2 * g + H) ^ sw);
      pb.rd[H][1] = sb + 4096 * wn + 64 * l + 16 * ((2 * g + H) ^ sw);
    }
    pb.wa = sa + 2048 * wave + 64 * (lane >> 2) + 16 * ((lane & 3) ^ ((lane >> 4) & 3));
#pragma unroll
    for (int q = 0; q < 2; ++q) pb.wr[q] = sb + 64 * br + 16 * ((2 * hh + q) ^ swz(br));
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x16){0};

  // Prologue: stages 0 and 1 written (chunk 0 of pair 0), pairs 0 and 1 in
  // slots 0 and 1, activations of steps 2 and 3 in flight, pass 0 of step 0
  // read.
  u32x4 ra[2][2];
  Q6Pair pp[2];  // [slot]
  {
    u32x4 a0[2], a1[2];
    load_a8(asrc, 0, a0);
    load_a8(asrc, 1, a1);
    pp[0] = load_q6_pair(w, aux, rk0, 0, hh);
    load_a8(asrc, 2 < nk ? 2 : last, ra[0]);
    load_a8(asrc, 3 < nk ? 3 : last, ra[1]);
    pp[1] = load_q6_pair(w, aux, rk0, np > 1 ? 1 : 0, hh);
    write_a8<0>(pb, a0);
    write_a8<1>(pb, a1);
    uint32_t o[8];
    q6_pair_run<0, 0>(pp[0], hh, o);
    write_run8<0>(pb, o);
    q6_pair_run<0, 1>(pp[0], hh, o);
    write_run8<1>(pb, o);
  }
  wait_lds_all();
  Pass8 P0, P1;

  // Step s = 8u + B: pass 0 of stage s % 4 (read after the barrier on even
  // steps, during the previous step on odd ones), pass 1 of it, and
  // the run of step s + 2 (pair (s + 2) / 4, chunk ((s + 2) / 2) % 2, run
  // (s + 2) % 2) from slot ((B + 2) / 4) % 2 into stage (s + 2) % 4; slot 0
  // is free after step 8u + 1 and takes pair 2u + 2, slot 1 after 8u + 5 and
  // takes pair 2u + 3.
  auto step = [&](int64_t s, auto Bc) {
    constexpr int B = decltype(Bc)::value;
    constexpr int T = (B + 2) & 7, CC = (T >> 1) & 1, RR = T & 1, SLOT = ((B + 2) >> 2) & 1;
    constexpr int ST = B & 3, ST1 = (B + 1) & 3, ST2 = (B + 2) & 3;
    if constexpr ((B & 1) == 0) {
      __builtin_amdgcn_s_barrier();
      static_for<6>([&](auto F) {
        constexpr int f = decltype(F)::value;
        P0.x[f] = ds_read16_off<ST * P8_A + 2048 * (f < 4 ? f : f - 4)>(pb.rd[0][f < 4 ? 0 : 1]);
      });
      wait_pass8(P0);
    }
    // stage (s + 2) % 4 was last read in steps s - 3 and s - 2: its activation
    // part is written first, the decoded run (during the first pass) early in
    // the second, so that no write is left to complete at the end of the step
    write_a8<ST2>(pb, ra[B & 1]);
    load_a8(asrc, s + 4 < nk ? s + 4 : last, ra[B & 1]);
    uint32_t o0[8];
    const RunScale sc = q6_run_scale<CC, RR>(pp[SLOT], hh);
    mfma_pass8<ST, 1>(P0, P1, pb, acc, [&](auto F) {
      constexpr int f = decltype(F)::value;
      if constexpr (f & 1) q6_run_part<CC, RR, f / 2>(pp[SLOT], sc, o0);
    });
    wait_pass8(P1);
    mfma_pass8<ST1, 0>(P1, P0, pb, acc, [&](auto F) {
      if constexpr (decltype(F)::value == 0) write_run8<ST2>(pb, o0);
    }, std::integral_constant<bool, (B & 1) == 0>{});
    if constexpr (B == 1 || B == 5) {
      const int64_t jn = (s + 7) >> 2 < np ? (s + 7) >> 2 : np - 1;
      pp[B == 1 ? 0 : 1] = load_q6_pair(w, aux, rk0, jn, hh);
    }
    if constexpr ((B & 1) == 0) wait_pass8(P0);
    else wait_lds_all();
  };
  for (int64_t t = 0; t < nk; t += 8) {
    step(t, std::integral_constant<int, 0>{});
    step(t + 1, std::integral_constant<int, 1>{});
    step(t + 2, std::integral_constant<int, 2>{});
    step(t + 3, std::integral_constant<int, 3>{});
    step(t + 4, std::integral_constant<int, 4>{});
    step(t + 5, std::integral_constant<int, 5>{});
    step(t + 6, std::integral_constant<int, 6>{});
    step(t + 7, std::integral_constant<int, 7>{});
  }

  // The tile to y: 16-bit outputs of whole tiles staged in LDS (the four
  // stages, free after the loop), other tiles straight from the accumulators.
  const bool vec = vec_stores_ok(o.y, n);
  float bb[2][4];  // biases, loaded before the first store
#pragma unroll
  for (int j = 0; j < 2; ++j) tile_col_bias(o, n, n0 + 64 * wn + j * 32, lane, bb[j]);
  if (o.ytype != RQ_F32 && vec && n % 8 == 0 && m0 + 256 <= m && n0 + 256 <= n) {
    __syncthreads();  // every wave's stage reads are done
    const float unused_x[4][4] = {}, unused_w[2][4] = {};  // scales: none (SCALED false)
    stage_block_2b<false>(acc, SM, 128 * wm, 64 * wn, o.ytype, unused_x, unused_w, bb, o.bias != nullptr, lane);
    __syncthreads();
    store_staged_2b<512>(SM, o.y, n, m0, n0, tid);
    return;
  }
  const float one[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  static_for<4>([&](auto I) {
    static_for<2>([&](auto J) {
      store_tile32<false>(acc[I][J], o, m, n, m0 + 128 * wm + I * 32, n0 + 64 * wn + J * 32, one, one, bb[J],
                          nullptr, nullptr, lane, vec);
    });
  });
}

// ---- generic formats on eight waves -------------------------------------
//
// Each format's pieces (64-element chunks, run 0 of piece 2c + h holding
// inputs 16h .. 16h + 15 of K-step 2c and run 1 those of K-step 2c + 1, so a
// chunk fills the weight rows of two consecutive stages) on the eight waves
// and LDS layout of k_q6_pipe8: each thread decodes piece t % 2 of
// weight row t / 2 every other step (chunk (s + 2) / 2 in step s, s even),
// and the pieces of chunks c + 1 and c + 2 are in flight in two register
// slots.  Indices past the end are clamped (their loads and writes land in
// stages that are never read); k must be a multiple of 128.
template <int ST>
__device__ __forceinline__ void write_run16(const PipeBases8 &pb, const uint32_t *o) {
  ds_write16_off<ST * P8_A>(pb.wr[0], (u32x4){o[0], o[1], o[2], o[3]});
  ds_write16_off<ST * P8_A>(pb.wr[1], (u32x4){o[4], o[5], o[6], o[7]});
}

template <class F>
__global__ __launch_bounds__(512) void k_qgemm_pipe8(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                                     const uint16_t *__restrict__ x, int64_t m, int64_t n,
                                                     int64_t k, const Out o) {
  __shared__ __attribute__((aligned(1024))) uint8_t SM[4 * P_STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int64_t gm = gridDim.y, tiles = (int64_t)gridDim.x * gridDim.y;
  const int64_t b = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
  const int64_t lin = tiles % 8 == 0 ? (b % 8) * (tiles / 8) + b / 8 : b;
  const int64_t m0 = (lin % gm) * 256, n0 = (lin / gm) * 256;
  const int64_t nk = k / 32;
  const int last = (int)nk - 1;

  const uint8_t *asrc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t gr = m0 + 32 * wave + 16 * j + (lane >> 2);
    asrc[j] = reinterpret_cast<const uint8_t *>(x + (gr < m ? gr : m - 1) * k) + 16 * (lane & 3);
  }
  const int h = tid & 1, br = tid >> 1;
  const uint64_t rk0 = (uint64_t)(n0 + br < n ? n0 + br : n - 1) * (uint64_t)k;

  PipeBases8 pb;
  {
    const uint32_t sa = lds_addr(SM), sb = sa + P8_B;
    const int l = lane & 31, g = lane >> 5, sw = (l >> 2) & 3;
#pragma unroll
    for (int H = 0; H < 2; ++H) {
      pb.rd[H][0] = sa + 8192 * wm + 64 * l + 16 * ((2 * g + H) ^ sw);
      pb.rd[H][1] = sb + 4096 * wn + 64 * l + 16 * ((2 * g + H) ^ sw);
    }
    pb.wa = sa + 2048 * wave + 64 * (lane >> 2) + 16 * ((lane & 3) ^ ((lane >> 4) & 3));
#pragma unroll
    for (int q = 0; q < 2; ++q) pb.wr[q] = sb + 64 * br + 16 * ((2 * h + q) ^ swz(br));
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x16){0};

  // Prologue: stages 0 and 1 written (chunk 0), activations of steps 2 and 3
  // and the pieces of chunks 1 and 2 in flight, pass 0 of step 0 read.
  u32x4 ra[2][2];
  typename F::Piece pc[2];  // [chunk % 2]
  {
    u32x4 a0[2], a1[2];
    load_a8(asrc, 0, a0);
    load_a8(asrc, 1, a1);
    const typename F::Piece p0 = F::load_e(w, aux, rk0, h);
    load_a8(asrc, 2 < nk ? 2 : last, ra[0]);
    load_a8(asrc, 3 < nk ? 3 : last, ra[1]);
    const int c1 = (2 < nk ? 2 : last - 1) + h, c2 = (4 < nk ? 4 : last - 1) + h;
    pc[1] = F::load_e(w, aux, rk0, c1);
    pc[0] = F::load_e(w, aux, rk0, c2);
    write_a8<0>(pb, a0);
    write_a8<1>(pb, a1);
    uint32_t o[16];
    F::decode_bf16(p0, o);
    write_run16<0>(pb, o);
    write_run16<1>(pb, o + 8);
  }
  wait_lds_all();
  __builtin_amdgcn_s_barrier();
  Pass8 P0, P1;
  static_for<6>([&](auto Fc) {
    constexpr int f = decltype(Fc)::value;
    P0.x[f] = ds_read16_off<2048 * (f < 4 ? f : f - 4)>(pb.rd[0][f < 4 ? 0 : 1]);
  });
  wait_pass8(P0);

  // Step s = 4u + B: pass 1 of stage B, pass 0 of stage (B + 1) % 4; on even
  // steps the chunk (s + 2) / 2 (slot (B / 2 + 1) % 2) into stages
  // (B + 2) % 4 and (B + 3) % 4, whose last reads were in steps s - 2 and
  // s - 1, and the piece of chunk (s + 6) / 2 into that slot.
  auto step = [&](int64_t s, auto Bc) {
    constexpr int B = decltype(Bc)::value;
    constexpr int SL = ((B >> 1) + 1) & 1;
    __builtin_amdgcn_s_barrier();
    write_a8<(B + 2) & 3>(pb, ra[B & 1]);
    load_a8(asrc, s + 4 < nk ? s + 4 : last, ra[B & 1]);
    uint32_t o0[16];
    if constexpr ((B & 1) == 0) F::decode_bf16(pc[SL], o0);
    mfma_pass8<B, 1>(P0, P1, pb, acc, [](auto) {});
    wait_pass8(P1);
    mfma_pass8<(B + 1) & 3, 0>(P1, P0, pb, acc, [&](auto Fc) {
      if constexpr ((B & 1) == 0 && decltype(Fc)::value == 0) {
        write_run16<(B + 2) & 3>(pb, o0);
        write_run16<(B + 3) & 3>(pb, o0 + 8);
      }
    });
    if constexpr ((B & 1) == 0) {
      const int pn = (int)(s + 6 < nk ? s + 6 : last - 1) + h;  // piece h of chunk (s + 6) / 2
      pc[SL] = F::load_e(w, aux, rk0, pn);
    }
    wait_pass8(P0);
    wait_lds_all();
  };
  for (int64_t t = 0; t < nk; t += 4) {
    step(t, std::integral_constant<int, 0>{});
    step(t + 1, std::integral_constant<int, 1>{});
    step(t + 2, std::integral_constant<int, 2>{});
    step(t + 3, std::integral_constant<int, 3>{});
  }

  const bool vec = vec_stores_ok(o.y, n);
  float bb[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j) tile_col_bias(o, n, n0 + 64 * wn + j * 32, lane, bb[j]);
  if (o.ytype != RQ_F32 && vec && n % 8 == 0 && m0 + 256 <= m && n0 + 256 <= n) {
    __syncthreads();
    const float unused_x[4][4] = {}, unused_w[2][4] = {};
    stage_block_2b<false>(acc, SM, 128 * wm, 64 * wn, o.ytype, unused_x, unused_w, bb, o.bias != nullptr, lane);
    __syncthreads();
    store_staged_2b<512>(SM, o.y, n, m0, n0, tid);
    return;
  }
  const float one[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  static_for<4>([&](auto I) {
    static_for<2>([&](auto J) {
      store_tile32<false>(acc[I][J], o, m, n, m0 + 128 * wm + I * 32, n0 + 64 * wn + J * 32, one, one, bb[J],
                          nullptr, nullptr, lane, vec);
    });
  });
}

// y = sum over s < splits of part[s] (f32 partials of m * n outputs), with
// o's bias.
__global__ __launch_bounds__(256) void k_splitk_sum(const float *__restrict__ part, int splits, int64_t mn,
                                                    int64_t n, const Out o) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < mn; i += (int64_t)gridDim.x * 256) {
    float v = part[i];
    for (int s = 1; s < splits; ++s) v += part[s * mn + i];
    if (o.bias) v = with_bias(v, load_as_f32(o.bias, o.btype, i % n), o.ytype);
    store_one(o.y, o.ytype, i, v);
  }
}

// The same with four consecutive outputs a thread (m * n and n multiples of
// four, y 16-byte aligned): 16-byte partial loads, all S of a thread's loads
// issued before the sums, which run in split order as above (same results).
template <int S>
__global__ __launch_bounds__(256) void k_splitk_sum4(const float *__restrict__ part, int64_t mn, int64_t n,
                                                     const Out o) {
  const float4 *p4 = reinterpret_cast<const float4 *>(part);
  const int64_t mn4 = mn / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < mn4; i += (int64_t)gridDim.x * 256) {
    float4 t[S];
#pragma unroll
    for (int s = 0; s < S; ++s) t[s] = p4[s * mn4 + i];
    float4 v = t[0];
#pragma unroll
    for (int s = 1; s < S; ++s) {
      v.x += t[s].x;
      v.y += t[s].y;
      v.z += t[s].z;
      v.w += t[s].w;
    }
    if (o.bias) {
      const int64_t c = (4 * i) % n;
      v.x = with_bias(v.x, load_as_f32(o.bias, o.btype, c), o.ytype);
      v.y = with_bias(v.y, load_as_f32(o.bias, o.btype, c + 1), o.ytype);
      v.z = with_bias(v.z, load_as_f32(o.bias, o.btype, c + 2), o.ytype);
      v.w = with_bias(v.w, load_as_f32(o.bias, o.btype, c + 3), o.ytype);
    }
    store_four(o.y, o.ytype, 4 * i, v.x, v.y, v.z, v.w);
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

template <class F, int BM, int BN, int WM, int WN, int D = 3, int KG = 1, int XT = RQ_BF16, int NB = 2>
int launch(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease &ws,
           int sp_force = 0) {
  const int64_t nk = wt->k / BK;
  const int64_t gx = (wt->n + BN - 1) / BN, gy = (m + BM - 1) / BM;
  const int sp = sp_force > 0 ? sp_force : splits_for(gx * gy, nk);
  // K-groups need equal shares of every split's steps.
  if constexpr (KG > 1) {
    if (nk % ((int64_t)sp * KG) != 0) return launch<F, BM, BN, WM, WN, D, 1, XT, 2>(wt, x, m, o, s, ws, sp);
  }
  const int64_t steps = (nk + sp - 1) / sp;
  const int used = (int)((nk + steps - 1) / steps);  // splits that own at least one step
  float *part = nullptr;
  if (used > 1) {
    int rc = RQ_OK;
    part = static_cast<float *>(ws.get((size_t)used * m * wt->n * sizeof(float), &rc));
    if (!part) return rc;
  }
  const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)used);
  hipLaunchKernelGGL((k_qgemm<F, BM, BN, WM, WN, D, KG, XT, NB>), grid, dim3(64 * WM * WN * KG), 0, s, wt->data,
                     wt->data + wt->aux_off, x, m, wt->n, wt->k, o, steps, part);
  if (part) {
    const int64_t mn = m * wt->n;
    if (wt->n % 4 == 0 && (reinterpret_cast<uintptr_t>(o.y) & 15) == 0 && used <= 8) {
      const int64_t blocks = (mn / 4 + 255) / 256 < 4096 ? (mn / 4 + 255) / 256 : 4096;
      const dim3 g((unsigned)blocks), b(256);
      switch (used) {
        case 2: hipLaunchKernelGGL(k_splitk_sum4<2>, g, b, 0, s, part, mn, wt->n, o); break;
        case 3: hipLaunchKernelGGL(k_splitk_sum4<3>, g, b, 0, s, part, mn, wt->n, o); break;
        case 4: hipLaunchKernelGGL(k_splitk_sum4<4>, g, b, 0, s, part, mn, wt->n, o); break;
        case 5: hipLaunchKernelGGL(k_splitk_sum4<5>, g, b, 0, s, part, mn, wt->n, o); break;
        case 6: hipLaunchKernelGGL(k_splitk_sum4<6>, g, b, 0, s, part, mn, wt->n, o); break;
        case 7: hipLaunchKernelGGL(k_splitk_sum4<7>, g, b, 0, s, part, mn, wt->n, o); break;
        default: hipLaunchKernelGGL(k_splitk_sum4<8>, g, b, 0, s, part, mn, wt->n, o); break;
      }
    } else {
      const int64_t blocks = (mn + 255) / 256 < 4096 ? (mn + 255) / 256 : 4096;
      hipLaunchKernelGGL(k_splitk_sum, dim3((unsigned)blocks), dim3(256), 0, s, part, used, mn, wt->n, o);
    }
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemm launch failed");
}

template <class F>
int launch_pipe(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s) {
  const dim3 grid((unsigned)((wt->n + 255) / 256), (unsigned)((m + 255) / 256));
  if (std::is_same<F, FmtQ6KG>::value && wt->k % 256 == 0)
    hipLaunchKernelGGL(k_q6_pipe8, grid, dim3(512), 0, s, wt->data, wt->data + wt->aux_off,
                       static_cast<const uint16_t *>(x), m, wt->n, wt->k, o);
  else
    hipLaunchKernelGGL((k_qgemm_pipe8<F>), grid, dim3(512), 0, s, wt->data, wt->data + wt->aux_off,
                       static_cast<const uint16_t *>(x), m, wt->n, wt->k, o);
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "gemm launch failed");
}

template <class F>
int by_m(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease &ws) {
  if (m <= 64) return launch<F, 64, 128, 2, 2>(wt, x, m, o, s, ws);
  // 256 x 256 tiles when they still give every CU a workgroup (pipelined
  // when K is a multiple of 128), else 128 x 128.
  const int64_t big_tiles = ((m + 255) / 256) * ((wt->n + 255) / 256);
  if (big_tiles >= 256 && wt->k % 128 == 0) return launch_pipe<F>(wt, x, m, o, s);
  if (big_tiles >= 256) return launch<F, 256, 256, 2, 4, 1>(wt, x, m, o, s, ws);
  // Fewer than 128 tiles of 128 x 128 (2048-wide layers at M = 512): short K
  // takes 64 x 64 tiles of two waves (256 workgroups) in four K-groups (eight
  // waves a workgroup); long K keeps 128 x 128 and splits K four ways (at
  // most, 32 K-steps per split).  Other shapes: 128 x 128 in two K-groups.
  // Each K-step is latency-bound at these sizes (a 64-deep step is 8-16
  // MFMAs a wave), so more waves per tile help.  Measured on the 2048 / 8192
  // prefill shapes: q/k/o 36 -> 26 us (64 x 128) -> 25.3 us (64 x 64) ->
  // 18.4 us (four K-groups), v Q6_K 28.2 -> 27.2 -> 21.9 us, gate/up 37.9 ->
  // 34.4 us (two K-groups), down 67 -> 53 us (two K-groups: 56 us).
  // Register slots: the loop runs D steps an iteration, so a group's step
  // count should be a multiple of D (three slots on the 8, 16 and 32 steps
  // of these groups ran one dead step each); one slot on the 64 x 64 groups
  // (q/k/o 18.4 -> 15.4 us, v 20.0 -> 16.7 us; two slots 16.0 / 17.5) and
  // on 128 x 128 (gate/up 32.6 -> 29.0 us with two slots, 28.3 -> 27.8-28.2
  // with one).  The split down projection also takes two K-groups (eight
  // waves a workgroup): 42.7 -> 40.7 us, 44.5 -> 41.4 in alternating runs.
  const int64_t tiles128 = ((m + 127) / 128) * ((wt->n + 127) / 128), nk = wt->k / BK;
  if (tiles128 < 128 && nk <= 32) return launch<F, 64, 64, 2, 1, 1, 4>(wt, x, m, o, s, ws);
  if (tiles128 < 128 && nk >= 64) {
    const int sp = (int)(nk / 32 < 4 ? nk / 32 : 4);
    return launch<F, 128, 128, 2, 2, 1, 2>(wt, x, m, o, s, ws, sp);
  }
  return launch<F, 128, 128, 2, 2, 1, 2>(wt, x, m, o, s, ws);
}

// f32 / f16 activations, m > 64: the two-limb tiles (twice the LDS of the
// bf16 tiles).  One LDS buffer a K-group, so that two K-groups of 128 x 128
// or four of 64 x 64 (eight waves, two a SIMD) fit: against one group of
// 128 x 128 / two of 64 x 64 double-buffered (one wave a SIMD), M = 512
// q/k/o 33.6 -> 29.0 us, v 35.2 -> 31.5, gate/up 78.9 -> 73.9, down 91.8 ->
// 85.3, LM head 2.66 -> 2.51 ms.  Where those forms spill (more than 256
// registers at two waves a SIMD: Q8_0's pieces on both tiles, Q5_0's on
// 64 x 64) the double-buffered ones stay (Q8_0 2048 x 2048: 34.0 against
// 42.6 us with the spills).  Tile shapes follow by_m: 64 x 64 where 128 x 128
// tiles are too few for the CUs with short K, K split four ways for long K
// on few tiles.
template <class F, int XT>
int by_m_limbs(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease &ws) {
  constexpr bool Q8 = std::is_same<F, FmtQ8>::value;
  constexpr bool WIDE64 = !Q8 && !std::is_same<F, FmtQx0<true>>::value, WIDE128 = !Q8;
  constexpr int KG128 = WIDE128 ? 2 : 1, NB128 = WIDE128 ? 1 : 2;
  const int64_t tiles128 = ((m + 127) / 128) * ((wt->n + 127) / 128), nk = wt->k / BK;
  if (tiles128 < 128 && nk <= 32) {
    if constexpr (WIDE64) return launch<F, 64, 64, 2, 1, 1, 4, XT, 1>(wt, x, m, o, s, ws);
    else return launch<F, 64, 64, 2, 1, 1, 2, XT>(wt, x, m, o, s, ws);
  }
  if (tiles128 < 128 && nk >= 64) {
    const int sp = (int)(nk / 32 < 4 ? nk / 32 : 4);
    return launch<F, 128, 128, 2, 2, 1, KG128, XT, NB128>(wt, x, m, o, s, ws, sp);
  }
  return launch<F, 128, 128, 2, 2, 1, KG128, XT, NB128>(wt, x, m, o, s, ws);
}

template <int XT>
int limbs_fmt(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease &ws) {
  switch (wt->qtype) {
    case RQ_Q4_K: return by_m_limbs<FmtQ4K, XT>(wt, x, m, o, s, ws);
    case RQ_Q6_K: return by_m_limbs<FmtQ6KG, XT>(wt, x, m, o, s, ws);
    case RQ_Q8_0: return by_m_limbs<FmtQ8, XT>(wt, x, m, o, s, ws);
    case RQ_Q5_K: return by_m_limbs<FmtQ5K, XT>(wt, x, m, o, s, ws);
    case RQ_Q4_0: return by_m_limbs<FmtQx0<false>, XT>(wt, x, m, o, s, ws);
    case RQ_Q5_0: return by_m_limbs<FmtQx0<true>, XT>(wt, x, m, o, s, ws);
    default: return RQ_E_UNSUPPORTED;
  }
}

}  // namespace

// f32 / f16 activations, m > 64, k % 64 == 0, 16-byte aligned x: the
// two-limb tiles of k_qgemm.
int launch_linear_mfma_limbs(const rq_weight *wt, const void *x, int xtype, int64_t m, const Out &o, hipStream_t s,
                             WsLease &ws) {
  if (wt->k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  if (xtype == RQ_F32) return limbs_fmt<RQ_F32>(wt, x, m, o, s, ws);
  if (xtype == RQ_F16) return limbs_fmt<RQ_F16>(wt, x, m, o, s, ws);
  return RQ_E_UNSUPPORTED;
}

// bf16 activations, m > 1, k % 64 == 0, 16-byte aligned x.
int launch_linear_mfma(const rq_weight *wt, const void *x, int64_t m, const Out &o, hipStream_t s, WsLease &ws) {
  if (wt->k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  switch (wt->qtype) {
    case RQ_Q4_K: return by_m<FmtQ4K>(wt, x, m, o, s, ws);
    case RQ_Q6_K: return by_m<FmtQ6KG>(wt, x, m, o, s, ws);
    case RQ_Q8_0: return by_m<FmtQ8>(wt, x, m, o, s, ws);
    case RQ_Q5_K: return by_m<FmtQ5K>(wt, x, m, o, s, ws);
    case RQ_Q4_0: return by_m<FmtQx0<false>>(wt, x, m, o, s, ws);
    case RQ_Q5_0: return by_m<FmtQx0<true>>(wt, x, m, o, s, ws);
    default: return RQ_E_UNSUPPORTED;
  }
}

}  // namespace rq
