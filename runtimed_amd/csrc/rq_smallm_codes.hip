// rq_smallm_codes.hip -- quantized linear y = x W^T for 4 <= M <= 64 f32
// activation rows (speculative verify in the reference's compute type) on the
// bf16 matrix cores, with the weights as their integer codes.
//
// A Q4_K / Q6_K / Q8_0 weight is a small integer code times a scale shared by
// a run of 16 or 32 weights (plus, for Q4_K, a min term shared the same way):
// w = D q - M.  Codes below 128 are exact in bf16 as 128 + q (the byte permute
// 0x43nn, one instruction per two codes); int8 codes are exact in bf16 as
// they are.  So the matrix cores can take the codes as they are, and the
// scales are applied afterwards, per run, to the f32 sums:
//
//   sum_e x_e w_e = D sum_e x_e (128 + q_e) - (128 D + M) sum_e x_e
//                 = D S - M' X
//
// with S from one v_mfma_f32_16x16x32_bf16 on the codes and X from one on
// constant ones.  The activations are the A operand as two bf16 limbs each
// (hi = bf16(x), lo = bf16(x - hi): 16 significant bits), so an MFMA takes 16
// elements: lane group g supplies elements 4g .. 4g + 3 of a 16-element run,
// hi limbs in K slots 0..3 and lo limbs in 4..7, and the codes of the same
// elements twice.  The products are exact and summed in f32; what departs
// from the reference's f32 matmul is the limbs' 2^-17 and the summation order.
//
// Compared with decoding every weight to f32 (one FMA) and then to two bf16
// limbs (three more instructions), a code costs half an instruction and each
// run of 16 or 32 weights two FMAs per output held by the lane.
//
// Layout: the weights are the B operand (lane l holds weight row l % 16 and
// its four codes of lane group l / 16), so the lane's outputs -- rows
// 4 (l / 16) .. + 3 of the activation tile, weight row l % 16 -- take the
// lane's own scales.  Workgroups and waves as in the bf16 small-M kernel:
// NW waves split the K chunks of 16 weight rows, B chunks a batch, the wave
// tiles summed through LDS, K split over S workgroups for few row tiles, and
// the activation slice staged in LDS (already split into limbs) when it fits.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "rq_epilogue.h"
#include "rq_formats.h"
#include "rq_internal.h"
#include "rq_smallm_common.h"

namespace rq {
namespace {

// bf16 0x43nn = 128 + nn for nn < 128: v_perm_b32 over {kCodeMagic, codes}
// puts bytes 0 and 1 (2 and 3) of a code word below 0x43 in two bf16 halves.
constexpr uint32_t kCodeMagic = 0x43434343u;
constexpr uint32_t kCodeSel01 = 0x04010400u;
constexpr uint32_t kCodeSel23 = 0x04030402u;
__device__ __forceinline__ uint32_t cpair(uint32_t codes, uint32_t sel) {
  return __builtin_amdgcn_perm(kCodeMagic, codes, sel);
}
// Four codes below 128 (bytes of c) as the B fragment of one MFMA: 128 + q of
// elements 0..3, then the same for the lo limbs.
__device__ __forceinline__ bf16x8 codes_b(uint32_t c) {
  const uint32_t p0 = cpair(c, kCodeSel01), p1 = cpair(c, kCodeSel23);
  return pick(p0, p1, p0, p1);
}
// Four int8 codes (bytes of c, signed) as exact bf16, twice.
__device__ __forceinline__ bf16x8 codes_b_i8(uint32_t c) {
  const float f0 = (float)(int8_t)(c & 0xFFu), f1 = (float)(int8_t)((c >> 8) & 0xFFu);
  const float f2 = (float)(int8_t)((c >> 16) & 0xFFu), f3 = (float)(int8_t)(c >> 24);
  // the upper halves of the f32 values (exact: at most 8 significant bits)
  const uint32_t p0 = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  const uint32_t p1 = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  return pick(p0, p1, p0, p1);
}

// Weight chunks: 64 elements of a row (t-th chunk), four runs r of 16
// (chunk elements 16 r .. 16 r + 15); lane group g holds the codes of
// elements 16 r + 4 g .. + 3.  A format gives, per run, the B fragment and
// the scale D and min M' of  sum_e x_e w_e = D S - M' X  (S from the B
// fragment, X from ones); runs 2j and 2j + 1 share them where PAIR (32-weight
// groups), which lets their MFMAs chain into one S and one X.

// Q4_K (dequant_k.rs:19-44): chunk c of a block = sub-blocks 2c (low nibbles
// of qs[32c .. 32c + 31]) and 2c + 1 (high nibbles of the same bytes); runs 0,
// 1 are the low nibbles of qs[32c + 4g ..] and qs[32c + 16 + 4g ..], runs 2, 3
// their high nibbles.  Codes 128 + q: M' = 128 d sc + dmin m.
struct CdQ4K {
  static constexpr bool PAIR = true, MIN = true;
  struct Chunk {
    uint4 hd;
    uint32_t q0, q1;
    int c;
  };
  __device__ static Chunk load(const uint8_t *w, const uint8_t *, int64_t row, int64_t k, int64_t t, int g) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 64u * (uint64_t)t;
    const uint8_t *bp = w + (e >> 8) * 144u;
    Chunk ch;
    ch.c = (int)((e >> 6) & 3u);
    ch.hd = *reinterpret_cast<const uint4 *>(bp);
    ch.q0 = *reinterpret_cast<const uint32_t *>(bp + 16 + 32 * ch.c + 4 * g);
    ch.q1 = *reinterpret_cast<const uint32_t *>(bp + 16 + 32 * ch.c + 16 + 4 * g);
    return ch;
  }
  __device__ static void decode(const Chunk &ch, int, bf16x8 (&b)[4], float (&d)[4], float (&mn)[4]) {
    FmtQ4K::Piece pc;
    pc.hd = ch.hd;
    pc.c = ch.c;
    float a0, b0, a1, b1;
    FmtQ4K::scales(pc, a0, b0, a1, b1);
    b[0] = codes_b(ch.q0 & 0x0F0F0F0Fu);
    b[1] = codes_b(ch.q1 & 0x0F0F0F0Fu);
    b[2] = codes_b((ch.q0 >> 4) & 0x0F0F0F0Fu);
    b[3] = codes_b((ch.q1 >> 4) & 0x0F0F0F0Fu);
    d[0] = d[1] = a0;
    d[2] = d[3] = a1;
    mn[0] = mn[1] = fmaf(128.0f, a0, b0);
    mn[2] = mn[3] = fmaf(128.0f, a1, b1);
  }
};

// Q6_K (dequant_k.rs:87-111) on the split layout (208-byte records, f16 d
// array).  Chunk ch of half hf holds the half's outputs 64 ch .. 64 ch + 63:
// element j < 32 is code nibble ch of ql[j] with bits 4 ch .. 4 ch + 1 of
// qh[j], element 32 + l nibble ch of ql[l + 32] with bits 4 ch + 2 .. of
// qh[l]; run r takes scale sc[4 ch + r] of the half.  Codes 128 + q for
// q - 32: M' = 160 d sc.
struct CdQ6K {
  static constexpr bool PAIR = false, MIN = true;
  struct Chunk {
    uint32_t l0, l1, l2, l3, h0, h1, sc, d;
    int ch;
  };
  __device__ static Chunk load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int64_t t, int g) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 64u * (uint64_t)t;
    const uint64_t blk = e >> 8;
    const int hf = (int)((e >> 7) & 1u);
    const uint8_t *rec = w + blk * 208u;
    const uint8_t *ql = rec + 64 * hf + 4 * g, *qh = rec + 128 + 32 * hf + 4 * g;
    Chunk c;
    c.ch = (int)((e >> 6) & 1u);
    c.l0 = *reinterpret_cast<const uint32_t *>(ql);
    c.l1 = *reinterpret_cast<const uint32_t *>(ql + 16);
    c.l2 = *reinterpret_cast<const uint32_t *>(ql + 32);
    c.l3 = *reinterpret_cast<const uint32_t *>(ql + 48);
    c.h0 = *reinterpret_cast<const uint32_t *>(qh);
    c.h1 = *reinterpret_cast<const uint32_t *>(qh + 16);
    c.sc = *reinterpret_cast<const uint32_t *>(rec + 192 + 8 * hf + 4 * c.ch);
    c.d = reinterpret_cast<const uint16_t *>(aux)[blk];
    return c;
  }
  __device__ static void decode(const Chunk &c, int, bf16x8 (&b)[4], float (&d)[4], float (&mn)[4]) {
    const int sh = 4 * c.ch;
    const uint32_t hl0 = c.h0 >> sh, hl1 = c.h1 >> sh;
    b[0] = codes_b(((c.l0 >> sh) & 0x0F0F0F0Fu) | ((hl0 & 0x03030303u) << 4));
    b[1] = codes_b(((c.l1 >> sh) & 0x0F0F0F0Fu) | ((hl1 & 0x03030303u) << 4));
    b[2] = codes_b(((c.l2 >> sh) & 0x0F0F0F0Fu) | ((hl0 & 0x0C0C0C0Cu) << 2));
    b[3] = codes_b(((c.l3 >> sh) & 0x0F0F0F0Fu) | ((hl1 & 0x0C0C0C0Cu) << 2));
    const float dd = h2f(c.d);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      d[r] = dd * (float)(int8_t)((c.sc >> (8 * r)) & 0xFFu);
      mn[r] = 160.0f * d[r];
    }
  }
};

// Q8_0 (dequant.rs:40-47) on the split layout (int8 quants in element
// order, f16 d per 32 in the aux array): runs 0, 1 are block 2t, runs 2, 3
// block 2t + 1; int8 codes are exact in bf16 and there is no min term.
struct CdQ8 {
  static constexpr bool PAIR = true, MIN = false;
  struct Chunk {
    uint32_t q[4], d;
  };
  __device__ static Chunk load(const uint8_t *w, const uint8_t *aux, int64_t row, int64_t k, int64_t t, int g) {
    const uint64_t e = (uint64_t)row * (uint64_t)k + 64u * (uint64_t)t;
    Chunk c;
#pragma unroll
    for (int r = 0; r < 4; ++r) c.q[r] = *reinterpret_cast<const uint32_t *>(w + e + 16 * r + 4 * g);
    c.d = *reinterpret_cast<const uint32_t *>(aux + 2 * (e >> 5));
    return c;
  }
  __device__ static void decode(const Chunk &c, int, bf16x8 (&b)[4], float (&d)[4], float (&mn)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) b[r] = codes_b_i8(c.q[r]);
    d[0] = d[1] = h2f(c.d);
    d[2] = d[3] = h2f(c.d >> 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) mn[r] = 0.0f;
  }
};

// ---- activations ----------------------------------------------------------
//
// The A fragment of run r: four f32 activations split into hi / lo bf16
// limbs, hi limbs in slots 0..3 and lo limbs in 4..7.
__device__ __forceinline__ bf16x8 x_frag(const u32x4 &v) {
  uint32_t h0, l0, h1, l1;
  limbs2(__uint_as_float(v.x), __uint_as_float(v.y), h0, l0);
  limbs2(__uint_as_float(v.z), __uint_as_float(v.w), h1, l1);
  return pick(h0, h1, l0, l1);
}

// A chunk's activations for every column tile: raw f32 from global memory
// (xr: byte address of element 4g of chunk 0 in the lane's row of each
// column tile), or limb fragments from the LDS slice.
template <int MT>
struct CxRaw {
  u32x4 v[MT][4];
};
template <int MT>
struct CxFrag {
  bf16x8 a[MT][4];
};

template <int MT>
__device__ __forceinline__ void cx_load(CxRaw<MT> &f, const uint8_t *const (&xr)[MT], int64_t t) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) f.v[ct][r] = *reinterpret_cast<const u32x4 *>(xr[ct] + 256 * t + 64 * r);
}

template <int MT>
__device__ __forceinline__ void cx_split(const CxRaw<MT> &raw, CxFrag<MT> &f) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) f.a[ct][r] = x_frag(raw.v[ct][r]);
}

// The LDS slice holds every 4-element piece of f32 activations as its 16-byte
// limb fragment (hi 0..3, lo 0..3) at the piece's own offset (4 bytes an
// element); xs_row[ct]: the lane's row at its lane group's piece.
template <int MT>
__device__ __forceinline__ void cx_lds(CxFrag<MT> &f, const uint8_t *const (&xs_row)[MT], int64_t tl) {
#pragma unroll
  for (int ct = 0; ct < MT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) f.a[ct][r] = __builtin_bit_cast(bf16x8, ds_read16(xs_row[ct] + 256 * tl + 64 * r));
}

// The staged copy: 16-byte pieces of f32 activations, each written as its
// limb fragment, then the workgroup barrier.
template <int NT, int XR>
__device__ __forceinline__ void cx_stage(uint8_t *xs, u32x4 (&v)[XR], const XStage &st) {
  auto put = [&](int base) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
      int r, c;
      st.at(base + i * NT + (int)threadIdx.x, r, c);
      ds_write16(xs + r * st.xstr + 16 * c, __builtin_bit_cast(u32x4, x_frag(v[i])));
    }
  };
  put(0);
  for (int base = XR * NT; base < st.total; base += XR * NT) {
    xs_load<NT, XR>(v, st, base);
    put(base);
  }
  __syncthreads();
}

// One chunk of RT row tiles on MT column tiles: X = ones (per column tile and
// run, shared by the row tiles), S = codes; the lane's outputs += D S - M' X
// per run (or per run pair).  live false (a chunk past the end of the slice,
// loaded from a valid place) zeroes the scales, so it adds nothing.
template <class C, int MT, int RT>
__device__ __forceinline__ void codes_chunk(const typename C::Chunk (&c)[RT], const CxFrag<MT> &xf,
                                            f32x4 (&acc)[RT][MT], int g, bool live) {
  const bf16x8 ones = __builtin_bit_cast(bf16x8, (u32x4){0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int G = C::PAIR ? 2 : 1;  // runs sharing a scale
  f32x4 X[MT][4 / G];
  if constexpr (C::MIN) {
#pragma unroll
    for (int ct = 0; ct < MT; ++ct)
#pragma unroll
      for (int r0 = 0; r0 < 4; r0 += G) {
        X[ct][r0 / G] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.a[ct][r0], ones, zero, 0, 0, 0);
        if (G == 2)
          X[ct][r0 / G] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.a[ct][r0 + 1], ones, X[ct][r0 / G], 0, 0, 0);
      }
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    bf16x8 b[4];
    float d[4], mn[4];
    C::decode(c[rt], g, b, d, mn);
    if (!live) {
#pragma unroll
      for (int r = 0; r < 4; ++r) d[r] = mn[r] = 0.0f;
    }
#pragma unroll
    for (int r0 = 0; r0 < 4; r0 += G) {
#pragma unroll
      for (int ct = 0; ct < MT; ++ct) {
        f32x4 S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.a[ct][r0], b[r0], zero, 0, 0, 0);
        if (G == 2) S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.a[ct][r0 + 1], b[r0 + 1], S, 0, 0, 0);
        if constexpr (C::MIN) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[rt][ct][i] = fmaf(d[r0], S[i], fmaf(-mn[r0], X[ct][r0 / G][i], acc[rt][ct][i]));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[rt][ct][i] = fmaf(d[r0], S[i], acc[rt][ct][i]);
        }
      }
    }
  }
}

// Output slot q = (rt MT + ct) 64 + l of a workgroup: activation rows
// 16 ct + 4 (l / 16) + i, weight row n0 + 16 rt + l % 16.
template <int MT>
__device__ __forceinline__ void codes_store(float v, int q, int i, int64_t m, int64_t n, int64_t n0, const Out &o) {
  const int l = q & 63, ct = (q >> 6) % MT, rt = (q >> 6) / MT;
  const int64_t wr = n0 + 16 * rt + (l & 15), ar = 16 * ct + 4 * (l >> 4) + i;
  if (wr < n && ar < m) store_linear(o, ar, n, wr, v);
}

// The tiles of one workgroup: RT row tiles of 16 weight rows from tile
// group tg, K slice s of S, NW waves; xs / xstr: the LDS slice with XL.
template <class C, int MT, int NW, int B, int RT, bool XL>
__device__ __forceinline__ void codes_tiles(const uint8_t *__restrict__ w, const uint8_t *__restrict__ aux,
                                            const float *__restrict__ x, int64_t m, const Out &o, int64_t n,
                                            int64_t k, int64_t tg, int S, int s, f32x4 *__restrict__ wsp,
                                            uint32_t *__restrict__ cnt, f32x4 (&part)[NW][RT * MT * 64],
                                            uint8_t *xs, int xstr) {
  constexpr int NSLOT = RT * MT * 64;
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n0 = tg * 16 * RT;
  int64_t row[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int64_t r = n0 + 16 * rt + (lane & 15);
    row[rt] = r < n ? r : n - 1;
  }
  const int64_t nk = k / 64, cps = (nk + S - 1) / S;
  const int64_t lo = s * cps, hi = lo + cps < nk ? lo + cps : nk;
  typedef typename std::conditional<XL, CxFrag<MT>, CxRaw<MT>>::type XF;

  f32x4 acc[RT][MT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < MT; ++ct) acc[rt][ct] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  // The lane's activation row in each column tile (rows past m read row m - 1;
  // their outputs are not stored), at its lane group's element 4g.
  const uint8_t *xr[MT];
  const uint8_t *xsr[MT];
#pragma unroll
  for (int ct = 0; ct < MT; ++ct) {
    const int64_t mr = 16 * ct + (lane & 15) < m ? 16 * ct + (lane & 15) : m - 1;
    xr[ct] = reinterpret_cast<const uint8_t *>(x + mr * k + 4 * g);
    xsr[ct] = XL ? xs + mr * xstr + 16 * g : nullptr;
  }

  auto load_batch = [&](int64_t t, typename C::Chunk (&c)[B][RT], XF (&xf)[B]) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int64_t ti = t + i * NW < hi ? t + i * NW : (t < hi ? t : lo);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) c[i][rt] = C::load(w, aux, row[rt], k, ti, g);
      if constexpr (!XL) cx_load<MT>(xf[i], xr, ti);
    }
  };
  auto run_batch = [&](int64_t t, const typename C::Chunk (&c)[B][RT], XF (&xf)[B]) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int64_t ti = t + i * NW < hi ? t + i * NW : (t < hi ? t : lo);
      CxFrag<MT> f;
      if constexpr (XL) cx_lds<MT>(f, xsr, ti - lo);
      else cx_split<MT>(xf[i], f);
      codes_chunk<C, MT, RT>(c[i], f, acc, g, t + i * NW < hi);
    }
  };

  if (lo < hi) {
    const int64_t t0 = lo + wave;
    if constexpr (XL) {
      constexpr int NT = 64 * NW, XR = 8;
      const XStage st = make_stage(reinterpret_cast<const uint8_t *>(x + lo * 64), 4 * k, m, 4 * (hi - lo) * 64, xstr);
      u32x4 v[XR];
      xs_load<NT, XR>(v, st, 0);
      __builtin_amdgcn_sched_barrier(0);  // the copy's loads first: its wait then skips the weights
      typename C::Chunk c0[B][RT];
      XF xf0[B];
      load_batch(t0, c0, xf0);
      __builtin_amdgcn_sched_barrier(0);
      cx_stage<NT, XR>(xs, v, st);
      run_batch(t0, c0, xf0);
      for (int64_t t = t0 + B * NW; t < hi; t += B * NW) {
        typename C::Chunk c[B][RT];
        XF xf[B];
        load_batch(t, c, xf);
        __builtin_amdgcn_sched_barrier(0);
        run_batch(t, c, xf);
      }
    } else {
      for (int64_t t = t0; t < hi; t += B * NW) {
        typename C::Chunk c[B][RT];
        XF xf[B];
        load_batch(t, c, xf);
        __builtin_amdgcn_sched_barrier(0);
        run_batch(t, c, xf);
      }
    }
  }

#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < MT; ++ct) part[wave][(rt * MT + ct) * 64 + lane] = acc[rt][ct];
  __syncthreads();
  if (S > 1) {
    auto sum = [&](int q) {
      f32x4 v = part[0][q];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) v += part[w2][q];
      return v;
    };
    auto put = [&](int q, const f32x4 &v) {
#pragma unroll
      for (int i = 0; i < 4; ++i) codes_store<MT>(v[i], q, i, m, n, n0, o);
    };
    split_finish<NSLOT, 64 * NW>(sum, put, S, s, wsp, cnt);
    return;
  }
  // The waves' partials summed one float a thread (in wave order), every
  // thread of the workgroup taking part: all NW reads issued at once.
  const float *pf = reinterpret_cast<const float *>(&part[0][0]);
  for (int f = threadIdx.x; f < NSLOT * 4; f += 64 * NW) {
    float p[NW];
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) p[w2] = pf[w2 * NSLOT * 4 + f];
    float v = p[0];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) v += p[w2];
    codes_store<MT>(v, f >> 2, f & 3, m, n, n0, o);
  }
}

template <class C, int MT, int NW, int B, int RT, bool XL>
__global__ __launch_bounds__(64 * NW) void k_smallm_codes(const uint8_t *__restrict__ w,
                                                          const uint8_t *__restrict__ aux,
                                                          const float *__restrict__ x, int64_t m, const Out o,
                                                          int64_t n, int64_t k, int S, f32x4 *__restrict__ wsp,
                                                          uint32_t *__restrict__ cnt, int xstr) {
  __shared__ f32x4 part[NW][RT * MT * 64];
  extern __shared__ __attribute__((aligned(16))) uint8_t xs_dyn[];
  const int bid = split_order((int)blockIdx.x, (int)gridDim.x, S);
  const int64_t tg = bid / S;
  codes_tiles<C, MT, NW, B, RT, XL>(w, aux, x, m, o, n, k, tg, S, bid % S, wsp + tg * S * RT * MT * 64, cnt + tg,
                                    part, xs_dyn, xstr);
}

template <class C, int MT, int NW, int B, int RT, bool XL>
__global__ __launch_bounds__(64 * NW) void k_smallm_codes_set(const WeightSet set, const float *__restrict__ x,
                                                              int64_t m, int64_t k, int S, f32x4 *__restrict__ wsp,
                                                              uint32_t *__restrict__ cnt, int xstr) {
  __shared__ f32x4 part[NW][RT * MT * 64];
  extern __shared__ __attribute__((aligned(16))) uint8_t xs_dyn[];
  const int bid = split_order((int)blockIdx.x, (int)gridDim.x, S);
  const SetEntry e = pick_entry(set, bid);
  const int gt = bid / S;
  codes_tiles<C, MT, NW, B, RT, XL>(e.w, e.aux, x, m, e.o, e.n, k, (bid - e.g0) / S, S, bid % S,
                                    wsp + (int64_t)gt * S * RT * MT * 64, cnt + gt, part, xs_dyn, xstr);
}

// Tile groups (RT row tiles each) of a weight.
template <int RT>
int64_t tile_groups(const rq_weight *w) {
  return ((w->n + 15) / 16 + RT - 1) / RT;
}

template <class C, int MT, int NW, int B, int RT, bool XL>
int codes_launch(const rq_weight *const *w, int count, bool set, const float *x, int64_t m, const Out *o, int S,
                 f32x4 *wsp, uint32_t *cnt, hipStream_t s, int xstr, size_t xbytes) {
  if (XL && (size_t)NW * RT * MT * 64 * sizeof(f32x4) + xbytes > 160 * 1024) return RQ_E_UNSUPPORTED;
  if (!set) {
    const rq_weight *wt = w[0];
    if (!lds_allow<&k_smallm_codes<C, MT, NW, B, RT, XL>>(xbytes)) return RQ_E_UNSUPPORTED;
    hipLaunchKernelGGL((k_smallm_codes<C, MT, NW, B, RT, XL>), dim3((unsigned)(tile_groups<RT>(wt) * S)),
                       dim3(64 * NW), xbytes, s, wt->data, wt->data + wt->aux_off, x, m, o[0], wt->n, wt->k, S, wsp,
                       cnt, xstr);
  } else {
    WeightSet ws;
    int64_t total = 0;
    const int rc = fill_set(ws, w, count, o, [&](const rq_weight *wj) { return tile_groups<RT>(wj) * S; }, &total);
    if (rc) return rc;
    if (!lds_allow<&k_smallm_codes_set<C, MT, NW, B, RT, XL>>(xbytes)) return RQ_E_UNSUPPORTED;
    hipLaunchKernelGGL((k_smallm_codes_set<C, MT, NW, B, RT, XL>), dim3((unsigned)total), dim3(64 * NW), xbytes, s,
                       ws, x, m, w[0]->k, S, wsp, cnt, xstr);
  }
  return hipGetLastError() == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "small-M codes launch failed");
}

// Plan: K split over S workgroups (up to 4) where few row tiles leave CUs idle
// and there are 16 or more rows (or long rows); eight waves, one chunk a
// batch; two row tiles a workgroup from 256 workgroups (a launch that would
// fill the CUs more than once, or nearly); the activation slice in LDS from
// 16 rows when it fits.  Graph-timed, 32 distinct Q4_K copies of the 0.5B
// layer, us a launch, against the f32 matrix-core kernel (one weight) and the
// two-limb set kernel (q/k/v, gate/up) -> this kernel:
//   M = 4:  gate/up set 9.2 -> 7.1, q/k/v set 4.9 -> 3.9, o 4.5 -> 3.6,
//           down 9.3 -> 7.5, gate 6.8 -> 4.7
//   M = 16: gate/up set 10.7 -> 7.7, q/k/v set 5.5 -> 4.2, o 4.9 -> 3.9,
//           down 10.2 -> 8.6, gate 7.1 -> 5.2
//   M = 32: down 16.9 -> 10.9, gate 9.5 -> 7.0, q/k/v set 7.3 -> 5.8, gate/up
//           set 11.8 -> 12.1, but o 4.8 -> 5.6
//   M = 64: gate/up set 27.5 -> 22.9, gate 13.7 -> 12.6, but o 5.0 -> 10.2,
//           q/k/v set 9.8 -> 10.5, down 15.0 -> 15.3
// Four waves with batches of two or four chunks, sixteen waves and other K
// splits were slower; two row tiles on the 56- and 72-tile launches lost
// 10-25%.  So this kernel takes 4 <= m <= 16; 17..32 rows on rows longer
// than 2048 elements, on 256 or more row tiles and for sets; 33..64 rows on
// 256 or more row tiles; the rest stay on the other kernels.
template <class C, int MT, int RT>
int codes_go(const rq_weight *const *w, int count, bool set, const float *x, int64_t m, const Out *o, hipStream_t s,
             WsLease *ws, int S) {
  int64_t groups = 0;
  for (int j = 0; j < count; ++j) groups += tile_groups<RT>(w[j]);
  f32x4 *wsp = nullptr;
  uint32_t *cnt = nullptr;
  if (S > 1) {
    int rc = RQ_OK;
    cnt = groups <= WsLease::kCounters ? ws->counters() : nullptr;
    wsp = cnt ? static_cast<f32x4 *>(ws->get((size_t)groups * S * RT * MT * 64 * sizeof(f32x4), &rc, true))
              : nullptr;
    if (!wsp) S = 1;
  }
  const int64_t nk = w[0]->k / 64, cps = (nk + S - 1) / S;
  const int xstr = (int)(cps * 64 * 4 + 16);
  const size_t xbytes = (size_t)m * (size_t)xstr;
  const bool xl = m >= 16 && cps * 64 <= 2048 && xbytes <= kSmXsMax;
  if (xl) {
    const int rc = codes_launch<C, MT, 8, 1, RT, true>(w, count, set, x, m, o, S, wsp, cnt, s, xstr, xbytes);
    if (rc != RQ_E_UNSUPPORTED) return rc;
  }
  return codes_launch<C, MT, 8, 1, RT, false>(w, count, set, x, m, o, S, wsp, cnt, s, 0, 0);
}

template <class C, int MT>
int codes_plan(const rq_weight *const *w, int count, bool set, const float *x, int64_t m, const Out *o,
               hipStream_t s, WsLease *ws) {
  int64_t tiles = 0;
  for (int j = 0; j < count; ++j) tiles += (w[j]->n + 15) / 16;
  const int64_t nk = w[0]->k / 64;
  int S = 1;
  if (ws != nullptr && tiles <= WsLease::kCounters && tiles < 128 && !(w[0]->k <= 1024 && m <= 64) &&
      (m >= 16 || nk > 32))
    while (S < 4 && tiles * S * 2 <= 512 && nk >= 4 * S) S *= 2;
  const int rt = tiles * S >= 256 ? 2 : 1;
  if (rt == 2) return codes_go<C, MT, 2>(w, count, set, x, m, o, s, ws, S);
  return codes_go<C, MT, 1>(w, count, set, x, m, o, s, ws, S);
}

template <class C>
int codes_run(const rq_weight *const *w, int count, bool set, const float *x, int64_t m, const Out *o, hipStream_t s,
              WsLease *ws) {
  if (m <= 16) return codes_plan<C, 1>(w, count, set, x, m, o, s, ws);
  int64_t tiles = 0;
  for (int j = 0; j < count; ++j) tiles += (w[j]->n + 15) / 16;
  if (m <= 32 && (w[0]->k > 2048 || tiles >= 256 || set)) return codes_plan<C, 2>(w, count, set, x, m, o, s, ws);
  if (m > 32 && tiles >= 256) return codes_plan<C, 4>(w, count, set, x, m, o, s, ws);
  return RQ_E_UNSUPPORTED;
}

}  // namespace

// f32 activations, 4 <= m <= 64 where the plan above takes them, k % 64 ==
// 0, 16-byte aligned x, one weight or a set of one format and k: Q4_K, Q6_K
// and Q8_0 (RQ_E_UNSUPPORTED otherwise: the two-limb or f32 kernels take
// those).
int launch_linear_smallm_codes(const rq_weight *const *w, int count, bool set, const void *x, int64_t m,
                               const Out *o, hipStream_t s, WsLease *ws) {
  const int64_t k = w[0]->k;
  if (m < 4 || m > 64 || k % 64 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return RQ_E_UNSUPPORTED;
  for (int j = 1; j < count; ++j)
    if (w[j]->qtype != w[0]->qtype || w[j]->k != k) return RQ_E_UNSUPPORTED;
  const float *xf = static_cast<const float *>(x);
  switch (w[0]->qtype) {
    case RQ_Q4_K: return codes_run<CdQ4K>(w, count, set, xf, m, o, s, ws);
    case RQ_Q6_K: return codes_run<CdQ6K>(w, count, set, xf, m, o, s, ws);
    case RQ_Q8_0: return codes_run<CdQ8>(w, count, set, xf, m, o, s, ws);
    default: return RQ_E_UNSUPPORTED;
  }
}

}  // namespace rq
