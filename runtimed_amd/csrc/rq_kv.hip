// rq_kv.hip -- paged-KV block quantizer on gfx950
// (crates/runtimed-model/src/cache/paged/quantize.rs).
//
// A K or V chunk is viewed as [b, h, sd] (sd = tokens * head_dim,
// quantize.rs:14-18).  FP8 and INT8 modes use one scale per head h over all
// b slabs: s[h] = max(max|t[:, h, :]| / D, 1e-8) with D = 448 (FP8) or 127
// (INT8); codes are f32_to_fp8_e4m3(t / s[h]) (the reference's encoder,
// ties to the lower magnitude) or (i8)clamp(round(t / s[h]), -128, 127).
// The reference runs both passes on the host after a device-to-host copy;
// here they are two stream-ordered kernels:
//   k_kv_absmax  grid (P, h): partial maxima of P ranges of each head;
//   k_kv_encode  grid (X, slabs): every workgroup folds its head's P partials
//                into s[h] (the batch-0 workgroup at x = 0 stores it), then
//                encodes its range.
// F16 mode is the attention-sink branch of quantize_block_kv
// (quantize.rs:109-122): a plain cast with every scale 1.
// Bound: HBM; per element 2-4 bytes read twice (max pass + encode pass), 1
// (FP8 / INT8) or 2 (F16) bytes written.
#include "rq_e4m3.h"
#include "rq_epilogue.h"
#include "rq_internal.h"

namespace rq {
namespace {

constexpr int KV_THREADS = 256;
constexpr int KV_MAX_PARTS = 256;
constexpr int64_t KV_MAX_SLABS_Y = 65535;

// Four elements at i (i % 4 == 0, 16-byte aligned data) as f32: the type a
// template parameter (TT < 0: the run-time ttype), so that a batch of loads
// is not split across type branches.
template <int TT>
__device__ __forceinline__ float4 ld4t(const void *t, int ttype, int64_t i) {
  if constexpr (TT < 0) {
    return load_x4(t, ttype, i);
  } else if constexpr (TT == RQ_F32) {
    return *reinterpret_cast<const float4 *>(static_cast<const float *>(t) + i);
  } else {
    const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(t) + i);
    if constexpr (TT == RQ_BF16)
      return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y << 16),
                         __uint_as_float(v.y & 0xFFFF0000u));
    else
      return make_float4((float)__builtin_bit_cast(_Float16, (uint16_t)(v.x & 0xFFFFu)),
                         (float)__builtin_bit_cast(_Float16, (uint16_t)(v.x >> 16)),
                         (float)__builtin_bit_cast(_Float16, (uint16_t)(v.y & 0xFFFFu)),
                         (float)__builtin_bit_cast(_Float16, (uint16_t)(v.y >> 16)));
  }
}

// Loads a thread issues together in the vector loops (one load per loop
// iteration waited for each load in turn).
constexpr int KV_U = 4;

// Elements of one 16-byte load: 4 f32 or 8 16-bit values.
template <int TT>
constexpr int kv_epl() {
  return TT == RQ_F32 ? 4 : 8;
}

// kv_epl<TT>() elements at i (a multiple of that count, 16-byte aligned data)
// as f32, from one 16-byte load.
template <int TT>
__device__ __forceinline__ void ld16(const void *t, int64_t i, float (&f)[8]) {
  if constexpr (TT == RQ_F32) {
    const float4 v = *reinterpret_cast<const float4 *>(static_cast<const float *>(t) + i);
    f[0] = v.x, f[1] = v.y, f[2] = v.z, f[3] = v.w;
  } else {
    const uint4 v = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(t) + i);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (TT == RQ_BF16) {
        f[2 * j] = __uint_as_float(w[j] << 16);
        f[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
      } else {
        f[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] & 0xFFFFu));
        f[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] >> 16));
      }
    }
  }
}

__device__ __forceinline__ float block_max(float v, float *red) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Partial max|t| of elements [p * chunk, (p+1) * chunk) of head hh's b * sd
// elements (slab-major).  NaN elements are skipped, as the reference's
// `a > max_abs` test skips them.  VEC: sd and chunk are multiples of the
// elements of a 16-byte load (4 f32, 8 16-bit) and t is 16-byte aligned, so
// each lane loads 16 bytes at once.
template <bool VEC, int TT>
__global__ __launch_bounds__(KV_THREADS) void k_kv_absmax(const void *__restrict__ t, int ttype, int64_t b,
                                                          int64_t h, int64_t sd, int64_t chunk,
                                                          float *__restrict__ part) {
  __shared__ float red[4];
  const int p = blockIdx.x, P = gridDim.x;
  const int64_t hh = blockIdx.y;
  const int64_t e0 = p * chunk;
  const int64_t e1 = e0 + chunk < b * sd ? e0 + chunk : b * sd;
  float mx = 0.0f;
  for (int64_t bb = e0 / sd; bb < b && bb * sd < e1; ++bb) {
    const int64_t lo = (e0 > bb * sd ? e0 : bb * sd) - bb * sd;
    const int64_t hi = (e1 < (bb + 1) * sd ? e1 : (bb + 1) * sd) - bb * sd;
    const int64_t base = (bb * h + hh) * sd;
    if constexpr (VEC) {
      constexpr int E = kv_epl<TT>();
      for (int64_t i0 = lo + E * threadIdx.x; i0 < hi; i0 += E * KV_THREADS * KV_U) {
        float v[KV_U][8];
#pragma unroll
        for (int u = 0; u < KV_U; ++u) {
          const int64_t i = i0 + E * KV_THREADS * u;
          ld16<TT>(t, base + (i < hi ? i : i0), v[u]);  // past the range: a repeat, not counted
        }
#pragma unroll
        for (int u = 0; u < KV_U; ++u) {
          if (i0 + E * KV_THREADS * u >= hi) break;
#pragma unroll
          for (int j = 0; j < E; ++j) {
            const float a = fabsf(v[u][j]);
            if (a > mx) mx = a;
          }
        }
      }
    } else {
      for (int64_t i = lo + threadIdx.x; i < hi; i += KV_THREADS) {
        const float a = fabsf(load_x1(t, ttype, base + i));
        if (a > mx) mx = a;
      }
    }
  }
  mx = block_max(mx, red);
  if (threadIdx.x == 0) part[hh * P + p] = mx;
}

__device__ __forceinline__ uint32_t encode_int8(float v) {
  const float r = roundf(v);
  if (r != r) return 0u;
  return (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(r, -128.0f), 127.0f);
}

template <int MODE>
__device__ __forceinline__ uint32_t encode_one(float v, float sc) {
  return MODE == RQ_KV_FP8 ? enc_e4m3_ref(v / sc) : encode_int8(v / sc);
}

// Encode slab `slab` (= batch * h + head), elements [x0, x1) of it.  VEC:
// sd and per_block are multiples of the elements of a 16-byte load (4 f32,
// 8 16-bit), t is 16-byte and q 8-byte aligned.
template <int MODE, bool VEC, int TT>
__global__ __launch_bounds__(KV_THREADS) void k_kv_encode(const void *__restrict__ t, int ttype, int64_t b,
                                                          int64_t h, int64_t sd, const float *__restrict__ part,
                                                          int P, int64_t per_block, void *__restrict__ q,
                                                          float *__restrict__ scales) {
  __shared__ float red[4];
  const int64_t x0 = (int64_t)blockIdx.x * per_block;
  const int64_t x1 = x0 + per_block < sd ? x0 + per_block : sd;
  for (int64_t slab = blockIdx.y; slab < b * h; slab += gridDim.y) {
    const int64_t hh = slab % h;
    const int64_t base = slab * sd;
    if (MODE == RQ_KV_F16) {
      if (blockIdx.x == 0 && slab < h && threadIdx.x == 0) scales[hh] = 1.0f;
      _Float16 *o = static_cast<_Float16 *>(q);
      if (VEC) {
        for (int64_t i = x0 + 4 * threadIdx.x; i < x1; i += 4 * KV_THREADS) {
          const float4 v = ld4t<TT>(t, ttype, base + i);
          *reinterpret_cast<uint2 *>(o + base + i) = make_uint2(pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w));
        }
      } else {
        for (int64_t i = x0 + threadIdx.x; i < x1; i += KV_THREADS) o[base + i] = (_Float16)load_x1(t, ttype, base + i);
      }
      continue;
    }
    uint8_t *o = static_cast<uint8_t *>(q);
    if constexpr (VEC) {
      // The first batch of elements is loaded before the head's partial
      // maxima are read and folded (it does not depend on them), so the two
      // reads overlap instead of following each other.
      constexpr int E = kv_epl<TT>();
      const int64_t i00 = x0 + E * threadIdx.x;
      const int64_t ic = i00 < x1 ? i00 : x0;
      float v[KV_U][8];
#pragma unroll
      for (int u = 0; u < KV_U; ++u) {
        const int64_t i = i00 + E * KV_THREADS * u;
        ld16<TT>(t, base + (i < x1 ? i : ic), v[u]);
      }
      float mx = threadIdx.x < P ? part[hh * P + threadIdx.x] : 0.0f;
      mx = block_max(mx, red);
      __syncthreads();  // red is reused by the next slab
      const float sc = fmaxf(mx / (MODE == RQ_KV_FP8 ? 448.0f : 127.0f), 1e-8f);
      if (blockIdx.x == 0 && slab < h && threadIdx.x == 0) scales[hh] = sc;
      auto put = [&](int64_t i, const float (&f)[8]) {
        uint32_t c[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < E; ++j) c[j >> 2] |= encode_one<MODE>(f[j], sc) << (8 * (j & 3));
        if constexpr (E == 8) *reinterpret_cast<uint2 *>(o + base + i) = make_uint2(c[0], c[1]);
        else *reinterpret_cast<uint32_t *>(o + base + i) = c[0];
      };
#pragma unroll
      for (int u = 0; u < KV_U; ++u) {
        const int64_t i = i00 + E * KV_THREADS * u;
        if (i < x1) put(i, v[u]);
      }
      for (int64_t i0 = i00 + E * KV_THREADS * KV_U; i0 < x1; i0 += E * KV_THREADS * KV_U) {
#pragma unroll
        for (int u = 0; u < KV_U; ++u) {
          const int64_t i = i0 + E * KV_THREADS * u;
          ld16<TT>(t, base + (i < x1 ? i : i0), v[u]);
        }
#pragma unroll
        for (int u = 0; u < KV_U; ++u) {
          const int64_t i = i0 + E * KV_THREADS * u;
          if (i < x1) put(i, v[u]);
        }
      }
      continue;
    }
    float mx = threadIdx.x < P ? part[hh * P + threadIdx.x] : 0.0f;
    mx = block_max(mx, red);
    __syncthreads();  // red is reused by the next slab
    const float sc = fmaxf(mx / (MODE == RQ_KV_FP8 ? 448.0f : 127.0f), 1e-8f);
    if (blockIdx.x == 0 && slab < h && threadIdx.x == 0) scales[hh] = sc;
    {
      for (int64_t i = x0 + threadIdx.x; i < x1; i += KV_THREADS)
        o[base + i] = (uint8_t)encode_one<MODE>(load_x1(t, ttype, base + i), sc);
    }
  }
}

template <int MODE>
__device__ __forceinline__ float decode_one(uint32_t c) {
  return MODE == RQ_KV_FP8 ? dec_e4m3(c & 0xFFu) : (float)(int8_t)(c & 0xFFu);
}

// dequantize_fp8 / dequantize_int8 (quantize.rs:48-57, 98-107) and the F16
// cast of QuantizedCacheBlock::dequantize_k (block.rs:98-104).  VEC: sd and
// per_block are multiples of 4, q is 8-byte and out 16-byte aligned.
template <int MODE, bool VEC>
__global__ __launch_bounds__(KV_THREADS) void k_kv_decode(const void *__restrict__ q, const float *__restrict__ scales,
                                                          int64_t b, int64_t h, int64_t sd, int64_t per_block,
                                                          void *__restrict__ out, int otype) {
  const int64_t x0 = (int64_t)blockIdx.x * per_block;
  const int64_t x1 = x0 + per_block < sd ? x0 + per_block : sd;
  for (int64_t slab = blockIdx.y; slab < b * h; slab += gridDim.y) {
    const int64_t base = slab * sd;
    const float sc = MODE == RQ_KV_F16 ? 1.0f : scales[slab % h];
    if (VEC) {
      for (int64_t i = x0 + 4 * threadIdx.x; i < x1; i += 4 * KV_THREADS) {
        if (MODE == RQ_KV_F16) {
          const float4 v = load_x4(q, RQ_F16, base + i);
          store_four(out, otype, base + i, v.x, v.y, v.z, v.w);
        } else {
          const uint32_t c = *reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(q) + base + i);
          store_four(out, otype, base + i, decode_one<MODE>(c) * sc, decode_one<MODE>(c >> 8) * sc,
                     decode_one<MODE>(c >> 16) * sc, decode_one<MODE>(c >> 24) * sc);
        }
      }
    } else {
      for (int64_t i = x0 + threadIdx.x; i < x1; i += KV_THREADS) {
        if (MODE == RQ_KV_F16) {
          store_out(out, otype, base + i, (float)static_cast<const _Float16 *>(q)[base + i]);
        } else {
          const uint8_t c = static_cast<const uint8_t *>(q)[base + i];
          store_out(out, otype, base + i, decode_one<MODE>(c) * sc);
        }
      }
    }
  }
}

// Every head's scale set to one value (the floor of a head with no
// elements).  A kernel, not a copy from host memory, so that a caller may
// capture it in a graph.
__global__ __launch_bounds__(256) void k_kv_fill_scales(float *__restrict__ scales, int64_t h, float v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < h) scales[i] = v;
}

int last_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "%s launch: %s", what, hipGetErrorString(e));
}

// Elements per workgroup along one slab: at least 4096 (a multiple of 8),
// and at most 1024 workgroups across a slab.
int64_t slab_split(int64_t sd, int64_t *blocks) {
  int64_t per = 4096;
  if ((sd + per - 1) / per > 1024) per = ((sd + 1023) / 1024 + 7) & ~(int64_t)7;
  *blocks = (sd + per - 1) / per;
  return per;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

template <int MODE>
void launch_encode(bool vec, dim3 grid, hipStream_t s, const void *t, int ttype, int64_t b, int64_t h, int64_t sd,
                   const float *part, int P, int64_t per, void *q, float *scales) {
#define RQ_KVE(V, TT) \
  hipLaunchKernelGGL((k_kv_encode<MODE, V, TT>), grid, dim3(KV_THREADS), 0, s, t, ttype, b, h, sd, part, P, per, q, scales)
  if (!vec) RQ_KVE(false, -1);
  else if (ttype == RQ_F32) RQ_KVE(true, RQ_F32);
  else if (ttype == RQ_BF16) RQ_KVE(true, RQ_BF16);
  else RQ_KVE(true, RQ_F16);
#undef RQ_KVE
}

template <int MODE>
void launch_decode(bool vec, dim3 grid, hipStream_t s, const void *q, const float *scales, int64_t b, int64_t h,
                   int64_t sd, int64_t per, void *out, int otype) {
  if (vec)
    hipLaunchKernelGGL((k_kv_decode<MODE, true>), grid, dim3(KV_THREADS), 0, s, q, scales, b, h, sd, per, out, otype);
  else
    hipLaunchKernelGGL((k_kv_decode<MODE, false>), grid, dim3(KV_THREADS), 0, s, q, scales, b, h, sd, per, out,
                       otype);
}

}  // namespace

int launch_kv_quantize(const void *t, int ttype, int64_t b, int64_t h, int64_t sd, int mode, void *q,
                       float *scales, hipStream_t s, WsLease &ws) {
  int64_t xb = 0;
  const int64_t per = slab_split(sd, &xb);
  const dim3 grid((unsigned)xb, (unsigned)(b * h < KV_MAX_SLABS_Y ? b * h : KV_MAX_SLABS_Y));
  // vector loads: 16 bytes of input (4 f32 or 8 16-bit elements) a lane
  const bool vec = sd % (ttype == RQ_F32 ? 4 : 8) == 0 && aligned(t, 16) && aligned(q, 8);
  if (mode == RQ_KV_F16) {
    launch_encode<RQ_KV_F16>(vec, grid, s, t, ttype, b, h, sd, nullptr, 0, per, q, scales);
    return last_launch("kv cast");
  }
  // Partial maxima: P ranges per head, each at least 4096 elements and a
  // multiple of 8 long.
  const int64_t per_head = b * sd;
  int64_t P = (per_head + 4095) / 4096;
  if (P > KV_MAX_PARTS) P = KV_MAX_PARTS;
  const int64_t chunk = ((per_head + P - 1) / P + 7) & ~(int64_t)7;
  int rc = RQ_OK;
  float *part = static_cast<float *>(ws.get((size_t)(h * P) * sizeof(float), &rc));
  if (!part) return rc;
  const dim3 pg((unsigned)P, (unsigned)h);
#define RQ_KVM(V, TT) hipLaunchKernelGGL((k_kv_absmax<V, TT>), pg, dim3(KV_THREADS), 0, s, t, ttype, b, h, sd, chunk, part)
  if (!vec) RQ_KVM(false, -1);
  else if (ttype == RQ_F32) RQ_KVM(true, RQ_F32);
  else if (ttype == RQ_BF16) RQ_KVM(true, RQ_BF16);
  else RQ_KVM(true, RQ_F16);
#undef RQ_KVM
  rc = last_launch("kv absmax");
  if (!rc) {
    if (mode == RQ_KV_FP8) launch_encode<RQ_KV_FP8>(vec, grid, s, t, ttype, b, h, sd, part, (int)P, per, q, scales);
    else launch_encode<RQ_KV_INT8>(vec, grid, s, t, ttype, b, h, sd, part, (int)P, per, q, scales);
    rc = last_launch("kv encode");
  }
  return rc;
}

int launch_kv_fill_scales(float *scales, int64_t h, float v, hipStream_t s) {
  hipLaunchKernelGGL(k_kv_fill_scales, dim3((unsigned)((h + 255) / 256)), dim3(256), 0, s, scales, h, v);
  return last_launch("kv scale fill");
}

int launch_kv_dequantize(const void *q, int mode, const float *scales, int64_t b, int64_t h, int64_t sd, void *out,
                         int otype, hipStream_t s) {
  int64_t xb = 0;
  const int64_t per = slab_split(sd, &xb);
  const dim3 grid((unsigned)xb, (unsigned)(b * h < KV_MAX_SLABS_Y ? b * h : KV_MAX_SLABS_Y));
  const bool vec = sd % 4 == 0 && aligned(q, 8) && aligned(out, 16);
  if (mode == RQ_KV_F16) launch_decode<RQ_KV_F16>(vec, grid, s, q, scales, b, h, sd, per, out, otype);
  else if (mode == RQ_KV_FP8) launch_decode<RQ_KV_FP8>(vec, grid, s, q, scales, b, h, sd, per, out, otype);
  else launch_decode<RQ_KV_INT8>(vec, grid, s, q, scales, b, h, sd, per, out, otype);
  return last_launch("kv decode");
}

}  // namespace rq
