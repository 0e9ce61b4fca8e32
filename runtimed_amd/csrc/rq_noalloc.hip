// rq_noalloc.hip -- the FP8 GEMM for callers that cannot allocate device
// memory (code under HIP graph capture that must not record allocation
// nodes, tight serving loops, harnesses that forbid hipMalloc).
//
// rq_fp8_gemm encodes its activations into scratch memory (e4m3 codes, m * k
// bytes, then m per-row scales) taken from the stream's workspace, which may
// grow -- an allocation.  rq_fp8_gemm_noalloc runs the same two kernels with
// that scratch in `scratch`, a fixed array of kNoAllocScratch bytes in the
// library's code object: each GPU the library runs on holds its own copy
// until the process ends.  Its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// handed to kernels: in host code the array's name is not a device address.
//
// Every call on a GPU shares that GPU's array: two calls that overlap on one
// GPU (different streams, or one stream's calls from several threads
// interleaved with a graph replay) race on it.  Nothing in it needs to start
// at zero: the encoder writes every code and scale the GEMM reads.
#include <mutex>

#include "rq_internal.h"

namespace rq {
namespace {

constexpr size_t kNoAllocScratch = RQ_NOALLOC_SCRATCH_BYTES;
static_assert(kNoAllocScratch % 256 == 0, "scratch is carved in 256-byte units");

__device__ __align__(256) uint8_t scratch[kNoAllocScratch];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint8_t *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on `device` (current), looked up on the
// first call there.
int scratch_on(int device, uint8_t **out) {
  if (device < 0 || device >= kMaxDevices) return set_error(RQ_E_DEVICE, "device %d out of range", device);
  std::lock_guard<std::mutex> g(g_mu);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(RQ_E_DEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g_scratch_ptr[device] = static_cast<uint8_t *>(p);
  }
  *out = g_scratch_ptr[device];
  return RQ_OK;
}

}  // namespace
}  // namespace rq

using namespace rq;

extern "C" int rq_fp8_gemm_noalloc(const void *x, int xtype, int64_t m, const uint8_t *w, const float *w_scale,
                                   int64_t n, int64_t k, void *y, int ytype, int mode, void *stream) {
  int rc = fp8_gemm_checks(xtype, m, n, k, ytype, mode);
  if (rc) return rc;
  if (m == 0) return RQ_OK;
  if (!x || !w || !y) return set_error(RQ_E_ARG, "null argument");
  const hipStream_t s = as_stream(stream);
  if (xtype == RQ_F8E4M3)  // codes as they are: no scratch
    return launch_fp8_gemm(static_cast<const uint8_t *>(x), nullptr, m, w, w_scale, n, k, y, ytype, s);
  const uint64_t qbytes = ((uint64_t)m * (uint64_t)k + 255) & ~(uint64_t)255;
  const uint64_t need = qbytes + (uint64_t)m * sizeof(float);
  if (need > kNoAllocScratch)
    return set_error(RQ_E_ARG, "rq_fp8_gemm_noalloc: m * k = %lld activations need %llu bytes of scratch, above "
                     "its fixed %llu (m * k rounded up to 256, plus 4 m)",
                     (long long)(m * k), (unsigned long long)need, (unsigned long long)kNoAllocScratch);
  int dev = 0;
  rc = hipGetDevice(&dev) == hipSuccess ? RQ_OK : set_error(RQ_E_DEVICE, "hipGetDevice failed");
  if (rc) return rc;
  uint8_t *base = nullptr;
  rc = scratch_on(dev, &base);
  if (rc) return rc;
  float *xs = reinterpret_cast<float *>(base + qbytes);
  rc = launch_fp8_quantize(x, xtype, m, k, mode, base, xs, s);
  if (!rc) rc = launch_fp8_gemm(base, xs, m, w, w_scale, n, k, y, ytype, s);
  return rc;
}
