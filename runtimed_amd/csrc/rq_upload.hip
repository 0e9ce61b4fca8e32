// rq_upload.hip -- host-to-device upload of GGUF block streams for
// rq_weight_create (the load path of load_gguf.rs:28-38, where the reference
// hands the mapped bytes to candle's qtensor_from_ggml).
//
// The source (typically a memory-mapped GGUF file) is copied in chunks into
// one of two pinned staging buffers, then DMA-ed to the device with
// hipMemcpyAsync while the host fills the other buffer.  Formats kept as
// the GGUF stream (Q4_K, Q5_K) land in place; for the split layouts (Q8_0,
// Q4_0, Q5_0, Q6_K; see rq_internal.h) the chunk lands in device staging
// memory and k_split_blocks scatters its blocks into the handle's quant and
// scale arrays.  The staging buffers are kept per device for the life of the
// process; uploads to one device are serialized by a mutex.
#include <string.h>

#include <mutex>
#include <thread>
#include <vector>

#include "rq_internal.h"

namespace rq {
namespace {

constexpr uint64_t kChunk = 64ull << 20;  // staging buffer size (bytes)

// One thread per block: copy block b of the GGUF stream (2-byte aligned,
// bbytes long) into the split layout.  16-bit loads and stores throughout.
__global__ __launch_bounds__(256) void k_split_blocks(int qtype, const uint16_t *__restrict__ src, uint64_t b0,
                                                      uint64_t nb, uint8_t *__restrict__ dst, uint64_t aux_off) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nb) return;
  const uint64_t b = b0 + i;
  if (qtype == RQ_Q8_0) {  // [d f16][32 int8] -> quants b*32, d at aux_off + b*2
    const uint16_t *s = src + i * 17;
    uint16_t *q = reinterpret_cast<uint16_t *>(dst + b * 32);
    for (int j = 0; j < 16; ++j) q[j] = s[1 + j];
    reinterpret_cast<uint16_t *>(dst + aux_off)[b] = s[0];
  } else if (qtype == RQ_Q4_0) {  // [d][16 qs] -> qs b*16, d at aux_off + b*2
    const uint16_t *s = src + i * 9;
    uint16_t *q = reinterpret_cast<uint16_t *>(dst + b * 16);
    for (int j = 0; j < 8; ++j) q[j] = s[1 + j];
    reinterpret_cast<uint16_t *>(dst + aux_off)[b] = s[0];
  } else if (qtype == RQ_Q5_0) {  // [d][qh 4][16 qs] -> qs b*16, {qh, d, 0} at aux_off + b*8
    const uint16_t *s = src + i * 11;
    uint16_t *q = reinterpret_cast<uint16_t *>(dst + b * 16);
    for (int j = 0; j < 8; ++j) q[j] = s[3 + j];
    uint16_t *r = reinterpret_cast<uint16_t *>(dst + aux_off + b * 8);
    r[0] = s[1];
    r[1] = s[2];
    r[2] = s[0];
    r[3] = 0;
  } else {  // Q6_K: [208 bytes][d] -> records b*208, d at aux_off + b*2
    const uint16_t *s = src + i * 105;
    uint16_t *q = reinterpret_cast<uint16_t *>(dst + b * 208);
    for (int j = 0; j < 104; ++j) q[j] = s[j];
    reinterpret_cast<uint16_t *>(dst + aux_off)[b] = s[104];
  }
}

struct Stager {
  std::mutex mu;
  bool ready = false;
  hipStream_t stream = nullptr;
  uint8_t *pinned[2] = {nullptr, nullptr};
  uint8_t *dstage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
};

int hip_fail(hipError_t e, const char *what) {
  return set_error(e == hipErrorOutOfMemory ? RQ_E_NOMEM : RQ_E_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

int stager_init(Stager &st) {
  if (st.ready) return RQ_OK;
  hipError_t e = hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
  for (int i = 0; i < 2; ++i) {
    if ((e = hipHostMalloc(reinterpret_cast<void **>(&st.pinned[i]), kChunk, hipHostMallocDefault)) != hipSuccess)
      return hip_fail(e, "hipHostMalloc");
    if ((e = hipMalloc(reinterpret_cast<void **>(&st.dstage[i]), kChunk)) != hipSuccess) return hip_fail(e, "hipMalloc");
    if ((e = hipEventCreateWithFlags(&st.done[i], hipEventDisableTiming)) != hipSuccess)
      return hip_fail(e, "hipEventCreate");
  }
  st.ready = true;
  return RQ_OK;
}

// Host copy of one chunk into pinned memory, split over threads for large
// chunks (a single core's memcpy, and the page faults of a freshly mapped
// file, cap a serial copy well below the DMA rate).
void copy_in(uint8_t *dst, const uint8_t *src, uint64_t len) {
  const unsigned hw = std::thread::hardware_concurrency();
  const int threads = (int)(len >= (8ull << 20) ? (hw > 8 ? 8 : (hw ? hw : 1)) : 1);
  if (threads <= 1) {
    memcpy(dst, src, len);
    return;
  }
  std::vector<std::thread> pool;
  const uint64_t part = (len / threads + 4095) & ~(uint64_t)4095;
  for (int t = 0; t < threads; ++t) {
    const uint64_t o = (uint64_t)t * part;
    if (o >= len) break;
    const uint64_t n = len - o < part ? len - o : part;
    pool.emplace_back([=] { memcpy(dst + o, src + o, n); });
  }
  for (auto &th : pool) th.join();
}

}  // namespace

// Uploads nblocks GGUF blocks (bbytes each) from host memory into the
// handle layout at dptr (aux_off = offset of the scale array for the split
// formats).  Returns when the data is on the device.
int upload_blocks(int qtype, const uint8_t *src, uint64_t nblocks, int bbytes, uint8_t *dptr, uint64_t aux_off,
                  int device) {
  static std::mutex table_mu;
  static std::vector<Stager *> table;
  Stager *st;
  {
    std::lock_guard<std::mutex> g(table_mu);
    if ((int)table.size() <= device) table.resize(device + 1, nullptr);
    if (!table[device]) table[device] = new Stager();  // kept until the process ends
    st = table[device];
  }
  std::lock_guard<std::mutex> g(st->mu);
  int rc = stager_init(*st);
  if (rc) return rc;
  const bool split = qtype == RQ_Q8_0 || qtype == RQ_Q4_0 || qtype == RQ_Q5_0 || qtype == RQ_Q6_K;
  const uint64_t per = kChunk / (uint64_t)bbytes;  // blocks per chunk
  int buf = 0;
  for (uint64_t b0 = 0; b0 < nblocks; b0 += per, buf ^= 1) {
    const uint64_t nb = nblocks - b0 < per ? nblocks - b0 : per;
    const uint64_t len = nb * (uint64_t)bbytes;
    hipError_t e = hipEventSynchronize(st->done[buf]);  // this buffer's last DMA (and split) finished
    if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
    copy_in(st->pinned[buf], src + b0 * (uint64_t)bbytes, len);
    if (!split) {
      e = hipMemcpyAsync(dptr + b0 * (uint64_t)bbytes, st->pinned[buf], len, hipMemcpyHostToDevice, st->stream);
      if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync");
    } else {
      e = hipMemcpyAsync(st->dstage[buf], st->pinned[buf], len, hipMemcpyHostToDevice, st->stream);
      if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync");
      hipLaunchKernelGGL(k_split_blocks, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st->stream, qtype,
                         reinterpret_cast<const uint16_t *>(st->dstage[buf]), b0, nb, dptr, aux_off);
      if ((e = hipGetLastError()) != hipSuccess) return hip_fail(e, "split launch");
    }
    if ((e = hipEventRecord(st->done[buf], st->stream)) != hipSuccess) return hip_fail(e, "hipEventRecord");
  }
  const hipError_t e = hipStreamSynchronize(st->stream);
  return e == hipSuccess ? RQ_OK : hip_fail(e, "hipStreamSynchronize");
}

}  // namespace rq
