// rq_workspace.cpp -- per-(device, stream) device memory that outlives a call.
//
// The entry points that need scratch (split-K partials of the tiled GEMM, an
// aligned copy of the activations, FP8 activation codes, embedding ids, the
// KV quantizer's partial maxima) take it from their stream's workspace
// instead of allocating per call: a stream-ordered allocation and free
// around a kernel cost 12-17 us per call on MI355X, more than many of the
// kernels they serve.
//
// Rules (rq_internal.h, WsLease):
//  * one buffer per (device, stream); hipStreamPerThread is keyed per thread,
//    since that handle names a different stream on every thread;
//  * a lease holds the slot's mutex while one entry point enqueues its
//    launches, so calls from several threads on one stream do not interleave
//    their use of the buffer (their kernels run in stream order anyway);
//  * growth allocates a larger buffer in stream order; the old one is freed
//    in stream order when the lease ends (after every launch of the call that
//    may still use it), unless a captured graph may refer to it, in which
//    case it is kept until the process ends;
//  * under stream capture a large enough buffer is used as it is and marked
//    as referred to by a graph; a larger need grows the buffer with a plain
//    allocation made with this thread's capture mode relaxed (no graph
//    node; the old buffer stays alive, as graphs may refer to it), and only
//    if that fails with a stream-ordered allocation and free that become
//    nodes of the graph (10-20 us per replay on MI355X).  Counters are not
//    created under capture (their zeroing would be a memset node): kernels
//    that need them run without split K there.
#include <map>
#include <mutex>
#include <thread>
#include <tuple>

#include "rq_internal.h"

namespace rq {

struct Slot {
  std::mutex mu;
  void *ptr = nullptr;
  size_t bytes = 0;
  bool graph_ref = false;  // a captured graph may refer to ptr: never free it
  uint32_t *counters = nullptr;  // zero between calls; never freed
};

namespace {

struct Key {
  int device;
  hipStream_t stream;
  std::thread::id thread;
  bool operator<(const Key &o) const {
    return std::tie(device, stream, thread) < std::tie(o.device, o.stream, o.thread);
  }
};

std::mutex g_slots_mu;

// Slots live until the process ends (their buffers may be referred to by
// graphs that outlive any owner here).
std::map<Key, Slot *> &slots() {
  static auto *m = new std::map<Key, Slot *>();
  return *m;
}

Slot *slot_for(int device, hipStream_t s) {
  const Key key{device, s, s == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id()};
  std::lock_guard<std::mutex> g(g_slots_mu);
  Slot *&p = slots()[key];
  if (!p) p = new Slot();
  return p;
}

constexpr size_t kGrain = 2u << 20;  // buffers grow in 2 MiB steps (at least doubling)

}  // namespace

WsLease::WsLease(int device, hipStream_t s) : device_(device), s_(s) {}

// The slot is taken at the first request, so calls that need no scratch
// (every decode GEMV) cost nothing here.
void WsLease::acquire() {
  slot_ = slot_for(device_, s_);
  slot_->mu.lock();
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s_, &st) != hipSuccess) {
    // An error here (the legacy stream while another stream captures in
    // global mode) means launches would fail too; treat it as capture so
    // that nothing grows, and let the launch report it.
    (void)hipGetLastError();
    capturing_ = true;
  } else {
    capturing_ = st == hipStreamCaptureStatusActive;
  }
}

WsLease::~WsLease() {
  for (void *p : async_) (void)hipFreeAsync(p, s_);
  if (slot_) slot_->mu.unlock();
}

void *WsLease::get(size_t bytes, int *rc, bool quiet) {
  auto fail = [&](int code, const char *what, size_t want, hipError_t e) -> void * {
    (void)hipGetLastError();
    *rc = quiet ? code : set_error(code, "%s of %zu bytes: %s", what, want, hipGetErrorString(e));
    return nullptr;
  };
  if (!slot_) acquire();
  bytes = (bytes + 255) & ~(size_t)255;
  if (bytes == 0) bytes = 256;
  if (capturing_) {
    if (slot_->ptr && used_ + bytes <= slot_->bytes) {
      slot_->graph_ref = true;
      void *p = static_cast<uint8_t *>(slot_->ptr) + used_;
      used_ += bytes;
      return p;
    }
    {
      // A new buffer outside the graph; earlier requests of this call keep
      // pointing into the old one, which is never freed.
      size_t want = bytes > 2 * slot_->bytes ? bytes : 2 * slot_->bytes;
      want = (want + kGrain - 1) / kGrain * kGrain;
      hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
      void *p = nullptr;
      if (hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess) {
        const hipError_t e = hipMalloc(&p, want);
        (void)hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) {
          (void)hipGetLastError();
          p = nullptr;
        }
      } else {
        (void)hipGetLastError();
      }
      if (p) {
        slot_->ptr = p;
        slot_->bytes = want;
        slot_->graph_ref = true;
        used_ = bytes;
        return p;
      }
    }
    void *p = nullptr;
    const hipError_t e = hipMallocAsync(&p, bytes, s_);
    if (e != hipSuccess) return fail(e == hipErrorOutOfMemory ? RQ_E_NOMEM : RQ_E_DEVICE, "workspace", bytes, e);
    async_.push_back(p);
    return p;
  }
  if (!slot_->ptr || used_ + bytes > slot_->bytes) {
    size_t want = used_ + bytes > 2 * slot_->bytes ? used_ + bytes : 2 * slot_->bytes;
    want = (want + kGrain - 1) / kGrain * kGrain;
    void *p = nullptr;
    const hipError_t e = hipMallocAsync(&p, want, s_);
    if (e != hipSuccess) return fail(e == hipErrorOutOfMemory ? RQ_E_NOMEM : RQ_E_DEVICE, "workspace", want, e);
    // The old buffer may still serve launches of this call (earlier
    // requests) and of earlier calls: freed in stream order at the end of
    // this lease, or kept if a graph may refer to it.
    if (slot_->ptr && !slot_->graph_ref) async_.push_back(slot_->ptr);
    slot_->ptr = p;
    slot_->bytes = want;
    slot_->graph_ref = false;
    used_ = 0;
  }
  void *p = static_cast<uint8_t *>(slot_->ptr) + used_;
  used_ += bytes;
  return p;
}

uint32_t *WsLease::counters() {
  if (!slot_) acquire();
  if (slot_->counters) return slot_->counters;
  if (capturing_) return nullptr;
  void *p = nullptr;
  if (hipMallocAsync(&p, kCounters * sizeof(uint32_t), s_) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (hipMemsetAsync(p, 0, kCounters * sizeof(uint32_t), s_) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFreeAsync(p, s_);
    return nullptr;
  }
  slot_->counters = static_cast<uint32_t *>(p);
  return slot_->counters;
}

}  // namespace rq
