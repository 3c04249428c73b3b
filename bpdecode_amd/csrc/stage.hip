// Host-to-device staging of the small int64 arrays the batch classes upload
// per step (slot lists, queued pool writes).
//
// Per (device, stream): pinned host buffers, each either free or carrying a
// copy in flight (a FIFO, with an event recorded after each copy).  A call
// retires the copies that have completed, takes a free buffer large enough
// (or allocates one), copies the values into it, enqueues the host-to-device
// copy on the stream and records its event.  The host therefore never waits
// for the device, however far ahead of it it runs (up to kMaxInflight
// copies; past that the oldest is waited for), and the caller's array may
// change as soon as the call returns.  One call replaces a pinned-tensor
// allocation, a fill and an asynchronous tensor copy.
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "bpd_common.hpp"

namespace bpd {
namespace {

constexpr size_t kMinStageBytes = 4096;
constexpr size_t kMaxInflight = 8192;

struct StageBuf {
  void* buf;
  size_t bytes;
  hipEvent_t ev;
};

struct Stager {
  std::deque<StageBuf> inflight;  // in enqueue order
  std::vector<StageBuf> free;
};

std::mutex g_stage_mu;
std::map<std::pair<int, hipStream_t>, Stager> g_stagers;

// Called with the stream's device current and the lock held.
int stage_copy(Stager& s, int64_t* dst, const int64_t* src, size_t bytes, hipStream_t st) {
  while (!s.inflight.empty()) {
    const hipError_t q = s.inflight.front().ev ? hipEventQuery(s.inflight.front().ev) : hipSuccess;
    if (q == hipErrorNotReady) {
      if (s.inflight.size() < kMaxInflight) break;
      BPD_HIP(hipEventSynchronize(s.inflight.front().ev));
    } else if (q != hipSuccess) {
      BPD_FAIL(BPD_ERR_HIP, "hipEventQuery: %s", hipGetErrorString(q));
    }
    s.free.push_back(s.inflight.front());
    s.inflight.pop_front();
  }
  StageBuf b{nullptr, 0, nullptr};
  for (size_t i = 0; i < s.free.size(); ++i) {
    if (s.free[i].bytes >= bytes) {
      b = s.free[i];
      s.free[i] = s.free.back();
      s.free.pop_back();
      break;
    }
  }
  if (!b.buf) {
    size_t want = kMinStageBytes;
    while (want < bytes) want *= 2;
    BPD_HIP(hipHostMalloc(&b.buf, want, hipHostMallocDefault));
    b.bytes = want;
    const hipError_t e = hipEventCreateWithFlags(&b.ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      (void)hipHostFree(b.buf);
      BPD_FAIL(BPD_ERR_HIP, "hipEventCreateWithFlags: %s", hipGetErrorString(e));
    }
  }
  std::memcpy(b.buf, src, bytes);
  hipError_t e = hipMemcpyAsync(dst, b.buf, bytes, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipEventRecord(b.ev, st);
  if (e != hipSuccess) {
    s.free.push_back(b);  // nothing was left in flight from it
    BPD_FAIL(BPD_ERR_HIP, "staged copy: %s", hipGetErrorString(e));
  }
  s.inflight.push_back(b);
  return BPD_OK;
}

}  // namespace
}  // namespace bpd

using namespace bpd;

extern "C" int bpd_stage_int64(int64_t* dst, const int64_t* src, int64_t n, void* stream) {
  BPD_REQUIRE(n >= 0, "negative count");
  if (n == 0) return BPD_OK;
  BPD_REQUIRE(dst && src, "null pointer argument");
  const size_t bytes = size_t(n) * sizeof(int64_t);
  hipStream_t st = as_stream(stream);
  // events belong to the stream's device: make it current for the call
  int dev = 0, cur = 0;
  BPD_HIP(hipGetDevice(&cur));
  if (st) {
    BPD_HIP(hipStreamGetDevice(st, &dev));
  } else {
    dev = cur;
  }
  if (dev != cur) BPD_HIP(hipSetDevice(dev));
  int rc;
  {
    std::lock_guard<std::mutex> lock(g_stage_mu);
    rc = stage_copy(g_stagers[std::make_pair(dev, st)], dst, src, bytes, st);
  }
  if (dev != cur) BPD_HIP(hipSetDevice(cur));
  return rc;
}
