// Host-to-device staging of the small int64 arrays the batch classes upload
// per step (slot lists, queued pool writes).
//
// Per (device, stream): a ring of pinned host memory.  A call copies the
// values to the ring's head and enqueues the host-to-device copy from there
// on the stream; every kCheckpointCalls calls (and whenever the ring runs
// short) it records an event after its copy, which marks every ring byte
// before it as reusable once the event completes.  Space is reclaimed by
// querying the oldest checkpoints once less than half the ring is free, and
// only when the ring is full does a call wait for one.  So the host never
// waits for the device while the copies in flight fit in the ring, a call
// costs one memcpy and one asynchronous copy (plus an event record once in
// kCheckpointCalls calls), and the caller's array may change as soon as the
// call returns.  Uploads
// larger than a quarter of the ring take a pinned buffer of their own
// (with an event of its own), freed once that event completes.
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <utility>

#include "bpd_common.hpp"

namespace bpd {
namespace {

constexpr size_t kRingBytes = size_t(4) << 20;
constexpr size_t kRingAlign = 256;
constexpr int kCheckpointCalls = 32;

struct Checkpoint {
  hipEvent_t ev;
  uint64_t end;  // ring bytes (monotonic count) consumed up to this copy
};

struct Big {
  void* buf;
  hipEvent_t ev;
};

struct Stager {
  char* ring = nullptr;
  uint64_t head = 0;     // monotonic byte count of the ring handed out
  uint64_t retired = 0;  // every ring byte before this is free again
  int since_checkpoint = 0;
  std::deque<Checkpoint> checkpoints;  // in enqueue order
  std::deque<hipEvent_t> spare;        // completed checkpoint events, reused
  std::deque<Big> big;                 // oversize uploads in flight
};

std::mutex g_stage_mu;
std::map<std::pair<int, hipStream_t>, Stager> g_stagers;

// Reclaims the ring up to every completed checkpoint (waiting for the oldest
// while fewer than `need` bytes are free).  Called with the lock held and the
// stream's device current.
int reclaim(Stager& s, size_t need) {
  while (!s.checkpoints.empty()) {
    Checkpoint& c = s.checkpoints.front();
    const bool short_of_space = kRingBytes - (s.head - s.retired) < need;
    hipError_t q = hipEventQuery(c.ev);
    if (q == hipErrorNotReady) {
      if (!short_of_space) break;
      q = hipEventSynchronize(c.ev);
    }
    if (q != hipSuccess) BPD_FAIL(BPD_ERR_HIP, "staging event: %s", hipGetErrorString(q));
    s.retired = c.end;
    s.spare.push_back(c.ev);
    s.checkpoints.pop_front();
  }
  return BPD_OK;
}

int checkpoint(Stager& s, hipStream_t st) {
  hipEvent_t ev = nullptr;
  if (!s.spare.empty()) {
    ev = s.spare.front();
    s.spare.pop_front();
  } else {
    BPD_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  }
  const hipError_t e = hipEventRecord(ev, st);
  if (e != hipSuccess) {
    s.spare.push_back(ev);
    BPD_FAIL(BPD_ERR_HIP, "staging event record: %s", hipGetErrorString(e));
  }
  s.checkpoints.push_back(Checkpoint{ev, s.head});
  s.since_checkpoint = 0;
  return BPD_OK;
}

int stage_big(Stager& s, int64_t* dst, const int64_t* src, size_t bytes, hipStream_t st) {
  while (!s.big.empty() && hipEventQuery(s.big.front().ev) == hipSuccess) {
    (void)hipHostFree(s.big.front().buf);
    (void)hipEventDestroy(s.big.front().ev);
    s.big.pop_front();
  }
  Big b{nullptr, nullptr};
  BPD_HIP(hipHostMalloc(&b.buf, bytes, hipHostMallocDefault));
  hipError_t e = hipEventCreateWithFlags(&b.ev, hipEventDisableTiming);
  if (e != hipSuccess) {
    (void)hipHostFree(b.buf);
    BPD_FAIL(BPD_ERR_HIP, "hipEventCreateWithFlags: %s", hipGetErrorString(e));
  }
  std::memcpy(b.buf, src, bytes);
  e = hipMemcpyAsync(dst, b.buf, bytes, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipEventRecord(b.ev, st);
  if (e != hipSuccess) {
    (void)hipStreamSynchronize(st);  // nothing of this copy may still read the buffer
    (void)hipHostFree(b.buf);
    (void)hipEventDestroy(b.ev);
    BPD_FAIL(BPD_ERR_HIP, "staged copy: %s", hipGetErrorString(e));
  }
  s.big.push_back(b);
  return BPD_OK;
}

// Called with the stream's device current and the lock held.
int stage_copy(Stager& s, int64_t* dst, const int64_t* src, size_t bytes, hipStream_t st) {
  if (bytes > kRingBytes / 4) return stage_big(s, dst, src, bytes, st);
  if (!s.ring) BPD_HIP(hipHostMalloc(reinterpret_cast<void**>(&s.ring), kRingBytes, hipHostMallocDefault));
  const size_t span = (bytes + kRingAlign - 1) / kRingAlign * kRingAlign;
  uint64_t at = s.head;
  const size_t off = size_t(at % kRingBytes);
  const size_t skip = off + span > kRingBytes ? kRingBytes - off : 0;  // never wrap inside a copy
  const size_t need = skip + span;
  if (kRingBytes - (s.head - s.retired) < need) {
    // short of space: make every byte handed out so far reclaimable, then wait
    if (s.since_checkpoint > 0 || s.checkpoints.empty() || s.checkpoints.back().end != s.head)
      if (int rc = checkpoint(s, st)) return rc;
    if (int rc = reclaim(s, need)) return rc;
  } else if (!s.checkpoints.empty() && kRingBytes - (s.head - s.retired) < kRingBytes / 2) {
    if (int rc = reclaim(s, 0)) return rc;  // below half free: retire what has completed
  }
  at += skip;
  char* p = s.ring + size_t(at % kRingBytes);
  std::memcpy(p, src, bytes);
  const hipError_t e = hipMemcpyAsync(dst, p, bytes, hipMemcpyHostToDevice, st);
  if (e != hipSuccess) BPD_FAIL(BPD_ERR_HIP, "staged copy: %s", hipGetErrorString(e));
  s.head = at + span;
  if (++s.since_checkpoint >= kCheckpointCalls) return checkpoint(s, st);
  return BPD_OK;
}

// Device of a stream, cached per thread for the last stream asked about.
int stream_device(hipStream_t st, int* dev) {
  thread_local hipStream_t last = nullptr;
  thread_local int last_dev = -1;
  if (st && st == last && last_dev >= 0) {
    *dev = last_dev;
    return BPD_OK;
  }
  if (st) {
    BPD_HIP(hipStreamGetDevice(st, dev));
    last = st;
    last_dev = *dev;
  } else {
    BPD_HIP(hipGetDevice(dev));
  }
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
  if (int rc = stream_device(st, &dev)) return rc;
  BPD_HIP(hipGetDevice(&cur));
  if (dev != cur) BPD_HIP(hipSetDevice(dev));
  int rc;
  {
    std::lock_guard<std::mutex> lock(g_stage_mu);
    rc = stage_copy(g_stagers[std::make_pair(dev, st)], dst, src, bytes, st);
  }
  if (dev != cur) BPD_HIP(hipSetDevice(cur));
  return rc;
}
