// A second stream per device for the blocked drivers that run two halves of a batch side
// by side (launch_pf_large, launch_lu_large): a half's panel kernels, one latency-bound
// workgroup per matrix, then run beside the other half's trailing update, which streams
// the matrices through HBM or keeps the MFMA busy.
//
// The stream is created on first use with hipStreamNonBlocking (no implicit ordering
// with the null stream; every dependency is an explicit event) at the default priority,
// and kept, with its two events, until the process ends. A split run holds the
// device's mutex from its fork to its join, so two host threads never interleave their
// records of the shared events. A stream under graph capture runs unsplit.
#include <atomic>
#include <mutex>

#include "fermix_internal.h"

namespace fx {
namespace {

constexpr int SIDE_MAXDEV = 64;

struct Side {
  std::mutex mu;
  bool tried = false, ok = false;
  hipStream_t s2 = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

Side g_side[SIDE_MAXDEV];

}  // namespace

SideStream::SideStream(hipStream_t s, bool want) : s_(s) {
  if (!want) return;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SIDE_MAXDEV) return;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
  Side& d = g_side[dev];
  std::unique_lock<std::mutex> lk(d.mu);
  if (!d.tried) {
    d.tried = true;
    d.ok = hipStreamCreateWithFlags(&d.s2, hipStreamNonBlocking) == hipSuccess &&
           hipEventCreateWithFlags(&d.fork, hipEventDisableTiming) == hipSuccess &&
           hipEventCreateWithFlags(&d.join, hipEventDisableTiming) == hipSuccess;
  }
  if (!d.ok) return;
  lk_ = std::move(lk);
  side_ = &d.s2;
  fork_ = &d.fork;
  join_ = &d.join;
}

int SideStream::fork() {
  if (!side_ || forked_) return FX_ERR_LAUNCH;
  if (hipEventRecord(*fork_, s_) != hipSuccess || hipStreamWaitEvent(*side_, *fork_, 0) != hipSuccess)
    return FX_ERR_LAUNCH;
  forked_ = true;
  return FX_OK;
}

int SideStream::join() {
  if (!forked_) return FX_OK;
  forked_ = false;
  if (hipEventRecord(*join_, *side_) != hipSuccess || hipStreamWaitEvent(s_, *join_, 0) != hipSuccess)
    return FX_ERR_LAUNCH;
  return FX_OK;
}

SideStream::~SideStream() { join(); }

int device_cus() {
  static std::atomic<int> cache[SIDE_MAXDEV];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SIDE_MAXDEV) return 256;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) return 256;
  cache[dev].store(c, std::memory_order_relaxed);
  return c;
}

}  // namespace fx
