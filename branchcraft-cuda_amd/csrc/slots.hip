// Per-device pool of split-scratch slots for the entry points without a
// workspace argument (declared in bc_slots.h).
#include "bc_slots.h"

#include <mutex>

namespace {

using bch::kSlotBytes;
using bch::kSlots;

// File-scope device scratch: every device the library's code object is
// loaded on holds its own copy until the process ends.  In host code the
// name is a host-side stand-in, never a device address: the pool passes on
// the address hipGetSymbolAddress returns for the current device.
__device__ __align__(256) unsigned char slot_scratch[kSlots * kSlotBytes];

constexpr int kMaxDevices = 64;

enum SlotState : unsigned char {
  kFree,      // never used
  kOwned,     // last used on `last`, not recorded: only that stream reuses it
  kRecorded,  // last used on `last`, its completion recorded in `ev`
};

struct DevicePool {
  std::mutex mu;
  char* base = nullptr;            // device address of slot_scratch
  hipEvent_t ev[kSlots] = {};
  hipStream_t last[kSlots] = {};   // stream of the slot's last use
  SlotState state[kSlots] = {};
  unsigned long long stamp[kSlots] = {};
  unsigned long long clock = 0;
  // Set once a call found every slot owned by other streams: from then on
  // every use records its event, so slots can pass between streams.  Until
  // then no event is recorded (a record costs about 3 us of GPU time per
  // call, measured on MI355X, while waiting on a passed event costs none).
  bool record_all = false;
};

DevicePool pools[kMaxDevices];

// hipStreamPerThread names a different stream in every host thread, so its
// handle says nothing about stream order: it never owns a slot (its uses are
// always recorded) and always waits for a slot's previous use.
bool ordered(hipStream_t a, hipStream_t b) { return a == b && a != hipStreamPerThread; }

// The slot for a call on `st`: the one this stream used last (no wait:
// stream order), else a free slot, else the least recently used slot whose
// last use is recorded; -1 if none.
int pick(const DevicePool& p, hipStream_t st) {
  int best = -1;
  for (int i = 0; i < kSlots; ++i)
    if (p.state[i] != kFree && ordered(p.last[i], st) &&
        (best < 0 || p.stamp[i] > p.stamp[best]))
      best = i;
  if (best >= 0) return best;
  for (int i = 0; i < kSlots; ++i)
    if (p.state[i] == kFree) return i;
  for (int i = 0; i < kSlots; ++i)
    if (p.state[i] == kRecorded && (best < 0 || p.stamp[i] < p.stamp[best])) best = i;
  return best;
}

}  // namespace

namespace bch {

ScratchLease::ScratchLease(hipStream_t stream, size_t bytes) : stream_(stream) {
  if (bytes == 0 || bytes > kSlotBytes) return;
  // A captured call records no event that its replays could be ordered
  // by; it runs without scratch.  (A query that fails counts as captured.)
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return;
  DevicePool& p = pools[dev];
  p.mu.lock();
  if (!p.base) {
    void* addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(slot_scratch)) != hipSuccess || !addr) {
      p.mu.unlock();
      return;
    }
    p.base = static_cast<char*>(addr);
  }
  const int i = pick(p, stream);
  if (i < 0) {
    // Every slot is owned by another stream, with no recorded use to wait
    // for: run without scratch this time, and record every use from now on.
    p.record_all = true;
    p.mu.unlock();
    return;
  }
  if (p.state[i] == kRecorded && !ordered(p.last[i], stream) &&
      hipStreamWaitEvent(stream, p.ev[i], 0) != hipSuccess) {
    p.mu.unlock();
    return;
  }
  pool_ = &p;
  slot_ = i;
  ptr_ = p.base + (size_t)i * kSlotBytes;
}

ScratchLease::~ScratchLease() {
  if (!ptr_) return;
  DevicePool& p = *static_cast<DevicePool*>(pool_);
  const int i = slot_;
  bool rec = false;
  if (p.record_all || stream_ == hipStreamPerThread) {
    if (!p.ev[i] && hipEventCreateWithFlags(&p.ev[i], hipEventDisableTiming) != hipSuccess)
      p.ev[i] = nullptr;
    rec = p.ev[i] && hipEventRecord(p.ev[i], stream_) == hipSuccess;
  }
  // Without a record the slot stays this stream's (reused in stream order);
  // a per-thread-stream use that could not be recorded is never reused.
  p.last[i] = stream_;
  p.state[i] = rec ? kRecorded : kOwned;
  p.stamp[i] = ++p.clock;
  p.mu.unlock();
}

}  // namespace bch
