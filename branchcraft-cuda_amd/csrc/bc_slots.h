// Library-owned split scratch for the entry points that take no workspace
// (the reference's signatures: bc_packed_decode, bc_tree_verify).
//
// Each device the library runs on holds kSlots slots of kSlotBytes in a
// file-scope device array (see slots.hip).  A call leases one slot for the
// duration of its launches under the device's pool lock: the slot its stream
// used last (reused in stream order, with no event), else a free slot, else
// the least recently used slot whose last use was recorded in its event (the
// stream then waits for that event with hipStreamWaitEvent).  Events are
// recorded only once some call has found every slot owned by other streams
// (from then on after every use): up to kSlots streams each keep a slot of
// their own at no GPU cost, and calls on more streams still never touch one
// slot's memory at the same time.  Nothing is allocated per call (each
// slot's event is created once, at its first record).
//
// A lease is empty (get() == nullptr) -- and the call then runs its
// single-pass kernels, which need no scratch -- when the request is larger
// than a slot, when the stream is being captured into a graph (an event
// recorded outside the capture cannot order the replays), when every slot is
// owned by another stream with no recorded use, or when a HIP call of the
// pool fails.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "branchcraft.h"

namespace bch {

constexpr int kSlots = BC_SCRATCH_SLOTS;
constexpr size_t kSlotBytes = BC_SCRATCH_SLOT_BYTES;

// Internal to the library (not exported from the shared object).
class __attribute__((visibility("hidden"))) ScratchLease {
 public:
  ScratchLease(hipStream_t stream, size_t bytes);
  ~ScratchLease();
  ScratchLease(const ScratchLease&) = delete;
  ScratchLease& operator=(const ScratchLease&) = delete;

  // Device address of the leased slot (kSlotBytes, 256-byte aligned), or
  // null.
  void* get() const { return ptr_; }

 private:
  void* pool_ = nullptr;  // the device's pool, locked while ptr_ is set
  int slot_ = -1;
  hipStream_t stream_ = nullptr;
  void* ptr_ = nullptr;
};

}  // namespace bch
