// Library-owned per-device scratch buffers.
//
// A few entry points need device memory beyond their inputs and outputs
// (partial sums of a deterministic reduction, split-K GEMM partials, the dS
// tiles of the flash backward). They lease it for the duration of one call
// from a pool kept per (device, slot):
//
//   bmb::ScratchLease ws(bmb::SCRATCH_NN, bytes);
//   if (!ws) ...;            // could not be allocated (the error is cleared)
//   launch(..., ws.get());   // kernels queued on the null stream
//   // ~ScratchLease returns the buffer to the pool
//
// A buffer is held by one lease at a time, so calls made concurrently from
// several host threads never share one; the pool holds as many buffers as
// were ever leased at once (per device and slot), whatever the number of
// threads that come and go. Every user queues its kernels on the null stream
// of the device, where launches run in submission order whichever host thread
// made them: the next lessee's kernels therefore run after the previous
// lessee's, although the buffer returns to the pool as soon as the previous
// call has queued its work. A buffer that must grow is freed only after the
// device has gone idle (earlier work may still read it). Buffers are kept
// until the process ends.
#pragma once

#include <stddef.h>

namespace bmb {

enum ScratchSlot {
    SCRATCH_FLASH_DS = 0,  // flash backward dS tiles
    SCRATCH_NN = 1,        // nn.h reductions (partials, scalar results)
    SCRATCH_GEMM = 2,      // split-K partial sums of gemm()
    SCRATCH_SLOTS = 3
};

struct ScratchBuffer;

// Checks out a buffer of at least `bytes` bytes (256 if 0) of the current
// device for `slot`; get() is nullptr when it cannot be had.
class ScratchLease {
   public:
    ScratchLease(ScratchSlot slot, size_t bytes);
    ~ScratchLease();
    ScratchLease(const ScratchLease &) = delete;
    ScratchLease &operator=(const ScratchLease &) = delete;

    void *get() const { return ptr_; }
    explicit operator bool() const { return ptr_ != nullptr; }

   private:
    int dev_ = -1;
    ScratchSlot slot_;
    ScratchBuffer *buf_ = nullptr;
    void *ptr_ = nullptr;
};

}  // namespace bmb
