// Library-owned per-device scratch buffers.
//
// A few entry points need device memory beyond their inputs and outputs
// (partial sums of a deterministic reduction, split-K GEMM partials, the dS
// tiles of the flash backward). They lease it for the duration of one call
// from a pool kept per (device, slot):
//
//   bmb::ScratchLease ws(bmb::SCRATCH_NN, bytes, stream);
//   if (!ws) ...;            // could not be allocated (the error is cleared)
//   launch(..., ws.get());   // kernels queued on `stream`
//   // ~ScratchLease returns the buffer to the pool
//
// A buffer is held by one lease at a time, so calls made concurrently from
// several host threads never share one; the pool holds as many buffers as
// were ever leased at once (per device and slot), whatever the number of
// threads that come and go. The buffer returns to the pool as soon as the
// call has queued its work, so reuse is ordered on the device by an event:
// the lease's destructor records the buffer's event on the lessee's stream
// (after every kernel the call queued there), and the next lease makes its
// own stream wait for that event before anything it queues. A lessee on the
// null stream records nothing when it returns the buffer: a next lease on
// the null stream queues after its work anyway, and a next lease on another
// stream records the event on the null stream then (after everything queued
// there so far, the last lessee's work included) and waits for it. Two calls
// on different streams, or on the null stream from several host threads,
// therefore never touch one buffer at the same time. A lease prefers an idle
// buffer last used on its own stream, so that work on two streams does not
// wait on each other through the pool. A buffer that must grow is freed only
// after its event has completed. Buffers are kept until the process ends.
#pragma once

#include <stddef.h>

#include <hip/hip_runtime_api.h>

namespace bmb {

enum ScratchSlot {
    SCRATCH_FLASH_DS = 0,  // flash backward dS tiles
    SCRATCH_NN = 1,        // nn.h reductions (partials, scalar results)
    SCRATCH_GEMM = 2,      // split-K partial sums of gemm()
    SCRATCH_SLOTS = 3
};

struct ScratchBuffer;

// Checks out a buffer of at least `bytes` bytes (256 if 0) of the current
// device for `slot`, for kernels queued on `stream` (0: the null stream);
// get() is nullptr when it cannot be had.
class ScratchLease {
   public:
    ScratchLease(ScratchSlot slot, size_t bytes, hipStream_t stream = nullptr);
    ~ScratchLease();
    ScratchLease(const ScratchLease &) = delete;
    ScratchLease &operator=(const ScratchLease &) = delete;

    void *get() const { return ptr_; }
    explicit operator bool() const { return ptr_ != nullptr; }

   private:
    int dev_ = -1;
    ScratchSlot slot_;
    hipStream_t stream_;
    ScratchBuffer *buf_ = nullptr;
    void *ptr_ = nullptr;
};

}  // namespace bmb
