// Library-owned per-device scratch buffers.
//
// A few entry points need device memory beyond their inputs and outputs
// (partial sums of a deterministic reduction, split-K GEMM partials, the dS
// tiles of the flash backward). They take it from here: one grow-only buffer
// per (host thread, device, slot), allocated on first use and kept until the
// process ends. Growing waits for the device to go idle before freeing the
// old buffer, so work already queued on it is never left reading freed
// memory. The users launch on the null stream, where one host thread's
// launches run in order, so a thread's calls never overlap on its buffers.
#pragma once

#include <stddef.h>

namespace bmb {

enum ScratchSlot {
    SCRATCH_FLASH_DS = 0,  // flash backward dS tiles
    SCRATCH_NN = 1,        // nn.h reductions (partials, scalar results)
    SCRATCH_GEMM = 2,      // split-K partial sums of gemm()
    SCRATCH_SLOTS = 3
};

// Returns a device pointer to at least `bytes` bytes for the current device
// and calling thread, or nullptr if it cannot be allocated (the allocation
// error is cleared). The memory is shared by every use of that slot from this
// thread on this device, so work on two streams must not use one slot
// concurrently.
void *device_scratch(ScratchSlot slot, size_t bytes);

}  // namespace bmb
