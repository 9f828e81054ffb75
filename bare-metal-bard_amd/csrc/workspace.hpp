// Library-owned per-device scratch buffers.
//
// A few entry points need device memory beyond their inputs and outputs
// (partial sums of a deterministic reduction, the dS tiles of the flash
// backward). They take it from here: one grow-only buffer per (device, slot),
// allocated on first use and kept until the process ends. Growing waits for
// the device to go idle before freeing the old buffer, so work already queued
// on it is never left reading freed memory.
#pragma once

#include <stddef.h>

namespace bmb {

enum ScratchSlot {
    SCRATCH_FLASH_DS = 0,  // flash backward dS tiles
    SCRATCH_NN = 1,        // nn.h reductions (partials, scalar results)
    SCRATCH_SLOTS = 2
};

// Returns a device pointer to at least `bytes` bytes for the current device,
// or nullptr if it cannot be allocated (the allocation error is cleared).
// Calls for one device are serialised by a mutex; the memory is shared by
// every caller of that slot on that device, so two streams must not use one
// slot concurrently.
void *device_scratch(ScratchSlot slot, size_t bytes);

}  // namespace bmb
