// Kernel launch helper: every launch in the library goes through here so the
// launch status is captured for bmb_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include "status.hpp"

namespace bmb {

template <typename... KArgs, typename... Args>
inline void launch(void (*kern)(KArgs...), dim3 grid, dim3 block, size_t smem,
                   hipStream_t stream, Args... args) {
    kern<<<grid, block, smem, stream>>>(static_cast<KArgs>(args)...);
    note_launch_status(hipGetLastError());
}

}  // namespace bmb
