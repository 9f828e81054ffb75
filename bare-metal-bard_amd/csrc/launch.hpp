// Kernel launch helper: every launch in the library goes through here so the
// launch status is captured for bmb_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>

#include "status.hpp"

namespace bmb {

// Kernels whose dynamic LDS exceeds the 64 KiB default get their limit raised
// once per device (gfx950 has 160 KiB per CU).
template <typename K>
inline void allow_smem(K kern, size_t bytes) {
    if (bytes <= 65536) return;
    static std::once_flag once[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return;
    std::call_once(once[dev], [&] {
        note_launch_status(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)bytes));
    });
}

template <typename... KArgs, typename... Args>
inline void launch(void (*kern)(KArgs...), dim3 grid, dim3 block, size_t smem,
                   hipStream_t stream, Args... args) {
    kern<<<grid, block, smem, stream>>>(static_cast<KArgs>(args)...);
    note_launch_status(hipGetLastError());
}

}  // namespace bmb
