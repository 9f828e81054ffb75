// Kernel launch helper: every launch in the library goes through here so the
// launch status is captured for bmb_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>
#include <set>
#include <utility>

#include "status.hpp"

namespace bmb {

// Kernels whose dynamic LDS exceeds the 64 KiB default get their limit raised
// once per kernel and device (gfx950 has 160 KiB per CU). Keyed on the
// kernel's address: kernels of one signature share this instantiation.
template <typename K>
inline void allow_smem(K kern, size_t bytes) {
    if (bytes <= 65536) return;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    const void *f = reinterpret_cast<const void *>(kern);
    static std::mutex mu;
    static std::set<std::pair<int, const void *>> done;
    std::lock_guard<std::mutex> lock(mu);  // held until the attribute is set
    if (!done.insert({dev, f}).second) return;
    note_launch_status(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)bytes));
}

// True when `stream` is being captured into a graph. The null stream is never
// asked (querying it while another stream captures is itself an error).
inline bool stream_capturing(hipStream_t stream) {
    if (stream == nullptr) return false;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;  // unknown: behave as under capture (allocate nothing)
    }
    return st != hipStreamCaptureStatusNone;
}

template <typename... KArgs, typename... Args>
inline void launch(void (*kern)(KArgs...), dim3 grid, dim3 block, size_t smem,
                   hipStream_t stream, Args... args) {
    kern<<<grid, block, smem, stream>>>(static_cast<KArgs>(args)...);
    note_launch_status(hipGetLastError());
}

}  // namespace bmb
