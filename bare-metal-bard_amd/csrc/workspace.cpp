// Per-device grow-only scratch buffers (see workspace.hpp).
#include "workspace.hpp"

#include <hip/hip_runtime_api.h>


namespace bmb {

namespace {
constexpr int MAX_DEVICES = 64;
// Per host thread: kernels a thread queues on the null stream run in its
// order, so one thread's calls never overlap on its own buffers, and two
// threads never share one.
thread_local void *g_ptr[MAX_DEVICES][SCRATCH_SLOTS] = {};
thread_local size_t g_cap[MAX_DEVICES][SCRATCH_SLOTS] = {};
}  // namespace

void *device_scratch(ScratchSlot slot, size_t bytes) {
    int dev = 0;
    if (slot < 0 || slot >= SCRATCH_SLOTS) return nullptr;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    if (bytes == 0) bytes = 256;
    void *&ptr = g_ptr[dev][slot];
    size_t &cap = g_cap[dev][slot];
    if (cap < bytes) {
        if (ptr != nullptr) {
            if (hipDeviceSynchronize() != hipSuccess) return nullptr;
            (void)hipFree(ptr);
            ptr = nullptr;
            cap = 0;
        }
        void *p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            (void)hipGetLastError();  // clear the allocation failure
            return nullptr;
        }
        ptr = p;
        cap = bytes;
    }
    return ptr;
}

}  // namespace bmb
