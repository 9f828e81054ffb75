// Per-device grow-only scratch buffers (see workspace.hpp).
#include "workspace.hpp"

#include <hip/hip_runtime_api.h>

#include <mutex>

namespace bmb {

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_ptr[MAX_DEVICES][SCRATCH_SLOTS] = {};
size_t g_cap[MAX_DEVICES][SCRATCH_SLOTS] = {};
}  // namespace

void *device_scratch(ScratchSlot slot, size_t bytes) {
    int dev = 0;
    if (slot < 0 || slot >= SCRATCH_SLOTS) return nullptr;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    if (bytes == 0) bytes = 256;
    std::lock_guard<std::mutex> lock(g_mu);
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
