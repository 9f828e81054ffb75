// SGEMM kernel table (src/registry.cu:4-23) and the library's launch-status
// bookkeeping.
#include <hip/hip_runtime_api.h>

#include "../../include/kernels.h"
#include "status.hpp"

extern "C" {

// Ids 1-9 keep the reference's names (src/registry.cu:5-13). Tolerances are
// the normwise bound each stage is held to against an fp32 reference:
//   * 1-8 are bit-identical to a sequential fmaf loop; 1e-4 is the
//     reference's bar for fp32 kernels, kept so the table reads the same.
//   * 9 is fp32 in / fp32 products / fp32 accumulate on matrix cores; only the
//     summation order differs (measured ~1e-7), so it keeps the fp32 1e-4.
//   * 10 (bf16x3) carries the lower precision of its split products.
const KernelEntry KERNELS[] = {
    {1, "naive",      sgemm_naive,        "one lane per output, rows across lanes (uncoalesced)", 1e-4},
    {2, "coalesced",  sgemm_coalesced,    "columns across the wave64 lanes", 1e-4},
    {3, "smem",       sgemm_smem,         "32x32 LDS tiling", 1e-4},
    {4, "tile1d",     sgemm_tile1d,       "1D register tiling, TM=8", 1e-4},
    {5, "tile2d",     sgemm_tile2d,       "2D register tiling, 8x8 per lane", 1e-4},
    {6, "vectorized", sgemm_vectorized,   "128-bit loads + k-major A in LDS", 1e-4},
    {7, "warptile",   sgemm_warptile,     "wave64 tiling, conflict-free 4x4 strips", 1e-4},
    {8, "dbuffer",    sgemm_doublebuffer, "double-buffered LDS + register prefetch, fp32 VALU, bit-exact", 1e-4},
    {9, "tensorcore", sgemm_tensorcore,   "MFMA v_mfma_f32_32x32x2_f32, fp32 in/out", 1e-4},
    {10, "mfma_bf16x3", sgemm_mfma_bf16x3, "MFMA bf16 hi/lo split, 3 products, fp32 accumulate", 1e-4},
};

const int NUM_KERNELS = sizeof(KERNELS) / sizeof(KERNELS[0]);

const KernelEntry *find_kernel(int id) {
    for (int i = 0; i < NUM_KERNELS; ++i)
        if (KERNELS[i].id == id) return &KERNELS[i];
    return nullptr;
}

}  // extern "C"

namespace {
thread_local hipError_t g_launch_status = hipSuccess;
}

void bmb::note_launch_status(hipError_t e) {
    if (e != hipSuccess && g_launch_status == hipSuccess) g_launch_status = e;
}

extern "C" int bmb_last_error(void) {
    const hipError_t e = g_launch_status;
    g_launch_status = hipSuccess;
    return (int)e;
}
