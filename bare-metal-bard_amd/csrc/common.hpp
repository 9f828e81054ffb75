// Shared device/host helpers for the gfx950 kernels.
//
// Every kernel in this library is written for CDNA4 (gfx950): wave64, MFMA
// matrix cores, 160 KB LDS per CU, 256 CUs in 8 XCDs. Nothing here targets
// any other architecture.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bmb {

constexpr int WAVE = 64;

__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Fused multiply-add with one rounding, written out so that the k-ordered
// accumulation of the fp32 VALU kernels never depends on -ffp-contract.
__device__ __forceinline__ float fma_rn(float a, float b, float c) {
    return __builtin_fmaf(a, b, c);
}

// BLAS-style epilogue shared by every SGEMM path: beta == 0 never reads C.
// Otherwise C = fma(alpha, acc, beta * C). The CPU oracle uses the same form,
// which is what makes the VALU kernels bit-identical to it.
__device__ __forceinline__ float epilogue(float acc, float alpha, float beta,
                                          const float *c) {
    return beta == 0.0f ? alpha * acc : fma_rn(alpha, acc, beta * (*c));
}

// GPT-2's tanh GELU (src/nn.cu:116-121) and its derivative (:132-139),
// shared by gelu_forward/backward and the fused GEMM epilogue so that both
// produce the same bits.
constexpr float GELU_S = 0.7978845608028654f;  // sqrt(2/pi)
constexpr float GELU_C = 0.044715f;
__device__ __forceinline__ float gelu(float x) {
    return 0.5f * x * (1.0f + tanhf(GELU_S * (x + GELU_C * x * x * x)));
}
__device__ __forceinline__ float gelu_grad(float x, float g) {
    const float t = tanhf(GELU_S * (x + GELU_C * x * x * x));
    const float sech2 = 1.0f - t * t;
    const float dinner = GELU_S * (1.0f + 3.0f * GELU_C * x * x);
    return g * (0.5f * (1.0f + t) + 0.5f * x * sech2 * dinner);
}

// 128-bit global/LDS moves.
__device__ __forceinline__ float4 ld4(const float *p) {
    return *reinterpret_cast<const float4 *>(p);
}
__device__ __forceinline__ void st4(float *p, float4 v) {
    *reinterpret_cast<float4 *>(p) = v;
}

// XCD-aware tile order. The hardware hands workgroup ids to the 8 XCDs
// round-robin, so ids x, x+8, x+16, ... share one XCD and its L2. This maps
// them to a contiguous range of logical ids, so that a group of neighbouring
// output tiles -- which read the same A row-panel and B column-panel -- lands
// on one L2 instead of being spread over all eight.
__device__ __forceinline__ int xcd_remap(int pid, int nblocks) {
    constexpr int NXCD = 8;
    if (nblocks % NXCD != 0) return pid;
    return (pid % NXCD) * (nblocks / NXCD) + pid / NXCD;
}

// Grouped row-major tile order over a tiles_m x tiles_n grid: GROUP tile-rows
// are walked column by column, so consecutive ids reuse the same B panels.
__device__ __forceinline__ void group_tile(int pid, int tiles_m, int tiles_n,
                                           int group, int &tm, int &tn) {
    const int per_group = group * tiles_n;
    const int g = pid / per_group;
    const int first_m = g * group;
    const int gsz = min(tiles_m - first_m, group);
    const int local = pid % per_group;
    tm = first_m + local % gsz;
    tn = local / gsz;
}

}  // namespace bmb
