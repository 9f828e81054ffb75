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
// shared by gelu_forward/backward and the fused GEMM epilogues so that both
// produce the same bits. With u = sqrt(2/pi) (x + 0.044715 x^3) and the
// logistic s = 1 / (1 + e^(-2u)) = (1 + tanh u) / 2, exactly
//   gelu(x)  = 0.5 x (1 + tanh u)                      = x s
//   gelu'(x) = 0.5 (1 + tanh u) + 0.5 x sech^2(u) u'(x) = s + 2 x s (1 - s) u'(x)
// since sech^2 u = (1 - tanh u)(1 + tanh u) = 4 s (1 - s), and 1 - s =
// e^(-2u) s. One v_exp_f32 and one v_rcp_f32 (about 1 ulp each) replace
// tanhf's ~30 instructions, which made the fused GEMM epilogues 10% slower
// than the plain ones. Nothing cancels: 1 + tanh u and 1 - tanh u are
// products, so the relative error stays ~1e-7 also where gelu(x) is tiny
// (x << 0). The exponent is capped at 126 so e^(-2u) stays finite (then s
// ~ 2^-126 and the results are ~0, not NaN).
constexpr float GELU_S = 0.7978845608028654f;  // sqrt(2/pi)
constexpr float GELU_C = 0.044715f;
constexpr float GELU_M2LOG2E = -2.0f * 1.4426950408889634f;  // e^(-2u) = 2^(u * this)
__device__ __forceinline__ float gelu_logistic(float x, float &e) {
    const float u = GELU_S * (x + GELU_C * x * x * x);
    e = __builtin_amdgcn_exp2f(fminf(u * GELU_M2LOG2E, 126.0f));
    return __builtin_amdgcn_rcpf(1.0f + e);
}
__device__ __forceinline__ float gelu(float x) {
    float e;
    return x * gelu_logistic(x, e);
}
__device__ __forceinline__ float gelu_grad(float x, float g) {
    float e;
    const float s = gelu_logistic(x, e);
    const float dinner = GELU_S * (1.0f + 3.0f * GELU_C * x * x);
    return g * (s + 2.0f * x * s * (e * s) * dinner);
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
