// Device query and measured peak rates for the roofline denominators -- the
// counterpart of bare-metal-bard's tools/device_query.cu:28-32,52, which
// prints the fp32 peak at the locked clock and the ridge point.
//
// Besides the device properties this measures, with HIP events, what the
// kernels of this library can actually issue on this GPU:
//   * fp32 FMA on the vector ALU as v_fmac_f32 (no packed-fp32 instructions),
//     at 1, 2, 4 and 8 waves per SIMD;
//   * the VALU SGEMM's inner loop without its global loads and barriers: an
//     8 x 8 outer product per lane per k (64 accumulators), from registers
//     and with its operands read from LDS as KERNELS id 8 reads them (two
//     128-bit reads of A and two of B per k, shared by 8 lanes each);
//   * fp32 MFMA v_mfma_f32_32x32x2_f32 and v_mfma_f32_16x16x4_f32;
//   * bf16 and fp16 MFMA v_mfma_f32_32x32x16_bf16 / _f16;
//   * a plain 1 GiB device-to-device copy (read + write bytes).
// Every kernel has a fixed trip count and touches only its own outputs.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#define CHECK(x)                                                              \
    do {                                                                      \
        hipError_t e_ = (x);                                                  \
        if (e_ != hipSuccess) {                                               \
            fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            exit(1);                                                          \
        }                                                                     \
    } while (0)

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int THREADS = 256;

// 16 independent accumulators per lane; each step is acc += x_i * x_{i+1}.
__global__ __launch_bounds__(THREADS) void valu_fma_k(float *out, float m, int iters) {
    float a[16], x[16];
    for (int i = 0; i < 16; ++i) { a[i] = threadIdx.x * 1e-3f + i; x[i] = m + i * 1e-3f; }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i) a[i] = __builtin_fmaf(x[i], x[(i + 1) & 15], a[i]);
    }
    float s = 0.0f;
    for (int i = 0; i < 16; ++i) s += a[i];
    out[blockIdx.x * THREADS + threadIdx.x] = s;
}

// 8 x 8 outer product per lane and k: acc[i][j] += a[i] * b[j]. LDS = false:
// a and b stay in registers. LDS = true: per k, a comes from two 128-bit reads
// of a k-major A row and b from two of a B row, at the lane offsets of the
// id-8 SGEMM's 128 x 128 tile (8 lanes share each address).
template <bool LDS>
__global__ __launch_bounds__(THREADS) void valu_outer_k(float *out, int iters) {
    constexpr int LDA = 132, LDB = 128, BK = 16;
    __shared__ float lds[BK * LDA + BK * LDB];
    for (int i = threadIdx.x; i < BK * (LDA + LDB); i += THREADS) lds[i] = i * 1e-3f;
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float *as = lds + (wave >> 1) * 64 + (lane >> 3) * 4;
    const float *bs = lds + BK * LDA + (wave & 1) * 64 + (lane & 7) * 4;
    float a[8], b[8], acc[64];
    for (int i = 0; i < 8; ++i) { a[i] = threadIdx.x * 1e-3f + i; b[i] = 1.0f + i; }
    for (int i = 0; i < 64; ++i) acc[i] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll 8
        for (int k = 0; k < BK; ++k) {
            if (LDS) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const float4 x = *reinterpret_cast<const float4 *>(as + k * LDA + 32 * s);
                    const float4 y = *reinterpret_cast<const float4 *>(bs + k * LDB + 32 * s);
                    a[4 * s] = x.x; a[4 * s + 1] = x.y; a[4 * s + 2] = x.z; a[4 * s + 3] = x.w;
                    b[4 * s] = y.x; b[4 * s + 1] = y.y; b[4 * s + 2] = y.z; b[4 * s + 3] = y.w;
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i * 8 + j] = __builtin_fmaf(a[i], b[j], acc[i * 8 + j]);
            if (!LDS) asm volatile("" : "+v"(a[0]), "+v"(b[0]));
        }
    }
    float s = 0.0f;
    for (int i = 0; i < 64; ++i) s += acc[i];
    out[blockIdx.x * THREADS + threadIdx.x] = s;
}

__global__ __launch_bounds__(THREADS) void mfma_f32_32_k(float *out, float x, int iters) {
    f32x16 acc[4];
    for (int j = 0; j < 4; ++j) for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    const float a = x * threadIdx.x, b = x + threadIdx.x;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.0f;
    for (int j = 0; j < 4; ++j) for (int r = 0; r < 16; ++r) s += acc[j][r];
    out[blockIdx.x * THREADS + threadIdx.x] = s;
}

// One dependent accumulation chain per wave (each MFMA reads the previous
// one's result), for the issue rate of back-to-back dependent MFMAs.
__global__ __launch_bounds__(THREADS) void mfma_f32_chain_k(float *out, float x, int iters) {
    f32x16 acc;
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const float a = x * threadIdx.x, b = x + threadIdx.x;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
    }
    float s = 0.0f;
    for (int r = 0; r < 16; ++r) s += acc[r];
    out[blockIdx.x * THREADS + threadIdx.x] = s;
}

__global__ __launch_bounds__(THREADS) void mfma_f32_16_k(float *out, float x, int iters) {
    f32x4 acc[4];
    for (int j = 0; j < 4; ++j) for (int r = 0; r < 4; ++r) acc[j][r] = 0.0f;
    const float a = x * threadIdx.x, b = x + threadIdx.x;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.0f;
    for (int j = 0; j < 4; ++j) for (int r = 0; r < 4; ++r) s += acc[j][r];
    out[blockIdx.x * THREADS + threadIdx.x] = s;
}

__global__ __launch_bounds__(THREADS) void mfma_bf16_k(float *out, float x, int iters) {
    f32x16 acc[4];
    for (int j = 0; j < 4; ++j) for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (__bf16)(x * (threadIdx.x + i)); b[i] = (__bf16)(x + i); }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.0f;
    for (int j = 0; j < 4; ++j) for (int r = 0; r < 16; ++r) s += acc[j][r];
    out[blockIdx.x * THREADS + threadIdx.x] = s;
}

__global__ __launch_bounds__(THREADS) void mfma_f16_k(float *out, float x, int iters) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    f32x16 acc[4];
    for (int j = 0; j < 4; ++j) for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    h8 a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (_Float16)(x * (threadIdx.x + i)); b[i] = (_Float16)(x + i); }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.0f;
    for (int j = 0; j < 4; ++j) for (int r = 0; r < 16; ++r) s += acc[j][r];
    out[blockIdx.x * THREADS + threadIdx.x] = s;
}

__global__ __launch_bounds__(THREADS) void copy_k(float4 *dst, const float4 *src, size_t n) {
    const size_t stride = (size_t)gridDim.x * THREADS;
    for (size_t i = blockIdx.x * (size_t)THREADS + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

template <class F>
static float time_ms(F launch, int reps) {
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    launch();
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    float best = 1e30f;
    for (int r = 0; r < reps; ++r) {
        CHECK(hipEventRecord(a, 0));
        launch();
        CHECK(hipEventRecord(b, 0));
        CHECK(hipEventSynchronize(b));
        float ms;
        CHECK(hipEventElapsedTime(&ms, a, b));
        if (ms < best) best = ms;
    }
    CHECK(hipEventDestroy(a));
    CHECK(hipEventDestroy(b));
    return best;
}

int main() {
    hipDeviceProp_t p;
    CHECK(hipGetDeviceProperties(&p, 0));
    int clk_khz = 0;
    CHECK(hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeClockRate, 0));
    const int cus = p.multiProcessorCount;
    const double ghz = clk_khz / 1e6;
    printf("device %s (%s): %d CUs, max engine clock %.3f GHz, LDS %zu KiB per workgroup, "
           "%.1f GiB HBM, wave %d\n", p.name, p.gcnArchName, cus, ghz,
           p.sharedMemPerBlock / 1024, p.totalGlobalMem / 1073741824.0, p.warpSize);
    const double fp32_peak = 256.0 * cus * ghz / 1e3;  // 128 fp32 FMA per clock per CU
    printf("published-form peaks at that clock: fp32 vector/matrix %.1f TFLOP/s; "
           "ridge at 8 TB/s %.1f FLOP/B\n", fp32_peak, fp32_peak * 1e12 / 8e12);

    const int blocks_cu = 8;  // 8 workgroups of 4 waves per CU = 8 waves per SIMD
    float *out;
    CHECK(hipMalloc(&out, sizeof(float) * (size_t)cus * blocks_cu * THREADS));

    // Settle the clock first: from idle it ramps over a few tens of
    // milliseconds of load.
    {
        hipEvent_t a, b;
        CHECK(hipEventCreate(&a));
        CHECK(hipEventCreate(&b));
        float total = 0.0f;
        while (total < 300.0f) {
            CHECK(hipEventRecord(a, 0));
            valu_fma_k<<<cus * 4, THREADS>>>(out, 0.999f, 1 << 16);
            CHECK(hipEventRecord(b, 0));
            CHECK(hipEventSynchronize(b));
            float ms;
            CHECK(hipEventElapsedTime(&ms, a, b));
            total += ms;
        }
        CHECK(hipEventDestroy(a));
        CHECK(hipEventDestroy(b));
    }
    for (int wps : {1, 2, 4, 8}) {
        const int blocks = cus * wps, iters = 4096;
        const float ms = time_ms([&] { valu_fma_k<<<blocks, THREADS>>>(out, 0.999f, iters); }, 5);
        const double fl = 2.0 * 16 * iters * (double)blocks * THREADS;
        printf("vector fp32 v_fmac_f32, %d wave(s) per SIMD: %.1f TFLOP/s\n", wps, fl / ms / 1e9);
    }
    for (int wps : {1, 2, 4}) {
        const int blocks = cus * wps, iters = 1024;
        const double fl = 2.0 * 64 * 16 * iters * (double)blocks * THREADS;
        float ms = time_ms([&] { valu_outer_k<false><<<blocks, THREADS>>>(out, iters); }, 10);
        const double reg = fl / ms / 1e9;
        ms = time_ms([&] { valu_outer_k<true><<<blocks, THREADS>>>(out, iters); }, 10);
        printf("vector fp32 8x8 outer product per lane, %d wave(s) per SIMD: registers %.1f, "
               "operands from LDS %.1f TFLOP/s\n", wps, reg, fl / ms / 1e9);
    }
    {
        const int blocks = cus * blocks_cu, iters = 1024;
        const double waves = (double)blocks * (THREADS / 64);
        float ms = time_ms([&] { mfma_f32_32_k<<<blocks, THREADS>>>(out, 1e-3f, iters); }, 5);
        printf("matrix fp32 v_mfma_f32_32x32x2_f32: %.1f TFLOP/s\n",
               4.0 * iters * 32 * 32 * 2 * 2 * waves / ms / 1e9);
        for (int wps : {1, 2}) {
            const int cb = cus * wps;
            ms = time_ms([&] { mfma_f32_chain_k<<<cb, THREADS>>>(out, 1e-3f, iters); }, 5);
            printf("matrix fp32 32x32x2, one dependent chain per wave, %d wave(s) per SIMD: "
                   "%.1f TFLOP/s\n", wps,
                   4.0 * iters * 32 * 32 * 2 * 2 * (double)cb * (THREADS / 64) / ms / 1e9);
        }
        ms = time_ms([&] { mfma_f32_16_k<<<blocks, THREADS>>>(out, 1e-3f, iters); }, 5);
        printf("matrix fp32 v_mfma_f32_16x16x4_f32: %.1f TFLOP/s\n",
               4.0 * iters * 16 * 16 * 4 * 2 * waves / ms / 1e9);
        ms = time_ms([&] { mfma_bf16_k<<<blocks, THREADS>>>(out, 1e-3f, iters); }, 5);
        printf("matrix bf16 v_mfma_f32_32x32x16_bf16: %.1f TFLOP/s\n",
               4.0 * iters * 32 * 32 * 16 * 2 * waves / ms / 1e9);
        ms = time_ms([&] { mfma_f16_k<<<blocks, THREADS>>>(out, 1e-3f, iters); }, 5);
        printf("matrix fp16 v_mfma_f32_32x32x16_f16: %.1f TFLOP/s\n",
               4.0 * iters * 32 * 32 * 16 * 2 * waves / ms / 1e9);
    }
    {
        const size_t n = (size_t)1 << 26;  // float4 elements: 1 GiB per buffer
        float4 *src, *dst;
        CHECK(hipMalloc(&src, n * sizeof(float4)));
        CHECK(hipMalloc(&dst, n * sizeof(float4)));
        CHECK(hipMemset(src, 0, n * sizeof(float4)));
        const float ms = time_ms([&] { copy_k<<<cus * 16, THREADS>>>(dst, src, n); }, 10);
        printf("copy 1 GiB device to device: %.1f GB/s (read + write bytes)\n",
               2.0 * n * sizeof(float4) / ms / 1e6);
        CHECK(hipFree(src));
        CHECK(hipFree(dst));
    }
    CHECK(hipFree(out));
    return 0;
}
