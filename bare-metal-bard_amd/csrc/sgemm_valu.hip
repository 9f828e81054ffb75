// Stage 8: the true-fp32 VALU SGEMM ("dbuffer" in the reference ladder,
// src/kernels/k08_doublebuffer.cu:40-216), designed for gfx950.
//
// Numerics. Each output is acc = fma(a_k, b_k, acc) for k = 0..K-1 in order,
// one v_fma_f32 per term, then bmb::epilogue(). That is exactly the CPU
// oracle's sequential fmaf loop, so this kernel is bit-identical to it (and to
// stages 1-7). Split-K, reassociation or MFMA would all break that, which is
// why this stage stays on the vector ALU.
//
// Ceiling. This build never emits packed fp32 (v_pk_fma_f32). A single wave
// issues one v_fmac_f32 every 4 clocks, but several waves on one SIMD issue
// concurrently: a loop of nothing but FMAs reaches ~112 TFLOP/s (71% of the
// 157.3 TFLOP/s vector peak) with 8 waves per SIMD, which is the practical
// ceiling of a kernel that also has to read its operands from LDS.
//
// Structure.
//   * 256 lanes = 4 wave64 per workgroup, 128x128 output tile, BK = 16.
//   * Each wave owns a 64x64 quadrant; each lane an 8x8 patch made of two
//     4-row strips 32 rows apart and two 4-column strips 32 columns apart.
//     The 8 lanes sharing a strip row read one float4 each of a 32-float
//     LDS span, so every per-k LDS read is conflict-free and 128-bit.
//   * A is stored k-major in LDS (As[k][m], +4 pad so the transposing
//     stores spread over all banks); B is stored as it lies (Bs[k][n]).
//   * Double-buffered LDS with the next tile prefetched into registers while
//     the current one is consumed: one barrier per BK chunk.
//   * Ragged M, N, K are handled in-kernel: guarded, zero-filled loads and
//     guarded stores. There is no fallback kernel. VEC selects aligned 128-bit
//     global access when K % 4 == 0, N % 4 == 0 and the pointers are 16-byte
//     aligned; otherwise interior chunks still use dword-aligned 128-bit loads
//     and only a chunk that straddles a row end uses 32-bit loads.
//   * Workgroup ids are remapped so the tiles one XCD runs share panels.
#include "common.hpp"
#include "../../include/kernels.h"
#include "launch.hpp"

using bmb::epilogue;
using bmb::fma_rn;

namespace {

constexpr int BM = 128, BN = 128, BK = 16, NT = 256;
constexpr int APAD = 4;
constexpr int LDA = BM + APAD;  // As row (one k) width
constexpr int LDB = BN;         // Bs row width

// Per-thread share of one tile: A is BM x BK = 2048 floats, B is BK x BN =
// 2048 floats, i.e. 8 floats of each per lane.
struct Prefetch {
    float a[8];
    float b[8];
};

template <bool VEC>
__device__ __forceinline__ void load_tile(Prefetch &p, const float *A,
                                          const float *B, int M, int N, int K,
                                          int cRow, int cCol, int k0, int tid) {
    // A chunk e = tid + r*NT (r = 0,1): row m = e / 4, k offset (e % 4) * 4.
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int e = tid + r * NT;
        const int m = e >> 2, kc = (e & 3) * 4;
        const int gm = cRow + m, gk = k0 + kc;
        if (VEC) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gm < M && gk < K) v = bmb::ld4(&A[(size_t)gm * K + gk]);
            p.a[r * 4 + 0] = v.x; p.a[r * 4 + 1] = v.y;
            p.a[r * 4 + 2] = v.z; p.a[r * 4 + 3] = v.w;
        } else if (gm < M && gk + 3 < K) {
            // Interior chunk of an unaligned row: one dword-aligned 128-bit load.
            float4 v;
            __builtin_memcpy(&v, &A[(size_t)gm * K + gk], sizeof(v));
            p.a[r * 4 + 0] = v.x; p.a[r * 4 + 1] = v.y;
            p.a[r * 4 + 2] = v.z; p.a[r * 4 + 3] = v.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                p.a[r * 4 + i] = (gm < M && gk + i < K) ? A[(size_t)gm * K + gk + i] : 0.0f;
        }
    }
    // B chunk e: row k = e / 32, n offset (e % 32) * 4.
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int e = tid + r * NT;
        const int k = e >> 5, nc = (e & 31) * 4;
        const int gk = k0 + k, gn = cCol + nc;
        if (VEC) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gk < K && gn < N) v = bmb::ld4(&B[(size_t)gk * N + gn]);
            p.b[r * 4 + 0] = v.x; p.b[r * 4 + 1] = v.y;
            p.b[r * 4 + 2] = v.z; p.b[r * 4 + 3] = v.w;
        } else if (gk < K && gn + 3 < N) {
            float4 v;
            __builtin_memcpy(&v, &B[(size_t)gk * N + gn], sizeof(v));
            p.b[r * 4 + 0] = v.x; p.b[r * 4 + 1] = v.y;
            p.b[r * 4 + 2] = v.z; p.b[r * 4 + 3] = v.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                p.b[r * 4 + i] = (gk < K && gn + i < N) ? B[(size_t)gk * N + gn + i] : 0.0f;
        }
    }
}

__device__ __forceinline__ void store_tile(const Prefetch &p, float *As,
                                           float *Bs, int tid) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int e = tid + r * NT;
        const int m = e >> 2, kc = (e & 3) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) As[(kc + i) * LDA + m] = p.a[r * 4 + i];
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int e = tid + r * NT;
        const int k = e >> 5, nc = (e & 31) * 4;
        bmb::st4(&Bs[k * LDB + nc],
                 make_float4(p.b[r * 4 + 0], p.b[r * 4 + 1], p.b[r * 4 + 2], p.b[r * 4 + 3]));
    }
}

template <bool VEC>
__global__ __launch_bounds__(NT) void sgemm_valu_k(int M, int N, int K,
                                                   float alpha,
                                                   const float *__restrict__ A,
                                                   const float *__restrict__ B,
                                                   float beta, float *C,
                                                   int tiles_m, int tiles_n) {
    __shared__ float As[2][BK * LDA];
    __shared__ float Bs[2][BK * LDB];

    const int nblocks = tiles_m * tiles_n;
    int tm, tn;
    bmb::group_tile(bmb::xcd_remap(blockIdx.x, nblocks), tiles_m, tiles_n, 8, tm, tn);
    const int cRow = tm * BM, cCol = tn * BN;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int lr = lane >> 3, lc = lane & 7;

    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;

    const int nkt = (K + BK - 1) / BK;
    Prefetch pf;
    if (nkt > 0) {
        load_tile<VEC>(pf, A, B, M, N, K, cRow, cCol, 0, tid);
        store_tile(pf, As[0], Bs[0], tid);
    }
    __syncthreads();

    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) load_tile<VEC>(pf, A, B, M, N, K, cRow, cCol, (kt + 1) * BK, tid);

        const float *as = As[cur] + wm + lr * 4;
        const float *bs = Bs[cur] + wn + lc * 4;
        // Unrolled by 2 only: a full unroll lets the scheduler hoist all 16
        // k-steps' LDS reads and pushes the lane past 256 VGPRs.
#pragma unroll 2
        for (int k = 0; k < BK; ++k) {
            float ra[8], rb[8];
            const float4 a0 = bmb::ld4(as + k * LDA);
            const float4 a1 = bmb::ld4(as + k * LDA + 32);
            const float4 b0 = bmb::ld4(bs + k * LDB);
            const float4 b1 = bmb::ld4(bs + k * LDB + 32);
            ra[0] = a0.x; ra[1] = a0.y; ra[2] = a0.z; ra[3] = a0.w;
            ra[4] = a1.x; ra[5] = a1.y; ra[6] = a1.z; ra[7] = a1.w;
            rb[0] = b0.x; rb[1] = b0.y; rb[2] = b0.z; rb[3] = b0.w;
            rb[4] = b1.x; rb[5] = b1.y; rb[6] = b1.z; rb[7] = b1.w;
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = fma_rn(ra[i], rb[j], acc[i][j]);
        }

        if (more) store_tile(pf, As[cur ^ 1], Bs[cur ^ 1], tid);
        __syncthreads();
    }

    // Epilogue. Row of acc[i][.]: wm + (i/4)*32 + lr*4 + i%4; column of
    // acc[.][h*4+x]: wn + h*32 + lc*4 + x.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = cRow + wm + (i >> 2) * 32 + lr * 4 + (i & 3);
        if (r >= M) continue;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c = cCol + wn + h * 32 + lc * 4;
            float *dst = C + (size_t)r * N + c;
            if (VEC && c + 3 < N) {
                float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
                if (beta != 0.0f) o = bmb::ld4(dst);
                o.x = epilogue(acc[i][h * 4 + 0], alpha, beta, &o.x);
                o.y = epilogue(acc[i][h * 4 + 1], alpha, beta, &o.y);
                o.z = epilogue(acc[i][h * 4 + 2], alpha, beta, &o.z);
                o.w = epilogue(acc[i][h * 4 + 3], alpha, beta, &o.w);
                bmb::st4(dst, o);
            } else {
#pragma unroll
                for (int x = 0; x < 4; ++x)
                    if (c + x < N) dst[x] = epilogue(acc[i][h * 4 + x], alpha, beta, &dst[x]);
            }
        }
    }
}

}  // namespace

extern "C" void sgemm_doublebuffer(int M, int N, int K, float alpha,
                                   const float *A, const float *B, float beta,
                                   float *C) {
    if (M <= 0 || N <= 0) return;
    const int tiles_m = bmb::ceil_div(M, BM), tiles_n = bmb::ceil_div(N, BN);
    const bool vec = (K % 4 == 0) && (N % 4 == 0) && (((uintptr_t)A & 15) == 0) &&
                     (((uintptr_t)B & 15) == 0) && (((uintptr_t)C & 15) == 0);
    const dim3 grid(tiles_m * tiles_n);
    if (vec)
        bmb::launch(sgemm_valu_k<true>, grid, dim3(NT), 0, nullptr, M, N, K,
                    alpha, A, B, beta, C, tiles_m, tiles_n);
    else
        bmb::launch(sgemm_valu_k<false>, grid, dim3(NT), 0, nullptr, M, N, K,
                    alpha, A, B, beta, C, tiles_m, tiles_n);
}
