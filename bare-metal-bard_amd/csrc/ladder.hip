// SGEMM ladder, stages 1-7, for gfx950.
//
// Each stage mirrors one rung of bare-metal-bard's optimisation ladder
// (src/kernels/k01..k07) as a wave64 kernel of this build's own design. They
// exist so that the id -> stage table keeps its meaning and so that the bench
// can show the ladder on this hardware; the production fp32 VALU kernel is
// stage 8 (sgemm_valu.hip) and the matrix-core kernel is stage 9.
//
// One invariant holds for every stage: each output is accumulated as
// acc = fma(a_k, b_k, acc) for k = 0..K-1 in order, starting from +0, and the
// epilogue is bmb::epilogue(). Zero padding of ragged tiles only ever adds
// fma(0, 0, acc) = acc. So every stage is bit-identical to every other and to
// the CPU oracle's sequential fmaf loop.
#include "common.hpp"
#include "../../include/kernels.h"
#include "launch.hpp"

using bmb::ceil_div;
using bmb::epilogue;
using bmb::fma_rn;

namespace {

// ---------------------------------------------------------------- stage 1
// One lane per output; threadIdx.x walks ROWS, so a wave's 64 lanes read A at
// addresses K floats apart (uncoalesced), as in src/kernels/k01_naive.cu:18-30.
__global__ void naive_k(int M, int N, int K, float alpha, const float *A,
                        const float *B, float beta, float *C) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    const int col = blockIdx.y * blockDim.y + threadIdx.y;
    if (row >= M || col >= N) return;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k)
        acc = fma_rn(A[(size_t)row * K + k], B[(size_t)k * N + col], acc);
    const size_t idx = (size_t)row * N + col;
    C[idx] = epilogue(acc, alpha, beta, &C[idx]);
}

// ---------------------------------------------------------------- stage 2
// threadIdx.x walks COLUMNS: a wave reads 64 consecutive floats of B (256 B)
// and broadcasts one A element (src/kernels/k02_coalesced.cu:19-32).
__global__ void coalesced_k(int M, int N, int K, float alpha, const float *A,
                            const float *B, float beta, float *C) {
    const int col = blockIdx.x * blockDim.x + threadIdx.x;
    const int row = blockIdx.y * blockDim.y + threadIdx.y;
    if (row >= M || col >= N) return;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k)
        acc = fma_rn(A[(size_t)row * K + k], B[(size_t)k * N + col], acc);
    const size_t idx = (size_t)row * N + col;
    C[idx] = epilogue(acc, alpha, beta, &C[idx]);
}

// ---------------------------------------------------------------- stage 3
// 32x32 LDS tiles, two barriers per chunk, guarded zero fill
// (src/kernels/k03_smem.cu:26-68). Bs rows are 32 floats, so the 64 lanes of
// a wave (two rows of 32 threads) read two different Bs rows: no conflict.
template <int BS>
__global__ __launch_bounds__(BS *BS) void smem_k(int M, int N, int K, float alpha,
                                                const float *A, const float *B,
                                                float beta, float *C) {
    __shared__ float As[BS][BS + 1];
    __shared__ float Bs[BS][BS];
    const int col = threadIdx.x, row = threadIdx.y;
    const int cRow = blockIdx.y * BS, cCol = blockIdx.x * BS;
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += BS) {
        As[row][col] = (cRow + row < M && k0 + col < K)
                           ? A[(size_t)(cRow + row) * K + k0 + col] : 0.0f;
        Bs[row][col] = (k0 + row < K && cCol + col < N)
                           ? B[(size_t)(k0 + row) * N + cCol + col] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < BS; ++k) acc = fma_rn(As[row][k], Bs[k][col], acc);
        __syncthreads();
    }
    if (cRow + row < M && cCol + col < N) {
        const size_t idx = (size_t)(cRow + row) * N + cCol + col;
        C[idx] = epilogue(acc, alpha, beta, &C[idx]);
    }
}

// ---------------------------------------------------------------- stage 4
// 1-D register tiling: each lane owns TM outputs of one column, holding the B
// element in a register across them (src/kernels/k04_tile1d.cu:24-83). One
// wave spans the 64 columns of the tile, so B reads are conflict-free and A
// reads are wave-wide broadcasts.
template <int BM, int BN, int BK, int TM>
__global__ __launch_bounds__((BM / TM) * BN) void tile1d_k(
    int M, int N, int K, float alpha, const float *A, const float *B,
    float beta, float *C) {
    constexpr int NT = (BM / TM) * BN;
    __shared__ float As[BK][BM + 1];
    __shared__ float Bs[BK][BN];
    const int tid = threadIdx.x;
    const int tc = tid % BN, tr = tid / BN;
    const int cRow = blockIdx.y * BM, cCol = blockIdx.x * BN;
    float acc[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) acc[i] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += BK) {
        for (int e = tid; e < BM * BK; e += NT) {
            const int m = e / BK, k = e % BK;
            const int gm = cRow + m, gk = k0 + k;
            As[k][m] = (gm < M && gk < K) ? A[(size_t)gm * K + gk] : 0.0f;
        }
        for (int e = tid; e < BK * BN; e += NT) {
            const int k = e / BN, n = e % BN;
            const int gk = k0 + k, gn = cCol + n;
            Bs[k][n] = (gk < K && gn < N) ? B[(size_t)gk * N + gn] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < BK; ++k) {
            const float b = Bs[k][tc];
#pragma unroll
            for (int i = 0; i < TM; ++i) acc[i] = fma_rn(As[k][tr * TM + i], b, acc[i]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int r = cRow + tr * TM + i, c = cCol + tc;
        if (r < M && c < N) {
            const size_t idx = (size_t)r * N + c;
            C[idx] = epilogue(acc[i], alpha, beta, &C[idx]);
        }
    }
}

// ---------------------------------------------------------------- stage 5
// 2-D register tiling, 8x8 outputs per lane as an outer product per k
// (src/kernels/k05_tile2d.cu:27-105). Fully guarded: any M, N, K. Stages 6
// and 7 fall back to it for shapes their vector paths cannot take, as the
// reference does (k06_vectorized.cu:119-122, k07_warptile.cu:180-183).
template <int BM, int BN, int BK, int TM, int TN>
__global__ __launch_bounds__((BM / TM) * (BN / TN)) void tile2d_k(
    int M, int N, int K, float alpha, const float *A, const float *B,
    float beta, float *C) {
    constexpr int NT = (BM / TM) * (BN / TN);
    __shared__ float As[BK][BM + 4];
    __shared__ float Bs[BK][BN + 4];
    const int tid = threadIdx.x;
    const int tc = tid % (BN / TN), tr = tid / (BN / TN);
    const int cRow = blockIdx.y * BM, cCol = blockIdx.x * BN;
    float acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += BK) {
        for (int e = tid; e < BM * BK; e += NT) {
            const int m = e / BK, k = e % BK;
            const int gm = cRow + m, gk = k0 + k;
            As[k][m] = (gm < M && gk < K) ? A[(size_t)gm * K + gk] : 0.0f;
        }
        for (int e = tid; e < BK * BN; e += NT) {
            const int k = e / BN, n = e % BN;
            const int gk = k0 + k, gn = cCol + n;
            Bs[k][n] = (gk < K && gn < N) ? B[(size_t)gk * N + gn] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < BK; ++k) {
            float ra[TM], rb[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) ra[i] = As[k][tr * TM + i];
#pragma unroll
            for (int j = 0; j < TN; ++j) rb[j] = Bs[k][tc * TN + j];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = fma_rn(ra[i], rb[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int r = cRow + tr * TM + i;
        if (r >= M) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int c = cCol + tc * TN + j;
            if (c < N) {
                const size_t idx = (size_t)r * N + c;
                C[idx] = epilogue(acc[i][j], alpha, beta, &C[idx]);
            }
        }
    }
}

// ---------------------------------------------------------------- stage 6
// 128-bit global loads, A stored transposed in LDS so each lane's TM rows are
// one vector read (src/kernels/k06_vectorized.cu:38-111). Needs M, N % 128
// and K % 8 (and hence 16-byte aligned rows).
template <int BM, int BN, int BK, int TM, int TN>
__global__ __launch_bounds__((BM / TM) * (BN / TN)) void vectorized_k(
    int M, int N, int K, float alpha, const float *A, const float *B,
    float beta, float *C) {
    constexpr int NT = (BM / TM) * (BN / TN);
    __shared__ float As[BK][BM];
    __shared__ float Bs[BK][BN];
    const int tid = threadIdx.x;
    const int tc = tid % (BN / TN), tr = tid / (BN / TN);
    const int cRow = blockIdx.y * BM, cCol = blockIdx.x * BN;
    float acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += BK) {
        for (int e = tid; e < BM * BK / 4; e += NT) {
            const int m = e / (BK / 4), kc = (e % (BK / 4)) * 4;
            const float4 a = bmb::ld4(&A[(size_t)(cRow + m) * K + k0 + kc]);
            As[kc + 0][m] = a.x; As[kc + 1][m] = a.y;
            As[kc + 2][m] = a.z; As[kc + 3][m] = a.w;
        }
        for (int e = tid; e < BK * BN / 4; e += NT) {
            const int k = e / (BN / 4), nc = (e % (BN / 4)) * 4;
            bmb::st4(&Bs[k][nc], bmb::ld4(&B[(size_t)(k0 + k) * N + cCol + nc]));
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < BK; ++k) {
            float ra[TM], rb[TN];
#pragma unroll
            for (int i = 0; i < TM; i += 4) {
                const float4 v = bmb::ld4(&As[k][tr * TM + i]);
                ra[i] = v.x; ra[i + 1] = v.y; ra[i + 2] = v.z; ra[i + 3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < TN; j += 4) {
                const float4 v = bmb::ld4(&Bs[k][tc * TN + j]);
                rb[j] = v.x; rb[j + 1] = v.y; rb[j + 2] = v.z; rb[j + 3] = v.w;
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = fma_rn(ra[i], rb[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const size_t r = (size_t)(cRow + tr * TM + i);
#pragma unroll
        for (int j = 0; j < TN; j += 4) {
            float *dst = &C[r * N + cCol + tc * TN + j];
            float4 o;
            if (beta == 0.0f) o = make_float4(0.f, 0.f, 0.f, 0.f);
            else o = bmb::ld4(dst);
            o.x = epilogue(acc[i][j + 0], alpha, beta, &o.x);
            o.y = epilogue(acc[i][j + 1], alpha, beta, &o.y);
            o.z = epilogue(acc[i][j + 2], alpha, beta, &o.z);
            o.w = epilogue(acc[i][j + 3], alpha, beta, &o.w);
            bmb::st4(dst, o);
        }
    }
}

// ---------------------------------------------------------------- stage 7
// Wave-level tiling for wave64 (src/kernels/k07_warptile.cu:42-162 is the
// warp32 original). A 256-lane block owns 128x128; each wave owns 64x64 and
// each lane an 8x8 patch made of two 4-row by two 4-column strips placed 32
// apart. With that split the 16 lanes that share a row of the wave's lane grid
// read 16 consecutive float4 of Bs (256 B, every bank once), so the per-k LDS
// reads are conflict-free without padding. Needs M, N % 128 and K % 16.
template <int BM, int BN, int BK>
__global__ __launch_bounds__(256) void warptile_k(int M, int N, int K,
                                                  float alpha, const float *A,
                                                  const float *B, float beta,
                                                  float *C) {
    constexpr int NT = 256;
    __shared__ float As[BK][BM];
    __shared__ float Bs[BK][BN];
    const int tid = threadIdx.x;
    const int wave = tid / 64, lane = tid % 64;
    const int wm = (wave / 2) * 64, wn = (wave % 2) * 64;
    const int lr = lane / 8, lc = lane % 8;  // 8x8 lane grid over 64x64
    const int cRow = blockIdx.y * BM, cCol = blockIdx.x * BN;
    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += BK) {
        for (int e = tid; e < BM * BK / 4; e += NT) {
            const int m = e / (BK / 4), kc = (e % (BK / 4)) * 4;
            const float4 a = bmb::ld4(&A[(size_t)(cRow + m) * K + k0 + kc]);
            As[kc + 0][m] = a.x; As[kc + 1][m] = a.y;
            As[kc + 2][m] = a.z; As[kc + 3][m] = a.w;
        }
        for (int e = tid; e < BK * BN / 4; e += NT) {
            const int k = e / (BN / 4), nc = (e % (BN / 4)) * 4;
            bmb::st4(&Bs[k][nc], bmb::ld4(&B[(size_t)(k0 + k) * N + cCol + nc]));
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < BK; ++k) {
            float ra[8], rb[8];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float4 a = bmb::ld4(&As[k][wm + h * 32 + lr * 4]);
                ra[h * 4 + 0] = a.x; ra[h * 4 + 1] = a.y;
                ra[h * 4 + 2] = a.z; ra[h * 4 + 3] = a.w;
                const float4 b = bmb::ld4(&Bs[k][wn + h * 32 + lc * 4]);
                rb[h * 4 + 0] = b.x; rb[h * 4 + 1] = b.y;
                rb[h * 4 + 2] = b.z; rb[h * 4 + 3] = b.w;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = fma_rn(ra[i], rb[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const size_t r = (size_t)(cRow + wm + (i / 4) * 32 + lr * 4 + i % 4);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float *dst = &C[r * N + cCol + wn + h * 32 + lc * 4];
            float4 o;
            if (beta == 0.0f) o = make_float4(0.f, 0.f, 0.f, 0.f);
            else o = bmb::ld4(dst);
            o.x = epilogue(acc[i][h * 4 + 0], alpha, beta, &o.x);
            o.y = epilogue(acc[i][h * 4 + 1], alpha, beta, &o.y);
            o.z = epilogue(acc[i][h * 4 + 2], alpha, beta, &o.z);
            o.w = epilogue(acc[i][h * 4 + 3], alpha, beta, &o.w);
            bmb::st4(dst, o);
        }
    }
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

void sgemm_naive(int M, int N, int K, float alpha, const float *A,
                 const float *B, float beta, float *C) {
    if (M <= 0 || N <= 0) return;
    dim3 block(16, 16);
    dim3 grid(ceil_div(M, 16), ceil_div(N, 16));
    bmb::launch(naive_k, grid, block, 0, nullptr, M, N, K, alpha, A, B, beta, C);
}

void sgemm_coalesced(int M, int N, int K, float alpha, const float *A,
                     const float *B, float beta, float *C) {
    if (M <= 0 || N <= 0) return;
    dim3 block(64, 4);
    dim3 grid(ceil_div(N, 64), ceil_div(M, 4));
    bmb::launch(coalesced_k, grid, block, 0, nullptr, M, N, K, alpha, A, B, beta, C);
}

void sgemm_smem(int M, int N, int K, float alpha, const float *A,
                const float *B, float beta, float *C) {
    if (M <= 0 || N <= 0) return;
    constexpr int BS = 32;
    dim3 grid(ceil_div(N, BS), ceil_div(M, BS));
    bmb::launch(smem_k<BS>, grid, dim3(BS, BS), 0, nullptr, M, N, K, alpha, A, B, beta, C);
}

void sgemm_tile1d(int M, int N, int K, float alpha, const float *A,
                  const float *B, float beta, float *C) {
    if (M <= 0 || N <= 0) return;
    constexpr int BM = 64, BN = 64, BK = 8, TM = 8;
    dim3 grid(ceil_div(N, BN), ceil_div(M, BM));
    bmb::launch(tile1d_k<BM, BN, BK, TM>, grid, dim3((BM / TM) * BN), 0, nullptr,
                M, N, K, alpha, A, B, beta, C);
}

void sgemm_tile2d(int M, int N, int K, float alpha, const float *A,
                  const float *B, float beta, float *C) {
    if (M <= 0 || N <= 0) return;
    constexpr int BM = 128, BN = 128, BK = 8, TM = 8, TN = 8;
    dim3 grid(ceil_div(N, BN), ceil_div(M, BM));
    bmb::launch(tile2d_k<BM, BN, BK, TM, TN>, grid, dim3((BM / TM) * (BN / TN)),
                0, nullptr, M, N, K, alpha, A, B, beta, C);
}

void sgemm_vectorized(int M, int N, int K, float alpha, const float *A,
                      const float *B, float beta, float *C) {
    constexpr int BM = 128, BN = 128, BK = 8, TM = 8, TN = 8;
    if (M % BM || N % BN || K % BK || !aligned16(A) || !aligned16(B) ||
        !aligned16(C) || M <= 0 || N <= 0) {
        sgemm_tile2d(M, N, K, alpha, A, B, beta, C);
        return;
    }
    dim3 grid(N / BN, M / BM);
    bmb::launch(vectorized_k<BM, BN, BK, TM, TN>, grid, dim3((BM / TM) * (BN / TN)),
                0, nullptr, M, N, K, alpha, A, B, beta, C);
}

void sgemm_warptile(int M, int N, int K, float alpha, const float *A,
                    const float *B, float beta, float *C) {
    constexpr int BM = 128, BN = 128, BK = 16;
    if (M % BM || N % BN || K % BK || !aligned16(A) || !aligned16(B) ||
        !aligned16(C) || M <= 0 || N <= 0) {
        sgemm_tile2d(M, N, K, alpha, A, B, beta, C);
        return;
    }
    dim3 grid(N / BN, M / BM);
    bmb::launch(warptile_k<BM, BN, BK>, grid, dim3(256), 0, nullptr, M, N, K,
                alpha, A, B, beta, C);
}

}  // extern "C"
