// SGEMM stage 10: fp32 GEMM from three bf16 matrix-core products.
//
// Each fp32 operand x is split as hi = bf16(x), lo = bf16(x - hi) (both
// round-to-nearest-even; x - hi is exact in fp32), so x = hi + lo up to
// 2^-18 |x|. The product a*b is taken as hi_a*hi_b + hi_a*lo_b + lo_a*hi_b,
// dropping lo_a*lo_b (<= 2^-18 |ab|). Each bf16 x bf16 product is exact in
// fp32 and accumulation is fp32 on v_mfma_f32_32x32x16_bf16, so the error is a
// few 2^-17 per product -- well inside the 1e-4 normwise bar, an order of
// magnitude better than the TF32 stage it stands in for (src/kernels/
// k09_tensorcore.cu:119-128 rounds to 10 mantissa bits), and 3 bf16 MFMAs
// cost 96 cycles per 32x32x16 step against 512 for fp32 MFMA.
//
// MFMA operand layout (v_mfma_f32_32x32x16_bf16): lane l supplies 8
// consecutive-k bf16 of row (A) or column (B) l % 32, k = 8 * (l / 32) + 0..7;
// the D layout matches v_mfma_f32_32x32x2_f32.
//
// LDS: four bf16 planes (A hi, A lo, B hi, B lo), each stored [row][k] with k
// contiguous (row = m for A, n for B), so every fragment is one 128-bit read.
// The row stride is BK + 8 bf16 (48 B at BK = 16): 16 consecutive rows of a
// 128-bit read then start on 16 distinct 4-bank groups. An operand whose k
// axis is contiguous in global memory is staged with 128-bit loads; one whose
// k axis is strided is staged with 4 scalar loads per lane that are coalesced
// across lanes (consecutive lanes take consecutive m or n).
#include "common.hpp"
#include "../../include/kernels.h"
#include "launch.hpp"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256, BK = 16, NT = 512;
constexpr int WAVES_N = 4;
constexpr int WM = 128, WN = 64, FM = WM / 32, FN = WN / 32;
constexpr int LDK = BK + 8;              // bf16 per LDS row
constexpr int A_PLANE = BM * LDK;        // bf16 per A plane
constexpr int B_PLANE = BN * LDK;
constexpr int STAGE = 2 * A_PLANE + 2 * B_PLANE;  // bf16 per stage
constexpr size_t SMEM_BYTES = 2 * (size_t)STAGE * sizeof(__bf16);
constexpr int A_PER_T = BM * BK / 4 / NT;  // 4-element chunks per lane
constexpr int B_PER_T = BN * BK / 4 / NT;
static_assert(A_PER_T == 2 && B_PER_T == 2, "staging split");

struct Chunk {
    float v[4];
};

// Chunk e of an operand tile with R rows (m or n) and BK columns (k).
// Returns the tile row and the first k of the chunk. With a k-contiguous
// operand consecutive lanes walk k first (128-bit loads); with a k-strided
// one they walk rows first (coalesced scalar loads).
template <bool KCONTIG, int R>
__device__ __forceinline__ void chunk_pos(int e, int &row, int &kc) {
    if (KCONTIG) { row = e / (BK / 4); kc = (e % (BK / 4)) * 4; }
    else         { row = e % R;        kc = (e / R) * 4; }
}

// Loads 4 k-consecutive elements of logical row `grow` starting at `gk` from
// a stored matrix. KCONTIG: stored [rows][K] (element (r,k) at r*K + k);
// otherwise stored [K][rows] (element at k*rows + r).
template <bool KCONTIG, bool VEC>
__device__ __forceinline__ Chunk load4(const float *P, int rows, int K,
                                       int grow, int gk) {
    Chunk c = {{0.f, 0.f, 0.f, 0.f}};
    if (grow >= rows) return c;
    if (KCONTIG) {
        const float *p = P + (size_t)grow * K + gk;
        if (VEC) {
            if (gk < K) {
                const float4 v = bmb::ld4(p);
                c.v[0] = v.x; c.v[1] = v.y; c.v[2] = v.z; c.v[3] = v.w;
            }
        } else if (gk + 3 < K) {
            // Interior chunk of an unaligned row: one dword-aligned 128-bit load.
            float4 v;
            __builtin_memcpy(&v, p, sizeof(v));
            c.v[0] = v.x; c.v[1] = v.y; c.v[2] = v.z; c.v[3] = v.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (gk + i < K) c.v[i] = p[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (gk + i < K) c.v[i] = P[(size_t)(gk + i) * rows + grow];
    }
    return c;
}

__device__ __forceinline__ void split_store(const Chunk &c, __bf16 *hi,
                                            __bf16 *lo) {
    bf16x4 h, l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 x = (__bf16)c.v[i];
        h[i] = x;
        l[i] = (__bf16)(c.v[i] - (float)x);
    }
    *reinterpret_cast<bf16x4 *>(hi) = h;
    *reinterpret_cast<bf16x4 *>(lo) = l;
}

// TA: A stored K x M (m contiguous, k strided); else M x K (k contiguous).
// TB: B stored N x K (k contiguous); else K x N (k strided).
template <bool TA, bool TB, bool VEC>
__global__ __launch_bounds__(NT) void bf16x3_k(int M, int N, int K, float alpha,
                                               const float *__restrict__ A,
                                               const float *__restrict__ B,
                                               float beta, float *C,
                                               int tiles_m, int tiles_n) {
    extern __shared__ __bf16 lds[];
    constexpr bool AK = !TA, BKc = TB;  // is the k axis contiguous?
    int tm, tn;
    bmb::group_tile(bmb::xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m,
                    tiles_n, 8, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = (wave / WAVES_N) * WM, wn = (wave % WAVES_N) * WN;
    const int l32 = lane & 31, half = lane >> 5;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int fi = 0; fi < FM; ++fi)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fi][fn][r] = 0.0f;

    Chunk ga[A_PER_T], gb[B_PER_T];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            int row, kc;
            chunk_pos<AK, BM>(tid + i * NT, row, kc);
            ga[i] = load4<AK, VEC>(A, M, K, m0 + row, k0 + kc);
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            int row, kc;
            chunk_pos<BKc, BN>(tid + i * NT, row, kc);
            gb[i] = load4<BKc, VEC>(B, N, K, n0 + row, k0 + kc);
        }
    };
    auto sstore = [&](__bf16 *st) {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            int row, kc;
            chunk_pos<AK, BM>(tid + i * NT, row, kc);
            split_store(ga[i], st + row * LDK + kc, st + A_PLANE + row * LDK + kc);
        }
        __bf16 *bst = st + 2 * A_PLANE;
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            int row, kc;
            chunk_pos<BKc, BN>(tid + i * NT, row, kc);
            split_store(gb[i], bst + row * LDK + kc, bst + B_PLANE + row * LDK + kc);
        }
    };

    const int nkt = (K + BK - 1) / BK;
    if (nkt > 0) {
        gload(0);
        sstore(lds);
    }
    __syncthreads();

    for (int kt = 0; kt < nkt; ++kt) {
        const __bf16 *st = lds + (kt & 1) * STAGE;
        const bool more = kt + 1 < nkt;
        if (more) gload((kt + 1) * BK);

        bf16x8 ah[FM], al[FM], bh[FN], bl[FN];
#pragma unroll
        for (int fi = 0; fi < FM; ++fi) {
            const int off = (wm + fi * 32 + l32) * LDK + half * 8;
            ah[fi] = *reinterpret_cast<const bf16x8 *>(st + off);
            al[fi] = *reinterpret_cast<const bf16x8 *>(st + A_PLANE + off);
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const int off = 2 * A_PLANE + (wn + fn * 32 + l32) * LDK + half * 8;
            bh[fn] = *reinterpret_cast<const bf16x8 *>(st + off);
            bl[fn] = *reinterpret_cast<const bf16x8 *>(st + B_PLANE + off);
        }
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
                acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[fi], bh[fn], acc[fi][fn], 0, 0, 0);
                acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[fi], bl[fn], acc[fi][fn], 0, 0, 0);
                acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[fi], bh[fn], acc[fi][fn], 0, 0, 0);
            }

        if (more) sstore(lds + ((kt + 1) & 1) * STAGE);
        __syncthreads();
    }

#pragma unroll
    for (int fi = 0; fi < FM; ++fi)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const int col = n0 + wn + fn * 32 + l32;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + fi * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (row < M) {
                    float *dst = C + (size_t)row * N + col;
                    *dst = bmb::epilogue(acc[fi][fn][r], alpha, beta, dst);
                }
            }
        }
}

template <bool VEC>
void launch_nn(int M, int N, int K, float alpha, const float *A, const float *B,
               float beta, float *C) {
    auto kern = bf16x3_k<false, false, VEC>;
    bmb::allow_smem(kern, SMEM_BYTES);
    const int tiles_m = bmb::ceil_div(M, BM), tiles_n = bmb::ceil_div(N, BN);
    bmb::launch(kern, dim3(tiles_m * tiles_n), dim3(NT), SMEM_BYTES, nullptr, M,
                N, K, alpha, A, B, beta, C, tiles_m, tiles_n);
}

}  // namespace

extern "C" void sgemm_mfma_bf16x3(int M, int N, int K, float alpha,
                                  const float *A, const float *B, float beta,
                                  float *C) {
    if (M <= 0 || N <= 0) return;
    const bool vec = K % 4 == 0 && (((uintptr_t)A & 15) == 0);
    if (vec) launch_nn<true>(M, N, K, alpha, A, B, beta, C);
    else     launch_nn<false>(M, N, K, alpha, A, B, beta, C);
}
