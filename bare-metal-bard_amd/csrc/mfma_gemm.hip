// Host side of the fp32 MFMA GEMM: SGEMM stage 9, gemm() and batched_gemm().
//
// The reference dispatches gemm() to a fast kernel only when M, N % 128 and
// K % 16 are all zero and otherwise to a 16x16 scalar kernel
// (src/gemm.cu:204-217); batched_gemm() always uses a guarded 64x64 kernel
// (src/bgemm.cu:88-97). Here one kernel template handles every shape and
// transpose in-kernel (guarded, zero-filled staging; guarded stores), and the
// host only picks the tile size from the amount of parallel work and whether
// 128-bit global loads are legal.
#include "mfma_gemm.hpp"
#include "../../include/gemm.h"
#include "../../include/kernels.h"
#include "launch.hpp"

namespace {

using bmb::MfmaTile;
using TileL = MfmaTile<256, 256, 16, 2, 4>;  // 512 lanes, 128x64 per wave
using TileM = MfmaTile<128, 128, 16, 2, 2>;  // 256 lanes, 64x64 per wave
using TileS = MfmaTile<64, 64, 16, 2, 2>;    // 256 lanes, 32x32 per wave

// Enough workgroups to give every one of the 256 CUs at least one.
constexpr long long FILL = 224;

template <bool TA, bool TB, class Tile>
void launch_tile(int batch, int M, int N, int K, float alpha, const float *A,
                 long long sA, const float *B, long long sB, float beta,
                 float *C, long long sC, hipStream_t stream, bool vec) {
    using L = bmb::MfmaLayout<TA, TB, Tile>;
    const int tiles_m = bmb::ceil_div(M, Tile::BM), tiles_n = bmb::ceil_div(N, Tile::BN);
    const dim3 grid(tiles_m * tiles_n, batch);
    bmb::allow_smem(bmb::mfma_gemm_k<TA, TB, Tile, true>, L::SMEM_BYTES);
    bmb::allow_smem(bmb::mfma_gemm_k<TA, TB, Tile, false>, L::SMEM_BYTES);
    if (vec)
        bmb::launch(bmb::mfma_gemm_k<TA, TB, Tile, true>, grid, dim3(Tile::NT),
                    L::SMEM_BYTES, stream, M, N, K, alpha, A, sA, B, sB, beta, C,
                    sC, tiles_m, tiles_n);
    else
        bmb::launch(bmb::mfma_gemm_k<TA, TB, Tile, false>, grid, dim3(Tile::NT),
                    L::SMEM_BYTES, stream, M, N, K, alpha, A, sA, B, sB, beta, C,
                    sC, tiles_m, tiles_n);
}

inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

template <bool TA, bool TB>
void dispatch(int batch, int M, int N, int K, float alpha, const float *A,
              long long sA, const float *B, long long sB, float beta, float *C,
              long long sC, hipStream_t stream) {
    if (M <= 0 || N <= 0 || batch <= 0) return;
    // 128-bit loads need the contiguous axis of each stored operand to be a
    // multiple of 4 floats, 16-byte aligned bases, and batch strides that keep
    // that alignment.
    const int a_contig = TA ? M : K, b_contig = TB ? K : N;
    const bool vec = a_contig % 4 == 0 && b_contig % 4 == 0 && al16(A) && al16(B) &&
                     (batch == 1 || (sA % 4 == 0 && sB % 4 == 0));
    auto work = [&](int bm, int bn) {
        return (long long)bmb::ceil_div(M, bm) * bmb::ceil_div(N, bn) * batch;
    };
    if (work(TileL::BM, TileL::BN) >= FILL)
        launch_tile<TA, TB, TileL>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream, vec);
    else if (work(TileM::BM, TileM::BN) >= FILL)
        launch_tile<TA, TB, TileM>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream, vec);
    else
        launch_tile<TA, TB, TileS>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream, vec);
}

void gemm_any(bool ta, bool tb, int batch, int M, int N, int K, float alpha,
              const float *A, long long sA, const float *B, long long sB,
              float beta, float *C, long long sC, hipStream_t stream) {
    if (!ta && !tb)     dispatch<false, false>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream);
    else if (!ta && tb) dispatch<false, true >(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream);
    else if (ta && !tb) dispatch<true,  false>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream);
    else                dispatch<true,  true >(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream);
}

}  // namespace

extern "C" {

void gemm(bool transA, bool transB, int M, int N, int K, float alpha,
          const float *A, const float *B, float beta, float *C,
          hipStream_t stream) {
    gemm_any(transA, transB, 1, M, N, K, alpha, A, 0, B, 0, beta, C, 0, stream);
}

void batched_gemm(bool transA, bool transB, int batch, int M, int N, int K,
                  float alpha, const float *A, long long strideA,
                  const float *B, long long strideB, float beta, float *C,
                  long long strideC, hipStream_t stream) {
    gemm_any(transA, transB, batch, M, N, K, alpha, A, strideA, B, strideB, beta,
             C, strideC, stream);
}

void sgemm_tensorcore(int M, int N, int K, float alpha, const float *A,
                      const float *B, float beta, float *C) {
    gemm_any(false, false, 1, M, N, K, alpha, A, 0, B, 0, beta, C, 0, nullptr);
}

}  // extern "C"
