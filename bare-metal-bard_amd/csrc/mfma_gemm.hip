// Host side of the fp32 MFMA GEMM: SGEMM stage 9, gemm() and batched_gemm().
//
// The reference dispatches gemm() to a fast kernel only when M, N % 128 and
// K % 16 are all zero and otherwise to a 16x16 scalar kernel
// (src/gemm.cu:204-217); batched_gemm() always uses a guarded 64x64 kernel
// (src/bgemm.cu:88-97). Here one kernel template handles every shape and
// transpose in-kernel (guarded, zero-filled staging; guarded stores), and the
// host only picks the tile size (pick_tile) and whether every row of the
// operands is 16-byte aligned.
#include "mfma_gemm.hpp"
#include "../../include/gemm.h"
#include "../../include/kernels.h"
#include "launch.hpp"

namespace {

using bmb::MfmaTile;
using TileL = MfmaTile<256, 256, 16, 2, 4>;  // 512 lanes, 128x64 per wave
using TileM = MfmaTile<128, 128, 16, 2, 2>;  // 256 lanes, 64x64 per wave
using TileS = MfmaTile<64, 64, 16, 2, 2>;    // 256 lanes, 32x32 per wave

// Number of CUs of the current device (256 on MI355X), cached per device.
int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

// Tile choice. Measured on MI355X at fp32 (N=4096/8192): the 256x256 tile
// (8 waves, one workgroup per CU) reaches ~86% of the MFMA peak, 128x128 (4
// waves, three per CU) ~82% and 64x64 (4 waves, eight per CU) ~78%. The big
// tiles lose badly when their count leaves a partial round of workgroups
// (4097^3 on 256x256: 17*17 = 289 tiles = 1.13 rounds, 63 TFLOP/s against
// 102 on 64x64), and small problems need the small tile to occupy every CU.
// So a big tile is used only when it fills whole rounds of the machine.
enum class TileKind { L, M, S };
TileKind pick_tile(long long tiles_l, long long tiles_m, int cus) {
    if (tiles_l >= cus && tiles_l % cus == 0) return TileKind::L;
    if (tiles_m >= 3LL * cus && tiles_m % (3LL * cus) == 0) return TileKind::M;
    return TileKind::S;
}

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
    switch (pick_tile(work(TileL::BM, TileL::BN), work(TileM::BM, TileM::BN), device_cus())) {
    case TileKind::L:
        launch_tile<TA, TB, TileL>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream, vec);
        break;
    case TileKind::M:
        launch_tile<TA, TB, TileM>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream, vec);
        break;
    case TileKind::S:
        launch_tile<TA, TB, TileS>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream, vec);
        break;
    }
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
