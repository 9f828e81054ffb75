// Stage 8: the true-fp32 VALU SGEMM ("dbuffer" in the reference ladder,
// src/kernels/k08_doublebuffer.cu:40-216), designed for gfx950.
//
// Numerics. Each output is acc = fma(a_k, b_k, acc) for k = 0..K-1 in order,
// one v_fma_f32 per term, then bmb::epilogue(). That is exactly the CPU
// oracle's sequential fmaf loop, so this kernel is bit-identical to it (and to
// stages 1-7). Split-K, reassociation or MFMA would all break that, which is
// why this stage stays on the vector ALU.
//
// Ceiling. This build never emits packed fp32 (v_pk_fma_f32). gfx950 issues
// plain v_fmac_f32 from two waves of one SIMD at once (its second VALU port):
// a loop of nothing but FMAs with 32 or more independent accumulators per lane
// reaches 128-136 TFLOP/s (81-86% of the 157.3 TFLOP/s vector peak) with 2 to
// 8 waves per SIMD, ~70 with one. A GEMM also reads its operands from LDS;
// the counters of the 128 x 128 tile at N = 4096 show 94% of its VALU
// instructions are FMAs, a third of them issued on the second port.
//
// Structure.
//   * 256 lanes = 4 wave64 per workgroup; tiles of 128 x 128, 64 x 128,
//     64 x 64 and 64 x 32 outputs, chosen per shape (pick_tile): the small
//     tiles fill the device when M x N is small, the large one reads less LDS
//     per FMA.
//   * Each wave owns a quarter of the tile; each lane a patch of 4 x 4 strips
//     (two 4-row strips 32 rows apart and two 4-column strips 32 columns
//     apart in the 128 x 128 tile). The 8 lanes sharing a strip row read one
//     float4 each of a 32-float LDS span, so every per-k LDS read is 128-bit.
//   * A is stored k-major in LDS (As[k][m], +4 pad so the transposing
//     stores spread over the banks); B is stored as it lies (Bs[k][n]).
//   * Double-buffered LDS with the next k-tile prefetched into registers while
//     the current one is consumed: one barrier per k-tile.
//   * Ragged M, N, K are handled in-kernel: guarded, zero-filled loads and
//     guarded stores. There is no fallback kernel. VEC selects aligned 128-bit
//     global access when K % 4 == 0, N % 4 == 0 and the pointers are 16-byte
//     aligned; otherwise interior chunks still use dword-aligned 128-bit loads
//     and only a chunk that straddles a row end uses 32-bit loads.
//   * Workgroup ids are remapped so the tiles one XCD runs share panels.
#include <math.h>

#include <mutex>

#include "common.hpp"
#include "../../include/kernels.h"
#include "launch.hpp"

using bmb::epilogue;
using bmb::fma_rn;

namespace {

constexpr int NT = 256;
constexpr int APAD = 4;

// Tile of 64*TMS x 16*SW*TNS outputs for 4 waves (2 x 2), each wave a
// 32*TMS x 8*SW*TNS quadrant; each lane a patch of TMS x TNS strips of
// 4 x SW outputs, strips 32 rows / 8*SW columns apart, so the 8 lanes sharing
// a strip row (or column) read one float4 (float2) each of a contiguous LDS
// span per k: every LDS read is conflict-free and 128-bit (64-bit for SW = 2).
// 128 x 128 (TMS = TNS = 2, SW = 4) keeps 64 accumulators per lane and reads
// 1 byte of LDS per FMA; 64 x 64 (1, 1) has 4x the workgroups for a small C at
// 2 bytes per FMA; 64 x 32 (SW = 2: 4 x 2 outputs per lane) has 8x.
template <int TMS_, int TNS_, int BK_, int UNROLL_, int SW_ = 4>
struct ValuTile {
    static constexpr int TMS = TMS_, TNS = TNS_;
    static constexpr int SW = SW_;          // columns per lane strip (4 or 2)
    static constexpr int BK = BK_;          // k per LDS stage
    static constexpr int UNROLL = UNROLL_;  // k-loop unroll within a stage
    static constexpr int BM = 64 * TMS, BN = 16 * SW * TNS;
    static constexpr int LDA = BM + APAD;  // As row (one k) width
    static constexpr int LDB = BN;         // Bs row width
    static constexpr int A_CH = BM * BK / 4 / NT;  // float4 chunks per lane
    static constexpr int B_CH = BK * BN / 4 / NT;
    static constexpr int KCH = BK / 4;             // float4 chunks per A row
};

// A chunk e (four consecutive k of one row m): four lanes along k (one
// 64-byte row segment), then consecutive rows, then the next segment. The
// transposed LDS stores of a wave then cover 16 rows of 4 segments each, so
// every bank takes one of them (row stride BM + 4: segments 16 banks apart);
// with 8 or 16 lanes along k they would fall on the same 4 offsets (2- and
// 4-way conflicts for 32- and 64-deep stages).
template <class Tl>
__device__ __forceinline__ void a_chunk(int e, int &m, int &kc) {
    static_assert(Tl::BK % 16 == 0, "whole 16-k segments per stage");
    const int kq = e & 3, kseg = e / (4 * Tl::BM);
    m = (e >> 2) % Tl::BM;
    kc = (kseg * 4 + kq) * 4;
}

// Per-thread share of one k-tile of A (BM x BK) and B (BK x BN).
template <class Tl>
struct Prefetch {
    float a[4 * Tl::A_CH];
    float b[4 * Tl::B_CH];
};

template <class Tl, bool VEC>
__device__ __forceinline__ void load_tile(Prefetch<Tl> &p, const float *A,
                                          const float *B, int M, int N, int K,
                                          int cRow, int cCol, int k0, int tid) {
    // A chunk e = tid + r*NT (a_chunk).
#pragma unroll
    for (int r = 0; r < Tl::A_CH; ++r) {
        const int e = tid + r * NT;
        int m, kc;
        a_chunk<Tl>(e, m, kc);
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
    // B chunk e: row k = e / (BN/4), n offset (e % (BN/4)) * 4.
#pragma unroll
    for (int r = 0; r < Tl::B_CH; ++r) {
        const int e = tid + r * NT;
        const int k = e / (Tl::BN / 4), nc = (e % (Tl::BN / 4)) * 4;
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

template <class Tl>
__device__ __forceinline__ void store_tile(const Prefetch<Tl> &p, float *As,
                                           float *Bs, int tid) {
#pragma unroll
    for (int r = 0; r < Tl::A_CH; ++r) {
        const int e = tid + r * NT;
        int m, kc;
        a_chunk<Tl>(e, m, kc);
#pragma unroll
        for (int i = 0; i < 4; ++i) As[(kc + i) * Tl::LDA + m] = p.a[r * 4 + i];
    }
#pragma unroll
    for (int r = 0; r < Tl::B_CH; ++r) {
        const int e = tid + r * NT;
        const int k = e / (Tl::BN / 4), nc = (e % (Tl::BN / 4)) * 4;
        bmb::st4(&Bs[k * Tl::LDB + nc],
                 make_float4(p.b[r * 4 + 0], p.b[r * 4 + 1], p.b[r * 4 + 2], p.b[r * 4 + 3]));
    }
}

template <class Tl, bool VEC>
__global__ __launch_bounds__(NT) void sgemm_valu_k(int M, int N, int K,
                                                   float alpha,
                                                   const float *__restrict__ A,
                                                   const float *__restrict__ B,
                                                   float beta, float *C,
                                                   int tiles_m, int tiles_n) {
    constexpr int TM = 4 * Tl::TMS, TN = Tl::SW * Tl::TNS;  // outputs per lane
    constexpr int SW = Tl::SW;
    constexpr int BK = Tl::BK;
    __shared__ float As[2][BK * Tl::LDA];
    __shared__ float Bs[2][BK * Tl::LDB];

    const int nblocks = tiles_m * tiles_n;
    int tm, tn;
    bmb::group_tile(bmb::xcd_remap(blockIdx.x, nblocks), tiles_m, tiles_n, 8, tm, tn);
    const int cRow = tm * Tl::BM, cCol = tn * Tl::BN;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * (Tl::BM / 2), wn = (wave & 1) * (Tl::BN / 2);
    const int lr = lane >> 3, lc = lane & 7;

    float acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = 0.0f;

    const int nkt = (K + BK - 1) / BK;
    Prefetch<Tl> pf;
    if (nkt > 0) {
        load_tile<Tl, VEC>(pf, A, B, M, N, K, cRow, cCol, 0, tid);
        store_tile<Tl>(pf, As[0], Bs[0], tid);
    }
    __syncthreads();

    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) load_tile<Tl, VEC>(pf, A, B, M, N, K, cRow, cCol, (kt + 1) * BK, tid);

        const float *as = As[cur] + wm + lr * 4;
        const float *bs = Bs[cur] + wn + lc * SW;
        // The 128 x 128 tile unrolls by 2 only: a full unroll lets the
        // scheduler hoist all k-steps' LDS reads and pushes the lane past 256
        // VGPRs. The small tiles (one wave per SIMD at small N) unroll fully,
        // so the reads of later k-steps are in flight during the FMAs.
#pragma unroll Tl::UNROLL
        for (int k = 0; k < BK; ++k) {
            float ra[TM], rb[TN];
#pragma unroll
            for (int s = 0; s < Tl::TMS; ++s) {
                const float4 a = bmb::ld4(as + k * Tl::LDA + 32 * s);
                ra[4 * s + 0] = a.x; ra[4 * s + 1] = a.y; ra[4 * s + 2] = a.z; ra[4 * s + 3] = a.w;
            }
#pragma unroll
            for (int s = 0; s < Tl::TNS; ++s) {
                if (SW == 4) {
                    const float4 b = bmb::ld4(bs + k * Tl::LDB + 32 * s);
                    rb[4 * s + 0] = b.x; rb[4 * s + 1] = b.y; rb[4 * s + 2] = b.z; rb[4 * s + 3] = b.w;
                } else {
                    const float2 b = *reinterpret_cast<const float2 *>(bs + k * Tl::LDB + 16 * s);
                    rb[2 * s + 0] = b.x; rb[2 * s + 1] = b.y;
                }
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = fma_rn(ra[i], rb[j], acc[i][j]);
        }

        if (more) store_tile<Tl>(pf, As[cur ^ 1], Bs[cur ^ 1], tid);
        __syncthreads();
    }

    // Epilogue. Row of acc[i][.]: wm + (i/4)*32 + lr*4 + i%4; column of
    // acc[.][h*SW+x]: wn + h*8*SW + lc*SW + x.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int r = cRow + wm + (i >> 2) * 32 + lr * 4 + (i & 3);
        if (r >= M) continue;
#pragma unroll
        for (int h = 0; h < Tl::TNS; ++h) {
            const int c = cCol + wn + h * 8 * SW + lc * SW;
            float *dst = C + (size_t)r * N + c;
            if (VEC && SW == 4 && c + 3 < N) {
                float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
                if (beta != 0.0f) o = bmb::ld4(dst);
                o.x = epilogue(acc[i][h * 4 + 0], alpha, beta, &o.x);
                o.y = epilogue(acc[i][h * 4 + 1], alpha, beta, &o.y);
                o.z = epilogue(acc[i][h * 4 + 2], alpha, beta, &o.z);
                o.w = epilogue(acc[i][h * 4 + 3], alpha, beta, &o.w);
                bmb::st4(dst, o);
            } else if (VEC && SW == 2 && c + 1 < N) {
                float2 o = make_float2(0.f, 0.f);
                if (beta != 0.0f) o = *reinterpret_cast<const float2 *>(dst);
                o.x = epilogue(acc[i][h * 2 + 0], alpha, beta, &o.x);
                o.y = epilogue(acc[i][h * 2 + 1], alpha, beta, &o.y);
                *reinterpret_cast<float2 *>(dst) = o;
            } else {
#pragma unroll
                for (int x = 0; x < SW; ++x)
                    if (c + x < N) dst[x] = epilogue(acc[i][h * SW + x], alpha, beta, &dst[x]);
            }
        }
    }
}

template <class Tl>
void launch_valu(int M, int N, int K, float alpha, const float *A, const float *B, float beta,
                 float *C, bool vec) {
    const int tiles_m = bmb::ceil_div(M, Tl::BM), tiles_n = bmb::ceil_div(N, Tl::BN);
    const dim3 grid(tiles_m * tiles_n);
    if (vec)
        bmb::launch(sgemm_valu_k<Tl, true>, grid, dim3(NT), 0, nullptr, M, N, K, alpha, A, B,
                    beta, C, tiles_m, tiles_n);
    else
        bmb::launch(sgemm_valu_k<Tl, false>, grid, dim3(NT), 0, nullptr, M, N, K, alpha, A, B,
                    beta, C, tiles_m, tiles_n);
}

// The tiles (bit-identical to one another: every one keeps each output's
// sequential k order) and their measured throughput on MI355X when the device
// is full of them (TFLOP/s at N = 8192).
using TileL = ValuTile<2, 2, 16, 8>;  // 128 x 128: 88
using TileW = ValuTile<1, 2, 16, 2>;  // 64 x 128: 84.5
using TileS = ValuTile<1, 1, 32, 8>;  // 64 x 64: 78
// 64 x 32 with 4 x 2 outputs per lane, for C too small to give every SIMD two
// waves otherwise (N = 1024: 51.0 TFLOP/s against 37.0 for 64 x 64; N = 512:
// 13.7 against 8.9). It reads 64 k per stage: one wave per SIMD of 64 x 64
// tiles, or two of these with 32-deep stages, leave the next stage's HBM
// latency exposed.
using TileX = ValuTile<1, 1, 64, 8, 2>;

struct ValuCand {
    int bm, bn;
    double tflops;
};
constexpr ValuCand VCANDS[] = {{128, 128, 88.0}, {64, 128, 84.5}, {64, 64, 78.0}};

template <class Tl>
int valu_occupancy() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, sgemm_valu_k<Tl, true>, NT, 0) !=
        hipSuccess) {
        (void)hipGetLastError();
        n = 1;
    }
    return n < 1 ? 1 : n;
}

// Tile choice: a tile's workgroups run in rounds of cus * occupancy; a last,
// part-filled round runs each CU's workgroups faster (fewer share its SIMDs),
// by (held / fit)^0.88 of a full round (the GEMM planner's fit). A larger tile
// reads less LDS per FMA; a smaller one fills the device at small M x N (at
// N = 1024: 64 workgroups of 128 x 128 for 256 CUs). Measured on the square
// sweep: 64 x 64 up to N = 3072 (N = 1024: 37 instead of 11 TFLOP/s),
// 64 x 128 at the ragged 4097, 128 x 128 from 4096. Below that, when 64 x 64
// tiles would put at most one workgroup on each CU (one wave per SIMD, which
// cannot use the second VALU issue port) and the 64 x 32 tiles fit in one
// round, the 64 x 32 tile runs two or three waves per SIMD instead.
int pick_tile(int M, int N) {
    static std::once_flag once[64];
    static int occ[64][4], cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    std::call_once(once[dev], [&] {
        occ[dev][0] = valu_occupancy<TileL>();
        occ[dev][1] = valu_occupancy<TileW>();
        occ[dev][2] = valu_occupancy<TileS>();
        occ[dev][3] = valu_occupancy<TileX>();
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            c <= 0) {
            (void)hipGetLastError();
            c = 256;
        }
        cus[dev] = c;
    });
    const long long tiles_s = (long long)bmb::ceil_div(M, 64) * bmb::ceil_div(N, 64);
    const long long tiles_x = (long long)bmb::ceil_div(M, 64) * bmb::ceil_div(N, 32);
    if (tiles_s <= cus[dev] && tiles_x <= (long long)cus[dev] * occ[dev][3]) return 3;
    int best = 0;
    double best_t = -1.0;
    for (int t = 0; t < 3; ++t) {
        const ValuCand &v = VCANDS[t];
        const long long tiles = (long long)bmb::ceil_div(M, v.bm) * bmb::ceil_div(N, v.bn);
        const long long slots = (long long)cus[dev] * occ[dev][t];
        const double t_item = (double)v.bm * v.bn * occ[dev][t] / v.tflops;
        const long long full = tiles / slots, rem = tiles % slots;
        double time = full * t_item;
        if (rem) {
            const long long per_cu = (rem + cus[dev] - 1) / cus[dev];
            time += per_cu < occ[dev][t] ? t_item * pow((double)per_cu / occ[dev][t], 0.88)
                                         : t_item;
        }
        if (best_t < 0 || time < best_t) {
            best_t = time;
            best = t;
        }
    }
    return best;
}

// tile: 0 = 128x128, 1 = 64x128, 2 = 64x64, 3 = 64x32.
void run_valu(int tile, int M, int N, int K, float alpha, const float *A, const float *B,
              float beta, float *C) {
    const bool vec = (K % 4 == 0) && (N % 4 == 0) && (((uintptr_t)A & 15) == 0) &&
                     (((uintptr_t)B & 15) == 0) && (((uintptr_t)C & 15) == 0);
    switch (tile) {
    case 0: launch_valu<TileL>(M, N, K, alpha, A, B, beta, C, vec); break;
    case 1: launch_valu<TileW>(M, N, K, alpha, A, B, beta, C, vec); break;
    case 2: launch_valu<TileS>(M, N, K, alpha, A, B, beta, C, vec); break;
    default: launch_valu<TileX>(M, N, K, alpha, A, B, beta, C, vec); break;
    }
}

}  // namespace

extern "C" void sgemm_doublebuffer(int M, int N, int K, float alpha,
                                   const float *A, const float *B, float beta,
                                   float *C) {
    if (M <= 0 || N <= 0) return;
    run_valu(pick_tile(M, N), M, N, K, alpha, A, B, beta, C);
}
