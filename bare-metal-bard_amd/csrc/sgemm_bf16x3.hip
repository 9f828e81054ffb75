// SGEMM stage 10: fp32 GEMM from three bf16 matrix-core products.
//
// Numerics. Each fp32 operand x is split as hi = bf16(x), lo = bf16(x - hi)
// (both round-to-nearest-even; x - hi is exact in fp32), so x = hi + lo up to
// 2^-16 |x|. The product a*b is taken as hi_a*hi_b + hi_a*lo_b + lo_a*hi_b,
// dropping lo_a*lo_b (<= 2^-16 |ab|). Each bf16 x bf16 product is exact in
// fp32 and accumulation is fp32 on v_mfma_f32_32x32x16_bf16, so the result is
// the split's exact value up to fp32 summation of 3K terms: a few 2^-17 per
// product against the exact product, an order of magnitude better than the
// TF32 stage it stands in for (src/kernels/k09_tensorcore.cu:119-128 rounds
// to 10 mantissa bits). Three bf16 MFMAs (8 passes each) cost 96 cycles per
// 32x32x16 step against 512 for the fp32 MFMA, so the ceiling is a third of
// the bf16 peak: 833 TFLOP/s of fp32-equivalent work.
//
// MFMA operand layout (v_mfma_f32_32x32x16_bf16): lane l supplies 8
// consecutive-k bf16 of row (A) or column (B) l % 32, k = 8 * (l / 32) + 0..7;
// the D layout matches v_mfma_f32_32x32x2_f32.
//
// Tiles. 256x256 (8 waves of 128x64), 128x128 (4 waves of 64x64) and 64x64
// (4 waves of 32x32) outputs, K in stages of 32 (two 16-k MFMA steps), and a
// split of K into ranges whose fp32 partials one reduce adds in range order
// (deterministic). A planner picks tile and split per shape, as gemm() does
// for the fp32 MFMA path: the 256x256 tile alone leaves most CUs idle below
// N = 4096 (16 workgroups at N = 1024).
//
// LDS: per stage four bf16 planes (A hi, A lo, B hi, B lo), each stored
// [row][k] with k contiguous (row = m for A, n for B), so every fragment is
// one 128-bit read. Rows are 64 bytes with their 16-byte chunks XOR-swizzled
// by row (lds_off), so neither the fragment reads nor the staging stores
// conflict on banks. A (k contiguous
// in global memory) is staged with 128-bit loads, four k per lane, split and
// written as two 64-bit stores. B (n contiguous) is staged as 4 x 4 blocks:
// four 128-bit loads (rows k..k+3, columns n..n+3; a wave covers 32
// consecutive column blocks of two k rows, so each load is two 512-byte
// coalesced accesses), a transpose in registers, then per column one 64-bit
// store of its 4 k per plane.
//
// Schedule: double-buffered LDS stages with register prefetch. While a stage
// is consumed, the next one is split and stored from registers (after the
// first 16-k step's MFMAs are issued, so the conversion overlaps them) and
// the global loads for the stage after it are issued; one barrier per stage.
#include <math.h>

#include <mutex>
#include <optional>

#include "common.hpp"
#include "gemm_fused.hpp"
#include "mfma_gemm.hpp"
#include "../../include/kernels.h"
#include "launch.hpp"
#include "workspace.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
using bmb::f32x16;

constexpr int BK = 32;   // k per LDS stage: two 16-k MFMA steps
constexpr int LDK = BK;  // bf16 per LDS row (64 bytes, no padding: see lds_off)

template <int BM_, int BN_, int WAVES_M_, int WAVES_N_>
struct B3Tile {
    static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int NT = 64 * WAVES_M * WAVES_N;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    static constexpr int FM = WM / 32, FN = WN / 32;
    static constexpr int A_PLANE = BM * LDK, B_PLANE = BN * LDK;  // bf16 elements
    static constexpr int STAGE = 2 * A_PLANE + 2 * B_PLANE;
    static constexpr size_t SMEM_BYTES = 2 * (size_t)STAGE * sizeof(__bf16);
    static constexpr int A_CH = BM * BK / 4 / NT;         // float4 chunks of A per lane
    static constexpr int B_BLK = BK * BN / 16;             // 4 x 4 blocks of B per stage
    static constexpr int B_PER_T = (B_BLK + NT - 1) / NT;  // blocks per lane
    static_assert((BM * BK / 4) % NT == 0, "A staging splits evenly over the lanes");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile is whole 32x32 blocks");
};

using TileL = B3Tile<256, 256, 2, 4>;
using TileM = B3Tile<128, 128, 2, 2>;
using TileS = B3Tile<64, 64, 2, 2>;

// Offset (in bf16) of element k (a multiple of 4) of LDS row `row`. Rows are
// 64 bytes (four 16-byte chunks); row r is stored in slot p = r ^ ((r >> 2)
// & 1) (rows swap pairwise in every other group of four), and chunk k / 8 of
// it at position chunk ^ g(r), g(r) = ((r >> 2) ^ (r >> 4)) & 3. gfx950
// serves a 128-bit LDS read 16 lanes per cycle from 256 bytes (64 banks) and
// a 64-bit write 16 lanes per cycle into 128 bytes (32 banks): fragment reads
// (16 consecutive rows, one chunk) hit 16 distinct 16-byte slots; A stores
// (two rows x eight 8-byte units per 16 lanes) and the B planes' transposed
// stores (rows 4m + c of eight consecutive column blocks m, two units; the
// slot swap alternates their parity, i.e. which 64-byte half of the write
// window they fall in) hit 16 distinct 8-byte slots. No bank conflict in any
// of them; a padded 80-byte row made the transposed stores 16-way conflicted.
__device__ __forceinline__ int lds_off(int row, int k) {
    const int p = row ^ ((row >> 2) & 1);
    return p * LDK + 8 * ((k >> 3) ^ (((row >> 2) ^ (row >> 4)) & 3)) + (k & 7);
}

// x -> (bf16(x), bf16(x - bf16(x))) for four values.
__device__ __forceinline__ void split4(const float (&x)[4], bf16x4 &hi, bf16x4 &lo) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 h = (__bf16)x[i];
        hi[i] = h;
        lo[i] = (__bf16)(x[i] - (float)h);
    }
}

template <class Tl, bool VEC>
struct Bf16x3Gemm {
    static constexpr int BM = Tl::BM, BN = Tl::BN, NT = Tl::NT;
    static constexpr int FM = Tl::FM, FN = Tl::FN;

    struct Regs {
        float4 a[Tl::A_CH];
        float4 b[Tl::B_PER_T][4];  // rows k..k+3 of a 4 x 4 block
    };

    // One 128-bit load from a 4-byte aligned address wholly inside the row.
    __device__ static __forceinline__ float4 ld_in(const float *p) {
        if (VEC) return bmb::ld4(p);
        float4 v;
        __builtin_memcpy(&v, p, sizeof(v));
        return v;
    }

    // Stage loads with zero fill outside [0, M) x [0, K) of A and
    // [0, K) x [0, N) of B (K is the range's length; lda = full K, ldb = N).
    __device__ static __forceinline__ void load_guarded(Regs &g, const float *A, const float *B,
                                                        int M, int N, int K, int lda, int ldb,
                                                        int m0, int n0, int k0, int tid) {
#pragma unroll
        for (int i = 0; i < Tl::A_CH; ++i) {
            const int e = tid + i * NT, r = e / (BK / 4), c = (e % (BK / 4)) * 4;
            g.a[i] = bmb::load_chunk<VEC>(A, M, K, lda, m0 + r, k0 + c);
        }
#pragma unroll
        for (int j = 0; j < Tl::B_PER_T; ++j) {
            const int e = tid + j * NT;
            if (Tl::B_BLK % NT != 0 && e >= Tl::B_BLK) continue;
            int kb, nb;
            b_block(e, kb, nb);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                g.b[j][i] = bmb::load_chunk<VEC>(B, K, N, ldb, k0 + 4 * kb + i, n0 + nb);
        }
    }

    // Byte offsets of this lane's chunks from the tile's stage base (A at
    // (m0, k0), B at (k0, n0)): loop-invariant and 32-bit, so an interior
    // stage's loads take a uniform base and no 64-bit address arithmetic.
    struct Offs {
        unsigned a[Tl::A_CH];
        unsigned b[Tl::B_PER_T][4];
    };
    __device__ static __forceinline__ void offsets(Offs &o, int lda, int ldb, int tid) {
#pragma unroll
        for (int i = 0; i < Tl::A_CH; ++i) {
            const int e = tid + i * NT, r = e / (BK / 4), c = (e % (BK / 4)) * 4;
            o.a[i] = 4u * ((unsigned)r * (unsigned)lda + (unsigned)c);
        }
#pragma unroll
        for (int j = 0; j < Tl::B_PER_T; ++j) {
            const int e = min(tid + j * NT, Tl::B_BLK - 1);
            int kb, nb;
            b_block(e, kb, nb);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                o.b[j][i] = 4u * ((unsigned)(4 * kb + i) * (unsigned)ldb + (unsigned)nb);
        }
    }
    __device__ static __forceinline__ float4 ld_at(const float *base, unsigned off) {
        return ld_in(reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) + off));
    }
    // Interior stage: every chunk inside the operands.
    __device__ static __forceinline__ void load_interior(Regs &g, const Offs &o, const float *a0,
                                                         const float *b0, int tid) {
#pragma unroll
        for (int i = 0; i < Tl::A_CH; ++i) g.a[i] = ld_at(a0, o.a[i]);
#pragma unroll
        for (int j = 0; j < Tl::B_PER_T; ++j) {
            if (Tl::B_BLK % NT != 0 && tid + j * NT >= Tl::B_BLK) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) g.b[j][i] = ld_at(b0, o.b[j][i]);
        }
    }

    // 4 x 4 block e of B: k rows 4kb..4kb+3 and columns nb..nb+3 of the stage.
    // Neighbouring lanes take the two halves of a 16-byte k chunk (kb even,
    // odd) of one column block; pairs of lanes walk the column blocks.
    __device__ static __forceinline__ void b_block(int e, int &kb, int &nb) {
        const int m = (e >> 1) % (BN / 4);
        kb = 2 * ((e >> 1) / (BN / 4)) + (e & 1);
        nb = 4 * m;
    }

    // Split the prefetched stage into the four planes of `st`.
    __device__ static __forceinline__ void store(const Regs &g, __bf16 *st, int tid) {
#pragma unroll
        for (int i = 0; i < Tl::A_CH; ++i) {
            const int e = tid + i * NT, r = e / (BK / 4), c = (e % (BK / 4)) * 4;
            const float x[4] = {g.a[i].x, g.a[i].y, g.a[i].z, g.a[i].w};
            bf16x4 h, l;
            split4(x, h, l);
            *reinterpret_cast<bf16x4 *>(st + lds_off(r, c)) = h;
            *reinterpret_cast<bf16x4 *>(st + Tl::A_PLANE + lds_off(r, c)) = l;
        }
        __bf16 *bh = st + 2 * Tl::A_PLANE, *bl = bh + Tl::B_PLANE;
#pragma unroll
        for (int j = 0; j < Tl::B_PER_T; ++j) {
            const int e = tid + j * NT;
            if (Tl::B_BLK % NT != 0 && e >= Tl::B_BLK) continue;
            int kb, nb;
            b_block(e, kb, nb);
            const float4 *b = g.b[j];
            const float cols[4][4] = {{b[0].x, b[1].x, b[2].x, b[3].x},
                                      {b[0].y, b[1].y, b[2].y, b[3].y},
                                      {b[0].z, b[1].z, b[2].z, b[3].z},
                                      {b[0].w, b[1].w, b[2].w, b[3].w}};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                bf16x4 h, l;
                split4(cols[c], h, l);
                *reinterpret_cast<bf16x4 *>(bh + lds_off(nb + c, 4 * kb)) = h;
                *reinterpret_cast<bf16x4 *>(bl + lds_off(nb + c, 4 * kb)) = l;
            }
        }
    }

    // One 16-k step of MFMAs on stage `st`: for every 32 x 32 block,
    // acc += lo_a hi_b, then hi_a lo_b, then hi_a hi_b (small terms first).
    __device__ static __forceinline__ void step(const __bf16 *st, int kk, int wm, int wn, int lane,
                                                f32x16 (&acc)[FM][FN]) {
        const int l32 = lane & 31, koff = kk * 16 + 8 * (lane >> 5);
        bf16x8 ah[FM], al[FM], bh[FN], bl[FN];
#pragma unroll
        for (int fi = 0; fi < FM; ++fi) {
            const int off = lds_off(wm + fi * 32 + l32, koff);
            ah[fi] = *reinterpret_cast<const bf16x8 *>(st + off);
            al[fi] = *reinterpret_cast<const bf16x8 *>(st + Tl::A_PLANE + off);
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const int off = 2 * Tl::A_PLANE + lds_off(wn + fn * 32 + l32, koff);
            bh[fn] = *reinterpret_cast<const bf16x8 *>(st + off);
            bl[fn] = *reinterpret_cast<const bf16x8 *>(st + Tl::B_PLANE + off);
        }
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
                acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[fi], bh[fn], acc[fi][fn], 0, 0, 0);
                acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[fi], bl[fn], acc[fi][fn], 0, 0, 0);
                acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[fi], bh[fn], acc[fi][fn], 0, 0, 0);
            }
    }

    // One output tile over k in [0, K) (A, B positioned at that range's
    // start). INTERIOR: the tile lies inside M x N and K is a positive whole
    // number of stages, so no load or store needs a bounds check. PARTIAL:
    // C receives the raw sums (a split-K partial, row stride N).
    template <bool INTERIOR, bool PARTIAL>
    __device__ static __forceinline__ void run(int M, int N, int K, int lda, int ldb, float alpha,
                                               const float *__restrict__ A,
                                               const float *__restrict__ B, float beta, float *C,
                                               int m0, int n0, __bf16 *smem) {
        const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
        const int wm = (wave / Tl::WAVES_N) * Tl::WM, wn = (wave % Tl::WAVES_N) * Tl::WN;

        f32x16 acc[FM][FN];
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fi][fn][r] = 0.0f;

        const int nkt = (K + BK - 1) / BK;
        Regs g;
        Offs o;
        if (INTERIOR) offsets(o, lda, ldb, tid);
        // Stage kt's tile bases (uniform): A at (m0, kt*BK), B at (kt*BK, n0).
        auto a_at = [&](int kt) { return A + (size_t)m0 * lda + (size_t)kt * BK; };
        auto b_at = [&](int kt) { return B + (size_t)kt * BK * ldb + n0; };
        auto load = [&](int kt) {
            if (INTERIOR) load_interior(g, o, a_at(kt), b_at(kt), tid);
            else load_guarded(g, A, B, M, N, K, lda, ldb, m0, n0, kt * BK, tid);
        };
        if (nkt > 0) {
            load(0);
            store(g, smem, tid);
            if (nkt > 1) load(1);
        }
        __syncthreads();
        for (int kt = 0; kt < nkt; ++kt) {
            const __bf16 *st = smem + (kt & 1) * Tl::STAGE;
            step(st, 0, wm, wn, lane, acc);
            if (kt + 1 < nkt) {
                // The other stage was last read before the previous barrier.
                store(g, smem + ((kt + 1) & 1) * Tl::STAGE, tid);
                if (kt + 2 < nkt) load(kt + 2);
            }
            step(st, 1, wm, wn, lane, acc);
            __syncthreads();
        }

        // Epilogue: lanes 0-31 of a register cover 32 consecutive columns.
        // The C values a row of FN blocks needs (beta != 0) are gathered
        // before any result is stored: 16 * FN loads in flight per lane.
        const int l32 = lane & 31, half = lane >> 5;
        const bool reads = !PARTIAL && beta != 0.0f;
#pragma unroll
        for (int fi = 0; fi < FM; ++fi) {
            float in[FN][16];
            if (reads) {
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) {
                    const int col = n0 + wn + fn * 32 + l32;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = m0 + wm + fi * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                        in[fn][r] = (INTERIOR || (row < M && col < N))
                                        ? C[(size_t)row * N + col] : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
                const int col = n0 + wn + fn * 32 + l32;
                if (!INTERIOR && col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm + fi * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (!INTERIOR && row >= M) continue;
                    const float a = acc[fi][fn][r];
                    C[(size_t)row * N + col] =
                        PARTIAL ? a : (reads ? bmb::fma_rn(alpha, a, beta * in[fn][r]) : alpha * a);
                }
            }
        }
    }
};

// Grid: x = output tiles (XCD-remapped, grouped), y = K range s, covering
// k in [s*kchunk, min(K, (s+1)*kchunk)) (kchunk a multiple of BK when
// gridDim.y > 1). PARTIAL: write the range's raw sums to C + s*M*N.
template <class Tl, bool VEC, bool PARTIAL>
__global__ __launch_bounds__(Tl::NT) void bf16x3_k(int M, int N, int K, int kchunk, float alpha,
                                                   const float *__restrict__ A,
                                                   const float *__restrict__ B, float beta,
                                                   float *C, int tiles_m, int tiles_n) {
    extern __shared__ __bf16 lds[];
    using G = Bf16x3Gemm<Tl, VEC>;
    int tm, tn;
    bmb::group_tile(bmb::xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int m0 = tm * Tl::BM, n0 = tn * Tl::BN;
    const int kb = blockIdx.y * kchunk, klen = min(K, kb + kchunk) - kb;
    const float *Ak = A + kb;
    const float *Bk = B + (size_t)kb * N;
    float *Cs = PARTIAL ? C + (size_t)blockIdx.y * M * N : C;
    if (m0 + Tl::BM <= M && n0 + Tl::BN <= N && klen > 0 && klen % BK == 0)
        G::template run<true, PARTIAL>(M, N, klen, K, N, alpha, Ak, Bk, beta, Cs, m0, n0, lds);
    else
        G::template run<false, PARTIAL>(M, N, klen, K, N, alpha, Ak, Bk, beta, Cs, m0, n0, lds);
}

// ------------------------------------------------------------- host side

// Tile and split choice, the fp32 MFMA planner's time model (mfma_gemm.hip)
// with this path's own measured constants: a work item is one output tile
// over one K range; the device runs cus x occupancy of them per round; a
// part-filled last round runs each CU's items faster by (held / fit)^0.5,
// and a single round that leaves CUs idle runs faster again by
// (busy CUs / cus)^0.3; a split adds the partials' round trip and the
// reduce. Fitted to every tile x {1, 2, 4, 8} splits on the square sweep
// N = 512 ... 8192 on MI355X, the model picks the measured best plan at every
// size of that sweep.
struct B3Cand {
    int bm, bn;
    double tflops;  // fp32-equivalent TFLOP/s when the device is full of them
};
constexpr B3Cand CANDS[] = {{256, 256, 417.0}, {128, 128, 326.0}, {64, 64, 233.0}};
constexpr int N_CANDS = 3;
constexpr int SPLITS[] = {1, 2, 4, 8};
constexpr double PARTIAL_EXP = 0.5;
constexpr double FILL_EXP = 0.3;
constexpr double K_OVERHEAD = 96.0;               // per-item prologue/epilogue, in k
constexpr double PARTIALS_BYTES_PER_S = 1.35e13;  // the partials' round trip
constexpr double LAUNCH_S = 1.6e-6;               // the reduce launch
constexpr int MIN_SPLIT_K = 64;  // two stages
constexpr long long MAX_SPLIT_FLOATS = 64LL << 20;  // 256 MiB of partials

template <class Tl>
int occupancy_of() {
    int n = 0;
    bmb::allow_smem(bf16x3_k<Tl, true, false>, Tl::SMEM_BYTES);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, bf16x3_k<Tl, true, false>, Tl::NT,
                                                     Tl::SMEM_BYTES) != hipSuccess) {
        (void)hipGetLastError();
        n = 1;
    }
    return n < 1 ? 1 : n;
}

struct Plan {
    int tile, splits, kchunk;
};

Plan pick(int M, int N, int K) {
    static std::once_flag once[64];
    static int occ[64][N_CANDS], cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    std::call_once(once[dev], [&] {
        occ[dev][0] = occupancy_of<TileL>();
        occ[dev][1] = occupancy_of<TileM>();
        occ[dev][2] = occupancy_of<TileS>();
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            c <= 0) {
            (void)hipGetLastError();
            c = 256;
        }
        cus[dev] = c;
    });
    Plan best{0, 1, K};
    double best_t = -1.0;
    for (int t = 0; t < N_CANDS; ++t) {
        const B3Cand &c = CANDS[t];
        const long long tiles = (long long)bmb::ceil_div(M, c.bm) * bmb::ceil_div(N, c.bn);
        for (int s : SPLITS) {
            int splits = 1, kchunk = K;
            if (s > 1) {
                if (K < 2 * MIN_SPLIT_K) continue;
                kchunk = (K + s - 1) / s;
                kchunk = (kchunk + BK - 1) / BK * BK;
                if (kchunk < MIN_SPLIT_K) continue;
                splits = (K + kchunk - 1) / kchunk;
                if (splits < 2 || (long long)splits * M * N > MAX_SPLIT_FLOATS) continue;
            }
            const long long items = tiles * splits;
            const long long slots = (long long)cus[dev] * occ[dev][t];
            const double t_item = 2.0 * c.bm * c.bn * (kchunk + K_OVERHEAD) * occ[dev][t] /
                                  (c.tflops * 1e12 / cus[dev]);
            const long long full = items / slots, rem = items % slots;
            double time = full * t_item;
            if (rem) {
                const long long per_cu = (rem + cus[dev] - 1) / cus[dev];
                double last = per_cu < occ[dev][t]
                                  ? t_item * pow((double)per_cu / occ[dev][t], PARTIAL_EXP)
                                  : t_item;
                if (full == 0 && rem < cus[dev]) last *= pow((double)rem / cus[dev], FILL_EXP);
                time += last;
            }
            if (splits > 1)
                time += (splits + 2.0) * M * N * 4.0 / PARTIALS_BYTES_PER_S + LAUNCH_S;
            if (best_t < 0 || time < best_t) {
                best_t = time;
                best = Plan{t, splits, kchunk};
            }
        }
    }
    return best;
}

template <class Tl, bool VEC, bool PARTIAL>
void launch(int M, int N, int K, int kchunk, int splits, float alpha, const float *A,
            const float *B, float beta, float *C) {
    auto kern = bf16x3_k<Tl, VEC, PARTIAL>;
    bmb::allow_smem(kern, Tl::SMEM_BYTES);
    const int tiles_m = bmb::ceil_div(M, Tl::BM), tiles_n = bmb::ceil_div(N, Tl::BN);
    bmb::launch(kern, dim3(tiles_m * tiles_n, splits), dim3(Tl::NT), Tl::SMEM_BYTES, nullptr, M,
                N, K, kchunk, alpha, A, B, beta, C, tiles_m, tiles_n);
}

template <class Tl>
void run_plan(const Plan &p, int M, int N, int K, float alpha, const float *A, const float *B,
              float beta, float *C, bool vec, float *P) {
    if (P != nullptr) {
        if (vec) launch<Tl, true, true>(M, N, K, p.kchunk, p.splits, 1.0f, A, B, 0.0f, P);
        else     launch<Tl, false, true>(M, N, K, p.kchunk, p.splits, 1.0f, A, B, 0.0f, P);
        bmb::splitk_reduce(C, P, p.splits, (long long)M * N, N, alpha, beta, nullptr);
    } else {
        if (vec) launch<Tl, true, false>(M, N, K, K, 1, alpha, A, B, beta, C);
        else     launch<Tl, false, false>(M, N, K, K, 1, alpha, A, B, beta, C);
    }
}

}  // namespace

extern "C" void sgemm_mfma_bf16x3(int M, int N, int K, float alpha,
                                  const float *A, const float *B, float beta,
                                  float *C) {
    if (M <= 0 || N <= 0) return;
    const bool vec = K % 4 == 0 && N % 4 == 0 && (((uintptr_t)A & 15) == 0) &&
                     (((uintptr_t)B & 15) == 0);
    Plan p = pick(M, N, K);
    float *P = nullptr;
    std::optional<bmb::ScratchLease> lease;
    if (p.splits > 1) {
        lease.emplace(bmb::SCRATCH_GEMM, (size_t)p.splits * M * N * sizeof(float));
        P = static_cast<float *>(lease->get());
        if (P == nullptr) p = Plan{p.tile, 1, K};  // no scratch: no split
    }
    switch (p.tile) {
    case 0: run_plan<TileL>(p, M, N, K, alpha, A, B, beta, C, vec, P); break;
    case 1: run_plan<TileM>(p, M, N, K, alpha, A, B, beta, C, vec, P); break;
    default: run_plan<TileS>(p, M, N, K, alpha, A, B, beta, C, vec, P); break;
    }
}
