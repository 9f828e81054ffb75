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
// Tiles. 256x256 (8 waves of 128x64), 128x256 (8 waves of 64x64), 128x128
// (4 waves of 64x64) and 64x64 (4 waves of 32x32) outputs, K in stages of 32
// (two 16-k MFMA steps), and a
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
// Schedule: double-buffered LDS stages with register prefetch; one barrier
// per stage. While a stage is consumed, the next one is split and stored from
// registers and the global loads for the stage after it are issued. In the
// interior steady state (step0_fused) the split and its LDS stores are cut
// into pieces (one float4 chunk, or one column of a 4 x 4 block) placed
// between the first 16-k step's MFMAs behind scheduling fences, and each
// piece's registers are refilled by the next loads as soon as it is stored.
// Left to the compiler, the first step's MFMAs went out back to back and the
// conversion ran after them, so the two waves of a SIMD, kept in phase by the
// barrier, converted at the same time while the matrix core idled. The fenced
// order is 1-5% faster on the GPT-2 shapes and 2% at N = 4096, bit-identical.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <optional>
#include <tuple>
#include <type_traits>

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
using TileT = B3Tile<128, 256, 2, 4>;
using TileXS = B3Tile<32, 32, 1, 1>;  // one wave (k-sliced kernels only)

// Offset (in bf16) of element k (a multiple of 4) of LDS row `row`. Rows are
// 64 bytes (four 16-byte chunks); row r is stored in slot p = r ^ ((r >> 2)
// & 1) (rows swap pairwise in every other group of four), and chunk k / 8 of
// it at position chunk ^ ((r >> 3) & 3).
//
// gfx950's LDS has 64 four-byte banks. Measured with SQ_LDS_BANK_CONFLICT
// on single-pattern probes:
// - A 128-bit read is served in four cycles of 16 lanes each, and the
//   groups are not consecutive lanes: {0-3, 12-15, 20-27}, {4-11, 16-19,
//   28-31} and the same two shapes over lanes 32-63. A group is conflict-free
//   when its 16 addresses fall in 16 distinct 16-byte slots modulo 256 bytes.
//   A fragment read covers rows 0-31 of a 32-row block at one chunk. The
//   rows of the first group, 0-3, 12-15, 20-23 and 24-27, occupy four slot
//   pairs (row slot mod 4) and take the XORs 0, 1, 2, 3; so do those of the
//   second group.
// - A 64-bit write is served in groups of 16 consecutive lanes. A stores
//   (two rows x eight 8-byte units per 16 lanes) and the B planes' transposed
//   stores (rows 4m + c of eight consecutive column blocks m, two 8-byte
//   units each) land in 16 distinct 8-byte slots under this mapping.
// The bf16x3 kernel reads no conflict cycle at all (N = 4096), down from
// 2.5e7 per launch for the XOR ((r >> 2) ^ (r >> 4)) & 3, which assumed 16
// consecutive lanes per read cycle. A padded 80-byte row made the transposed
// stores 16-way conflicted.
__device__ __forceinline__ int lds_off(int row, int k) {
    const int p = row ^ ((row >> 2) & 1);
    return p * LDK + 8 * ((k >> 3) ^ ((row >> 3) & 3)) + (k & 7);
}

// The largest float that rounds to a finite bfloat16 (0x7F7F7FFF): above it
// round-to-nearest gives infinity, although x is finite.
constexpr float BF16_FINITE_MAX = 0x1.fefffep+127f;

// x -> (hi, lo) = (bf16(c), bf16(x - hi)) for four values, with c = x clamped
// to +-BF16_FINITE_MAX (one v_med3_f32). For |x| <= BF16_FINITE_MAX, c = x.
// Above it (finite x up to FLT_MAX, or +-inf) hi is bf16's largest finite
// value with x's sign and x - hi is exact (Sterbenz) or +-inf, so a huge
// finite x still splits exactly instead of into (inf, -inf), and an infinite
// x gives (+-3.39e38, +-inf), whose products with a nonzero b are +-inf and
// with b = 0 NaN, as in fp32. NaN stays NaN in lo.
__device__ __forceinline__ void split4(const float (&x)[4], bf16x4 &hi, bf16x4 &lo) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 h =
            (__bf16)__builtin_amdgcn_fmed3f(x[i], -BF16_FINITE_MAX, BF16_FINITE_MAX);
        hi[i] = h;
        lo[i] = (__bf16)(x[i] - (float)h);
    }
}

// f(integral_constant<int, i>) for i = I .. N - 1.
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Staging of one operand's tile per stage: ROWS rows (m of A, n of B) x BK k,
// into a hi and a lo plane. KCONT: k is the contiguous axis of the stored
// operand (A not transposed, B transposed): 128-bit loads of four k, split,
// one 64-bit store per plane. Otherwise rows are contiguous (A transposed, B
// not): 4 x 4 blocks (four k rows of four consecutive m or n; a wave covers
// 32 consecutive blocks of two k rows, so each load is two 512-byte coalesced
// accesses), transposed in registers, one 64-bit store of four k per row and
// plane.
template <int ROWS, int NT, bool KCONT, bool VEC>
struct OpStage {
    static constexpr int CH = ROWS * BK / 4 / NT;      // KCONT: chunks per lane
    static constexpr int BLK = BK * ROWS / 16;         // otherwise: 4 x 4 blocks per stage
    static constexpr int PER_T = (BLK + NT - 1) / NT;  // blocks per lane
    static constexpr int NLD = KCONT ? CH : 4 * PER_T;
    static_assert(!KCONT || (ROWS * BK / 4) % NT == 0, "staging splits evenly over the lanes");
    float4 v[NLD];

    __device__ static __forceinline__ bool skip(int j, int tid) {
        return !KCONT && BLK % NT != 0 && tid + j * NT >= BLK;
    }
    // Chunk e (KCONT): row r, k c..c+3.
    __device__ static __forceinline__ void chunk(int e, int &r, int &c) {
        r = e / (BK / 4);
        c = (e % (BK / 4)) * 4;
    }
    // Block e: k rows 4kb..4kb+3, rows rb..rb+3. Neighbouring lanes take the
    // two halves of a 16-byte k chunk (kb even, odd) of one row block.
    __device__ static __forceinline__ void block(int e, int &kb, int &rb) {
        const int m = (e >> 1) % (ROWS / 4);
        kb = 2 * ((e >> 1) / (ROWS / 4)) + (e & 1);
        rb = 4 * m;
    }
    __device__ static __forceinline__ float4 ld_in(const float *p) {
        if (VEC) return bmb::ld4(p);
        float4 x;
        __builtin_memcpy(&x, p, sizeof(x));
        return x;
    }
    // Byte offsets of this lane's loads from the stage base (row 0, k 0 of the
    // tile): loop-invariant and 32-bit.
    __device__ static __forceinline__ void offsets(unsigned (&o)[NLD], int ld, int tid) {
        if (KCONT) {
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                int r, c;
                chunk(tid + i * NT, r, c);
                o[i] = 4u * ((unsigned)r * (unsigned)ld + (unsigned)c);
            }
        } else {
#pragma unroll
            for (int j = 0; j < PER_T; ++j) {
                int kb, rb;
                block(min(tid + j * NT, BLK - 1), kb, rb);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[4 * j + i] = 4u * ((unsigned)(4 * kb + i) * (unsigned)ld + (unsigned)rb);
            }
        }
    }
    // Interior stage: base = the stage's (row 0, k 0) element.
    __device__ __forceinline__ void load_interior(const float *base, const unsigned (&o)[NLD],
                                                  int tid) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            if (skip(i / 4, tid)) continue;
            v[i] = ld_in(reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) + o[i]));
        }
    }
    // Zero fill outside the operand: P is the K range's origin, R its rows
    // (M or N), K the range's length, ld the stored row stride.
    __device__ __forceinline__ void load_guarded(const float *P, int R, int K, int ld, int r0,
                                                 int k0, int tid) {
        if (KCONT) {
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                int r, c;
                chunk(tid + i * NT, r, c);
                v[i] = bmb::load_chunk<VEC>(P, R, K, ld, r0 + r, k0 + c);
            }
        } else {
#pragma unroll
            for (int j = 0; j < PER_T; ++j) {
                if (skip(j, tid)) continue;
                int kb, rb;
                block(tid + j * NT, kb, rb);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    v[4 * j + i] = bmb::load_chunk<VEC>(P, K, R, ld, k0 + 4 * kb + i, r0 + rb);
            }
        }
    }
    __device__ __forceinline__ void store(__bf16 *hi, __bf16 *lo, int tid) const {
        if (KCONT) {
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                int r, c;
                chunk(tid + i * NT, r, c);
                const float x[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
                bf16x4 h, l;
                split4(x, h, l);
                *reinterpret_cast<bf16x4 *>(hi + lds_off(r, c)) = h;
                *reinterpret_cast<bf16x4 *>(lo + lds_off(r, c)) = l;
            }
        } else {
#pragma unroll
            for (int j = 0; j < PER_T; ++j) {
                if (skip(j, tid)) continue;
                int kb, rb;
                block(tid + j * NT, kb, rb);
                const float4 *b = v + 4 * j;
                const float cols[4][4] = {{b[0].x, b[1].x, b[2].x, b[3].x},
                                          {b[0].y, b[1].y, b[2].y, b[3].y},
                                          {b[0].z, b[1].z, b[2].z, b[3].z},
                                          {b[0].w, b[1].w, b[2].w, b[3].w}};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    bf16x4 h, l;
                    split4(cols[c], h, l);
                    *reinterpret_cast<bf16x4 *>(hi + lds_off(rb + c, 4 * kb)) = h;
                    *reinterpret_cast<bf16x4 *>(lo + lds_off(rb + c, 4 * kb)) = l;
                }
            }
        }
    }
    // The store in pieces: chunk P (KCONT), or column P % 4 of block P / 4.
    static constexpr int NPIECE = KCONT ? NLD : 4 * PER_T;
    template <int P>
    __device__ __forceinline__ void store_piece(__bf16 *hi, __bf16 *lo, int tid) const {
        if constexpr (KCONT) {
            int r, c;
            chunk(tid + P * NT, r, c);
            const float x[4] = {v[P].x, v[P].y, v[P].z, v[P].w};
            bf16x4 h, l;
            split4(x, h, l);
            *reinterpret_cast<bf16x4 *>(hi + lds_off(r, c)) = h;
            *reinterpret_cast<bf16x4 *>(lo + lds_off(r, c)) = l;
        } else {
            constexpr int j = P / 4, c = P % 4;
            if (skip(j, tid)) return;
            int kb, rb;
            block(tid + j * NT, kb, rb);
            const float4 *b = v + 4 * j;
            auto col = [](const float4 &x) {
                return c == 0 ? x.x : c == 1 ? x.y : c == 2 ? x.z : x.w;
            };
            const float x[4] = {col(b[0]), col(b[1]), col(b[2]), col(b[3])};
            bf16x4 h, l;
            split4(x, h, l);
            *reinterpret_cast<bf16x4 *>(hi + lds_off(rb + c, 4 * kb)) = h;
            *reinterpret_cast<bf16x4 *>(lo + lds_off(rb + c, 4 * kb)) = l;
        }
    }
    // The interior loads into the registers that piece P was the last to read.
    template <int P>
    __device__ __forceinline__ void load_after_piece(const float *base, const unsigned (&o)[NLD],
                                                     int tid) {
        auto at = [&](int i) {
            return reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) + o[i]);
        };
        if constexpr (KCONT) {
            v[P] = ld_in(at(P));
        } else if constexpr (P % 4 == 3) {
            constexpr int j = P / 4;
            if (skip(j, tid)) return;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[4 * j + i] = ld_in(at(4 * j + i));
        }
    }
};

// op(A) is M x K, op(B) K x N; stored A is M x K (lda = K) or, TA, K x M
// (lda = M); stored B is K x N (ldb = N) or, TB, N x K (ldb = K). C is M x N.
template <class Tl, bool TA, bool TB, bool VEC>
struct Bf16x3Gemm {
    static constexpr int BM = Tl::BM, BN = Tl::BN, NT = Tl::NT;
    static constexpr int FM = Tl::FM, FN = Tl::FN;
    using SA = OpStage<BM, NT, !TA, VEC>;
    using SB = OpStage<BN, NT, TB, VEC>;

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

    // MFMA MI of a step in round-robin order over the accumulators: every
    // lo_a hi_b term, then every hi_a lo_b, then every hi_a hi_b. Each
    // accumulator takes its three terms in step()'s order.
    template <int MI>
    __device__ static __forceinline__ void mfma_rr(const bf16x8 (&ah)[FM], const bf16x8 (&al)[FM],
                                                   const bf16x8 (&bh)[FN], const bf16x8 (&bl)[FN],
                                                   f32x16 (&acc)[FM][FN]) {
        constexpr int round = MI / (FM * FN), idx = MI % (FM * FN), fi = idx / FN, fn = idx % FN;
        if constexpr (round == 0)
            acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[fi], bh[fn], acc[fi][fn], 0, 0, 0);
        else if constexpr (round == 1)
            acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[fi], bl[fn], acc[fi][fn], 0, 0, 0);
        else
            acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[fi], bh[fn], acc[fi][fn], 0, 0, 0);
    }

    // Step 0 of stage st with the next stage's split and LDS stores (into nx)
    // between its MFMAs: piece P follows MFMAs [P NM / NP, (P + 1) NM / NP)
    // behind a scheduling fence, and is followed by the loads (stage bases an,
    // bn) that refill its registers.
    __device__ static __forceinline__ void step0_fused(const __bf16 *st, __bf16 *nx, SA &ga, SB &gb,
                                                       const float *an, const float *bn,
                                                       const unsigned (&oa)[SA::NLD],
                                                       const unsigned (&ob)[SB::NLD], int wm,
                                                       int wn, int lane, int tid,
                                                       f32x16 (&acc)[FM][FN]) {
        const int l32 = lane & 31, koff = 8 * (lane >> 5);
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
        constexpr int NPA = SA::NPIECE, NP = NPA + SB::NPIECE, NM = FM * FN * 3;
        static_for<0, NP>([&](auto pc) {
            constexpr int P = decltype(pc)::value;
            static_for<P * NM / NP, (P + 1) * NM / NP>([&](auto mc) {
                mfma_rr<decltype(mc)::value>(ah, al, bh, bl, acc);
            });
            if constexpr (P < NPA) {
                ga.template store_piece<P>(nx, nx + Tl::A_PLANE, tid);
                ga.template load_after_piece<P>(an, oa, tid);
            } else {
                gb.template store_piece<P - NPA>(nx + 2 * Tl::A_PLANE,
                                                 nx + 2 * Tl::A_PLANE + Tl::B_PLANE, tid);
                gb.template load_after_piece<P - NPA>(bn, ob, tid);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    }

    // One output tile over k in [0, K) (A, B positioned at that range's
    // start). INTERIOR: the tile lies inside M x N and K > 0, so no store
    // and no load of a whole stage needs a bounds check. KTAIL (INTERIOR
    // only): K is not a whole number of stages, and the last stage's loads
    // are guarded (zero fill past K); every other stage runs the interior
    // loop. EPI: what the epilogue stores (bmb::Epi; EPI_PARTIAL: the raw
    // sums). C's rows (and those of ep.act, ep.pre) are ldc floats apart.
    // KS > 1: the workgroup is KS k-slices of NT lanes (bf16x3_ks_k); this
    // slice's stages are at smem, K is its range's length (<= 0: none of its
    // stages holds data) and every slice runs kloop stages, so that all of
    // them meet at the same barriers. The slices' sums are then added in LDS,
    // in slice order, and slice 0 runs the epilogue.
    template <bool INTERIOR, int EPI, bool KTAIL = false, int KS = 1>
    __device__ static __forceinline__ void run(int M, int N, int K, int lda, int ldb, float alpha,
                                               const float *__restrict__ A,
                                               const float *__restrict__ B, float beta, float *C,
                                               int ldc, int m0, int n0, __bf16 *smem,
                                               const bmb::EpiArgs &ep, int kloop = 0) {
        const int tid = KS > 1 ? (int)(threadIdx.x % NT) : (int)threadIdx.x;
        const int wave = tid >> 6, lane = tid & 63;
        const int wm = (wave / Tl::WAVES_N) * Tl::WM, wn = (wave % Tl::WAVES_N) * Tl::WN;

        f32x16 acc[FM][FN];
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fi][fn][r] = 0.0f;

        const int nkt = KS > 1 ? kloop : (K + BK - 1) / BK;
        SA ga;
        SB gb;
        unsigned oa[SA::NLD], ob[SB::NLD];
        if (INTERIOR) {
            SA::offsets(oa, lda, tid);
            SB::offsets(ob, ldb, tid);
        }
        // Stage kt's bases (uniform): the (row 0, k 0) element of each tile.
        auto a_at = [&](int kt) {
            return TA ? A + (size_t)kt * BK * lda + m0 : A + (size_t)m0 * lda + (size_t)kt * BK;
        };
        auto b_at = [&](int kt) {
            return TB ? B + (size_t)n0 * ldb + (size_t)kt * BK : B + (size_t)kt * BK * ldb + n0;
        };
        auto load = [&](int kt) {
            if (INTERIOR && !(KTAIL && kt == nkt - 1)) {
                ga.load_interior(a_at(kt), oa, tid);
                gb.load_interior(b_at(kt), ob, tid);
            } else {
                ga.load_guarded(A, M, K, lda, m0, kt * BK, tid);
                gb.load_guarded(B, N, K, ldb, n0, kt * BK, tid);
            }
        };
        auto store = [&](__bf16 *st) {
            ga.store(st, st + Tl::A_PLANE, tid);
            gb.store(st + 2 * Tl::A_PLANE, st + 2 * Tl::A_PLANE + Tl::B_PLANE, tid);
        };
        if (nkt > 0) {
            load(0);
            store(smem);
            if (nkt > 1) load(1);
        }
        __syncthreads();
        int kt0 = 0;
        if (INTERIOR) {
            // Stages with a next stage to store and a whole stage after it to
            // load (KTAIL: the last stage is loaded by the loop below).
            for (; kt0 + 2 < nkt - (KTAIL ? 1 : 0); ++kt0) {
                const __bf16 *st = smem + (kt0 & 1) * Tl::STAGE;
                step0_fused(st, smem + ((kt0 + 1) & 1) * Tl::STAGE, ga, gb, a_at(kt0 + 2),
                            b_at(kt0 + 2), oa, ob, wm, wn, lane, tid, acc);
                step(st, 1, wm, wn, lane, acc);
                __syncthreads();
            }
        }
        for (int kt = kt0; kt < nkt; ++kt) {
            const __bf16 *st = smem + (kt & 1) * Tl::STAGE;
            step(st, 0, wm, wn, lane, acc);
            if (kt + 1 < nkt) {
                // The other stage was last read before the previous barrier.
                store(smem + ((kt + 1) & 1) * Tl::STAGE);
                if (kt + 2 < nkt) load(kt + 2);
            }
            step(st, 1, wm, wn, lane, acc);
            __syncthreads();
        }

        if constexpr (KS > 1) {
            // Slices 1 .. KS-1 leave their sums in LDS (over the stages, which
            // every slice has finished reading at the loop's last barrier);
            // slice 0 adds them in slice order.
            const int slice = (int)(threadIdx.x / NT);
            float *red = reinterpret_cast<float *>(smem - (size_t)slice * 2 * Tl::STAGE);
            static_assert((size_t)(KS - 1) * FM * FN * 16 * NT * sizeof(float) <=
                              (size_t)KS * Tl::SMEM_BYTES,
                          "the slices' sums fit in the workgroup's stages");
            if (slice > 0) {
#pragma unroll
                for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            red[((((size_t)slice - 1) * FM + fi) * FN + fn) * 16 * NT + r * NT + tid] =
                                acc[fi][fn][r];
            }
            __syncthreads();
            if (slice > 0) return;
#pragma unroll 1
            for (int sl = 1; sl < KS; ++sl)
#pragma unroll
                for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[fi][fn][r] +=
                                red[((((size_t)sl - 1) * FM + fi) * FN + fn) * 16 * NT + r * NT + tid];
        }

        // Epilogue: lanes 0-31 of a register cover 32 consecutive columns.
        // Whatever a row of FN blocks reads (C for beta != 0, the GELU input)
        // is gathered before any result is stored: 16 * FN loads in flight.
        const int l32 = lane & 31, half = lane >> 5;
        const bool reads = (EPI == bmb::EPI_BLAS && beta != 0.0f) || EPI == bmb::EPI_GELU_GRAD;
        float bias[FN];
        if (EPI == bmb::EPI_BIAS || EPI == bmb::EPI_BIAS_GELU) {
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
                const int col = n0 + wn + fn * 32 + l32;
                bias[fn] = (INTERIOR || col < N) ? ep.bias[col] : 0.0f;
            }
        }
#pragma unroll
        for (int fi = 0; fi < FM; ++fi) {
            float in[FN][16];
            if (reads) {
                const float *src = EPI == bmb::EPI_GELU_GRAD ? ep.pre : C;
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) {
                    const int col = n0 + wn + fn * 32 + l32;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = m0 + wm + fi * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                        in[fn][r] = (INTERIOR || (row < M && col < N))
                                        ? src[(size_t)row * ldc + col] : 0.0f;
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
                    const size_t idx = (size_t)row * ldc + col;
                    if (EPI == bmb::EPI_PARTIAL) {
                        C[idx] = a;
                    } else if (EPI == bmb::EPI_BLAS) {
                        C[idx] = reads ? bmb::fma_rn(alpha, a, beta * in[fn][r]) : alpha * a;
                    } else if (EPI == bmb::EPI_GELU_GRAD) {
                        C[idx] = bmb::gelu_grad(in[fn][r], a);
                    } else {
                        const float v = a + bias[fn];
                        C[idx] = v;
                        if (EPI == bmb::EPI_BIAS_GELU) ep.act[idx] = bmb::gelu(v);
                    }
                }
            }
        }
    }
};

// Grid: x = output tiles (XCD-remapped, grouped), y = K range s, covering
// k in [s*kchunk, min(K, (s+1)*kchunk)) (kchunk a multiple of BK when
// gridDim.y > 1). EPI_PARTIAL: write the range's raw sums to C + s*M*N
// (packed rows). lda, ldb, ldc: the row strides of the stored A (at least M
// when TA, K otherwise), B (at least K when TB, N otherwise) and C (at least
// N), so that a block of rows and columns of a larger problem (its operands
// offset to its first row and column) runs as a problem of its own.
// KT: K is not a whole number of stages; interior tiles then run the
// interior loop with a guarded last stage (Bf16x3Gemm::run's KTAIL). A
// separate instantiation: the extra path costs the 256 x 256 kernels about a
// dozen spilled registers, which the other shapes need not pay.
template <class Tl, bool TA, bool TB, bool VEC, int EPI, bool KT = false>
__global__ __launch_bounds__(Tl::NT) void bf16x3_k(int M, int N, int K, int kchunk, float alpha,
                                                   const float *__restrict__ A, int lda,
                                                   const float *__restrict__ B, int ldb,
                                                   float beta, float *C, int ldc, int tiles_m,
                                                   int tiles_n, bmb::EpiArgs ep) {
    extern __shared__ __bf16 lds[];
    using G = Bf16x3Gemm<Tl, TA, TB, VEC>;
    int tm, tn;
    bmb::group_tile(bmb::xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int m0 = tm * Tl::BM, n0 = tn * Tl::BN;
    const int kb = blockIdx.y * kchunk, klen = min(K, kb + kchunk) - kb;
    const float *Ak = TA ? A + (size_t)kb * lda : A + kb;
    const float *Bk = TB ? B + kb : B + (size_t)kb * ldb;
    float *Cs = EPI == bmb::EPI_PARTIAL ? C + (size_t)blockIdx.y * M * N : C;
    const int ldcs = EPI == bmb::EPI_PARTIAL ? N : ldc;
    if (m0 + Tl::BM <= M && n0 + Tl::BN <= N && klen > 0 && klen % BK == 0)
        G::template run<true, EPI>(M, N, klen, lda, ldb, alpha, Ak, Bk, beta, Cs, ldcs, m0, n0,
                                   lds, ep);
    else if (KT && m0 + Tl::BM <= M && n0 + Tl::BN <= N && klen > 0)
        G::template run<true, EPI, true>(M, N, klen, lda, ldb, alpha, Ak, Bk, beta, Cs, ldcs, m0,
                                         n0, lds, ep);
    else
        G::template run<false, EPI>(M, N, klen, lda, ldb, alpha, Ak, Bk, beta, Cs, ldcs, m0, n0,
                                    lds, ep);
}

// The same tile as KS k-slices of Tl::NT lanes each (any epilogue but a
// split-K partial: it never splits). Every slice runs per = ceil(stages / KS)
// stages, slice s those from s * per on, in its own KS-th of the LDS, and the
// slices' sums meet in LDS (Bf16x3Gemm::run). For problems with too few
// output tiles to fill the device, where split-K would need a second launch
// for its reduce. A slice of an interior tile whose range is `per` whole
// stages takes the unguarded loop, the others the guarded one (both loops
// pass the same number of barriers).
template <class Tl, bool TA, bool TB, bool VEC, int EPI, int KS>
__global__ __launch_bounds__(Tl::NT * KS) void bf16x3_ks_k(int M, int N, int K, float alpha,
                                                           const float *__restrict__ A, int lda,
                                                           const float *__restrict__ B, int ldb,
                                                           float beta, float *C, int ldc,
                                                           int tiles_m, int tiles_n,
                                                           bmb::EpiArgs ep) {
    extern __shared__ __bf16 lds[];
    using G = Bf16x3Gemm<Tl, TA, TB, VEC>;
    int tm, tn;
    bmb::group_tile(bmb::xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int m0 = tm * Tl::BM, n0 = tn * Tl::BN;
    const int slice = (int)(threadIdx.x / Tl::NT);
    const int per = ((K + BK - 1) / BK + KS - 1) / KS;
    const int kb = slice * per * BK;
    const int klen = min(K - kb, per * BK);  // <= 0: a slice past K (zero stages of data)
    const float *Ak = TA ? A + (size_t)min(kb, K) * lda : A + min(kb, K);
    const float *Bk = TB ? B + min(kb, K) : B + (size_t)min(kb, K) * ldb;
    __bf16 *st = lds + (size_t)slice * 2 * Tl::STAGE;
    if (m0 + Tl::BM <= M && n0 + Tl::BN <= N && klen == per * BK)
        G::template run<true, EPI, false, KS>(M, N, klen, lda, ldb, alpha, Ak, Bk, beta, C, ldc,
                                              m0, n0, st, ep, per);
    else
        G::template run<false, EPI, false, KS>(M, N, klen, lda, ldb, alpha, Ak, Bk, beta, C, ldc,
                                               m0, n0, st, ep, per);
}

// ------------------------------------------------------------- host side

// Tile and split choice, the fp32 MFMA planner's time model (mfma_gemm.hip)
// with this path's own constants: a work item is one output tile over one K
// range; the device runs cus x occupancy of them per round; a part-filled
// last round runs each CU's items faster by (held / fit)^PARTIAL_EXP, and a
// single round that leaves CUs idle runs faster again by
// (busy CUs / cus)^FILL_EXP; a split adds the partials' round trip and the
// reduce. The tile rates and PARTIAL_EXP are fitted to a forced sweep on
// MI355X of every tile x split count below over the GPT-2 shapes and the
// square sweep N = 512 ... 8192 (810 timed plans): the model's plan is the
// measured best, or within 3% of it (the sweep's run-to-run spread), on all
// of them but N = 2048 (5%). The 128 x 256 tile serves the N = 768 and
// 3072-wide GPT-2 layers with K = 768 or 3072 (4-9% faster than 128 x 128
// there); a 256 x 128 tile was never chosen and is not built.
//
// Row bands. A tile count just above a whole number of rounds (4097^2 on
// 256 x 256: 289 tiles on 256 CUs; 6144^2: 576 tiles, 2.25 rounds; the GPT-2
// QKV forward, 8192 x 2304: 288 tiles) leaves most CUs idle for a whole
// extra tile time. A plan may therefore run C as two bands of full-width
// rows, one launch each on the same stream: rows [0, m1) on one tile with
// whole K, sized to whole rounds, and rows [m1, M) on the plan (tile and
// split) that suits that remainder, typically a smaller tile or a K split
// that spreads it over every CU.
struct B3Cand {
    int bm, bn;
    double tflops;  // fitted fp32-equivalent TFLOP/s when the device is full of them
    int ks;         // k-slices per workgroup (bf16x3_ks_k; never split)
};
constexpr B3Cand CANDS[] = {{256, 256, 452.0, 1}, {128, 128, 326.0, 1}, {64, 64, 233.0, 1},
                            {128, 256, 345.0, 1}, {64, 64, 233.0, 2},  {64, 64, 233.0, 4},
                            {32, 32, 180.0, 4},   {32, 32, 180.0, 8}};
constexpr int N_CANDS = 8;
// A k-sliced workgroup: each slice beyond the first adds KS_OVERHEAD k to its
// item (its own prologue and the slices' sum in LDS); the 32 x 32 tile only
// for problems of at most XS_MAX_OUTPUTS outputs, every slice at least
// MIN_SLICE_K of k. Fitted to a forced sweep of every plan on ten problems
// of 0.06-1.1 M outputs (the squares 512-2048, 256 x 256 x 4096, 512 x 512
// x 2048, 384 x 384 x 1000, 128 x 1024 x 8192): the model's plan is the
// measured best on all but N = 2048 (5%, as before). The k-sliced plans
// replace split-K plus its reduce at N = 512 (9.5 -> 5.6 us), 768, 1000 and
// 1024 (19.4 -> 15.0 us); no GPT-2 shape or square above 1024 changes plan.
constexpr double KS_OVERHEAD = 64.0;
constexpr long long XS_MAX_OUTPUTS = 1LL << 20;
constexpr int MIN_SLICE_K = 64;
// Split counts that are not powers of two fill the device in one round where
// {2, 4, 8} do not (the GPT-2 weight gradients: 36 tiles of 256 x 256 in 7
// ranges on 256 CUs, 36 of 128 x 128 in 14 on 512 slots: 18-36% faster). The
// model undercharges short ranges, so these are only considered when every
// range keeps MIN_ODD_SPLIT_K of k (a 7-way split of K = 1536, 224 per
// range, measured 5.5% slower than the 4-way split the model ranked second).
constexpr int SPLITS[] = {1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16};
constexpr int MIN_ODD_SPLIT_K = 512;
constexpr double PARTIAL_EXP = 0.63;
constexpr double FILL_EXP = 0.3;
constexpr double K_OVERHEAD = 96.0;               // per-item prologue/epilogue, in k
constexpr double PARTIALS_BYTES_PER_S = 1.35e13;  // the partials' round trip
constexpr double LAUNCH_S = 1.6e-6;               // the reduce launch
// A second band: its launch and the drain between the bands. Bands are only
// tried for K >= MIN_BAND_K, with K ranges of at least MIN_BAND_SPLIT_K in a
// split remainder band, and taken when modelled 3% faster than one band:
// measured on MI355X, bands gained 15-18% at N = 4097 and 6144 and on the
// GPT-2 LM-head weight gradient (K = 8192), and 4.5% on the GPT-2 QKV
// forward (8192 x 2304 x 768: 7168 rows on 256 x 256 tiles in two whole
// rounds, the last 1024 on 128 x 128). Without the bound on the remainder's
// K ranges they lost 3-7% on the K = 768 and 3072 GPT-2 GEMMs, whose short
// split ranges the model undercharges; with it, no other GPT-2 or square
// sweep shape changes plan. Corner plans (below) are tried for
// K >= MIN_CORNER_K only, the range they were measured on.
constexpr double BAND_S = 12.0e-6;
constexpr double BAND_GAIN = 0.97;
constexpr int MIN_BAND_K = 768;
constexpr int MIN_CORNER_K = 4096;
constexpr int MIN_BAND_SPLIT_K = 512;
constexpr int MIN_SPLIT_K = 64;  // two stages
constexpr long long MAX_SPLIT_FLOATS = 64LL << 20;  // 256 MiB of partials

template <class Kern>
int occupancy_of(Kern kern, int threads, size_t smem) {
    int n = 0;
    bmb::allow_smem(kern, smem);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, smem) != hipSuccess) {
        (void)hipGetLastError();
        n = 1;
    }
    return n < 1 ? 1 : n;
}
template <class Tl>
int occupancy_of() {
    return occupancy_of(bf16x3_k<Tl, false, false, true, bmb::EPI_BLAS>, Tl::NT, Tl::SMEM_BYTES);
}
template <class Tl, int KS>
int ks_occupancy_of() {
    return occupancy_of(bf16x3_ks_k<Tl, false, false, true, bmb::EPI_BLAS, KS>, Tl::NT * KS,
                        KS * Tl::SMEM_BYTES);
}

// One band's launch: tile candidate, K ranges and the K per range.
struct Part {
    int tile, splits, kchunk;
};

// Rows [0, m1) run on part[0], rows [m1, M) on part[1] (m1 == M: one band).
// A corner plan (edges) instead runs rows [0, m1) x columns [0, n1) on
// part[0], a block of whole tiles, and the at most EDGE_MAX columns right of
// it and rows below it on the edge kernels (edge_gemm.hip): 4097^2 as
// 4096^2 on 256 x 256 tiles plus a 4096 x 1 and a 1 x 4097 edge, where a
// plan of tiles alone computes 289 tiles (13% more than C) or runs a second
// band.
struct Plan {
    Part part[2];
    int m1, n1;
    bool edges;
};

struct Device {
    int occ[N_CANDS], cus;
};

const Device &device_info(int dev) {
    static std::once_flag once[64];
    static Device info[64];
    std::call_once(once[dev], [&] {
        Device &d = info[dev];
        d.occ[0] = occupancy_of<TileL>();
        d.occ[1] = occupancy_of<TileM>();
        d.occ[2] = occupancy_of<TileS>();
        d.occ[3] = occupancy_of<TileT>();
        d.occ[4] = ks_occupancy_of<TileS, 2>();
        d.occ[5] = ks_occupancy_of<TileS, 4>();
        d.occ[6] = ks_occupancy_of<TileXS, 4>();
        d.occ[7] = ks_occupancy_of<TileXS, 8>();
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            c <= 0) {
            (void)hipGetLastError();
            c = 256;
        }
        d.cus = c;
    });
    return info[dev];
}

// Modelled time of an M x N x K band on tile t with K split s ways; false if
// that split is not allowed (may_split, max_floats caps splits * M * N).
bool part_time(const Device &dv, int M, int N, int K, int t, int s, bool may_split,
               long long max_floats, Part &out, double &time) {
    const B3Cand &c = CANDS[t];
    int splits = 1, kchunk = K;
    if (c.ks > 1) {
        if (s > 1 || K < c.ks * MIN_SLICE_K) return false;
        if (c.bm == 32 && (long long)M * N > XS_MAX_OUTPUTS) return false;
    }
    if (s > 1) {
        if (!may_split || K < 2 * MIN_SPLIT_K) return false;
        kchunk = (K + s - 1) / s;
        kchunk = (kchunk + BK - 1) / BK * BK;
        if (kchunk < MIN_SPLIT_K) return false;
        splits = (K + kchunk - 1) / kchunk;
        if (splits < 2 || (long long)splits * M * N > max_floats) return false;
        if ((s & (s - 1)) != 0 && kchunk < MIN_ODD_SPLIT_K) return false;
    }
    const long long tiles = (long long)bmb::ceil_div(M, c.bm) * bmb::ceil_div(N, c.bn);
    const long long items = tiles * splits;
    const int occ = dv.occ[t], cus = dv.cus;
    const long long slots = (long long)cus * occ;
    const double t_item = 2.0 * c.bm * c.bn * (kchunk + K_OVERHEAD + (c.ks - 1) * KS_OVERHEAD) *
                          occ / (c.tflops * 1e12 / cus);
    const long long full = items / slots, rem = items % slots;
    time = full * t_item;
    if (rem) {
        const long long per_cu = (rem + cus - 1) / cus;
        double last =
            per_cu < occ ? t_item * pow((double)per_cu / occ, PARTIAL_EXP) : t_item;
        if (full == 0 && rem < cus) last *= pow((double)rem / cus, FILL_EXP);
        time += last;
    }
    if (splits > 1) time += (splits + 2.0) * M * N * 4.0 / PARTIALS_BYTES_PER_S + LAUNCH_S;
    out = Part{t, splits, kchunk};
    return true;
}

// The fastest single-band plan of an M x N x K band (split K ranges of at
// least min_split_k; k-sliced tiles only if ks_ok).
double best_part(const Device &dv, int M, int N, int K, bool may_split, long long max_floats,
                 Part &best, int min_split_k = 0, bool ks_ok = false) {
    double best_t = -1.0;
    best = Part{0, 1, K};
    for (int t = 0; t < N_CANDS; ++t)
        for (int s : SPLITS) {
            if (CANDS[t].ks > 1 && !ks_ok) continue;
            Part p;
            double tm;
            if (part_time(dv, M, N, K, t, s, may_split, max_floats, p, tm) &&
                (p.splits == 1 || p.kchunk >= min_split_k) && (best_t < 0 || tm < best_t)) {
                best_t = tm;
                best = p;
            }
        }
    return best_t;
}

// ks_ok: the k-sliced tiles may run the problem (single-band plans only).
Plan plan_for(int dev, int M, int N, int K, bool may_split, long long max_floats,
              bool edges_ok, bool ks_ok) {
    const Device &dv = device_info(dev);
    Plan best{{Part{0, 1, K}, Part{0, 1, K}}, M, N, false};
    const double single_t =
        best_part(dv, M, N, K, may_split, max_floats, best.part[0], 0, ks_ok);
    double best_t = single_t;
    // Two bands: the first whole rounds of one tile, the rest on its own plan.
    for (int t = 0; K >= MIN_BAND_K && t < N_CANDS; ++t) {
        const B3Cand &c = CANDS[t];
        if (c.ks > 1) continue;
        const long long tiles_n = bmb::ceil_div(N, c.bn);
        const long long slots = (long long)dv.cus * dv.occ[t];
        for (long long k = 1;; ++k) {
            const long long rows = k * slots / tiles_n;  // tile rows in k whole rounds
            if (rows <= 0) continue;
            if (rows * c.bm >= M) break;
            const int m1 = (int)(rows * c.bm);
            Part p0, p1;
            double t0, t1;
            if (!part_time(dv, m1, N, K, t, 1, false, 0, p0, t0)) continue;
            t1 = best_part(dv, M - m1, N, K, may_split, max_floats, p1, MIN_BAND_SPLIT_K);
            if (t1 < 0) continue;
            const double tm = t0 + t1 + BAND_S;
            if (tm < BAND_GAIN * single_t && tm < best_t) {
                best_t = tm;
                best = Plan{{p0, p1}, m1, N, false};
            }
        }
    }
    // Corner plans: whole tiles of one candidate over [0, m1) x [0, n1), the
    // edges on the edge kernels (row-major A and B, BLAS epilogue; their
    // scratch only where K may be split).
    for (int t = 0; edges_ok && may_split && K >= MIN_CORNER_K && t < N_CANDS; ++t) {
        const B3Cand &c = CANDS[t];
        if (c.ks > 1) continue;
        const int m1 = M / c.bm * c.bm, n1 = N / c.bn * c.bn;
        if (m1 == 0 || n1 == 0 || (m1 == M && n1 == N) || M - m1 > bmb::EDGE_MAX ||
            N - n1 > bmb::EDGE_MAX || bmb::edge_partial_floats(M - m1, N - n1, N, K) > max_floats)
            continue;
        Part p0;
        double t0;
        if (!part_time(dv, m1, n1, K, t, 1, false, 0, p0, t0)) continue;
        const double tm = t0 + bmb::edge_model_s(m1, N - n1, M - m1, N, K);
        if (tm < BAND_GAIN * single_t && tm < best_t) {
            best_t = tm;
            best = Plan{{p0, Part{0, 1, K}}, m1, n1, true};
        }
    }
    if (getenv("BMB_GEMM_PLAN_TRACE") != nullptr)
        fprintf(stderr, "bf16x3 gemm plan %dx%dx%d: m1 %d n1 %d edges %d parts (%d,%d,%d) "
                        "(%d,%d,%d) model %.1f us (one band %.1f us)\n",
                M, N, K, best.m1, best.n1, (int)best.edges, best.part[0].tile,
                best.part[0].splits, best.part[0].kchunk, best.part[1].tile, best.part[1].splits,
                best.part[1].kchunk, best_t * 1e6, single_t * 1e6);
    return best;
}

// Plans are memoised per (device, shape, split permission and cap): the
// search above costs tens of microseconds, a GEMM call in a training step
// a few hundred.
Plan pick(int M, int N, int K, bool may_split, long long max_floats, bool edges_ok,
          bool ks_ok) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    using Key = std::tuple<int, int, int, int, bool, long long, bool, bool>;
    static std::mutex mu;
    static std::map<Key, Plan> memo;
    const Key key{dev, M, N, K, may_split, max_floats, edges_ok, ks_ok};
    {
        std::lock_guard<std::mutex> lock(mu);
        auto it = memo.find(key);
        if (it != memo.end()) return it->second;
    }
    const Plan p = plan_for(dev, M, N, K, may_split, max_floats, edges_ok, ks_ok);
    std::lock_guard<std::mutex> lock(mu);
    if (memo.size() > 4096) memo.clear();
    memo.emplace(key, p);
    return p;
}

// The row strides of a launch's operands (see bf16x3_k).
struct Strides {
    int lda, ldb, ldc;
};

template <class Tl, bool TA, bool TB, int EPI>
void launch(int M, int N, int K, int kchunk, int splits, float alpha, const float *A,
            const float *B, float beta, float *C, const Strides &ld, bool vec,
            hipStream_t stream, bmb::EpiArgs ep) {
    const int tiles_m = bmb::ceil_div(M, Tl::BM), tiles_n = bmb::ceil_div(N, Tl::BN);
    const dim3 grid(tiles_m * tiles_n, splits);
    auto go = [&](auto kern) {
        bmb::allow_smem(kern, Tl::SMEM_BYTES);
        bmb::launch(kern, grid, dim3(Tl::NT), Tl::SMEM_BYTES, stream, M, N, K, kchunk, alpha, A,
                    ld.lda, B, ld.ldb, beta, C, ld.ldc, tiles_m, tiles_n, ep);
    };
    // (A ragged K has the guarded-tail interior kernels for the BLAS and
    // split-K epilogues; the fused ones run at K = 768 and 3072.)
    constexpr bool KT_OK = EPI == bmb::EPI_BLAS || EPI == bmb::EPI_PARTIAL;
    const bool kt = KT_OK && K % BK != 0;
    if (vec) {
        if (kt) go(bf16x3_k<Tl, TA, TB, true, EPI, KT_OK>);
        else go(bf16x3_k<Tl, TA, TB, true, EPI>);
    } else {
        if (kt) go(bf16x3_k<Tl, TA, TB, false, EPI, KT_OK>);
        else go(bf16x3_k<Tl, TA, TB, false, EPI>);
    }
}

// One band on tile Tl: one launch with the epilogue, or the split partials
// (EPI_PARTIAL into P) and the shared reduce with the epilogue.
template <class Tl, bool TA, bool TB, int EPI>
void run_part(const Part &p, int M, int N, int K, float alpha, const float *A, const float *B,
              float beta, float *C, const Strides &ld, bool vec, float *P, hipStream_t stream,
              bmb::EpiArgs ep) {
    if (p.splits > 1) {
        launch<Tl, TA, TB, bmb::EPI_PARTIAL>(M, N, K, p.kchunk, p.splits, 1.0f, A, B, 0.0f, P,
                                             ld, vec, stream, ep);
        bmb::splitk_reduce_epi(EPI, C, P, p.splits, (long long)M * N, N, ld.ldc, alpha, beta,
                               stream, ep.bias, ep.act, ep.pre);
    } else {
        launch<Tl, TA, TB, EPI>(M, N, K, K, 1, alpha, A, B, beta, C, ld, vec, stream, ep);
    }
}

// One k-sliced launch: one workgroup of KS slices per tile.
template <class Tl, bool TA, bool TB, int EPI, int KS>
void launch_ks(int M, int N, int K, float alpha, const float *A, const float *B, float beta,
               float *C, const Strides &ld, bool vec, hipStream_t stream, bmb::EpiArgs ep) {
    const int tiles_m = bmb::ceil_div(M, Tl::BM), tiles_n = bmb::ceil_div(N, Tl::BN);
    const size_t smem = (size_t)KS * Tl::SMEM_BYTES;
    auto go = [&](auto kern) {
        bmb::allow_smem(kern, smem);
        bmb::launch(kern, dim3(tiles_m * tiles_n), dim3(Tl::NT * KS), smem, stream, M, N, K,
                    alpha, A, ld.lda, B, ld.ldb, beta, C, ld.ldc, tiles_m, tiles_n, ep);
    };
    if (vec) go(bf16x3_ks_k<Tl, TA, TB, true, EPI, KS>);
    else go(bf16x3_ks_k<Tl, TA, TB, false, EPI, KS>);
}

template <bool TA, bool TB, int EPI>
void run_band(const Part &p, int M, int N, int K, float alpha, const float *A, const float *B,
              float beta, float *C, const Strides &ld, bool vec, float *P, hipStream_t stream,
              bmb::EpiArgs ep) {
    if (CANDS[p.tile].ks > 1) {
        // (never planned for a split-K partial)
        if constexpr (EPI != bmb::EPI_PARTIAL) {
            switch (p.tile) {
            case 4: launch_ks<TileS, TA, TB, EPI, 2>(M, N, K, alpha, A, B, beta, C, ld, vec, stream, ep); break;
            case 5: launch_ks<TileS, TA, TB, EPI, 4>(M, N, K, alpha, A, B, beta, C, ld, vec, stream, ep); break;
            case 6: launch_ks<TileXS, TA, TB, EPI, 4>(M, N, K, alpha, A, B, beta, C, ld, vec, stream, ep); break;
            default: launch_ks<TileXS, TA, TB, EPI, 8>(M, N, K, alpha, A, B, beta, C, ld, vec, stream, ep); break;
            }
        }
        return;
    }
    switch (p.tile) {
    case 0: run_part<TileL, TA, TB, EPI>(p, M, N, K, alpha, A, B, beta, C, ld, vec, P, stream, ep); break;
    case 1: run_part<TileM, TA, TB, EPI>(p, M, N, K, alpha, A, B, beta, C, ld, vec, P, stream, ep); break;
    case 2: run_part<TileS, TA, TB, EPI>(p, M, N, K, alpha, A, B, beta, C, ld, vec, P, stream, ep); break;
    default: run_part<TileT, TA, TB, EPI>(p, M, N, K, alpha, A, B, beta, C, ld, vec, P, stream, ep); break;
    }
}

// Both bands of a plan, in row order on one stream (the second band's split
// partials reuse P after the first band's reduce has read it).
template <bool TA, bool TB, int EPI>
void run_plan(const Plan &p, int M, int N, int K, float alpha, const float *A, const float *B,
              float beta, float *C, bool vec, float *P, hipStream_t stream, bmb::EpiArgs ep) {
    const Strides ld{TA ? M : K, TB ? K : N, N};
    run_band<TA, TB, EPI>(p.part[0], p.m1, p.n1, K, alpha, A, B, beta, C, ld, vec, P, stream, ep);
    if (p.edges) {
        bmb::gemm_edges(true, M, N, K, p.m1, p.n1, alpha, A, ld.lda, B, ld.ldb, beta, C, ld.ldc,
                        P, stream);
        return;
    }
    if (p.m1 >= M) return;
    const size_t r = (size_t)p.m1;
    bmb::EpiArgs e1 = ep;
    if (e1.act) e1.act += r * N;
    if (e1.pre) e1.pre += r * N;
    // A band of rows starts r rows (TA: r columns of the stored K x M) in.
    const float *A1 = TA ? A + r : A + r * K;
    // 16-byte loads of the band need its first row aligned as well.
    const bool vec1 = vec && (((uintptr_t)A1 & 15) == 0);
    run_band<TA, TB, EPI>(p.part[1], M - p.m1, N, K, alpha, A1, B, beta, C + r * N, ld, vec1, P,
                          stream, e1);
}

long long partial_floats(const Plan &p, int M, int N, int K) {
    long long f = 0;
    if (p.edges) return bmb::edge_partial_floats(M - p.m1, N - p.n1, N, K);
    if (p.part[0].splits > 1) f = (long long)p.part[0].splits * p.m1 * N;
    if (p.m1 < M && p.part[1].splits > 1)
        f = std::max(f, (long long)p.part[1].splits * (M - p.m1) * N);
    return f;
}

}  // namespace

// The bf16x3 GEMM behind gemm(), gemm_noalloc() and the GPT's fused linear
// layers (gemm_fused.hpp). Split-K partials go to `fixed` (at most
// fixed_floats), or else to scratch leased for `stream` (its reuse is ordered
// by the lease's event), except under graph capture, where a lease could
// allocate: there K is not split. The epilogue is one of
// EPI_BLAS (any transposes), EPI_BIAS / EPI_BIAS_GELU (A @ W^T) and
// EPI_GELU_GRAD (A @ B). Returns false, with nothing launched, for another
// combination.
bool bmb::bf16x3_gemm(bool ta, bool tb, int M, int N, int K, float alpha, const float *A,
                      const float *B, float beta, float *C, hipStream_t stream, int epi,
                      const float *bias, float *act, const float *pre, float *fixed,
                      long long fixed_floats) {
    if (M <= 0 || N <= 0) return true;
    const bmb::EpiArgs ep{bias, act, pre};
    const int a_contig = ta ? M : K, b_contig = tb ? K : N;
    const bool vec = a_contig % 4 == 0 && b_contig % 4 == 0 && (((uintptr_t)A & 15) == 0) &&
                     (((uintptr_t)B & 15) == 0);
    const bool may_split = fixed != nullptr || !bmb::stream_capturing(stream);
    const bool edges_ok = !ta && !tb && epi == bmb::EPI_BLAS;
    // (Every epilogue has k-sliced kernels, so a fused linear layer and
    // gemm() plus the separate bias/GELU pass plan a shape alike and give the
    // same bits.)
    const bool ks_ok = true;
    Plan p = pick(M, N, K, may_split, fixed ? fixed_floats : MAX_SPLIT_FLOATS, edges_ok, ks_ok);
    float *P = fixed;
    std::optional<bmb::ScratchLease> lease;
    const long long pf = partial_floats(p, M, N, K);
    if (pf > 0 && fixed == nullptr) {
        lease.emplace(bmb::SCRATCH_GEMM, (size_t)pf * sizeof(float), stream);
        P = static_cast<float *>(lease->get());
        if (P == nullptr) p = pick(M, N, K, false, 0, edges_ok, ks_ok);  // no scratch: no split
    }
#define BMB_B3(TA_, TB_, EPI_)                                                              \
    run_plan<TA_, TB_, EPI_>(p, M, N, K, alpha, A, B, beta, C, vec, P, stream, ep);         \
    return true;
    if (epi == bmb::EPI_BLAS) {
        if (!ta && !tb) { BMB_B3(false, false, bmb::EPI_BLAS) }
        if (!ta && tb) { BMB_B3(false, true, bmb::EPI_BLAS) }
        if (ta && !tb) { BMB_B3(true, false, bmb::EPI_BLAS) }
        BMB_B3(true, true, bmb::EPI_BLAS)
    }
    if (epi == bmb::EPI_BIAS && !ta && tb) { BMB_B3(false, true, bmb::EPI_BIAS) }
    if (epi == bmb::EPI_BIAS_GELU && !ta && tb) { BMB_B3(false, true, bmb::EPI_BIAS_GELU) }
    if (epi == bmb::EPI_GELU_GRAD && !ta && !tb) { BMB_B3(false, false, bmb::EPI_GELU_GRAD) }
#undef BMB_B3
    return false;
}

extern "C" void sgemm_mfma_bf16x3(int M, int N, int K, float alpha,
                                  const float *A, const float *B, float beta,
                                  float *C) {
    bmb::bf16x3_gemm(false, false, M, N, K, alpha, A, B, beta, C, nullptr, bmb::EPI_BLAS,
                     nullptr, nullptr, nullptr, nullptr, 0);
}
