// fp32 matrix-core GEMM for gfx950: v_mfma_f32_32x32x2_f32.
//
// One kernel template serves SGEMM stage 9 (sgemm_tensorcore), the
// transpose-aware gemm() and batched_gemm() (src/gemm.cu, src/bgemm.cu are the
// reference's counterparts). Inputs are fp32, each product is an exact fp32
// product and accumulation is fp32, so the result differs from the sequential
// fp32 oracle only by summation order (normwise ~1e-7 at K = 4096).
//
// MFMA operand layout used (v_mfma_f32_32x32x2_f32, one block):
//   A operand: lane l supplies A[m = l % 32][kk = l / 32]
//   B operand: lane l supplies B[kk = l / 32][n = l % 32]
//   D: lane l holds column n = l % 32, register r holds row
//      8 * (r / 4) + 4 * (l / 32) + r % 4.
// A K-chunk of 8 is consumed as 4 MFMAs; MFMA j pairs k = j (lanes 0-31) with
// k = 4 + j (lanes 32-63). The pairing is a permutation of the 8 k values
// applied identically to A and B, so the sum is unchanged; it lets a lane
// fetch its 4 k values of a k-contiguous LDS row with one 128-bit read.
//
// LDS layouts (each a direct copy of the operand's global layout, so staging
// is 128-bit loads and 128-bit stores with no transposition):
//   A, transA = false: As[m][k] (row stride BK + 4)  -> 128-bit fragment reads
//   A, transA = true : As[k][m] (row stride BM + 8)  -> 32-bit fragment reads
//   B, transB = false: Bs[k][n] (row stride BN + 8)  -> 32-bit fragment reads
//   B, transB = true : Bs[n][k] (row stride BK + 4)  -> 128-bit fragment reads
// gfx950 serves a 128-bit LDS read 16 lanes per cycle, in the lane groups
// {0-3, 12-15, 20-27} and {4-11, 16-19, 28-31} (and the same over lanes
// 32-63), and a 32-bit read 32 consecutive lanes per cycle (measured with
// SQ_LDS_BANK_CONFLICT). With the +4 pad a k-contiguous row is 9 16-byte
// slots long, so the 16 rows of a 128-bit read group (distinct residues mod
// 16) fall in 16 distinct slots. A 32-bit read has each half-wave read 32
// consecutive floats of one row: distinct banks with any pad (the +8 keeps
// the two half-waves, rows 4 apart, in opposite bank halves, which the
// hardware does not need since it serves them in separate cycles). The
// counter reads no conflict cycle for these layouts.
//
// Schedule. K is consumed in tiles of BK (a multiple of 16: an even number of
// 8-k groups) through two LDS stages. Fragments are double-buffered in
// registers: while the MFMAs of group g run, the LDS reads of group g+1 are in
// flight. The last group of a tile is issued AFTER the barrier that publishes
// the next stage, together with the reads of that stage's first group, so the
// MFMA pipe stays busy across the barrier; the global loads for the stage
// after next are issued right before the barrier and have a whole tile of
// MFMAs to land.
#pragma once

#include "common.hpp"

namespace bmb {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// What the epilogue does with a finished fp32 sum `acc` of output (row, col).
enum Epi {
    EPI_BLAS = 0,       // C = alpha * acc + beta * C (beta == 0: C write-only)
    EPI_PARTIAL = 1,    // C = acc (a split-K partial)
    EPI_BIAS = 2,       // C = acc + bias[col]
    EPI_BIAS_GELU = 3,  // C = acc + bias[col] and act = gelu(C), both stored
    EPI_GELU_GRAD = 4,  // C = gelu'(pre) * acc, i.e. gelu_grad(pre, acc)
};
struct EpiArgs {
    const float *bias;  // EPI_BIAS*: N floats
    float *act;         // EPI_BIAS_GELU: M x N, same layout as C
    const float *pre;   // EPI_GELU_GRAD: the GELU input, M x N, same layout as C
};

// The fused epilogues are the reference's separate passes in one: gemm with
// alpha = 1, beta = 0 stores acc, bias_forward adds bias[col] (one rounding),
// gelu_forward maps the sum (src/gpt.cu:256-277), gelu_backward maps the dX
// product (src/gpt.cu:336-337) -- the same fp32 results.
template <int EPI>
__device__ __forceinline__ void store_out(float *C, const EpiArgs &ep, size_t idx, float acc,
                                          float alpha, float beta, float bias) {
    if (EPI == EPI_PARTIAL) {
        C[idx] = acc;
    } else if (EPI == EPI_BLAS) {
        C[idx] = epilogue(acc, alpha, beta, C + idx);
    } else if (EPI == EPI_GELU_GRAD) {
        C[idx] = gelu_grad(ep.pre[idx], acc);
    } else {
        const float v = acc + bias;
        C[idx] = v;
        if (EPI == EPI_BIAS_GELU) ep.act[idx] = gelu(v);
    }
}

template <int BM_, int BN_, int BK_, int WAVES_M_, int WAVES_N_>
struct MfmaTile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int NT = WAVES_M * WAVES_N * 64;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    static constexpr int FM = WM / 32, FN = WN / 32;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile is whole 32x32 MFMA tiles");
    static_assert(BK % 16 == 0, "BK is an even number of 8-k groups");
};

template <bool TA, bool TB, class Tile>
struct MfmaLayout {
    static constexpr int BM = Tile::BM, BN = Tile::BN, BK = Tile::BK, NT = Tile::NT;
    // A
    static constexpr int LDA = TA ? BM + 8 : BK + 4;
    static constexpr int A_ROWS = TA ? BK : BM;  // rows of the LDS A array
    static constexpr int A_SZ = A_ROWS * LDA;
    static constexpr int A_CHUNKS = BM * BK / 4;  // float4 chunks per tile
    static constexpr int A_PER_T = A_CHUNKS / NT;
    // B
    static constexpr int LDB = TB ? BK + 4 : BN + 8;
    static constexpr int B_ROWS = TB ? BN : BK;
    static constexpr int B_SZ = B_ROWS * LDB;
    static constexpr int B_CHUNKS = BK * BN / 4;
    static constexpr int B_PER_T = B_CHUNKS / NT;
    static_assert(A_CHUNKS % NT == 0 && B_CHUNKS % NT == 0, "staging tiles evenly");
    static constexpr int STAGE = A_SZ + B_SZ;  // floats per pipeline stage
    static constexpr size_t SMEM_BYTES = 2 * (size_t)STAGE * sizeof(float);
};

// Loads one operand chunk (4 floats along the operand's contiguous axis) from
// global memory, zero filling whatever lies outside [0, rows) x [0, cols).
// `row` and `col0` index the stored matrix (row stride ld floats).
// VEC: ld % 4 == 0 and a 16-byte aligned base, so an in-range chunk is one
// aligned 128-bit load (cols is then a multiple of 4 too). Otherwise a chunk
// that lies wholly inside the row is still one 128-bit load (global loads on
// gfx950 need only dword alignment) and only a chunk straddling the row end
// falls back to guarded 32-bit loads.
template <bool VEC>
__device__ __forceinline__ float4 load_chunk(const float *P, int rows, int cols, int ld,
                                             int row, int col0) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row >= rows) return v;
    const float *p = P + (size_t)row * ld + col0;
    if (VEC) {
        if (col0 < cols) v = ld4(p);
    } else if (col0 + 3 < cols) {
        __builtin_memcpy(&v, p, sizeof(v));
    } else {
        if (col0 + 0 < cols) v.x = p[0];
        if (col0 + 1 < cols) v.y = p[1];
        if (col0 + 2 < cols) v.z = p[2];
    }
    return v;
}

// Epilogues whose edge tiles are shifted back inside C (see MfmaGemm::run).
template <int EPI>
constexpr bool SHIFT = EPI == EPI_BLAS || EPI == EPI_PARTIAL;

template <bool TA, bool TB, class Tile, bool VEC>
struct MfmaGemm {
    using L = MfmaLayout<TA, TB, Tile>;
    static constexpr int BM = Tile::BM, BN = Tile::BN, BK = Tile::BK, NT = Tile::NT;
    static constexpr int WM = Tile::WM, WN = Tile::WN, FM = Tile::FM, FN = Tile::FN;

    struct Regs {
        float4 a[L::A_PER_T];
        float4 b[L::B_PER_T];
    };

    // Chunk e of the A tile: which stored row and which 4-column group.
    __device__ static __forceinline__ void a_chunk(int e, int &r, int &c) {
        if (TA) { r = e / (BM / 4); c = (e % (BM / 4)) * 4; }  // stored K x M
        else    { r = e / (BK / 4); c = (e % (BK / 4)) * 4; }  // stored M x K
    }
    __device__ static __forceinline__ void b_chunk(int e, int &r, int &c) {
        if (TB) { r = e / (BK / 4); c = (e % (BK / 4)) * 4; }  // stored N x K
        else    { r = e / (BN / 4); c = (e % (BN / 4)) * 4; }  // stored K x N
    }

    // K bounds the k index (a split's length); lda / ldb are the stored
    // row strides (TA ? M : full K, TB ? full K : N).
    __device__ static __forceinline__ void load(Regs &g, const float *A,
                                                const float *B, int M, int N,
                                                int K, int lda, int ldb, int m0,
                                                int n0, int k0, int tid) {
#pragma unroll
        for (int i = 0; i < L::A_PER_T; ++i) {
            int r, c;
            a_chunk(tid + i * NT, r, c);
            g.a[i] = TA ? load_chunk<VEC>(A, K, M, lda, k0 + r, m0 + c)
                        : load_chunk<VEC>(A, M, K, lda, m0 + r, k0 + c);
        }
#pragma unroll
        for (int i = 0; i < L::B_PER_T; ++i) {
            int r, c;
            b_chunk(tid + i * NT, r, c);
            g.b[i] = TB ? load_chunk<VEC>(B, N, K, ldb, n0 + r, k0 + c)
                        : load_chunk<VEC>(B, K, N, ldb, k0 + r, n0 + c);
        }
    }

    __device__ static __forceinline__ void store(const Regs &g, float *as,
                                                 float *bs, int tid) {
#pragma unroll
        for (int i = 0; i < L::A_PER_T; ++i) {
            int r, c;
            a_chunk(tid + i * NT, r, c);
            st4(as + r * L::LDA + c, g.a[i]);
        }
#pragma unroll
        for (int i = 0; i < L::B_PER_T; ++i) {
            int r, c;
            b_chunk(tid + i * NT, r, c);
            st4(bs + r * L::LDB + c, g.b[i]);
        }
    }

    // Fragments of one 8-k group for this lane: fa[fi][j], fb[fn][j].
    __device__ static __forceinline__ void fragments(const float *as,
                                                     const float *bs, int g,
                                                     int wm, int wn, int lane,
                                                     float (&fa)[FM][4],
                                                     float (&fb)[FN][4]) {
        const int l32 = lane & 31, half = lane >> 5;
        const int kq = g * 8 + half * 4;
#pragma unroll
        for (int fi = 0; fi < FM; ++fi) {
            const int m = wm + fi * 32 + l32;
            if (TA) {
#pragma unroll
                for (int j = 0; j < 4; ++j) fa[fi][j] = as[(kq + j) * L::LDA + m];
            } else {
                const float4 v = ld4(as + m * L::LDA + kq);
                fa[fi][0] = v.x; fa[fi][1] = v.y; fa[fi][2] = v.z; fa[fi][3] = v.w;
            }
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const int n = wn + fn * 32 + l32;
            if (TB) {
                const float4 v = ld4(bs + n * L::LDB + kq);
                fb[fn][0] = v.x; fb[fn][1] = v.y; fb[fn][2] = v.z; fb[fn][3] = v.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) fb[fn][j] = bs[(kq + j) * L::LDB + n];
            }
        }
    }

    __device__ static __forceinline__ void mma(const float (&fa)[FM][4],
                                               const float (&fb)[FN][4],
                                               f32x16 (&acc)[FM][FN]) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                    acc[fi][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[fi][j], fb[fn][j],
                                                                       acc[fi][fn], 0, 0, 0);
    }

    // One 128-bit load of an in-range chunk: an aligned float4 (VEC), or a
    // 16-byte copy from a 4-byte aligned address, which is still one
    // global_load_dwordx4 on gfx950 (global loads need only dword alignment).
    __device__ static __forceinline__ float4 load4_in(const float *p) {
        if (VEC) return ld4(p);
        float4 v;
        __builtin_memcpy(&v, p, sizeof(v));
        return v;
    }

    // Loads of an interior tile: every row and column of the tile lies inside
    // the operands and K is a whole number of k-tiles, so no chunk needs a
    // bounds check and each is one 128-bit load.
    __device__ static __forceinline__ void load_interior(Regs &g, const float *A, const float *B,
                                                         int lda, int ldb, int m0, int n0, int k0,
                                                         int tid) {
#pragma unroll
        for (int i = 0; i < L::A_PER_T; ++i) {
            int r, c;
            a_chunk(tid + i * NT, r, c);
            g.a[i] = load4_in(TA ? A + (size_t)(k0 + r) * lda + m0 + c
                                 : A + (size_t)(m0 + r) * lda + k0 + c);
        }
#pragma unroll
        for (int i = 0; i < L::B_PER_T; ++i) {
            int r, c;
            b_chunk(tid + i * NT, r, c);
            g.b[i] = load4_in(TB ? B + (size_t)(n0 + r) * ldb + k0 + c
                                 : B + (size_t)(k0 + r) * ldb + n0 + c);
        }
    }

    // Instruction-order requests for the interior loop (a scheduling hint,
    // no effect on results). Per 8-k group a wave issues NMF MFMAs of 64
    // cycles each; one LDS read, LDS write or global load goes between two
    // MFMAs, so the matrix pipe never waits for a burst of memory
    // instructions. Measured on MI355X: +3-7% for the 128x128 and 256x256
    // tiles; the 64-row tiles gain only in the NT case and lose otherwise.
    static constexpr bool HINTS = (BM >= 128 && BN >= 128) || TB;
    static constexpr int NMF = 4 * FM * FN;                        // MFMAs per group
    static constexpr int NRD = (TA ? 2 * FM : FM) + (TB ? FN : 2 * FN);  // LDS read instrs
    static constexpr int NWR = L::A_PER_T + L::B_PER_T;            // LDS writes = loads

    // Before the barrier: the reads of groups 1..G-1 each behind one MFMA of
    // the group before, then the stage's LDS writes and the next global
    // loads behind the last MFMAs of group G-2.
    __device__ static __forceinline__ void hint_before_barrier() {
#pragma unroll
        for (int q = 0; q < BK / 8 - 1; ++q) {
#pragma unroll
            for (int i = 0; i < NMF; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                if (i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
                if (q == BK / 8 - 2 && i >= NMF - 2 * NWR && i < NMF - NWR)
                    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
                if (q == BK / 8 - 2 && i >= NMF - NWR)
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
            }
        }
    }
    // After the barrier: the next stage's first reads behind the last group's
    // MFMAs.
    __device__ static __forceinline__ void hint_after_barrier() {
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    }

    // The loads of k-tile t (k0 = t * BK) for run_tile's MODE: 1 every k-tile
    // is whole and the tile lies inside M x N (unguarded); 2 the same except
    // that the last k-tile is cut by K, so its loads are guarded (a uniform
    // branch); 0 guarded throughout (zero fill past M, N or K).
    template <int MODE>
    __device__ static __forceinline__ void load_tile(Regs &g, const float *A, const float *B,
                                                     int M, int N, int K, int lda, int ldb,
                                                     int m0, int n0, int t, int nkt, int tid) {
        if (MODE == 1 || (MODE == 2 && t < nkt - 1))
            load_interior(g, A, B, lda, ldb, m0, n0, t * BK, tid);
        else
            load(g, A, B, M, N, K, lda, ldb, m0, n0, t * BK, tid);
    }

    // One output tile (m0, n0) of one problem over k in [0, K); A and B are
    // positioned at k = 0 of that range, lda / ldb are their row strides.
    // smem holds two stages per k-slice. EPI selects what is stored (see
    // Epi). MODE (see load_tile): 1 and 2 need the tile inside M x N and
    // K > 0, 1 also K % (BK * KS) == 0.
    //
    // KS > 1 (a k-sliced workgroup of KS * NT threads): slice s stages and
    // multiplies k-tiles [s * per, (s + 1) * per) of the range in its own two
    // LDS stages, per = ceil(k-tiles / KS). Every slice runs `per` k-tiles, so
    // all reach the same barriers; a slice's k-tiles past K load zeros. The
    // slices' sums then meet in LDS and slice 0 adds them in slice order
    // (deterministic) and runs the epilogue. For tiles too few to give every
    // SIMD two waves (N <= 1024 or so), this doubles the waves per tile with
    // no split-K partials in global memory and no reduce launch.
    template <int EPI, int MODE, int KS = 1>
    __device__ static __forceinline__ void run_tile(int M, int N, int K, int lda, int ldb,
                                                    float alpha, const float *__restrict__ A,
                                                    const float *__restrict__ B, float beta,
                                                    float *C, int ldc, int m0, int n0,
                                                    float *smem, EpiArgs ep, int mlo, int nlo) {
        constexpr int G = BK / 8;  // 8-k groups per tile (even)
        constexpr bool INTERIOR = MODE != 0;             // no M / N bounds checks
        constexpr bool HINTED = MODE == 1 && HINTS;      // branch-free loop: scheduling hints
        const int slice = KS > 1 ? (int)threadIdx.x / NT : 0;
        const int tid = KS > 1 ? (int)threadIdx.x % NT : (int)threadIdx.x;
        const int wave = tid >> 6, lane = tid & 63;
        const int wm = (wave / Tile::WAVES_N) * WM;
        const int wn = (wave % Tile::WAVES_N) * WN;
        float *const smem0 = smem;

        f32x16 acc[FM][FN];
#pragma unroll
        for (int fi = 0; fi < FM; ++fi)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fi][fn][r] = 0.0f;

        // k-tiles every slice runs (the same in all slices: they share the
        // barriers), then this slice's own range and k-tiles.
        int nkt_iter = (K + BK - 1) / BK;
        if (KS > 1) {
            const int per = (nkt_iter + KS - 1) / KS;
            const int kb = min(K, slice * per * BK);
            const int klen = min(K, kb + per * BK) - kb;
            A += TA ? (size_t)kb * lda : (size_t)kb;
            B += TB ? (size_t)kb : (size_t)kb * ldb;
            K = klen;
            smem += slice * 2 * L::STAGE;
            nkt_iter = per;
        }
        const int nkt = (K + BK - 1) / BK;
        if (nkt_iter > 0) {
            Regs g;
            if (INTERIOR) {
                load_tile<MODE>(g, A, B, M, N, K, lda, ldb, m0, n0, 0, nkt, tid);
                store(g, smem, smem + L::A_SZ, tid);
                // (MODE 1: every slice has nkt whole k-tiles, clamp into
                // them; a k-sliced MODE 2 slice loads zeros past its range.)
                load_tile<MODE>(g, A, B, M, N, K, lda, ldb, m0, n0,
                                (MODE == 1 || KS == 1) ? min(1, nkt - 1) : 1, nkt, tid);
            } else {
                load(g, A, B, M, N, K, lda, ldb, m0, n0, 0, tid);
                store(g, smem, smem + L::A_SZ, tid);
                if (nkt_iter > 1) load(g, A, B, M, N, K, lda, ldb, m0, n0, BK, tid);
            }
            __syncthreads();

            float fa[2][FM][4], fb[2][FN][4];
            fragments(smem, smem + L::A_SZ, 0, wm, wn, lane, fa[0], fb[0]);
            for (int kt = 0; kt < nkt_iter; ++kt) {
                const float *as = smem + (kt & 1) * L::STAGE, *bs = as + L::A_SZ;
#pragma unroll
                for (int grp = 0; grp < G; ++grp) {
                    const int cb = grp & 1;  // G is even: group 0 of every tile is buffer 0
                    if (grp + 1 < G) {
                        fragments(as, bs, grp + 1, wm, wn, lane, fa[cb ^ 1], fb[cb ^ 1]);
                    } else {
                        // Publish the next stage, start the global loads of
                        // the one after, and read group 0 of the next stage
                        // while this tile's last MFMAs run. Unconditional on
                        // purpose: past the last tile the loads are zero fills
                        // (k >= K, no memory access) or, for an interior
                        // tile, repeat the last k-tile; the store and the
                        // reads touch the idle LDS stage; none of it is used.
                        // Guarding them makes the compiler copy the fragment
                        // registers and wait for the reads before this
                        // group's MFMAs.
                        // (A k-sliced MODE 2 tile loads zeros past its range
                        // instead: it may run k-tiles beyond it.)
                        float *nxt = smem + ((kt + 1) & 1) * L::STAGE;
                        store(g, nxt, nxt + L::A_SZ, tid);
                        if (INTERIOR)
                            load_tile<MODE>(g, A, B, M, N, K, lda, ldb, m0, n0,
                                            (MODE == 1 || KS == 1) ? min(kt + 2, nkt - 1) : kt + 2,
                                            nkt, tid);
                        else
                            load(g, A, B, M, N, K, lda, ldb, m0, n0, (kt + 2) * BK, tid);
                        if (HINTED) hint_before_barrier();
                        __syncthreads();
                        fragments(nxt, nxt + L::A_SZ, 0, wm, wn, lane, fa[cb ^ 1], fb[cb ^ 1]);
                    }
                    mma(fa[cb], fb[cb], acc);
                    if (HINTED && grp == G - 1) hint_after_barrier();
                }
            }
        }

        if (KS > 1) {
            // Slices 1.. leave their sums in LDS (the staging stages are
            // idle once every slice is past its last fragment read); slice 0
            // adds them in slice order. Lane-contiguous: no bank conflicts.
            static_assert(KS == 1 || (size_t)(KS - 1) * BM * BN <= (size_t)KS * 2 * L::STAGE,
                          "the slices' sums fit in the staging LDS");
            constexpr int PER = FM * FN * 16;
            __syncthreads();
            if (slice > 0) {
                float *dst = smem0 + (size_t)(slice - 1) * BM * BN + (size_t)wave * PER * 64 + lane;
#pragma unroll
                for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            dst[((fi * FN + fn) * 16 + r) * 64] = acc[fi][fn][r];
            }
            __syncthreads();
            if (slice > 0) return;
#pragma unroll
            for (int s = 1; s < KS; ++s) {
                const float *src =
                    smem0 + (size_t)(s - 1) * BM * BN + (size_t)wave * PER * 64 + lane;
#pragma unroll
                for (int fi = 0; fi < FM; ++fi)
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[fi][fn][r] += src[((fi * FN + fn) * 16 + r) * 64];
            }
        }

        if (INTERIOR && SHIFT<EPI> && (mlo > m0 || nlo > n0))
            epilogue<EPI, INTERIOR, SHIFT<EPI>>(M, N, alpha, beta, C, ldc, m0, n0, ep, mlo, nlo, wm,
                                                wn, lane, acc);
        else
            epilogue<EPI, INTERIOR, false>(M, N, alpha, beta, C, ldc, m0, n0, ep, mlo, nlo, wm, wn,
                                           lane, acc);
    }

    // Epilogue: lanes 0-31 of a register cover 32 consecutive columns, so
    // each C row segment is one 128-byte coalesced access. What an epilogue
    // reads (C when beta != 0, the GELU input) is gathered for a row of FN
    // blocks before any of their results is stored, so 16 * FN loads per lane
    // are in flight at once; read-use-store per element would cost one memory
    // round trip per output. Same arithmetic as store_out. WIN: a shifted edge
    // tile, storing only rows >= mlo and columns >= nlo (it may read the
    // others: they are inside C). C's rows (and those of ep.act and ep.pre)
    // are ldc floats apart.
    template <int EPI, bool INTERIOR, bool WIN>
    __device__ static __forceinline__ void epilogue(int M, int N, float alpha, float beta,
                                                    float *C, int ldc, int m0, int n0, EpiArgs ep,
                                                    int mlo, int nlo, int wm, int wn, int lane,
                                                    const f32x16 (&acc)[FM][FN]) {
        const int l32 = lane & 31, half = lane >> 5;
        const bool reads = EPI == EPI_GELU_GRAD || (EPI == EPI_BLAS && beta != 0.0f);
        const float *src = EPI == EPI_GELU_GRAD ? ep.pre : C;
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
                                        ? src[(size_t)row * ldc + col] : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
                const int col = n0 + wn + fn * 32 + l32;
                if (!INTERIOR && col >= N) continue;
                if (WIN && col < nlo) continue;
                const float bias = (EPI == EPI_BIAS || EPI == EPI_BIAS_GELU) ? ep.bias[col] : 0.0f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm + fi * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (!INTERIOR && row >= M) continue;
                    if (WIN && row < mlo) continue;
                    const size_t idx = (size_t)row * ldc + col;
                    const float a = acc[fi][fn][r];
                    float v;
                    if (EPI == EPI_PARTIAL) {
                        v = a;
                    } else if (EPI == EPI_BLAS) {
                        v = reads ? fma_rn(alpha, a, beta * in[fn][r]) : alpha * a;
                    } else if (EPI == EPI_GELU_GRAD) {
                        v = gelu_grad(in[fn][r], a);
                    } else {
                        v = a + bias;
                        if (EPI == EPI_BIAS_GELU) ep.act[idx] = gelu(v);
                    }
                    C[idx] = v;
                }
            }
        }
    }

    // Picks the interior path when it applies (a uniform branch per workgroup),
    // with or without 16-byte aligned operands; a K that is not a whole number
    // of k-tiles (per slice) guards only the last k-tile's loads.
    template <int EPI = EPI_BLAS, int KS = 1>
    __device__ static __forceinline__ void run(int M, int N, int K, int lda, int ldb,
                                               float alpha, const float *__restrict__ A,
                                               const float *__restrict__ B, float beta,
                                               float *C, int ldc, int m0, int n0, float *smem,
                                               EpiArgs ep = {}) {
        // A partial tile at the bottom or right edge of a C at least one tile
        // large is shifted back to end at the edge, overlapping its
        // neighbour: it then runs the interior path and stores only the rows
        // and columns it owns (from m0, n0 on). (BLAS and split-K epilogues
        // only: the fused ones, used at the GPT's whole-tile shapes, would
        // spill registers for the second epilogue.)
        if (SHIFT<EPI> ? (M >= BM && N >= BN && K > 0) : (m0 + BM <= M && n0 + BN <= N && K > 0)) {
            const int ms = min(m0, M - BM), ns = min(n0, N - BN);
            if (K % (BK * KS) == 0)
                run_tile<EPI, 1, KS>(M, N, K, lda, ldb, alpha, A, B, beta, C, ldc, ms, ns, smem, ep,
                                     m0, n0);
            else
                run_tile<EPI, 2, KS>(M, N, K, lda, ldb, alpha, A, B, beta, C, ldc, ms, ns, smem, ep,
                                     m0, n0);
        } else {
            run_tile<EPI, 0, KS>(M, N, K, lda, ldb, alpha, A, B, beta, C, ldc, m0, n0, smem, ep,
                                 m0, n0);
        }
    }
};

// Grid: x = output tiles (XCD-remapped, grouped), y = batch index. The
// fused epilogues (EPI_BIAS*) are used for single problems only. lda, ldb,
// ldc: the row strides of the stored A (at least M when TA, K otherwise), B
// (at least K when TB, N otherwise) and C (at least N), so that a block of
// rows and columns of a larger problem (its operands offset to its first row
// and column) runs as a problem of its own.
template <bool TA, bool TB, class Tile, bool VEC, int EPI>
__global__ __launch_bounds__(Tile::NT) void mfma_gemm_k(
    int M, int N, int K, float alpha, const float *__restrict__ A, int lda,
    long long sA, const float *__restrict__ B, int ldb, long long sB, float beta,
    float *C, int ldc, long long sC, int tiles_m, int tiles_n, EpiArgs ep) {
    extern __shared__ float smem_dyn[];
    const size_t z = blockIdx.y;
    int tm, tn;
    group_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    MfmaGemm<TA, TB, Tile, VEC>::template run<EPI>(M, N, K, lda, ldb, alpha, A + z * sA,
                                                   B + z * sB, beta, C + z * sC, ldc,
                                                   tm * Tile::BM, tn * Tile::BN, smem_dyn, ep);
}

// The same with KS k-slices per workgroup (KS * NT threads; LDS: KS times
// the stages of one).
template <bool TA, bool TB, class Tile, bool VEC, int EPI, int KS>
__global__ __launch_bounds__(Tile::NT * KS) void mfma_gemm_ks_k(
    int M, int N, int K, float alpha, const float *__restrict__ A, int lda,
    long long sA, const float *__restrict__ B, int ldb, long long sB, float beta,
    float *C, int ldc, long long sC, int tiles_m, int tiles_n, EpiArgs ep) {
    extern __shared__ float smem_dyn[];
    const size_t z = blockIdx.y;
    int tm, tn;
    group_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    MfmaGemm<TA, TB, Tile, VEC>::template run<EPI, KS>(M, N, K, lda, ldb, alpha, A + z * sA,
                                                       B + z * sB, beta, C + z * sC, ldc,
                                                       tm * Tile::BM, tn * Tile::BN, smem_dyn,
                                                       ep);
}

// Split-K: blockIdx.y = split s covers k in [s*kchunk, min(K, (s+1)*kchunk))
// (kchunk a multiple of 16; the host rounds it to a multiple of 32, whole
// k-tiles of every tile it uses) and writes its raw fp32 sums to the M x N
// partial P + s*M*N; splitk_reduce_k then adds the splits in order.
template <bool TA, bool TB, class Tile, bool VEC>
__global__ __launch_bounds__(Tile::NT) void mfma_gemm_splitk_k(
    int M, int N, int K, const float *__restrict__ A, int lda, const float *__restrict__ B,
    int ldb, float *P, int tiles_m, int tiles_n, int kchunk) {
    extern __shared__ float smem_dyn[];
    const int s = blockIdx.y;
    const int kb = s * kchunk;
    const int klen = min(K, kb + kchunk) - kb;
    int tm, tn;
    group_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const float *As = TA ? A + (size_t)kb * lda : A + kb;
    const float *Bs = TB ? B + kb : B + (size_t)kb * ldb;
    MfmaGemm<TA, TB, Tile, VEC>::template run<EPI_PARTIAL>(
        M, N, klen, lda, ldb, 1.0f, As, Bs, 0.0f, P + (size_t)s * M * N, N,
        tm * Tile::BM, tn * Tile::BN, smem_dyn);
}

// C = epilogue of sum_{s < splits} P[s]: one float4 of C per lane, splits
// added in ascending order, so the result depends only on the shape. N is
// the row length of the packed partials (and gives an element's bias
// column); C's rows (and those of ep.act, ep.pre) are ldc floats apart.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_k(float *C, const float *P, int splits,
                                                       long long mn, int N, int ldc,
                                                       float alpha, float beta, EpiArgs ep) {
    const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    const bool packed = ldc == N;
    const bool whole = packed && i + 3 < mn;
    float acc[4];
    if (whole) {
        float4 v;
        __builtin_memcpy(&v, P + i, sizeof(v));
        acc[0] = v.x; acc[1] = v.y; acc[2] = v.z; acc[3] = v.w;
        for (int s = 1; s < splits; ++s) {
            __builtin_memcpy(&v, P + (size_t)s * mn + i, sizeof(v));
            acc[0] += v.x; acc[1] += v.y; acc[2] += v.z; acc[3] += v.w;
        }
    } else {
        for (int k = 0; k < 4; ++k) {
            acc[k] = 0.0f;
            if (i + k < mn) {
                acc[k] = P[i + k];
                for (int s = 1; s < splits; ++s) acc[k] += P[(size_t)s * mn + i + k];
            }
        }
    }
    if (EPI == EPI_BLAS && whole) {
        float4 c = make_float4(0.f, 0.f, 0.f, 0.f);
        if (beta != 0.0f) __builtin_memcpy(&c, C + i, sizeof(c));
        c.x = epilogue(acc[0], alpha, beta, &c.x);
        c.y = epilogue(acc[1], alpha, beta, &c.y);
        c.z = epilogue(acc[2], alpha, beta, &c.z);
        c.w = epilogue(acc[3], alpha, beta, &c.w);
        __builtin_memcpy(C + i, &c, sizeof(c));
        return;
    }
    for (int k = 0; k < 4; ++k) {
        if (i + k >= mn) break;
        const long long row = (i + k) / N, col = (i + k) % N;
        const float bias = (EPI == EPI_BIAS || EPI == EPI_BIAS_GELU) ? ep.bias[col] : 0.0f;
        store_out<EPI>(C, ep, packed ? (size_t)(i + k) : (size_t)(row * ldc + col), acc[k], alpha,
                       beta, bias);
    }
}

}  // namespace bmb
