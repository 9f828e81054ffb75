// Host side of the fp32 MFMA GEMM: SGEMM stage 9, gemm() and batched_gemm().
//
// The reference dispatches gemm() to a fast kernel only when M, N % 128 and
// K % 16 are all zero and otherwise to a 16x16 scalar kernel
// (src/gemm.cu:204-217); batched_gemm() always uses a guarded 64x64 kernel
// (src/bgemm.cu:88-97). Here one kernel template handles every shape and
// transpose in-kernel (guarded, zero-filled staging; guarded stores), and the
// host picks the tile size and a split of K (pick()) and whether every row of
// the operands is 16-byte aligned.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <optional>
#include <tuple>

#include "mfma_gemm.hpp"
#include "../../include/gemm.h"
#include "../../include/kernels.h"
#include "gemm_fused.hpp"
#include "launch.hpp"
#include "workspace.hpp"

namespace {

using bmb::MfmaTile;
using TileL = MfmaTile<256, 256, 32, 2, 4>;  // 512 lanes, 128x64 per wave, K depth 32
using TileM = MfmaTile<128, 128, 16, 2, 2>;  // 256 lanes, 64x64 per wave
using TileN = MfmaTile<64, 128, 16, 2, 2>;   // 256 lanes, 32x64 per wave
using TileS = MfmaTile<64, 64, 16, 2, 2>;    // 256 lanes, 32x32 per wave
using TileXS = MfmaTile<32, 32, 16, 1, 1>;   // 64 lanes (k-sliced only: 4 or 8 slices)

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

// Tile and split-K choice from a time model fitted to MI355X measurements of
// every tile and split on the GPT-2 training shapes and a square sweep 512 ...
// 8192 (both transposes; 32 shapes, about 1500 timed plans): the fit picks
// the measured best plan on 28 of them and is within 3% on all but N = 1000.
// Per tile: `eff`, the fraction of the fp32 MFMA peak a CU reaches when it is
// full of such workgroups; per kernel (tile, transposes, epilogue, split or
// not): the workgroups that fit on a CU, from the runtime's occupancy query
// (registers and LDS decide it: the 128x128 tile runs 3 per CU, the 64x64
// tile 5-8). A work item is one output tile over one K split; the machine
// runs cus * occupancy of them per round, so an item count just above a whole
// number of rounds costs an extra round (4097^3 on 256x256: 289 tiles on 256
// CUs); a last round in which each CU holds fewer items than fit runs faster
// per item, by (held / fit)^PARTIAL_EXP. Splitting K multiplies the items of
// a problem with few output tiles (768 x 768 x 8192 has 144 on 64x64) and
// costs the partials' round trip (mostly through the 256 MB last-level
// cache, hence a rate above HBM's) plus one reduce launch. The model only
// compares candidates; its times are not predictions.
//
// A candidate with ks > 1 runs each output tile as ks k-slices of one
// workgroup (ks times the waves; the slices' sums meet in LDS, with no
// partials in global memory and no reduce launch): for few output tiles it
// puts more waves on each SIMD without split-K's round trip. Those kernels
// exist for the plain BLAS epilogue only (KERNELS id 9, gemm() in fp32 mode,
// batched_gemm()). The 32 x 32 tile exists only k-sliced (one wave per
// slice), for problems too small to give every CU a 64 x 64 tile (N = 512:
// 64 of them, or 256 split-K items plus a reduce launch), and is only
// considered up to XS_MAX_OUTPUTS outputs. Each slice beyond the first adds
// KS_OVERHEAD k steps to its workgroup's item (its own prologue, and the sum
// of the slices in LDS): without that charge the model put the GPT-2 forward
// and dX products with K = 768 (8192 x 2304 and 8192 x 768, thousands of
// tiles) on 4-sliced 64 x 128 tiles, 11-14% slower than the plain 64 x 128
// tile, while a forced sweep of every plan (23 shapes, 1000 plans) puts the
// charge anywhere in 16-28 k steps with the measured best plan picked on 21
// of them and the other two within 1.3%.
enum class TileKind { L, M, N, S, XS };
struct Cand {
    TileKind kind;
    int bm, bn;
    double eff;
    int ks;
};
constexpr Cand CANDS[] = {{TileKind::L, 256, 256, 0.909, 1},
                          {TileKind::M, 128, 128, 0.893, 1},
                          {TileKind::N, 64, 128, 0.823, 1},
                          {TileKind::S, 64, 64, 0.809, 1},
                          {TileKind::M, 128, 128, 0.893, 2},
                          {TileKind::N, 64, 128, 0.823, 2},
                          {TileKind::N, 64, 128, 0.823, 4},
                          {TileKind::S, 64, 64, 0.809, 2},
                          {TileKind::S, 64, 64, 0.809, 4},
                          {TileKind::XS, 32, 32, 0.5, 4},
                          {TileKind::XS, 32, 32, 0.5, 8}};
constexpr int N_CANDS = sizeof(CANDS) / sizeof(CANDS[0]);
constexpr long long XS_MAX_OUTPUTS = 1LL << 20;
constexpr int SPLITS[] = {1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 14, 16};
constexpr double K_OVERHEAD = 60.0;           // per-item prologue/epilogue, in k steps
constexpr double KS_OVERHEAD = 24.0;          // per k-slice beyond the first, in k steps
constexpr double PARTIAL_EXP = 0.88;          // speed of a part-filled last round
constexpr double PARTIALS_BYTES_PER_S = 1.35e13;  // the partials' round trip
constexpr double LAUNCH_S = 1.6e-6;           // the reduce launch
constexpr int MIN_SPLIT_K = 128;              // shortest K range a split may get
constexpr int MIN_SLICE_K = 64;               // shortest K range a k-slice may get
// A second band: its launch and the drain between the bands. Bands are only
// tried for K >= MIN_BAND_K, with K ranges of at least MIN_BAND_SPLIT_K in a
// split remainder band, and taken when modelled 3% faster than one band (as
// in the bf16x3 planner, sgemm_bf16x3.hip, where these bounds were measured).
constexpr double BAND_S = 12.0e-6;
constexpr double BAND_GAIN = 0.97;
constexpr int MIN_BAND_K = 4096;
constexpr int MIN_BAND_SPLIT_K = 512;
// Largest split-K partial buffer (floats): 640 MiB per call in flight on a device.
constexpr long long MAX_SPLIT_FLOATS = 160LL << 20;

}  // namespace

// Split-K partials of gemm_noalloc(): a fixed array of device memory instead
// of leased scratch (64 MiB; every GPU that loads this code object holds its
// own copy until the process ends). Host code never passes `scratch` itself
// to a kernel -- on the host that name is only a stand-in -- but the device
// address hipGetSymbolAddress returns for the current device.
constexpr long long NOALLOC_SPLIT_FLOATS = 16LL << 20;
static __device__ __align__(256) float scratch[NOALLOC_SPLIT_FLOATS];

namespace {

// The address of the current device's `scratch`, resolved on the first call
// on that device (with it current) and kept; nullptr (with a message) if the
// runtime cannot give it.
float *noalloc_scratch() {
    constexpr int MAX_DEV = 64;
    static std::mutex mu;
    static float *addr[MAX_DEV] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) {
        (void)hipGetLastError();
        fprintf(stderr, "gemm_noalloc: no current device (or more than %d devices)\n", MAX_DEV);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        float *p = nullptr;
        const hipError_t e = hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            fprintf(stderr, "gemm_noalloc: cannot resolve the scratch array on device %d: %s\n",
                    dev, hipGetErrorString(e));
            return nullptr;
        }
        addr[dev] = p;
    }
    return addr[dev];
}

// Workgroups per CU of each candidate's kernel: [tile][0 whole K, 1 split-K].
struct Occupancy {
    int wgs[N_CANDS][2];
};

template <class K>
int wgs_per_cu(K kern, int threads, size_t smem) {
    bmb::allow_smem(kern, smem);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, smem) != hipSuccess) {
        (void)hipGetLastError();  // the next launch must not report this query's failure
        n = 1;
    }
    if (n < 1) n = 1;
    return n;
}

template <bool TA, bool TB, class Tile, int EPI, bool VEC>
void tile_occupancy(int (&out)[2]) {
    using L = bmb::MfmaLayout<TA, TB, Tile>;
    out[0] = wgs_per_cu(bmb::mfma_gemm_k<TA, TB, Tile, VEC, EPI>, Tile::NT, L::SMEM_BYTES);
    out[1] = wgs_per_cu(bmb::mfma_gemm_splitk_k<TA, TB, Tile, VEC>, Tile::NT, L::SMEM_BYTES);
}

// The k-sliced kernel's workgroups per CU ([1]: unused, it never splits K
// across workgroups); 0 when the case has no k-sliced kernel.
template <bool TA, bool TB, class Tile, int EPI, bool VEC, int KS>
void ks_occupancy(int (&out)[2]) {
    using L = bmb::MfmaLayout<TA, TB, Tile>;
    out[0] = EPI == bmb::EPI_BLAS
                 ? wgs_per_cu(bmb::mfma_gemm_ks_k<TA, TB, Tile, VEC, bmb::EPI_BLAS, KS>,
                              Tile::NT * KS, KS * L::SMEM_BYTES)
                 : 0;
    out[1] = 0;
}

// One band's launch: tile candidate, K ranges (1: no split) and the K per
// range (a multiple of 16).
struct Part {
    int tile;  // index into CANDS (its ks: k-slices per workgroup)
    int splits;
    int kchunk;
};

// Rows [0, m1) x columns [0, n1) run on part[0], rows [0, m1) x columns
// [n1, N) on part[2], rows [m1, M) x all columns on part[1] (m1 == M: no row
// band; n1 == N: no column band), one launch after the other on the same
// stream. As in the bf16x3 planner (sgemm_bf16x3.hip), a tile count just
// above a whole number of rounds (4097^2 on 256 x 256: 289 tiles on 256 CUs)
// is run as a first band of whole rounds and a remainder band on its own
// tile and split. A corner plan instead runs the largest block of whole
// tiles (4096^2 of 4097^2) on them, and the thin right and bottom edges
// (4096 x 1 and 1 x 4097) as problems of their own, so no tile computes
// rows or columns outside C. edges: those edges are at most EDGE_MAX wide
// and run on the edge kernels (edge_gemm.hip) instead of part[1], part[2].
struct Plan {
    Part part[3];
    int m1, n1;
    bool edges;
};

inline int round_up16(long long x) { return (int)((x + 15) / 16 * 16); }
inline int round_up32(long long x) { return (int)((x + 31) / 32 * 32); }

double model_time(long long M, long long N, long long K, long long batch, const Cand &c,
                  int occ, int splits, int kchunk, int cus) {
    const long long tiles = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * batch;
    const long long items = tiles * splits;
    const long long slots = (long long)cus * occ;
    const double peak_cu = 157.3e12 / 256.0;
    const double t_item = 2.0 * c.bm * c.bn * (kchunk + K_OVERHEAD + (c.ks - 1) * KS_OVERHEAD) /
                          (c.eff * peak_cu) * occ;
    // (a k-sliced workgroup: occ counts workgroups of ks slices each)
    const long long full = items / slots, rem = items % slots;
    double t = full * t_item;
    if (rem) {
        // A partial round: CUs holding fewer items than fit run each faster.
        const long long per_cu = (rem + cus - 1) / cus;
        t += per_cu < occ ? t_item * pow((double)per_cu / occ, PARTIAL_EXP) : t_item;
    }
    if (splits > 1) t += (splits + 2.0) * M * N * 4.0 / PARTIALS_BYTES_PER_S + LAUNCH_S;
    return t;
}

// The fastest single-band plan (tile, split) of an M x N x K band, and its
// modelled time. Split-K is used only for single problems (KERNELS id 9,
// gemm() in fp32 mode; batched_gemm() never splits); max_floats caps the
// partials (splits * M * N).
double best_part(int M, int N, int K, int batch, bool may_split, const Occupancy &occ,
                 long long max_floats, int cus, Part &best, int min_split_k = 0) {
    best = Part{0, 1, round_up16(K)};
    double best_t = -1.0;
    for (int ci = 0; ci < N_CANDS; ++ci) {
        const Cand &c = CANDS[ci];
        if (occ.wgs[ci][0] <= 0) continue;  // no such kernel for this case
        if (c.ks > 1 && K < c.ks * MIN_SLICE_K) continue;
        if (c.kind == TileKind::XS && (long long)M * N * batch > XS_MAX_OUTPUTS) continue;
        for (int s : SPLITS) {
            int splits = 1, kchunk = round_up16(K);
            if (s > 1) {
                if (c.ks > 1 || !may_split || K < 2 * MIN_SPLIT_K) continue;
                kchunk = round_up32((K + s - 1) / s);  // whole k-tiles of every tile's BK
                if (kchunk < MIN_SPLIT_K) continue;
                splits = (K + kchunk - 1) / kchunk;
                if (splits < 2 || (long long)splits * M * N > max_floats) continue;
                if (kchunk < min_split_k) continue;
            }
            const double t =
                model_time(M, N, K, batch, c, occ.wgs[ci][splits > 1], splits, kchunk, cus);
            if (best_t < 0 || t < best_t) {
                best_t = t;
                best = Part{ci, splits, kchunk};
            }
        }
    }
    return best_t;
}

Plan plan_for(int M, int N, int K, int batch, bool may_split, const Occupancy &occ,
              long long max_floats, bool edges_ok) {
    const int cus = device_cus();
    const Part whole{0, 1, round_up16(K)};
    Plan best{{whole, whole, whole}, M, N, false};
    const double single_t = best_part(M, N, K, batch, may_split, occ, max_floats, cus,
                                      best.part[0]);
    if (batch != 1 || K < MIN_BAND_K) return best;
    double best_t = single_t;
    // Corner plans: whole tiles of one candidate over [0, m1) x [0, n1), the
    // edges on the best plan of their own.
    for (int ci = 0; ci < N_CANDS; ++ci) {
        const Cand &c = CANDS[ci];
        if (c.ks > 1) continue;
        const int m1 = M / c.bm * c.bm, n1 = N / c.bn * c.bn;
        if (m1 == 0 || n1 == 0 || (m1 == M && n1 == N)) continue;
        double tm = model_time(m1, n1, K, 1, c, occ.wgs[ci][0], 1, round_up16(K), cus);
        Part pr = whole, pb = whole;
        if (n1 < N) {
            const double t = best_part(m1, N - n1, K, 1, may_split, occ, max_floats, cus, pr,
                                       MIN_BAND_SPLIT_K);
            if (t < 0) continue;
            tm += t + BAND_S;
        }
        if (m1 < M) {
            const double t = best_part(M - m1, N, K, 1, may_split, occ, max_floats, cus, pb,
                                       MIN_BAND_SPLIT_K);
            if (t < 0) continue;
            tm += t + BAND_S;
        }
        if (tm < BAND_GAIN * single_t && tm < best_t) {
            best_t = tm;
            best = Plan{{Part{ci, 1, round_up16(K)}, pb, pr}, m1, n1, false};
        }
        // The same block with the edge kernels (row-major A and B, BLAS
        // epilogue, edges at most EDGE_MAX wide).
        // (The edges need scratch: only where K may be split.)
        if (edges_ok && M - m1 <= bmb::EDGE_MAX && N - n1 <= bmb::EDGE_MAX &&
            may_split && bmb::edge_partial_floats(M - m1, N - n1, N, K) <= max_floats) {
            const double te = model_time(m1, n1, K, 1, c, occ.wgs[ci][0], 1, round_up16(K), cus) +
                              bmb::edge_model_s(m1, N - n1, M - m1, N, K);
            if (te < BAND_GAIN * single_t && te < best_t) {
                best_t = te;
                best = Plan{{Part{ci, 1, round_up16(K)}, whole, whole}, m1, n1, true};
            }
        }
    }
    for (int ci = 0; ci < N_CANDS; ++ci) {
        const Cand &c = CANDS[ci];
        if (c.ks > 1) continue;  // a first band of whole rounds: plain tiles
        const long long tiles_n = (N + c.bn - 1) / c.bn;
        const long long slots = (long long)cus * occ.wgs[ci][0];
        for (long long k = 1;; ++k) {
            const long long rows = k * slots / tiles_n;  // tile rows in k whole rounds
            if (rows <= 0) continue;
            if (rows * c.bm >= M) break;
            const int m1 = (int)(rows * c.bm);
            const double t0 = model_time(m1, N, K, 1, c, occ.wgs[ci][0], 1, round_up16(K), cus);
            Part p1;
            const double t1 =
                best_part(M - m1, N, K, 1, may_split, occ, max_floats, cus, p1, MIN_BAND_SPLIT_K);
            if (t1 < 0) continue;
            const double tm = t0 + t1 + BAND_S;
            if (tm < BAND_GAIN * single_t && tm < best_t) {
                best_t = tm;
                best = Plan{{Part{ci, 1, round_up16(K)}, p1, whole}, m1, N, false};
            }
        }
    }
    if (getenv("BMB_GEMM_PLAN_TRACE") != nullptr)
        fprintf(stderr, "fp32 gemm plan %dx%dx%d: m1 %d n1 %d edges %d parts (%d,%d,%d) "
                        "(%d,%d,%d) (%d,%d,%d) model %.1f us (one band %.1f us)\n",
                M, N, K, best.m1, best.n1, (int)best.edges, best.part[0].tile, best.part[0].splits,
                best.part[0].kchunk, best.part[1].tile, best.part[1].splits, best.part[1].kchunk,
                best.part[2].tile, best.part[2].splits, best.part[2].kchunk, best_t * 1e6,
                single_t * 1e6);
    return best;
}

// Plans memoised per (device, case, shape, batch, split permission and cap).
template <bool TA, bool TB, int EPI>
Plan pick(int M, int N, int K, int batch, bool vec, bool may_split, const Occupancy &occ,
          long long max_floats = MAX_SPLIT_FLOATS) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    using Key = std::tuple<int, bool, int, int, int, int, bool, long long>;
    static std::mutex mu;
    static std::map<Key, Plan> memo;
    const Key key{dev, vec, M, N, K, batch, may_split, max_floats};
    {
        std::lock_guard<std::mutex> lock(mu);
        auto it = memo.find(key);
        if (it != memo.end()) return it->second;
    }
    const Plan p = plan_for(M, N, K, batch, may_split, occ, max_floats,
                            !TA && !TB && EPI == bmb::EPI_BLAS);
    std::lock_guard<std::mutex> lock(mu);
    if (memo.size() > 4096) memo.clear();
    memo.emplace(key, p);
    return p;
}

// The occupancy table of one (transposes, epilogue, alignment) case, queried
// once per device.
template <bool TA, bool TB, int EPI>
const Occupancy &occupancy(bool vec) {
    static Occupancy table[64][2];
    static std::once_flag once[64][2];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    std::call_once(once[dev][vec], [&] {
        Occupancy &o = table[dev][vec];
        if (vec) {
            tile_occupancy<TA, TB, TileL, EPI, true>(o.wgs[0]);
            tile_occupancy<TA, TB, TileM, EPI, true>(o.wgs[1]);
            tile_occupancy<TA, TB, TileN, EPI, true>(o.wgs[2]);
            tile_occupancy<TA, TB, TileS, EPI, true>(o.wgs[3]);
            ks_occupancy<TA, TB, TileM, EPI, true, 2>(o.wgs[4]);
            ks_occupancy<TA, TB, TileN, EPI, true, 2>(o.wgs[5]);
            ks_occupancy<TA, TB, TileN, EPI, true, 4>(o.wgs[6]);
            ks_occupancy<TA, TB, TileS, EPI, true, 2>(o.wgs[7]);
            ks_occupancy<TA, TB, TileS, EPI, true, 4>(o.wgs[8]);
            ks_occupancy<TA, TB, TileXS, EPI, true, 4>(o.wgs[9]);
            ks_occupancy<TA, TB, TileXS, EPI, true, 8>(o.wgs[10]);
        } else {
            tile_occupancy<TA, TB, TileL, EPI, false>(o.wgs[0]);
            tile_occupancy<TA, TB, TileM, EPI, false>(o.wgs[1]);
            tile_occupancy<TA, TB, TileN, EPI, false>(o.wgs[2]);
            tile_occupancy<TA, TB, TileS, EPI, false>(o.wgs[3]);
            ks_occupancy<TA, TB, TileM, EPI, false, 2>(o.wgs[4]);
            ks_occupancy<TA, TB, TileN, EPI, false, 2>(o.wgs[5]);
            ks_occupancy<TA, TB, TileN, EPI, false, 4>(o.wgs[6]);
            ks_occupancy<TA, TB, TileS, EPI, false, 2>(o.wgs[7]);
            ks_occupancy<TA, TB, TileS, EPI, false, 4>(o.wgs[8]);
            ks_occupancy<TA, TB, TileXS, EPI, false, 4>(o.wgs[9]);
            ks_occupancy<TA, TB, TileXS, EPI, false, 8>(o.wgs[10]);
        }
    });
    return table[dev][vec];
}

// The operands of one launch: a problem, or a block of rows and columns of
// one (pointers at its first row and column, the stored row strides).
struct Ops {
    const float *A;
    int lda;
    long long sA;
    const float *B;
    int ldb;
    long long sB;
    float *C;
    int ldc;
    long long sC;
};

template <bool TA, bool TB, class Tile, int EPI>
void launch_tile(int batch, int M, int N, int K, float alpha, const Ops &o, float beta,
                 hipStream_t stream, bool vec, bmb::EpiArgs ep) {
    using L = bmb::MfmaLayout<TA, TB, Tile>;
    const int tiles_m = bmb::ceil_div(M, Tile::BM), tiles_n = bmb::ceil_div(N, Tile::BN);
    const dim3 grid(tiles_m * tiles_n, batch);
    if (vec) {
        bmb::allow_smem(bmb::mfma_gemm_k<TA, TB, Tile, true, EPI>, L::SMEM_BYTES);
        bmb::launch(bmb::mfma_gemm_k<TA, TB, Tile, true, EPI>, grid, dim3(Tile::NT),
                    L::SMEM_BYTES, stream, M, N, K, alpha, o.A, o.lda, o.sA, o.B, o.ldb, o.sB,
                    beta, o.C, o.ldc, o.sC, tiles_m, tiles_n, ep);
    } else {
        bmb::allow_smem(bmb::mfma_gemm_k<TA, TB, Tile, false, EPI>, L::SMEM_BYTES);
        bmb::launch(bmb::mfma_gemm_k<TA, TB, Tile, false, EPI>, grid, dim3(Tile::NT),
                    L::SMEM_BYTES, stream, M, N, K, alpha, o.A, o.lda, o.sA, o.B, o.ldb, o.sB,
                    beta, o.C, o.ldc, o.sC, tiles_m, tiles_n, ep);
    }
}

// A tile as KS k-slices of one workgroup (EPI_BLAS only).
template <bool TA, bool TB, class Tile, int EPI, int KS>
void launch_tile_ks(int batch, int M, int N, int K, float alpha, const Ops &o, float beta,
                    hipStream_t stream, bool vec) {
    if constexpr (EPI == bmb::EPI_BLAS) {
        using L = bmb::MfmaLayout<TA, TB, Tile>;
        const int tiles_m = bmb::ceil_div(M, Tile::BM), tiles_n = bmb::ceil_div(N, Tile::BN);
        const dim3 grid(tiles_m * tiles_n, batch);
        const size_t smem = KS * L::SMEM_BYTES;
        if (vec) {
            auto k = bmb::mfma_gemm_ks_k<TA, TB, Tile, true, EPI, KS>;
            bmb::allow_smem(k, smem);
            bmb::launch(k, grid, dim3(Tile::NT * KS), smem, stream, M, N, K, alpha, o.A, o.lda,
                        o.sA, o.B, o.ldb, o.sB, beta, o.C, o.ldc, o.sC, tiles_m, tiles_n,
                        bmb::EpiArgs{});
        } else {
            auto k = bmb::mfma_gemm_ks_k<TA, TB, Tile, false, EPI, KS>;
            bmb::allow_smem(k, smem);
            bmb::launch(k, grid, dim3(Tile::NT * KS), smem, stream, M, N, K, alpha, o.A, o.lda,
                        o.sA, o.B, o.ldb, o.sB, beta, o.C, o.ldc, o.sC, tiles_m, tiles_n,
                        bmb::EpiArgs{});
        }
    }
}

// Split-K: the partial sums of each K range go to P (splits x M x N), then
// one reduce kernel adds them in range order and applies the epilogue.
template <bool TA, bool TB, class Tile, int EPI>
void launch_split(const Part &p, int M, int N, int K, float alpha, const Ops &o, float beta,
                  float *P, bool vec, bmb::EpiArgs ep, hipStream_t stream) {
    using L = bmb::MfmaLayout<TA, TB, Tile>;
    const int tiles_m = bmb::ceil_div(M, Tile::BM), tiles_n = bmb::ceil_div(N, Tile::BN);
    const dim3 grid(tiles_m * tiles_n, p.splits);
    if (vec) {
        bmb::allow_smem(bmb::mfma_gemm_splitk_k<TA, TB, Tile, true>, L::SMEM_BYTES);
        bmb::launch(bmb::mfma_gemm_splitk_k<TA, TB, Tile, true>, grid, dim3(Tile::NT),
                    L::SMEM_BYTES, stream, M, N, K, o.A, o.lda, o.B, o.ldb, P, tiles_m, tiles_n,
                    p.kchunk);
    } else {
        bmb::allow_smem(bmb::mfma_gemm_splitk_k<TA, TB, Tile, false>, L::SMEM_BYTES);
        bmb::launch(bmb::mfma_gemm_splitk_k<TA, TB, Tile, false>, grid, dim3(Tile::NT),
                    L::SMEM_BYTES, stream, M, N, K, o.A, o.lda, o.B, o.ldb, P, tiles_m, tiles_n,
                    p.kchunk);
    }
    const long long mn = (long long)M * N;
    bmb::launch(bmb::splitk_reduce_k<EPI>, dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0,
                stream, o.C, (const float *)P, p.splits, mn, N, o.ldc, alpha, beta, ep);
}

template <bool TA, bool TB, int EPI>
void run_band(const Part &p, int batch, int M, int N, int K, float alpha, const Ops &o,
              float beta, float *P, bool vec, bmb::EpiArgs ep, hipStream_t stream) {
    if (p.splits > 1) {
        switch (CANDS[p.tile].kind) {
        case TileKind::L: launch_split<TA, TB, TileL, EPI>(p, M, N, K, alpha, o, beta, P, vec, ep, stream); break;
        case TileKind::M: launch_split<TA, TB, TileM, EPI>(p, M, N, K, alpha, o, beta, P, vec, ep, stream); break;
        case TileKind::N: launch_split<TA, TB, TileN, EPI>(p, M, N, K, alpha, o, beta, P, vec, ep, stream); break;
        case TileKind::S: launch_split<TA, TB, TileS, EPI>(p, M, N, K, alpha, o, beta, P, vec, ep, stream); break;
        case TileKind::XS: break;  // (never split: k-sliced only)
        }
        return;
    }
    if (CANDS[p.tile].ks > 1) {
        const int ks = CANDS[p.tile].ks;
        switch (CANDS[p.tile].kind) {
        case TileKind::M:
            launch_tile_ks<TA, TB, TileM, EPI, 2>(batch, M, N, K, alpha, o, beta, stream, vec);
            break;
        case TileKind::N:
            if (ks == 2) launch_tile_ks<TA, TB, TileN, EPI, 2>(batch, M, N, K, alpha, o, beta, stream, vec);
            else launch_tile_ks<TA, TB, TileN, EPI, 4>(batch, M, N, K, alpha, o, beta, stream, vec);
            break;
        case TileKind::XS:
            if (ks == 4) launch_tile_ks<TA, TB, TileXS, EPI, 4>(batch, M, N, K, alpha, o, beta, stream, vec);
            else launch_tile_ks<TA, TB, TileXS, EPI, 8>(batch, M, N, K, alpha, o, beta, stream, vec);
            break;
        default:
            if (ks == 2) launch_tile_ks<TA, TB, TileS, EPI, 2>(batch, M, N, K, alpha, o, beta, stream, vec);
            else launch_tile_ks<TA, TB, TileS, EPI, 4>(batch, M, N, K, alpha, o, beta, stream, vec);
            break;
        }
        return;
    }
    switch (CANDS[p.tile].kind) {
    case TileKind::L: launch_tile<TA, TB, TileL, EPI>(batch, M, N, K, alpha, o, beta, stream, vec, ep); break;
    case TileKind::M: launch_tile<TA, TB, TileM, EPI>(batch, M, N, K, alpha, o, beta, stream, vec, ep); break;
    case TileKind::N: launch_tile<TA, TB, TileN, EPI>(batch, M, N, K, alpha, o, beta, stream, vec, ep); break;
    case TileKind::S: launch_tile<TA, TB, TileS, EPI>(batch, M, N, K, alpha, o, beta, stream, vec, ep); break;
    case TileKind::XS: break;  // (k-sliced only, above)
    }
}

inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Split-K partials go to `fixed` (at most fixed_floats), or else to scratch
// leased for `stream` (reuse ordered by the lease's event); under graph
// capture, where a lease could allocate, K is not split. The bands of a plan
// run in row order on the stream; a second band's split partials reuse P
// after the first band's reduce has read it.
template <bool TA, bool TB, int EPI = bmb::EPI_BLAS>
void dispatch(int batch, int M, int N, int K, float alpha, const float *A,
              long long sA, const float *B, long long sB, float beta, float *C,
              long long sC, hipStream_t stream, bmb::EpiArgs ep = {},
              float *fixed = nullptr, long long fixed_floats = 0) {
    if (M <= 0 || N <= 0 || batch <= 0) return;
    // 128-bit loads need the contiguous axis of each stored operand to be a
    // multiple of 4 floats, 16-byte aligned bases, and batch strides that keep
    // that alignment.
    const int a_contig = TA ? M : K, b_contig = TB ? K : N;
    const bool vec = a_contig % 4 == 0 && b_contig % 4 == 0 && al16(A) && al16(B) &&
                     (batch == 1 || (sA % 4 == 0 && sB % 4 == 0));
    const Occupancy &occ = occupancy<TA, TB, EPI>(vec);
    const bool may_split = batch == 1 && (fixed != nullptr || !bmb::stream_capturing(stream));
    Plan p = pick<TA, TB, EPI>(M, N, K, batch, vec, may_split, occ,
                               fixed ? fixed_floats : MAX_SPLIT_FLOATS);
    // Partials: the largest split band's splits x rows x columns.
    auto partials = [&](const Plan &q) {
        long long pf = 0;
        if (q.part[0].splits > 1) pf = (long long)q.part[0].splits * q.m1 * q.n1;
        if (q.edges) return std::max(pf, bmb::edge_partial_floats(M - q.m1, N - q.n1, N, K));
        if (q.m1 < M && q.part[1].splits > 1)
            pf = std::max(pf, (long long)q.part[1].splits * (M - q.m1) * N);
        if (q.n1 < N && q.part[2].splits > 1)
            pf = std::max(pf, (long long)q.part[2].splits * q.m1 * (N - q.n1));
        return pf;
    };
    const long long pf = partials(p);
    float *P = fixed;
    std::optional<bmb::ScratchLease> lease;
    if (pf > 0 && fixed == nullptr) {
        lease.emplace(bmb::SCRATCH_GEMM, (size_t)pf * sizeof(float), stream);
        P = static_cast<float *>(lease->get());
        if (P == nullptr) p = pick<TA, TB, EPI>(M, N, K, batch, vec, false, occ);  // no split
    }
    const int lda = TA ? M : K, ldb = TB ? K : N, ldc = N;
    const Ops whole{A, lda, sA, B, ldb, sB, C, ldc, sC};
    run_band<TA, TB, EPI>(p.part[0], batch, p.m1, p.n1, K, alpha, whole, beta, P, vec, ep,
                          stream);
    if (p.edges) {
        bmb::gemm_edges(false, M, N, K, p.m1, p.n1, alpha, A, lda, B, ldb, beta, C, ldc, P,
                        stream);
        return;
    }
    if (p.n1 < N) {
        // The right edge of the first rows: B and C n1 columns (TB: B n1
        // rows) in, bias n1 entries in.
        const size_t c = (size_t)p.n1;
        Ops o = whole;
        o.B = TB ? B + c * ldb : B + c;
        o.C = C + c;
        bmb::EpiArgs e = ep;
        if (e.bias) e.bias += c;
        if (e.act) e.act += c;
        if (e.pre) e.pre += c;
        run_band<TA, TB, EPI>(p.part[2], 1, p.m1, N - p.n1, K, alpha, o, beta, P,
                              vec && al16(o.B), e, stream);
    }
    if (p.m1 >= M) return;
    const size_t r = (size_t)p.m1;
    bmb::EpiArgs e1 = ep;
    if (e1.act) e1.act += r * ldc;
    if (e1.pre) e1.pre += r * ldc;
    // A band of rows starts r rows (TA: r columns of the stored K x M) in.
    Ops o = whole;
    o.A = TA ? A + r : A + r * K;
    o.C = C + r * ldc;
    run_band<TA, TB, EPI>(p.part[1], 1, M - p.m1, N, K, alpha, o, beta, P, vec && al16(o.A), e1,
                          stream);
}

void gemm_any(bool ta, bool tb, int batch, int M, int N, int K, float alpha,
              const float *A, long long sA, const float *B, long long sB,
              float beta, float *C, long long sC, hipStream_t stream) {
    if (!ta && !tb)     dispatch<false, false>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream);
    else if (!ta && tb) dispatch<false, true >(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream);
    else if (ta && !tb) dispatch<true,  false>(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream);
    else                dispatch<true,  true >(batch, M, N, K, alpha, A, sA, B, sB, beta, C, sC, stream);
}

// The arithmetic of gemm(), gemm_noalloc() and the GPT's linear layers
// (gemm_set_math): process-wide, read once per call.
std::atomic<int> g_math{GEMM_MATH_BF16X3};

bool fp32_math() { return g_math.load(std::memory_order_relaxed) == GEMM_MATH_FP32; }

// gemm() / gemm_noalloc() in fp32 mode: the KERNELS id 9 kernels (fp32
// matrix-core products), any transposes, split-K into `fixed` or leased
// scratch.
void fp32_gemm(bool ta, bool tb, int M, int N, int K, float alpha, const float *A,
               const float *B, float beta, float *C, hipStream_t stream, float *fixed,
               long long fixed_floats) {
    const bmb::EpiArgs ep{};
    if (!ta && !tb)
        dispatch<false, false>(1, M, N, K, alpha, A, 0, B, 0, beta, C, 0, stream, ep, fixed, fixed_floats);
    else if (!ta && tb)
        dispatch<false, true>(1, M, N, K, alpha, A, 0, B, 0, beta, C, 0, stream, ep, fixed, fixed_floats);
    else if (ta && !tb)
        dispatch<true, false>(1, M, N, K, alpha, A, 0, B, 0, beta, C, 0, stream, ep, fixed, fixed_floats);
    else
        dispatch<true, true>(1, M, N, K, alpha, A, 0, B, 0, beta, C, 0, stream, ep, fixed, fixed_floats);
}

}  // namespace

void bmb::gemm_bias_nt(int M, int N, int K, const float *A, const float *W, const float *bias,
                       float *C, float *gelu_out) {
    if (fp32_math()) {
        const bmb::EpiArgs ep{bias, gelu_out, nullptr};
        if (gelu_out != nullptr)
            dispatch<false, true, bmb::EPI_BIAS_GELU>(1, M, N, K, 1.0f, A, 0, W, 0, 0.0f, C, 0,
                                                      nullptr, ep);
        else
            dispatch<false, true, bmb::EPI_BIAS>(1, M, N, K, 1.0f, A, 0, W, 0, 0.0f, C, 0,
                                                 nullptr, ep);
        return;
    }
    bmb::bf16x3_gemm(false, true, M, N, K, 1.0f, A, W, 0.0f, C, nullptr,
                     gelu_out != nullptr ? bmb::EPI_BIAS_GELU : bmb::EPI_BIAS, bias, gelu_out,
                     nullptr, nullptr, 0);
}

void bmb::gemm_gelu_grad_nn(int M, int N, int K, const float *A, const float *B,
                            const float *pre, float *C) {
    if (fp32_math()) {
        dispatch<false, false, bmb::EPI_GELU_GRAD>(1, M, N, K, 1.0f, A, 0, B, 0, 0.0f, C, 0,
                                                   nullptr, bmb::EpiArgs{nullptr, nullptr, pre});
        return;
    }
    bmb::bf16x3_gemm(false, false, M, N, K, 1.0f, A, B, 0.0f, C, nullptr, bmb::EPI_GELU_GRAD,
                     nullptr, nullptr, pre, nullptr, 0);
}

void bmb::splitk_reduce(float *C, const float *P, int splits, long long mn, int N, float alpha,
                        float beta, hipStream_t stream) {
    bmb::launch(bmb::splitk_reduce_k<bmb::EPI_BLAS>, dim3((unsigned)((mn + 1023) / 1024)),
                dim3(256), 0, stream, C, P, splits, mn, N, N, alpha, beta, bmb::EpiArgs{});
}

void bmb::splitk_reduce_epi(int epi, float *C, const float *P, int splits, long long mn, int N,
                            int ldc, float alpha, float beta, hipStream_t stream,
                            const float *bias, float *act, const float *pre) {
    const dim3 grid((unsigned)((mn + 1023) / 1024)), block(256);
    const bmb::EpiArgs ep{bias, act, pre};
    switch (epi) {
    case bmb::EPI_BIAS:
        bmb::launch(bmb::splitk_reduce_k<bmb::EPI_BIAS>, grid, block, 0, stream, C, P, splits,
                    mn, N, ldc, alpha, beta, ep);
        break;
    case bmb::EPI_BIAS_GELU:
        bmb::launch(bmb::splitk_reduce_k<bmb::EPI_BIAS_GELU>, grid, block, 0, stream, C, P,
                    splits, mn, N, ldc, alpha, beta, ep);
        break;
    case bmb::EPI_GELU_GRAD:
        bmb::launch(bmb::splitk_reduce_k<bmb::EPI_GELU_GRAD>, grid, block, 0, stream, C, P,
                    splits, mn, N, ldc, alpha, beta, ep);
        break;
    default:
        bmb::launch(bmb::splitk_reduce_k<bmb::EPI_BLAS>, grid, block, 0, stream, C, P, splits, mn,
                    N, ldc, alpha, beta, ep);
        break;
    }
}

extern "C" {

void gemm(bool transA, bool transB, int M, int N, int K, float alpha,
          const float *A, const float *B, float beta, float *C,
          hipStream_t stream) {
    if (fp32_math()) {
        fp32_gemm(transA, transB, M, N, K, alpha, A, B, beta, C, stream, nullptr, 0);
        return;
    }
    bmb::bf16x3_gemm(transA, transB, M, N, K, alpha, A, B, beta, C, stream, bmb::EPI_BLAS,
                     nullptr, nullptr, nullptr, nullptr, 0);
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

int gemm_noalloc(bool transA, bool transB, int M, int N, int K, float alpha, const float *A,
                 const float *B, float beta, float *C, hipStream_t stream) {
    if (M <= 0 || N <= 0) return 0;
    float *fixed = noalloc_scratch();
    if (fixed == nullptr) return -1;
    if (fp32_math()) {
        fp32_gemm(transA, transB, M, N, K, alpha, A, B, beta, C, stream, fixed,
                  NOALLOC_SPLIT_FLOATS);
        return 0;
    }
    bmb::bf16x3_gemm(transA, transB, M, N, K, alpha, A, B, beta, C, stream, bmb::EPI_BLAS,
                     nullptr, nullptr, nullptr, fixed, NOALLOC_SPLIT_FLOATS);
    return 0;
}

int gemm_set_math(int math) {
    if (math != GEMM_MATH_BF16X3 && math != GEMM_MATH_FP32) {
        fprintf(stderr, "gemm_set_math: unknown mode %d (GEMM_MATH_BF16X3 = %d, "
                        "GEMM_MATH_FP32 = %d)\n", math, GEMM_MATH_BF16X3, GEMM_MATH_FP32);
        return -1;
    }
    return g_math.exchange(math);
}

int gemm_get_math(void) { return g_math.load(); }

}  // extern "C"
