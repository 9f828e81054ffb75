// Thin edges of a GEMM whose planner splits C into a block of whole tiles and
// its remainder (the corner plans of mfma_gemm.hip and sgemm_bf16x3.hip): at
// most EDGE_MAX columns right of the block and EDGE_MAX rows below it, row-
// major A and B (no transposes), C = alpha A B + beta C.
//
// Each edge is a handful of matrix-vector products: the right edge reads all
// of A's rows [0, m1) and a K x rn sliver of B, the bottom edge a rm x K
// sliver of A and all of B. On matrix-core tiles (64 wide at the least) nearly
// all of their work would be padding; here the VALU streams the large operand
// once, at HBM rate.
//  - right: B's K x rn sliver is first packed into rn contiguous rows (for
//    bf16x3, its split's hi and lo rows), then one 32-lane half-wave per row
//    of A, its lanes taking K in float4 steps, rn sums per lane, a
//    fixed-order butterfly over the half (every lane ends with the same
//    bits), and the lanes j < rn store C[row][n1 + j];
//  - bottom: one thread per 4 consecutive columns of B over one of `ranges`
//    consecutive K ranges, rm x 4 sums per thread, stored as partials
//    (ranges x rm x N); edge_reduce_k adds them in a fixed order and applies
//    the epilogue. Three launches: bottom partials (with the packing), right
//    edge, reduce.
// Every sum is an fp32 sum of exact products: fp32 products (the fp32 path),
// or, for the bf16x3 path, the three bf16 products hi*hi + hi*lo + lo*hi of
// the bf16x3 kernels' split, so an edge element meets the same bound as the
// rest of C.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "gemm_fused.hpp"
#include "launch.hpp"

namespace {

using bmb::EDGE_MAX;

// The bf16x3 kernels' split (sgemm_bf16x3.hip): hi = bf16(x clamped to
// bf16's largest finite value), lo = bf16(x - hi), both held as floats.
constexpr float BF16_FINITE_MAX = 0x1.fefffep+127f;
__device__ __forceinline__ void split_bf(float x, float &hi, float &lo) {
    const __bf16 h = (__bf16)__builtin_amdgcn_fmed3f(x, -BF16_FINITE_MAX, BF16_FINITE_MAX);
    hi = (float)h;
    lo = (float)(__bf16)(x - hi);
}

// acc += a * b as the path computes a product (a, b already split for BF).
template <bool BF>
__device__ __forceinline__ float madd(float a, float ah, float al, float b, float bh, float bl,
                                      float acc) {
    if (!BF) return fmaf(a, b, acc);
    acc = fmaf(ah, bh, acc);
    acc = fmaf(ah, bl, acc);
    return fmaf(al, bh, acc);
}

// B's right edge, K x rn floats rows ldb apart, packed to rn rows of K
// (Bs[j K + k]), so that the right edge reads it as 128-bit loads: read in
// place, every wave would touch one cache line per k for each 4 bytes. BF:
// the bf16x3 split's hi and lo of each value instead (Bs and Bs + rn K),
// split once here rather than by every row's wave.
template <bool BF>
__device__ __forceinline__ void edge_pack(long long e, int K, int rn, const float *__restrict__ B,
                                          int ldb, float *__restrict__ Bs) {
    if (e >= (long long)K * rn) return;
    const int j = (int)(e / K), k = (int)(e % K);
    const float b = B[(size_t)k * ldb + j];
    if (BF) {
        float hi, lo;
        split_bf(b, hi, lo);
        Bs[e] = hi;
        Bs[(size_t)rn * K + e] = lo;
    } else {
        Bs[e] = b;
    }
}

// The packing alone (no bottom edge to ride).
template <bool BF>
__global__ __launch_bounds__(256) void edge_pack_k(int K, int rn, const float *__restrict__ B,
                                                   int ldb, float *__restrict__ Bs) {
    edge_pack<BF>((long long)blockIdx.x * 256 + threadIdx.x, K, rn, B, ldb, Bs);
}

// Four consecutive floats of a row that may end inside them (zeros past n).
__device__ __forceinline__ void load4_tail(const float *p, int i, int n, float (&v)[4]) {
    if (i + 3 < n) {
        float4 x;
        __builtin_memcpy(&x, p + i, sizeof(x));  // one 128-bit load (dword alignment)
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = i + u < n ? p[i + u] : 0.0f;
    }
}

// Right edge: rows [0, m1), columns [0, RN) of the edge (A at row 0, C at
// column n1 of row 0; Bs the packed B edge). Each wave takes two rows, one
// per 32-lane half, so the two halves' loads of Bs are the same addresses
// (one fetch) and the packed edge is read once per two rows; four waves per
// workgroup. Each step loads U float4s of the row and of each Bs row before
// it multiplies, so that many loads per lane are in flight.
template <bool BF, int RN>
__global__ __launch_bounds__(256) void edge_right_k(int m1, int K, float alpha,
                                                    const float *__restrict__ A, int lda,
                                                    const float *__restrict__ Bs, float beta,
                                                    float *C, int ldc) {
    // (BF: Bs holds the split, hi rows then lo rows; twice the B loads per step.)
    constexpr int NB = BF ? 2 : 1;  // B rows per column: the value, or its hi and lo
    constexpr int U = NB * RN <= 2 ? 8 : NB * RN <= 4 ? 4 : 2;
    const int lane = threadIdx.x & 63, l32 = lane & 31;
    const int row = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * 2 + (lane >> 5);
    if (row - (lane >> 5) >= m1) return;  // both rows past the end (uniform over the wave)
    float acc[RN];
#pragma unroll
    for (int j = 0; j < RN; ++j) acc[j] = 0.0f;
    const float *a = A + (size_t)min(row, m1 - 1) * lda;  // (a row past the end stores nothing)
    for (int k0 = l32 * 4; k0 < K; k0 += 128 * U) {
        float av[U][4], bv[U][NB * RN][4];
#pragma unroll
        for (int s = 0; s < U; ++s) {
            const int k = k0 + 128 * s;
            load4_tail(a, k, K, av[s]);
#pragma unroll
            for (int j = 0; j < NB * RN; ++j) load4_tail(Bs + (size_t)j * K, k, K, bv[s][j]);
        }
#pragma unroll
        for (int s = 0; s < U; ++s)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float ah = 0.0f, al = 0.0f;
                if (BF) split_bf(av[s][u], ah, al);
#pragma unroll
                for (int j = 0; j < RN; ++j) {
                    const float b = bv[s][j][u];
                    const float bh = BF ? b : 0.0f, bl = BF ? bv[s][RN + j][u] : 0.0f;
                    acc[j] = madd<BF>(av[s][u], ah, al, b, bh, bl, acc[j]);
                }
            }
    }
    float out = 0.0f;
#pragma unroll
    for (int j = 0; j < RN; ++j) {
        float v = acc[j];
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off);  // within the half
        if (l32 == j) out = v;
    }
    if (l32 < RN && row < m1) {
        float *c = C + (size_t)row * ldc + l32;
        *c = bmb::epilogue(out, alpha, beta, c);
    }
}

// Bottom edge partials: rows [0, RM) of the edge (A at row m1), thread t of
// workgroup (cb, r) takes columns 4 (cb 256 + t) .. + 3 over K range r, U
// rows of B loaded ahead of their multiplies. Zeros past K (the zero rows
// add nothing).
// Workgroups past ncb * ranges pack B's right edge (edge_pack) instead, so
// that the packing rides this launch.
template <bool BF, int RM>
__global__ __launch_bounds__(256) void edge_bottom_k(int N, int K, int kr, int ncb, int nbot,
                                                     const float *__restrict__ A, int lda,
                                                     const float *__restrict__ B, int ldb,
                                                     float *__restrict__ P, int rn,
                                                     const float *__restrict__ Bn,
                                                     float *__restrict__ Bs) {
    constexpr int U = 8;
    if ((int)blockIdx.x >= nbot) {
        edge_pack<BF>((long long)(blockIdx.x - nbot) * 256 + threadIdx.x, K, rn, Bn, ldb, Bs);
        return;
    }
    const int cb = blockIdx.x % ncb, r = blockIdx.x / ncb;
    const int c0 = (cb * 256 + (int)threadIdx.x) * 4;
    if (c0 >= N) return;
    const int k0 = r * kr, k1 = min(K, k0 + kr);
    float acc[RM][4];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[i][u] = 0.0f;
    for (int kb = k0; kb < k1; kb += U) {
        float bv[U][4];
#pragma unroll
        for (int s = 0; s < U; ++s) {
            if (kb + s < k1) {
                load4_tail(B + (size_t)(kb + s) * ldb, c0, N, bv[s]);
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) bv[s][u] = 0.0f;
            }
        }
#pragma unroll
        for (int s = 0; s < U; ++s) {
            if (kb + s >= k1) break;
            float bh[4] = {}, bl[4] = {};
            if (BF)
#pragma unroll
                for (int u = 0; u < 4; ++u) split_bf(bv[s][u], bh[u], bl[u]);
#pragma unroll
            for (int i = 0; i < RM; ++i) {
                const float av = A[(size_t)i * lda + kb + s];
                float ah = 0.0f, al = 0.0f;
                if (BF) split_bf(av, ah, al);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc[i][u] = madd<BF>(av, ah, al, bv[s][u], bh[u], bl[u], acc[i][u]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RM; ++i) {
        float *p = P + ((size_t)r * RM + i) * N + c0;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (c0 + u < N) p[u] = acc[i][u];
    }
}

// C[i][c] = epilogue(sum over ranges r, in order, of P[r][i][c]) for the
// rm x N bottom edge (C at row m1, rows ldc apart). A workgroup takes 32
// elements; its 8 thread groups of 32 each add every 8th range (ranges g,
// g + 8, ... in order), and thread group 0 adds the 8 group sums in group
// order: a fixed order, with a few loads per thread instead of one per range.
__global__ __launch_bounds__(256) void edge_reduce_k(float *C, int ldc, const float *P,
                                                     int ranges, int rm, int N, float alpha,
                                                     float beta) {
    __shared__ float part[8][32];
    const int t = threadIdx.x, g = t >> 5;
    const long long per = (long long)rm * N;
    const long long e = (long long)blockIdx.x * 32 + (t & 31);
    float s = 0.0f;
    if (e < per) {
        int r = g;
        float v[4];
        for (; r + 24 < ranges; r += 32) {
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = P[(size_t)(r + 8 * u) * per + e];
#pragma unroll
            for (int u = 0; u < 4; ++u) s += v[u];
        }
        for (; r < ranges; r += 8) s += P[(size_t)r * per + e];
    }
    part[g][t & 31] = s;
    __syncthreads();
    if (g != 0 || e >= per) return;
    float tot = part[0][t];
#pragma unroll
    for (int q = 1; q < 8; ++q) tot += part[q][t];
    float *c = C + (size_t)(e / N) * ldc + e % N;
    *c = bmb::epilogue(tot, alpha, beta, c);
}

// Workgroups of the bottom edge: column blocks of 1024 columns, times K
// ranges of at least 16 rows, about 512 workgroups in all.
int bottom_ncb(int N) { return (N + 1023) / 1024; }
int bottom_ranges(int N, int K) {
    const int want = std::max(1, 512 / bottom_ncb(N));
    return std::max(1, std::min(want, (K + 15) / 16));
}

// f(integral_constant<int, w>) for a width w in 1 .. EDGE_MAX.
template <class F>
void with_width(int w, F &&f) {
    switch (w) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 5: f(std::integral_constant<int, 5>{}); break;
    case 6: f(std::integral_constant<int, 6>{}); break;
    case 7: f(std::integral_constant<int, 7>{}); break;
    default: f(std::integral_constant<int, 8>{}); break;
    }
}
static_assert(EDGE_MAX == 8, "with_width covers widths 1 .. 8");

}  // namespace

int bmb::edge_ranges(int N, int K) { return bottom_ranges(N, K); }

long long bmb::edge_partial_floats(int rm, int rn, int N, int K) {
    return (rm > 0 ? (long long)bottom_ranges(N, K) * rm * N : 0) + 2LL * rn * K;
}

double bmb::edge_model_s(long long m1, long long rn, long long rm, long long N, long long K) {
    // The streamed operand at a little below a plain copy's rate, plus the
    // launches.
    constexpr double BYTES_PER_S = 4.0e12, LAUNCH = 2.0e-6;
    double t = 0.0;
    if (rn > 0) t += 4.0 * m1 * K / BYTES_PER_S + 2.0 * LAUNCH;
    if (rm > 0) t += 4.0 * K * N / BYTES_PER_S + 2.0 * LAUNCH;
    return t;
}

void bmb::gemm_edges(bool bf16x3, int M, int N, int K, int m1, int n1, float alpha,
                     const float *A, int lda, const float *B, int ldb, float beta, float *C,
                     int ldc, float *P, hipStream_t stream) {
    const int rn = N - n1, rm = M - m1;
    const dim3 block(256);
    // P: the bottom edge's partials, then the packed right edge of B.
    const int ranges = rm > 0 ? bottom_ranges(N, K) : 0;
    const long long bottom = (long long)ranges * rm * N;
    float *Bs = P + bottom;
    const bool right = rn > 0 && m1 > 0;
    const int npack = right ? (int)(((long long)K * rn + 255) / 256) : 0;
    // 1. the bottom edge's partials, with the packing riding the launch
    if (rm > 0) {
        const int ncb = bottom_ncb(N);
        const int kr = (K + ranges - 1) / ranges, nbot = ncb * ranges;
        const float *Am = A + (size_t)m1 * lda;
        const dim3 grid((unsigned)(nbot + npack));
        auto bottom_k = [&](auto bf, auto rmc) {
            bmb::launch(edge_bottom_k<decltype(bf)::value, decltype(rmc)::value>, grid, block, 0,
                        stream, N, K, kr, ncb, nbot, Am, lda, B, ldb, P, rn, B + n1, Bs);
        };
        with_width(rm, [&](auto rmc) {
            if (bf16x3) bottom_k(std::true_type{}, rmc);
            else bottom_k(std::false_type{}, rmc);
        });
    } else if (right) {
        if (bf16x3)
            bmb::launch(edge_pack_k<true>, dim3((unsigned)npack), block, 0, stream, K, rn, B + n1,
                        ldb, Bs);
        else
            bmb::launch(edge_pack_k<false>, dim3((unsigned)npack), block, 0, stream, K, rn, B + n1,
                        ldb, Bs);
    }
    // 2. the right edge from the packed B
    if (right) {
        const dim3 grid((unsigned)((m1 + 7) / 8));
        const float *Bc = Bs;
        auto right_k = [&](auto bf, auto rnc) {
            bmb::launch(edge_right_k<decltype(bf)::value, decltype(rnc)::value>, grid, block, 0,
                        stream, m1, K, alpha, A, lda, Bc, beta, C + n1, ldc);
        };
        with_width(rn, [&](auto rnc) {
            if (bf16x3) right_k(std::true_type{}, rnc);
            else right_k(std::false_type{}, rnc);
        });
    }
    // 3. the bottom edge's reduce and epilogue
    if (rm > 0) {
        const long long per = (long long)rm * N;
        bmb::launch(edge_reduce_k, dim3((unsigned)((per + 31) / 32)), block, 0, stream,
                    C + (size_t)m1 * ldc, ldc, (const float *)P, ranges, rm, N, alpha, beta);
    }
}
