// Fused causal attention, forward and backward, for gfx950 -- the
// counterpart of bare-metal-bard's src/flash.cu (API: src/flash.h).
//
// The default forward (flash_fwd_h_k) and backward (flash_dsum_h_k, then
// flash_bwd_h_k's dK/dV and dQ passes) carry every fp32 operand as an fp16
// hi/lo pair on v_mfma_f32_32x32x16_f16 with exact power-of-two scaling; the
// "forward, fp16x3" and "backward, fp16x3" comment blocks give the error and
// range argument. The other configs' kernels, described first, use chains of
// v_mfma_f32_32x32x2_f32 (fp32 in, exact fp32 products, fp32 accumulate). In that instruction lane l supplies
// A[m = l%32][kk = l/32] and B[kk = l/32][n = l%32]; the 32x32 result leaves
// lane l holding column n = l%32, register r holding row
// res_row(r, l/32) = 8*(r/4) + 4*(l/32) + r%4. A 32-wide contraction over
// head dims uses dd = (l/32)*hs/2 + st for step st, so each lane's operand is
// hs/2 contiguous floats of one row: 128-bit LDS or register reads.
//
// Work split. A workgroup of WPB waves owns WPB consecutive 32-row tiles of
// one (batch, head): 32 queries per wave in the forward and the dQ pass,
// 32 keys per wave in the dK/dV pass. The tiles it streams (keys for the
// forward and dQ, queries for dK/dV) are staged through LDS once per
// workgroup, double-buffered with one barrier per tile, and read by every
// wave of the workgroup with 128-bit, bank-conflict-free LDS reads (rows
// padded by 4 floats). Causality is a loop bound; only the diagonal and a
// ragged last tile are masked.
//
// Forward (src/flash.cu:115-311 for the maths). The score tile is computed
// transposed, S^T = K Q^T (keys x queries), so each lane holds one query's
// scores for 16 keys and lane l^32 the other 16: the row max is an
// in-register reduction plus one v_permlane32_swap, the online-softmax
// rescale touches only the lane's own O^T registers, and the probabilities
// are already in the B-operand layout of O^T += V^T P^T. V is stored
// transposed in LDS so that the A operand of that product is 128-bit reads.
// Scores are in log2 units (q pre-multiplied by scale*log2 e), p = exp2(s-m)
// on v_exp_f32; lse is stored in natural-log units (lse = m ln2 + ln l), the
// quantity src/flash.cu:309 stores.
//
// Backward (src/flash.cu:434-466), default configs. dsum D = rowsum(dO * O);
// then the dK/dV pass (S = Q K^T so that P^T and dS^T are in A-operand layout
// for dV += P^T dO, dK += dS^T Q), which also stores the causal dS tiles in a
// library-owned workspace; then the dQ pass, dQ = scale * dS K, a light
// pass that streams those tiles. A long block may be split into two halves
// whose results are atomic adds onto rows the dsum kernel zeroed: exactly
// two addends onto zero, so the result does not depend on their order and
// repeated calls give the same bits. (Configs without the workspace
// recompute S and dP in the dQ workgroups instead.)
//
// Workgroup order. Forward: work items are handed out longest first (the
// causal triangle would otherwise leave a long tail) in a snake order over
// each XCD's CUs. Backward passes: persistent workgroups, as many as fit on
// the device at once, each running a host-planned list of (block, head)
// items placed so that every CU gets the same amount of work (see
// plan_schedule). When B*NH is a multiple of 8, every XCD gets a fixed set of
// heads: the hardware sends workgroup ids x, x+8, x+16, ... to one XCD, so a
// head's K/V (or Q/dO) is fetched from HBM into one L2 only.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <functional>
#include <map>
#include <mutex>
#include <optional>
#include <tuple>
#include <vector>

#include "common.hpp"
#include "../../include/flash.h"
#include "launch.hpp"
#include "workspace.hpp"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr int NXCD = 8;

__device__ __forceinline__ f32x16 mfma(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0.0f;
    return z;
}

// Row of the 32x32 MFMA result held in register r of a lane in half `hf`.
__device__ __forceinline__ int res_row(int r, int hf) {
    return 8 * (r >> 2) + 4 * hf + (r & 3);
}

// v_permlane32_swap exchanges the upper half of its first operand with the
// lower half of its second; with both operands = v, the two results hold
// v[l] and v[l^32] (in some order) in every lane l. Max and sum of the pair
// are therefore symmetric and identical in both lanes.
__device__ __forceinline__ float pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// One 32-row x HS-column fp32 tile in flight from global memory to LDS.
// Row r of the tile is at src + r*rs; rows >= nrows are zero. Chunk e of the
// tile (a float4) is row e / (HS/4), columns 4*(e % (HS/4)) + 0..3, so the
// lanes of a wave read whole rows: coalesced 128-bit loads.
template <int HS, int NT>
struct Tile32 {
    static constexpr int CPR = HS / 4;  // float4 chunks per row
    static constexpr int PER_T = 32 * CPR / NT;
    static_assert(PER_T >= 1 && (32 * CPR) % NT == 0, "tile splits evenly over the threads");
    float4 v[PER_T];

    __device__ __forceinline__ void load(const float *src, size_t rs, int nrows, int tid) {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * NT, r = e / CPR, c = (e % CPR) * 4;
            v[i] = r < nrows ? bmb::ld4(src + (size_t)r * rs + c) : zero4();
        }
    }
    // Row-major copy, LDS row stride ld floats.
    __device__ __forceinline__ void store_rows(float *lds, int ld, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * NT, r = e / CPR, c = (e % CPR) * 4;
            bmb::st4(lds + r * ld + c, v[i]);
        }
    }
};

// The same 32 x HS tile, staged transposed: LDS row d holds column d of the
// tile (32 floats, row stride ld). Each thread owns runs of 4 consecutive rows
// of one column: it loads them with four 32-bit loads (the lanes of a wave
// cover 64 consecutive columns of one row per load, so every load is a
// coalesced 256-byte access) and writes the run with one 128-bit LDS store;
// with ld = 36 the 16 lanes of each store phase hit 16 distinct 4-bank groups.
template <int HS, int NT>
struct TileT32 {
    static constexpr int PER_T = 8 * HS / NT;  // (column, 4-row run) pairs per thread
    static_assert(PER_T >= 1 && (8 * HS) % NT == 0, "tile splits evenly over the threads");
    float4 v[PER_T];

    __device__ __forceinline__ void load(const float *src, size_t rs, int nrows, int tid) {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * NT, c = e % HS, r0 = (e / HS) * 4;
            const float *p = src + (size_t)r0 * rs + c;
            v[i].x = r0 + 0 < nrows ? p[0] : 0.0f;
            v[i].y = r0 + 1 < nrows ? p[rs] : 0.0f;
            v[i].z = r0 + 2 < nrows ? p[2 * rs] : 0.0f;
            v[i].w = r0 + 3 < nrows ? p[3 * rs] : 0.0f;
        }
    }
    __device__ __forceinline__ void store(float *lds, int ld, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * NT, c = e % HS, r0 = (e / HS) * 4;
            bmb::st4(lds + c * ld + r0, v[i]);
        }
    }
};

// Global load at a uniform base plus a 32-bit byte offset: the offset stays
// in one VGPR and the base in SGPRs (no 64-bit address arithmetic per load).
__device__ __forceinline__ float4 ld4_at(const float *base, unsigned byte_off) {
    return *reinterpret_cast<const float4 *>(reinterpret_cast<const char *>(base) + byte_off);
}
__device__ __forceinline__ float ld1_at(const float *base, unsigned byte_off) {
    return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) + byte_off);
}

// TileT32 with every load issued and no 64-bit address arithmetic: the
// tile base is uniform (SGPRs) and each element is a 32-bit byte offset from
// it. For a full tile the offsets are loop-invariant; a ragged tile (nrows <
// 32, at most one per loop) re-reads row nrows-1 for the rows past the end
// and stores zeros for them.
template <int HS, int NT>
struct TileT32U {
    static constexpr int PER_T = 8 * HS / NT;
    static_assert(PER_T >= 1 && (8 * HS) % NT == 0, "tile splits evenly over the threads");
    float4 v[PER_T];
    int nr;

    __device__ __forceinline__ void load(const float *src, size_t rs, int nrows, int tid) {
        nr = nrows;
        const unsigned urs = (unsigned)rs;
        if (nrows == 32) {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                const int e = tid + i * NT, c = e % HS, r0 = (e / HS) * 4;
                const unsigned o = 4u * ((unsigned)r0 * urs + c);
                v[i].x = ld1_at(src, o);
                v[i].y = ld1_at(src, o + 4u * urs);
                v[i].z = ld1_at(src, o + 8u * urs);
                v[i].w = ld1_at(src, o + 12u * urs);
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                const int e = tid + i * NT, c = e % HS, r0 = (e / HS) * 4;
                v[i].x = ld1_at(src, 4u * ((unsigned)min(r0 + 0, nrows - 1) * urs + c));
                v[i].y = ld1_at(src, 4u * ((unsigned)min(r0 + 1, nrows - 1) * urs + c));
                v[i].z = ld1_at(src, 4u * ((unsigned)min(r0 + 2, nrows - 1) * urs + c));
                v[i].w = ld1_at(src, 4u * ((unsigned)min(r0 + 3, nrows - 1) * urs + c));
            }
        }
    }
    __device__ __forceinline__ void store(float *lds, int ld, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * NT, c = e % HS, r0 = (e / HS) * 4;
            const float4 w = make_float4(r0 + 0 < nr ? v[i].x : 0.0f, r0 + 1 < nr ? v[i].y : 0.0f,
                                         r0 + 2 < nr ? v[i].z : 0.0f, r0 + 3 < nr ? v[i].w : 0.0f);
            bmb::st4(lds + c * ld + r0, w);
        }
    }
};

// Tile32 with every load issued and 32-bit offsets from a uniform base, as
// TileT32U: rows past nrows re-read row nrows-1 and are stored as zeros.
template <int HS, int NT>
struct Tile32U {
    static constexpr int CPR = HS / 4;
    static constexpr int PER_T = 32 * CPR / NT;
    static_assert(PER_T >= 1 && (32 * CPR) % NT == 0, "tile splits evenly over the threads");
    float4 v[PER_T];
    int nr;

    __device__ __forceinline__ void load(const float *src, size_t rs, int nrows, int tid) {
        nr = nrows;
        const unsigned urs = (unsigned)rs;
        if (nrows == 32) {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                const int e = tid + i * NT, r = e / CPR, c = (e % CPR) * 4;
                v[i] = ld4_at(src, 4u * ((unsigned)r * urs + c));
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER_T; ++i) {
                const int e = tid + i * NT, r = min(e / CPR, nrows - 1), c = (e % CPR) * 4;
                v[i] = ld4_at(src, 4u * ((unsigned)r * urs + c));
            }
        }
    }
    __device__ __forceinline__ void store_rows(float *lds, int ld, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_T; ++i) {
            const int e = tid + i * NT, r = e / CPR, c = (e % CPR) * 4;
            bmb::st4(lds + r * ld + c, r < nr ? v[i] : zero4());
        }
    }
};

// Work item of workgroup `bid` among nblk tiles x BH heads.
// longest_hi: tile nblk-1 is the longest (forward, dQ); otherwise tile 0 is
// (dK/dV). Items are handed out longest first. With SNAKE, the k-th round of
// `cus` workgroups on one XCD walks the longest-first list in alternating
// direction, so that when a whole grid is resident at once every CU of the XCD
// receives a near-equal sum of work instead of the longest items together.
template <bool SNAKE>
__device__ __forceinline__ void work_item(int bid, int BH, int nblk, bool longest_hi, int cus,
                                          int &blk, int &bh) {
    int rank;
    if (BH % NXCD == 0) {
        const int xcd = bid % NXCD, hpx = BH / NXCD;
        int w = bid / NXCD;
        if (SNAKE) {
            const int per_xcd = hpx * nblk, round = w / cus, pos = w % cus;
            const int n = min(cus, per_xcd - round * cus);
            w = round * cus + ((round & 1) ? n - 1 - pos : pos);
        }
        rank = w / hpx;
        bh = (w % hpx) * NXCD + xcd;
    } else {
        rank = bid / BH;
        bh = bid % BH;
    }
    blk = longest_hi ? nblk - 1 - rank : rank;
}

// Per-head work list of a backward pass, built on the host and passed by
// value: item i streams tiles [t0[i], t1[i]) of block blk[i]; split[i] marks
// one of the two halves of a long block, whose results are added atomically
// into rows zeroed beforehand (exactly two addends onto zero, so the sum does
// not depend on their order). Items are listed longest first.
constexpr int MAX_ITEMS = 192;
struct Items {
    int n;
    unsigned short blk[MAX_ITEMS], t0[MAX_ITEMS], t1[MAX_ITEMS];
    unsigned char split[MAX_ITEMS];
};

// ------------------------------------------------------------------ forward

template <int HS>
struct FwdSmem {
    static constexpr int LDK = HS + 4;   // K rows (keys), 128-bit reads
    static constexpr int LDV = 32 + 4;   // V^T rows (head dims), 128-bit reads
    static constexpr int BUF = 32 * LDK + HS * LDV;
    static constexpr size_t BYTES = 2 * (size_t)BUF * sizeof(float);
};

// One 32-key tile of the forward for this wave's 32 queries: S^T = K Q^T in
// log2 units, online-softmax update of (m, l, O^T), O^T += V^T P^T.
// ks: K tile rows (stride LDK); vs: V^T rows (stride LDV). MASK: keys past
// the query (diagonal tile) or past T (ragged tile) get -inf.
template <int HS, bool MASK>
__device__ __forceinline__ void fwd_tile(const float *ks, const float *vs, const float (&qf)[HS / 2],
                                         f32x16 (&o)[HS / 32], float &m, float &l, int kb,
                                         int qi, int T, int l32, int hf) {
    constexpr int HH = HS / 2, DT = HS / 32;
    using S = FwdSmem<HS>;
    f32x16 s = zero16();
    const float *krow = ks + l32 * S::LDK + hf * HH;
#pragma unroll
    for (int j = 0; j < HH; j += 4) {
        const float4 kv = bmb::ld4(krow + j);
        s = mfma(kv.x, qf[j + 0], s);
        s = mfma(kv.y, qf[j + 1], s);
        s = mfma(kv.z, qf[j + 2], s);
        s = mfma(kv.w, qf[j + 3], s);
    }
    if (MASK) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kb + res_row(r, hf);
            s[r] = ((key > qi) | (key >= T)) ? -INFINITY : s[r];
        }
    }
    float mb = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mb = fmaxf(mb, s[r]);
    const float mn = fmaxf(m, pair_max(mb));  // finite: key 0 is live for every query
    const float alpha = exp2_hw(m - mn);      // 0 on the first tile
    float p[16], ls = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        p[r] = exp2_hw(s[r] - mn);
        ls += p[r];
    }
    l = l * alpha + ls;  // this half's keys; halves are combined at the end
    m = mn;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= alpha;

    // O^T += V^T P^T. Step st pairs key res_row(st, hf) of this half; keys
    // 8j + 4hf + 0..3 are 4 consecutive floats of a V^T row.
#pragma unroll
    for (int d = 0; d < DT; ++d) {
        const float *vrow = vs + (d * 32 + l32) * S::LDV + 4 * hf;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 vv = bmb::ld4(vrow + 8 * j);
            o[d] = mfma(vv.x, p[4 * j + 0], o[d]);
            o[d] = mfma(vv.y, p[4 * j + 1], o[d]);
            o[d] = mfma(vv.z, p[4 * j + 2], o[d]);
            o[d] = mfma(vv.w, p[4 * j + 3], o[d]);
        }
    }
}

template <int HS, int WPB, bool SNAKE, int MINW>
__global__ __launch_bounds__(WPB * 64) __attribute__((amdgpu_waves_per_eu(MINW))) void
flash_fwd_k(float *__restrict__ out, float *__restrict__ lse, const float *__restrict__ qkv,
            int T, int NH, int BH, float qscale, int cus, const unsigned *__restrict__ order) {
    constexpr int NT = WPB * 64, QB = 32 * WPB, HH = HS / 2, DT = HS / 32;
    using S = FwdSmem<HS>;
    extern __shared__ float smem[];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int nqb = (T + QB - 1) / QB;
    int qb, bh;
    if (order != nullptr) {  // host-planned placement (fwd_order)
        const unsigned e = order[blockIdx.x];
        qb = (int)(e & 0xffffu);
        bh = (int)(e >> 16);
    } else {
        work_item<SNAKE>(blockIdx.x, BH, nqb, true, cus, qb, bh);
    }
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;

    const int q0w = qb * QB + wave * 32;  // this wave's first query
    const int qi = q0w + l32;
    const bool active = q0w < T;

    // B operand of S^T = K Q^T: lane holds q[qi][hf*HH + st] * qscale.
    float qf[HH];
#pragma unroll
    for (int j = 0; j < HH; j += 4) {
        const float4 v = qi < T ? bmb::ld4(base + (size_t)qi * rs + hf * HH + j) : zero4();
        qf[j + 0] = v.x * qscale; qf[j + 1] = v.y * qscale;
        qf[j + 2] = v.z * qscale; qf[j + 3] = v.w * qscale;
    }

    f32x16 o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = zero16();
    float m = -INFINITY, l = 0.0f;

    const int kend = min(T, qb * QB + QB);
    const int nkt = (kend + 31) / 32;
    const int my_nkt = active ? (min(T, q0w + 32) + 31) / 32 : 0;

    Tile32U<HS, NT> kt;
    TileT32U<HS, NT> vt;
    kt.load(base + C, rs, min(32, T), tid);
    vt.load(base + 2 * C, rs, min(32, T), tid);
    kt.store_rows(smem, S::LDK, tid);
    vt.store(smem + 32 * S::LDK, S::LDV, tid);
    __syncthreads();

    for (int t = 0; t < nkt; ++t) {
        const int kb = t * 32;
        const bool more = t + 1 < nkt;
        {
            // next tile; the last one is loaded again at the end so that no
            // load sits behind a branch
            const int kn = min(kb + 32, (nkt - 1) * 32), nr = min(32, T - kn);
            kt.load(base + (size_t)kn * rs + C, rs, nr, tid);
            vt.load(base + (size_t)kn * rs + 2 * C, rs, nr, tid);
        }
        if (t < my_nkt) {
            const float *ks = smem + (t & 1) * S::BUF;
            // Only the diagonal and a ragged last tile need the mask; each
            // variant is straight-line code the scheduler can interleave.
            if (kb + 32 > q0w || kb + 32 > T)
                fwd_tile<HS, true>(ks, ks + 32 * S::LDK, qf, o, m, l, kb, qi, T, l32, hf);
            else
                fwd_tile<HS, false>(ks, ks + 32 * S::LDK, qf, o, m, l, kb, qi, T, l32, hf);
        }
        if (more) {
            float *nb = smem + ((t + 1) & 1) * S::BUF;
            kt.store_rows(nb, S::LDK, tid);
            vt.store(nb + 32 * S::LDK, S::LDV, tid);
        }
        __syncthreads();
    }

    l = pair_sum(l);
    if (active && qi < T) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float *dst = out + ((size_t)b * T + qi) * C + h * HS;
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                bmb::st4(dst + d * 32 + 8 * r4 + 4 * hf,
                         make_float4(o[d][4 * r4 + 0] * inv, o[d][4 * r4 + 1] * inv,
                                     o[d][4 * r4 + 2] * inv, o[d][4 * r4 + 3] * inv));
        if (hf == 0) lse[(size_t)bh * T + qi] = m * LN2 + logf(l);
    }
}

// ------------------------------------------------------- forward, fp16x3
//
// The same online-softmax forward with every contraction on
// v_mfma_f32_32x32x16_f16, whose fp16 products are exact in its fp32
// accumulator. Each fp32 operand x is carried as two fp16 values,
// hi = fp16(x) and lo = fp16(x - hi) (x - hi is exact in fp32), and a product
// a*b is accumulated as ah*bh + ah*bl + al*bh: what is dropped is al*bl and
// the rounding of lo, each within 2^-22 |a b|, so a score or output element
// carries about the error of an fp32 dot product (the fp32-MFMA forward above
// rounds only its accumulation). That is 16 fp32 products per lane in 3
// instructions of 32 cycles instead of 8 instructions of 64.
//
// Range. fp16 holds magnitudes up to 65504 and keeps 11 significant bits only
// down to 2^-14, so nothing is converted unscaled: each query row, and each
// 32-key tile of K and of V, is multiplied by a power of two 2^(14 - e), e the
// binary exponent of its largest magnitude, which puts that magnitude in
// [2^13, 2^14). Powers of two are exact and are undone exactly: a score is
// s' * 2^(eq - 14) * 2^(ek - 14), one factor per lane and tile that rides on
// the exp2 fma. For P V the tile factor of V moves onto P relative to the
// largest V exponent E the wave has seen: P'' = P * 2^(ev - E + 7). P itself
// may reach 2^8 (below), so P'' stays under 2^15, and when E grows the
// accumulated O is rescaled by 2^(E_old - E_new). Any finite fp32 input range
// works; within a tile, values far below the tile's largest lose digits only
// below 2^-36 of it.
//
// Softmax. The running max m is only moved when a query's tile max exceeds it
// by more than 8 (log2 units) or E grows -- a wave-uniform decision -- so the
// O rescale is skipped on almost every tile; the probabilities exp2(s - m) of
// the other tiles are then at most 2^8, and l and O carry the same stale m.
//
// Staging. The workgroup splits each K/V tile once into fp16 hi/lo planes in
// LDS. The tile exponents need a maximum over the whole workgroup's loads, so
// tile X is loaded into registers during tile X-3, its per-wave maxima are
// published in LDS at the end of tile X-2, and it is split into the third of
// three LDS buffers at the start of tile X-1: one barrier per tile, and more
// than a tile's work between each load and its first use.
//
// Register layout. For 32x32x16 lane l supplies A[m = l%32][k = 8*(l/32)+i]
// and B[k = 8*(l/32)+i][n = l%32], i = 0..7 (8 fp16 = 4 VGPRs), and gets the
// result as in 32x32x2 (res_row). The score tile is again S^T = K Q^T; step st
// of the head-dim contraction pairs lane half hf with dims hf*HS/2 + 8*st + i,
// so a lane's query operand is HS/2 contiguous dims, as in the fp32 forward.
// P^T then needs no data movement: registers 8*ks .. 8*ks+7 of a lane hold
// keys 16*ks + {0..3, 8..11} (half 0) or 16*ks + {4..7, 12..15} (half 1), and
// that set is the k index of step ks of O^T += V^T P^T; V^T rows in LDS store
// each 16-key group in the order 0-3, 8-11, 4-7, 12-15 so that those 8 keys
// are one 128-bit read.

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma_h(h8 a, h8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// x minus the fp16 value in half HIGH of the packed word h, in one
// v_fma_mix_f32 (fp16 operand read directly; exact, as x - fp16(x) is
// representable).
template <bool HIGH>
__device__ __forceinline__ float minus_half(unsigned h, float x) {
    float r;
    if (HIGH)
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "=v"(r) : "v"(h), "v"(x));
    else
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,0]"
            : "=v"(r) : "v"(h), "v"(x));
    return r;
}

// (a, b) -> hi = (fp16(a), fp16(b)), lo = (fp16(a - hi.a), fp16(b - hi.b)),
// each pair packed in one 32-bit word (round to nearest even).
__device__ __forceinline__ void split2(float a, float b, unsigned &hi, unsigned &lo) {
    hi = __builtin_bit_cast(unsigned, __builtin_convertvector((f2v){a, b}, h2v));
    const f2v r = {minus_half<false>(hi, a), minus_half<true>(hi, b)};
    lo = __builtin_bit_cast(unsigned, __builtin_convertvector(r, h2v));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

// Max over the wave of a non-negative float (compared as integers, which
// orders non-negative floats): DPP quad, half-row and row reductions, then the
// four row results.
__device__ __forceinline__ float wave_max_nonneg(float x) {
    int v = __float_as_int(x);
    v = max(v, dpp_i<0xb1>(v));   // quad_perm [1,0,3,2]
    v = max(v, dpp_i<0x4e>(v));   // quad_perm [2,3,0,1]
    v = max(v, dpp_i<0x141>(v));  // row_half_mirror
    v = max(v, dpp_i<0x140>(v));  // row_mirror
    const int m = max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
                      max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
    return __int_as_float(m);
}

__device__ __forceinline__ float absmax4(float4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Binary exponent e of a maximum m > 0 (2^(e-1) <= m < 2^e); NOEXP for m = 0.
constexpr int NOEXP = -1000;
__device__ __forceinline__ int max_exp(float m) {
    return m > 0.0f ? __builtin_amdgcn_frexp_expf(m) : NOEXP;
}


constexpr float SOFTMAX_SLACK = 8.0f;  // log2 units a stale running max may lag

template <int HS>
struct FwdSmemH {
    static constexpr int LDK = HS + 8;  // halves per K row (+16 bytes)
    static constexpr int LDV = 32 + 8;  // halves per V^T row (+16 bytes)
    static constexpr int KPLANE = 32 * LDK * 2;  // bytes
    static constexpr int VPLANE = HS * LDV * 2;
    static constexpr int OFF_KL = KPLANE, OFF_VH = 2 * KPLANE, OFF_VL = 2 * KPLANE + VPLANE;
    static constexpr int OFF_EXP = 2 * KPLANE + 2 * VPLANE;  // int2 (ek, ev) of the tile
    static constexpr int BUF = OFF_EXP + 16;
    static constexpr int NBUF = 3;
    static constexpr size_t SLOTS = NBUF * (size_t)BUF;  // 2 x (2 x waves) floats follow
    static size_t bytes(int waves) { return SLOTS + 2 * 2 * waves * sizeof(float); }
};

// Half-index of key kk (0..31) in a V^T row: 16-key groups in the order 0-3,
// 8-11, 4-7, 12-15 (the k order of the P fragment taken from the score
// accumulators).
__device__ __forceinline__ int vt_pos(int kk) {
    return (kk & 16) | (((kk >> 2) & 1) << 3) | (((kk >> 3) & 1) << 2) | (kk & 3);
}

// LDS slot of transposed row d (a head dim) of a V^T, Q^T, dO^T or K^T plane
// of 80-byte rows: rows permute within each group of four by d bits 4 and 5.
// gfx950 serves a 128-bit LDS read 16 lanes per cycle, in the lane groups
// {0-3, 12-15, 20-27} and {4-11, 16-19, 28-31} (and the same over lanes
// 32-63), and a 32-bit write 32 consecutive lanes per cycle (measured with
// SQ_LDS_BANK_CONFLICT). The 80-byte stride alone spreads the 16 rows of a
// read group over 16 distinct 16-byte slots; the stores of one phase write
// rows d = 4j + i (j = 0..15 at head size 64) at one or two key words, which
// the stride alone folds onto four 16-bank blocks, and the permutation
// spreads over all 64 banks. Reads and stores are then conflict-free at head
// sizes 32 and 64; at 128 a store phase writes 32 rows at one key word, at
// least two lanes per bank for any row placement.
__device__ __forceinline__ int t_row(int d) { return d ^ ((d >> 5) & 1) ^ (((d >> 4) & 1) << 1); }

// A 32-key tile of K and V for the fp16x3 forward in flight from global memory
// to LDS. Thread tid holds float4 column c = tid % G (G = HS/4 lanes per row) of
// keys 2p and 2p+1 of K and of V, p = tid / G + pass * (NT / G). Rows past
// nrows re-read row nrows-1.
template <int HS, int NT>
struct KVTileH {
    static constexpr int G = HS / 4;
    static constexpr int PAIRS = NT / G;
    static constexpr int PASSES = (16 + PAIRS - 1) / PAIRS;
    static constexpr int NW = NT / 64;
    float4 k[PASSES][2], v[PASSES][2];

    __device__ __forceinline__ static bool has(int p) { return PAIRS * PASSES <= 16 || p < 16; }

    __device__ __forceinline__ void load(const float *kb, const float *vb, size_t rs, int nrows,
                                         int tid) {
        const unsigned urs = (unsigned)rs;
        const int c = (tid % G) * 4;
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int p = tid / G + ps * PAIRS;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (!has(p)) {
                    k[ps][j] = v[ps][j] = zero4();
                    continue;
                }
                const unsigned o = 4u * ((unsigned)min(2 * p + j, nrows - 1) * urs + c);
                k[ps][j] = ld4_at(kb, o);
                v[ps][j] = ld4_at(vb, o);
            }
        }
    }

    // Publish this wave's max |K| and max |V| in slot[wave] and
    // slot[NW + wave] (every lane stores the same uniform value). Rows past
    // the end repeat row nrows-1, so they do not change the maxima; their
    // keys are masked (probability 0), so they need no zeroing either.
    __device__ __forceinline__ void publish(float *slot, int tid) const {
        float ak = 0.0f, av = 0.0f;
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                ak = fmaxf(ak, absmax4(k[ps][j]));
                av = fmaxf(av, absmax4(v[ps][j]));
            }
        ak = wave_max_nonneg(ak);
        av = wave_max_nonneg(av);
        slot[tid >> 6] = ak;
        slot[NW + (tid >> 6)] = av;
    }

    // Scale by the tile's powers of two, split and store (slot: the published
    // maxima of this tile).
    __device__ __forceinline__ void store(char *buf, const float *slot, int tid) const {
        using S = FwdSmemH<HS>;
        float mk = slot[0], mv = slot[NW];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            mk = fmaxf(mk, slot[w]);
            mv = fmaxf(mv, slot[NW + w]);
        }
        const int ek = max_exp(mk), ev = max_exp(mv);
        const int sk = ek == NOEXP ? 0 : 14 - ek, sv = ev == NOEXP ? 0 : 14 - ev;
        const int c = (tid % G) * 4;
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int p = tid / G + ps * PAIRS;
            if (!has(p)) continue;
            float4 vs[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float4 kx = k[ps][j], vx = v[ps][j];
                uint2 hi, lo;
                split2(ldexpf(kx.x, sk), ldexpf(kx.y, sk), hi.x, lo.x);
                split2(ldexpf(kx.z, sk), ldexpf(kx.w, sk), hi.y, lo.y);
                // K row 2p+j, dims c..c+3: one 64-bit store per plane.
                const int ko = (2 * p + j) * S::LDK * 2 + c * 2;
                *reinterpret_cast<uint2 *>(buf + ko) = hi;
                *reinterpret_cast<uint2 *>(buf + S::OFF_KL + ko) = lo;
                vs[j] = make_float4(ldexpf(vx.x, sv), ldexpf(vx.y, sv), ldexpf(vx.z, sv),
                                    ldexpf(vx.w, sv));
            }
            // V^T rows c..c+3, keys 2p and 2p+1 (adjacent positions): one
            // 32-bit store per row and plane.
            const float a0[4] = {vs[0].x, vs[0].y, vs[0].z, vs[0].w};
            const float a1[4] = {vs[1].x, vs[1].y, vs[1].z, vs[1].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                unsigned hi, lo;
                split2(a0[i], a1[i], hi, lo);
                const int vo = (t_row(c + i) * S::LDV + vt_pos(2 * p)) * 2;
                *reinterpret_cast<unsigned *>(buf + S::OFF_VH + vo) = hi;
                *reinterpret_cast<unsigned *>(buf + S::OFF_VL + vo) = lo;
            }
        }
        // Every thread stores the same (uniform) pair.
        *reinterpret_cast<int2 *>(buf + S::OFF_EXP) = make_int2(ek, ev);
    }
};

// One 32-key tile for this wave's 32 queries (see above). side1 and side2 are
// the workgroup's staging work for later tiles, placed after the score and
// after the P V MFMAs are issued so that their VALU work runs while the
// matrix cores are busy.
template <int HS, bool MASK, typename Side1, typename Side2>
__device__ __forceinline__ void fwd_tile_h(const char *buf, const h8 (&qh)[HS / 16],
                                           const h8 (&ql)[HS / 16], float fq,
                                           f32x16 (&o)[HS / 32], float &m, float &l, int &E,
                                           int kb, int qi, int T, int l32, int hf,
                                           Side1 &&side1, Side2 &&side2) {
    constexpr int NS = HS / 16, DT = HS / 32;
    using S = FwdSmemH<HS>;
    f32x16 s = zero16();
    const char *kh = buf + l32 * S::LDK * 2 + hf * HS;  // dims hf*HS/2 .. (bytes)
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        const h8 ah = *reinterpret_cast<const h8 *>(kh + 16 * st);
        const h8 al = *reinterpret_cast<const h8 *>(kh + S::OFF_KL + 16 * st);
        s = mfma_h(ah, qh[st], s);
        s = mfma_h(ah, ql[st], s);
        s = mfma_h(al, qh[st], s);
    }
    side1();
    const int2 ex = *reinterpret_cast<const int2 *>(buf + S::OFF_EXP);
    const int ek = __builtin_amdgcn_readfirstlane(ex.x), ev = __builtin_amdgcn_readfirstlane(ex.y);
    // Score = s' * fq * 2^(ek - 14); kept > 0 so that a masked -inf stays -inf.
    const float fqk = fmaxf(ldexpf(fq, ek == NOEXP ? 0 : ek - 14), 1.17549435e-38f);
    if (MASK) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kb + res_row(r, hf);
            s[r] = ((key > qi) | (key >= T)) ? -INFINITY : s[r];
        }
    }
    float mb = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mb = fmaxf(mb, s[r]);
    const float mt = pair_max(mb) * fqk;  // finite: key 0 of the tile is live for every query
    if (__builtin_amdgcn_ballot_w64(mt > m + SOFTMAX_SLACK) != 0 || ev > E) {
        const float mn = fmaxf(m, mt);
        const int En = max(E, ev);
        const float alpha = exp2_hw(m - mn);  // 0 on the first tile
        const float ao = ldexpf(alpha, E - En);
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[d][r] *= ao;
        l *= alpha;
        m = mn;
        E = En;
    }
    // P'' = exp2(score - m) * 2^g, g = ev - E + 7 <= 7.
    const int g = ev - E + 7;
    float pv[16], ls = 0.0f;
    if (g >= -80) {
        // 2^g folded into the exponent; l gets the sum back at scale 2^-g
        // (every exp2(score - m) above 2^-40 is still a normal float here).
        const float cm = m - (float)g;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pv[r] = exp2_hw(fmaf(s[r], fqk, -cm));
            ls += pv[r];
        }
        l += ldexpf(ls, -g);
    } else {
        // A tile of V far below the largest seen (or all zero).
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = exp2_hw(fmaf(s[r], fqk, -m));
            ls += p;
            pv[r] = ldexpf(p, g);
        }
        l += ls;
    }

    h8 ph[2], pl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        unsigned hw[4], lw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            split2(pv[8 * ks + 2 * u], pv[8 * ks + 2 * u + 1], hw[u], lw[u]);
        ph[ks] = __builtin_bit_cast(h8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
        pl[ks] = __builtin_bit_cast(h8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
    }
#pragma unroll
    for (int d = 0; d < DT; ++d) {
        const int row = d * 32 + l32;
        const char *vr = buf + S::OFF_VH + t_row(row) * S::LDV * 2;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int off = 32 * ks + 16 * hf;
            const h8 ah = *reinterpret_cast<const h8 *>(vr + off);
            const h8 al = *reinterpret_cast<const h8 *>(vr + (S::OFF_VL - S::OFF_VH) + off);
            o[d] = mfma_h(ah, ph[ks], o[d]);
            o[d] = mfma_h(ah, pl[ks], o[d]);
            o[d] = mfma_h(al, ph[ks], o[d]);
        }
    }
    side2();
}

template <int HS, int WPB, int MINW>
__global__ __launch_bounds__(WPB * 64) __attribute__((amdgpu_waves_per_eu(MINW))) void
flash_fwd_h_k(float *__restrict__ out, float *__restrict__ lse, const float *__restrict__ qkv,
              int T, int NH, int BH, float qscale, int cus, const unsigned *__restrict__ order) {
    constexpr int NT = WPB * 64, QB = 32 * WPB, HH = HS / 2, NS = HS / 16, DT = HS / 32;
    using S = FwdSmemH<HS>;
    extern __shared__ float smem[];
    char *sm = reinterpret_cast<char *>(smem);
    float *slots = reinterpret_cast<float *>(sm + S::SLOTS);  // 2 x (2 x WPB)

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int nqb = (T + QB - 1) / QB;
    int qb, bh;
    if (order != nullptr) {
        const unsigned e = order[blockIdx.x];
        qb = (int)(e & 0xffffu);
        bh = (int)(e >> 16);
    } else {
        work_item<true>(blockIdx.x, BH, nqb, true, cus, qb, bh);
    }
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;

    const int q0w = qb * QB + wave * 32;
    const int qi = q0w + l32;
    const bool active = q0w < T;

    // Query operand: dims hf*HH .. hf*HH+HH-1 of query qi, times qscale, scaled
    // by the query's power of two and split.
    h8 qh[NS], ql[NS];
    float fq;
    {
        float qv[HH];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < HH; j += 4) {
            const float4 v = qi < T ? bmb::ld4(base + (size_t)qi * rs + hf * HH + j) : zero4();
            qv[j + 0] = v.x * qscale; qv[j + 1] = v.y * qscale;
            qv[j + 2] = v.z * qscale; qv[j + 3] = v.w * qscale;
            amax = fmaxf(amax, absmax4(make_float4(qv[j], qv[j + 1], qv[j + 2], qv[j + 3])));
        }
        const int eq = max_exp(pair_max(amax));
        fq = eq == NOEXP ? 1.0f : ldexpf(1.0f, eq - 14);  // > 0: masked scores stay -inf
        const int sq = eq == NOEXP ? 0 : 14 - eq;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            unsigned hw[4], lw[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                split2(ldexpf(qv[8 * st + 2 * u], sq), ldexpf(qv[8 * st + 2 * u + 1], sq), hw[u],
                       lw[u]);
            qh[st] = __builtin_bit_cast(h8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
            ql[st] = __builtin_bit_cast(h8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
        }
    }

    f32x16 o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = zero16();
    float m = -INFINITY, l = 0.0f;
    int E = -200;  // below every finite fp32 exponent

    const int kend = min(T, qb * QB + QB);
    const int nkt = (kend + 31) / 32;
    const int my_nkt = active ? (min(T, q0w + 32) + 31) / 32 : 0;
    // Tile tt (clamped to the last one) of K and V.
    auto load_tile = [&](KVTileH<HS, NT> &kv, int tt) {
        const int kn = min(tt, nkt - 1) * 32;
        kv.load(base + (size_t)kn * rs + C, base + (size_t)kn * rs + 2 * C, rs, min(32, T - kn),
                tid);
    };

    // Tile X is loaded during tile X-3, its maxima published during X-2,
    // split into LDS at the start of X-1: two register sets in flight.
    KVTileH<HS, NT> ka, kb2;
    load_tile(ka, 0);
    load_tile(kb2, 1);
    ka.publish(slots, tid);
    __syncthreads();
    ka.store(sm, slots, tid);
    load_tile(ka, 2);
    kb2.publish(slots + 2 * WPB, tid);
    __syncthreads();

    // cur holds tile t+1 (split now, then reloaded with tile t+3); nxt holds
    // tile t+2 (maxima published after this tile's work).
    auto step = [&](int t, KVTileH<HS, NT> &cur, KVTileH<HS, NT> &nxt) {
        const int kb = t * 32;
        // Split tile t+1 and reload its registers with tile t+3; publish the
        // maxima of tile t+2.
        // (Past the last tile these repeat it into buffers nobody reads.)
        auto side1 = [&]() {
            cur.store(sm + ((t + 1) % 3) * S::BUF, slots + ((t + 1) & 1) * 2 * WPB, tid);
            load_tile(cur, t + 3);
        };
        auto side2 = [&]() { nxt.publish(slots + (t & 1) * 2 * WPB, tid); };
        const char *buf = sm + (t % 3) * S::BUF;
        if (t >= my_nkt) {
            side1();
            side2();
        } else if (kb + 32 > q0w || kb + 32 > T) {
            fwd_tile_h<HS, true>(buf, qh, ql, fq, o, m, l, E, kb, qi, T, l32, hf, side1, side2);
        } else {
            fwd_tile_h<HS, false>(buf, qh, ql, fq, o, m, l, E, kb, qi, T, l32, hf, side1, side2);
        }
        __syncthreads();
    };
    for (int t = 0; t < nkt; t += 2) {
        step(t, kb2, ka);
        if (t + 1 < nkt) step(t + 1, ka, kb2);
    }

    l = pair_sum(l);
    if (active && qi < T) {
        // O = O'' * 2^(E - 21) / l: the factors 2^(14 - ev) and 2^(ev - E + 7)
        // carried by the V and P operands.
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const int es = E - 21;
        float *dst = out + ((size_t)b * T + qi) * C + h * HS;
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                bmb::st4(dst + d * 32 + 8 * r4 + 4 * hf,
                         make_float4(ldexpf(o[d][4 * r4 + 0] * inv, es),
                                     ldexpf(o[d][4 * r4 + 1] * inv, es),
                                     ldexpf(o[d][4 * r4 + 2] * inv, es),
                                     ldexpf(o[d][4 * r4 + 3] * inv, es)));
        if (hf == 0) lse[(size_t)bh * T + qi] = m * LN2 + logf(l);
    }
}

// --------------------------------------------------------------- backward

// D[b,h,t] = sum_i dO[b,t,h*hs+i] * O[b,t,h*hs+i] (src/flash.cu:471-487).
// HS/4 lanes per row, one float4 each, reduced with cross-lane xor shuffles.
// Rows are walked in (b, h, t) order so that the D writes are contiguous.
// It also zeroes the dK/dV rows of key blocks (of `blk_rows` rows) whose bit
// is set in kv_zero, and the dQ rows of query blocks set in q_zero, in dqkv:
// the halves of a split backward item accumulate into them.
template <int HS>
__global__ __launch_bounds__(256) void flash_dsum_k(float *__restrict__ dsum,
                                                    const float *__restrict__ dout,
                                                    const float *__restrict__ out,
                                                    int T, int NH, long long rows,
                                                    float *__restrict__ dqkv, int blk_rows,
                                                    unsigned long long kv_zero,
                                                    unsigned long long q_zero) {
    constexpr int LPR = HS / 4;  // lanes per row
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long row = gid / LPR;  // row = (b*NH + h)*T + t
    const int sub = (int)(gid % LPR);
    float s = 0.0f;
    if (row < rows) {
        const int t = (int)(row % T);
        const long long bh = row / T;
        const int h = (int)(bh % NH);
        const long long b = bh / NH;
        const size_t off = ((size_t)b * T + t) * NH * HS + (size_t)h * HS + sub * 4;
        const float4 a = bmb::ld4(dout + off), c = bmb::ld4(out + off);
        s = a.x * c.x + a.y * c.y + a.z * c.z + a.w * c.w;
    }
#pragma unroll
    for (int w = 1; w < LPR; w <<= 1) s += __shfl_xor(s, w);
    if (row < rows && sub == 0) dsum[row] = s;
    if (row < rows && (kv_zero | q_zero) != 0) {
        const int t = (int)(row % T);
        const long long bh = row / T;
        const int h = (int)(bh % NH);
        const long long b = bh / NH;
        const int blk = t / blk_rows;
        const size_t C = (size_t)NH * HS;
        float *r = dqkv + ((size_t)b * T + t) * 3 * C + (size_t)h * HS + sub * 4;
        if (blk < 64 && ((q_zero >> blk) & 1)) bmb::st4(r, zero4());
        if (blk < 64 && ((kv_zero >> blk) & 1)) {
            bmb::st4(r + C, zero4());
            bmb::st4(r + 2 * C, zero4());
        }
    }
}

template <int HS>
struct BwdSmem {
    static constexpr int LD = HS + 4;
    // dK/dV pass: Q rows, dO rows, lse (log2 units), D.
    static constexpr int KV_BUF = 2 * 32 * LD + 64;
    // dQ pass: K rows, V rows.
    static constexpr int Q_BUF = 2 * 32 * LD;
    static constexpr int BUF = KV_BUF > Q_BUF ? KV_BUF : Q_BUF;
    static constexpr size_t BYTES = 2 * (size_t)BUF * sizeof(float);
};

// One 32-query tile of the dK/dV pass for this wave's 32 keys.
// qs: Q rows, then dO rows (stride LD), then lse*log2e and D (32 each).
// S = Q K^T and dP = dO V^T (lane holds key l32, register r holds query
// qb + res_row(r, hf)); P = exp2(S - lse), dS = P (dP - D); then
// dV += P^T dO and dK += dS^T Q, whose step st contracts over query
// res_row(st, hf). MASK: entries with key > query or query >= T are 0.
template <int HS, bool MASK>
__device__ __forceinline__ void kv_tile(const float *qs, const float (&kf)[HS / 2],
                                        const float (&vf)[HS / 2], f32x16 (&dv)[HS / 32],
                                        f32x16 (&dk)[HS / 32], int qb, int key, int T, int l32,
                                        int hf, float *__restrict__ ds_out) {
    constexpr int HH = HS / 2, DT = HS / 32;
    using S = BwdSmem<HS>;
    const float *os = qs + 32 * S::LD;
    const float *ls = qs + 2 * 32 * S::LD;
    f32x16 s = zero16(), dp = zero16();
    const float *qrow = qs + l32 * S::LD + hf * HH;
    const float *orow = os + l32 * S::LD + hf * HH;
#pragma unroll
    for (int j = 0; j < HH; j += 4) {
        const float4 qa = bmb::ld4(qrow + j), da = bmb::ld4(orow + j);
        s = mfma(qa.x, kf[j + 0], s);
        dp = mfma(da.x, vf[j + 0], dp);
        s = mfma(qa.y, kf[j + 1], s);
        dp = mfma(da.y, vf[j + 1], dp);
        s = mfma(qa.z, kf[j + 2], s);
        dp = mfma(da.z, vf[j + 2], dp);
        s = mfma(qa.w, kf[j + 3], s);
        dp = mfma(da.w, vf[j + 3], dp);
    }
    float p[16], ds[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 L4 = bmb::ld4(ls + 8 * j + 4 * hf);
        const float4 D4 = bmb::ld4(ls + 32 + 8 * j + 4 * hf);
        const float Lr[4] = {L4.x, L4.y, L4.z, L4.w};
        const float Dr[4] = {D4.x, D4.y, D4.z, D4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * j + i;
            float x = s[r] - Lr[i];
            if (MASK) {
                const int q = qb + res_row(r, hf);
                x = ((key > q) | (q >= T)) ? -INFINITY : x;  // exp2(-inf) = 0
            }
            p[r] = exp2_hw(x);
            ds[r] = p[r] * (dp[r] - Dr[i]);
        }
    }
    // dS tile for the dQ pass, row-major [query][key]: each half-wave stores
    // 32 consecutive keys of one query row per instruction.
    if (ds_out != nullptr) {
        float *dsl = ds_out + 128 * hf + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) dsl[(8 * (r >> 2) + (r & 3)) * 32] = ds[r];
    }
    const float *osl = os + 4 * hf * S::LD + l32, *qsl = qs + 4 * hf * S::LD + l32;
#pragma unroll
    for (int st = 0; st < 16; ++st) {
        const int qr = 8 * (st >> 2) + (st & 3);
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            dv[d] = mfma(p[st], osl[qr * S::LD + d * 32], dv[d]);
            dk[d] = mfma(ds[st], qsl[qr * S::LD + d * 32], dk[d]);
        }
    }
}

// One 32-key tile of the dQ pass for this wave's 32 queries. ks: K rows, then
// V rows (stride LD). S^T = K Q^T and dP^T = V dO^T (lane holds query l32,
// register r holds key kb + res_row(r, hf)); dS^T = P^T (dP^T - D);
// dQ^T += K^T dS^T, whose step st contracts over key res_row(st, hf).
// MASK: entries with key > query, key >= T or query >= T are 0.
template <int HS, bool MASK>
__device__ __forceinline__ void q_tile(const float *ks, const float (&qf)[HS / 2],
                                       const float (&df)[HS / 2], float L2, float Dq,
                                       f32x16 (&dq)[HS / 32], int kb, int qi, bool qv, int T,
                                       int l32, int hf) {
    constexpr int HH = HS / 2, DT = HS / 32;
    using S = BwdSmem<HS>;
    const float *vs = ks + 32 * S::LD;
    f32x16 s = zero16(), dp = zero16();
    const float *krow = ks + l32 * S::LD + hf * HH;
    const float *vrow = vs + l32 * S::LD + hf * HH;
#pragma unroll
    for (int j = 0; j < HH; j += 4) {
        const float4 ka = bmb::ld4(krow + j), va = bmb::ld4(vrow + j);
        s = mfma(ka.x, qf[j + 0], s);
        dp = mfma(va.x, df[j + 0], dp);
        s = mfma(ka.y, qf[j + 1], s);
        dp = mfma(va.y, df[j + 1], dp);
        s = mfma(ka.z, qf[j + 2], s);
        dp = mfma(va.z, df[j + 2], dp);
        s = mfma(ka.w, qf[j + 3], s);
        dp = mfma(va.w, df[j + 3], dp);
    }
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        float x = s[r] - L2;
        if (MASK) {
            const int kr = kb + res_row(r, hf);
            x = ((kr > qi) | (kr >= T) | !qv) ? -INFINITY : x;
        }
        ds[r] = exp2_hw(x) * (dp[r] - Dq);
    }
#pragma unroll
    for (int st = 0; st < 16; ++st) {
        const int kr = res_row(st, hf);
#pragma unroll
        for (int d = 0; d < DT; ++d)
            dq[d] = mfma(ks[kr * S::LD + d * 32 + l32], ds[st], dq[d]);
    }
}

// dS workspace layout: per head, the 32x32 tiles (query tile qt, key tile
// kt <= qt) of the causal lower triangle, tile (qt, kt) at index
// qt(qt+1)/2 + kt, each row-major [query][key] (the fp16x3 backward stores
// its tiles float4-major instead: kv_tile_h).
__host__ __device__ __forceinline__ size_t ds_tiles_per_head(int T) {
    const size_t n = (size_t)(T + 31) / 32;
    return n * (n + 1) / 2;
}
__device__ __forceinline__ float *ds_tile(float *ws, int bh, int T, int qt, int kt) {
    return ws + ((size_t)bh * ds_tiles_per_head(T) + (size_t)qt * (qt + 1) / 2 + kt) * 1024;
}

// dQ for the WPB*32 queries of query block qblk of head bh from the stored
// dS tiles: dQ = scale * dS K. The workgroup stages each 32-key K tile in LDS
// once; wave w multiplies its own dS tile (A operand: lane holds query l32
// and keys 16*hf + 0..15, read as four 128-bit loads) by it (B operand: K
// rows 16*hf + st). The result D[query][dim] leaves lane l with dim
// d*32 + l32 of query rows res_row(r, hf).
template <int HS, int WPB>
__device__ __forceinline__ void bwd_dq_from_ds_block(float *smem, float *__restrict__ dqkv,
                                                     const float *__restrict__ qkv,
                                                     const float *__restrict__ ws, int T,
                                                     int NH, int qblk, int bh, float scale,
                                                     int tk0, int tk1, bool accumulate) {
    constexpr int NT = WPB * 64, DT = HS / 32;
    using S = BwdSmem<HS>;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;

    const int qtw = qblk * WPB + wave, q0w = qtw * 32;
    const bool active = q0w < T;
    // Key tiles [tk0, tk1), each wave up to its diagonal.
    const int nkt = tk1 - tk0;
    const int my_nkt = active ? max(0, min(tk1, qtw + 1) - tk0) : 0;

    f32x16 dq[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) dq[d] = zero16();

    // dS tiles stream from HBM with little compute per tile, so each wave
    // keeps the next PF dS tiles in flight (a ring of registers whose slot u
    // serves tiles u, u + PF, ...; the loop is unrolled by PF so no slot is
    // ever copied). The K tiles are prefetched PF tiles ahead too: loads
    // complete in issue order, so a wait on a K tile loaded one tile ahead
    // would also wait for every dS tile issued before it. Every load is
    // issued (past its last tile a wave re-reads that tile; a wave with none
    // reads the head's first dS tile) so the compiler's wait counts are exact.
    constexpr int PF = 3, LDT = 36;
    const int last = max(my_nkt - 1, 0);
    const float *wsw = ws + ((size_t)bh * ds_tiles_per_head(T) +
                             (my_nkt > 0 ? (size_t)qtw * (qtw + 1) / 2 + tk0 : 0)) * 1024;
    const unsigned lane_off = 4u * (l32 * 32 + 16 * hf);
    auto ktile = [&](int j) { return base + (size_t)(tk0 + j) * 32 * rs + C; };
    auto krows = [&](int j) { return min(32, T - (tk0 + j) * 32); };
    float4 ring[PF][4];
    TileT32U<HS, NT> kt[PF];
    {
        TileT32U<HS, NT> k0;
        k0.load(ktile(0), rs, krows(0), tid);
#pragma unroll
        for (int j = 0; j < PF; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                ring[j][i] = ld4_at(wsw, 4096u * min(j, last) + lane_off + 16u * i);
            const int kj = min(j + 1, nkt - 1);
            kt[j].load(ktile(kj), rs, krows(kj), tid);
        }
        k0.store(smem, LDT, tid);
    }
    __syncthreads();

    for (int t0 = 0; t0 < nkt; t0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int t = t0 + u;
            if (t >= nkt) break;
            if (t < my_nkt) {
                const float *ks = smem + (t & 1) * S::BUF + l32 * LDT + 16 * hf;
                float4 kb[DT][4];
#pragma unroll
                for (int d = 0; d < DT; ++d)
#pragma unroll
                    for (int i = 0; i < 4; ++i) kb[d][i] = bmb::ld4(ks + d * 32 * LDT + 4 * i);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int d = 0; d < DT; ++d) {
                        dq[d] = mfma(ring[u][i].x, kb[d][i].x, dq[d]);
                        dq[d] = mfma(ring[u][i].y, kb[d][i].y, dq[d]);
                        dq[d] = mfma(ring[u][i].z, kb[d][i].z, dq[d]);
                        dq[d] = mfma(ring[u][i].w, kb[d][i].w, dq[d]);
                    }
            }
            const unsigned tn = 4096u * min(t + PF, last);
#pragma unroll
            for (int i = 0; i < 4; ++i) ring[u][i] = ld4_at(wsw, tn + lane_off + 16u * i);
            if (t + 1 < nkt) kt[u].store(smem + ((t + 1) & 1) * S::BUF, LDT, tid);
            const int kj = min(t + 1 + PF, nkt - 1);
            kt[u].load(ktile(kj), rs, krows(kj), tid);
            __syncthreads();
        }
    }

    if (!active) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int q = q0w + res_row(r, hf);
        if (q >= T) continue;
        float *dst = dqkv + ((size_t)b * T + q) * rs + h * HS;
        if (accumulate) {
#pragma unroll
            for (int d = 0; d < DT; ++d) atomicAdd(dst + d * 32 + l32, dq[d][r] * scale);
        } else {
#pragma unroll
            for (int d = 0; d < DT; ++d) dst[d * 32 + l32] = dq[d][r] * scale;
        }
    }
}

// dK, dV for the WPB*32 keys of key block kblk of head bh.
// ws: when not null, the dS tiles of head bh are stored there for the dQ
// pass (lower-triangular tile order, see ds_tile()).
template <int HS, int WPB>
__device__ __forceinline__ void bwd_kv_block(float *smem, float *__restrict__ dqkv,
                                             const float *__restrict__ qkv,
                                             const float *__restrict__ dout,
                                             const float *__restrict__ lse,
                                             const float *__restrict__ dsum, int T, int NH,
                                             int kblk, int bh, float scale, float qscale,
                                             float *__restrict__ ws, int tq0, int tq1,
                                             bool accumulate) {
    constexpr int NT = WPB * 64, KB = 32 * WPB, HH = HS / 2, DT = HS / 32;
    using S = BwdSmem<HS>;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;
    const float *dob = dout + (size_t)b * T * C + h * HS;
    const float *lrow = lse + (size_t)bh * T;
    const float *drow = dsum + (size_t)bh * T;

    const int k0w = kblk * KB + wave * 32, key = k0w + l32;
    const bool active = k0w < T;
    // B operands of S = Q K^T and dP = dO V^T: K (log2-scaled) and V rows.
    float kf[HH], vf[HH];
#pragma unroll
    for (int j = 0; j < HH; j += 4) {
        float4 kv = zero4(), vv = zero4();
        if (key < T) {
            kv = bmb::ld4(base + (size_t)key * rs + C + hf * HH + j);
            vv = bmb::ld4(base + (size_t)key * rs + 2 * C + hf * HH + j);
        }
        kf[j + 0] = kv.x * qscale; kf[j + 1] = kv.y * qscale;
        kf[j + 2] = kv.z * qscale; kf[j + 3] = kv.w * qscale;
        vf[j + 0] = vv.x; vf[j + 1] = vv.y; vf[j + 2] = vv.z; vf[j + 3] = vv.w;
    }

    f32x16 dv[DT], dk[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) { dv[d] = zero16(); dk[d] = zero16(); }

    // Query tiles [tq0, tq1); a wave skips the tiles before its diagonal.
    const int q_start = tq0 * 32;
    const int nqt = tq1 - tq0;
    Tile32<HS, NT> qt, ot;
    // Staging of lse (tid < 32, scaled to log2 units when stored) and D
    // (32 <= tid < 64). Nothing is computed on a loaded value before the
    // store, so the loads stay in flight across the compute of a tile.
    float lv = 0.0f;
    auto load_tile = [&](int qb) {
        const int nr = min(32, T - qb);
        qt.load(base + (size_t)qb * rs, rs, nr, tid);
        ot.load(dob + (size_t)qb * C, C, nr, tid);
        if (tid < 64) {
            const int q = qb + (tid & 31);
            lv = q < T ? (tid < 32 ? lrow[q] : drow[q]) : 0.0f;
        }
    };
    auto store_tile = [&](float *buf) {
        qt.store_rows(buf, S::LD, tid);
        ot.store_rows(buf + 32 * S::LD, S::LD, tid);
        if (tid < 64) buf[2 * 32 * S::LD + tid] = tid < 32 ? lv * LOG2E : lv;
    };
    load_tile(q_start);
    store_tile(smem);
    __syncthreads();

    for (int t = 0; t < nqt; ++t) {
        const int qb = q_start + 32 * t;
        const bool more = t + 1 < nqt;
        if (more) load_tile(qb + 32);
        if (active && qb >= k0w) {
            const float *qs = smem + (t & 1) * S::BUF;
            float *dso = ws ? ds_tile(ws, bh, T, qb >> 5, k0w >> 5) : nullptr;
            if (qb == k0w || qb + 32 > T || k0w + 32 > T)  // diagonal or ragged
                kv_tile<HS, true>(qs, kf, vf, dv, dk, qb, key, T, l32, hf, dso);
            else
                kv_tile<HS, false>(qs, kf, vf, dv, dk, qb, key, T, l32, hf, dso);
        }
        if (more) store_tile(smem + ((t + 1) & 1) * S::BUF);
        __syncthreads();
    }

    if (!active) return;
    // Lane holds column d*32 + l32 of key rows k0w + res_row(r, hf).
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int kr = k0w + res_row(r, hf);
        if (kr >= T) continue;
        float *dkp = dqkv + ((size_t)b * T + kr) * rs + C + h * HS;
        if (accumulate) {
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                atomicAdd(dkp + d * 32 + l32, dk[d][r] * scale);
                atomicAdd(dkp + C + d * 32 + l32, dv[d][r]);
            }
        } else {
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                dkp[d * 32 + l32] = dk[d][r] * scale;
                dkp[C + d * 32 + l32] = dv[d][r];
            }
        }
    }
}

// dQ for the WPB*32 queries of query block qblk of head bh.
template <int HS, int WPB>
__device__ __forceinline__ void bwd_q_block(float *smem, float *__restrict__ dqkv,
                                            const float *__restrict__ qkv,
                                            const float *__restrict__ dout,
                                            const float *__restrict__ lse,
                                            const float *__restrict__ dsum, int T, int NH,
                                            int qblk, int bh, float scale, float qscale) {
    constexpr int NT = WPB * 64, QB = 32 * WPB, HH = HS / 2, DT = HS / 32;
    using S = BwdSmem<HS>;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;
    const float *dob = dout + (size_t)b * T * C + h * HS;

    const int q0w = qblk * QB + wave * 32, qi = q0w + l32;
    const bool active = q0w < T, qv = qi < T;
    // B operands of S^T = K Q^T and dP^T = V dO^T: this lane's query row.
    float qf[HH], df[HH];
#pragma unroll
    for (int j = 0; j < HH; j += 4) {
        float4 qa = zero4(), da = zero4();
        if (qv) {
            qa = bmb::ld4(base + (size_t)qi * rs + hf * HH + j);
            da = bmb::ld4(dob + (size_t)qi * C + hf * HH + j);
        }
        qf[j + 0] = qa.x * qscale; qf[j + 1] = qa.y * qscale;
        qf[j + 2] = qa.z * qscale; qf[j + 3] = qa.w * qscale;
        df[j + 0] = da.x; df[j + 1] = da.y; df[j + 2] = da.z; df[j + 3] = da.w;
    }
    const float L2 = qv ? lse[(size_t)bh * T + qi] * LOG2E : 0.0f;
    const float Dq = qv ? dsum[(size_t)bh * T + qi] : 0.0f;

    f32x16 dq[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) dq[d] = zero16();

    const int kend = min(T, qblk * QB + QB);
    const int nkt = (kend + 31) / 32;
    const int my_nkt = active ? (min(T, q0w + 32) + 31) / 32 : 0;
    Tile32<HS, NT> kt, vt;
    kt.load(base + C, rs, min(32, T), tid);
    vt.load(base + 2 * C, rs, min(32, T), tid);
    kt.store_rows(smem, S::LD, tid);
    vt.store_rows(smem + 32 * S::LD, S::LD, tid);
    __syncthreads();

    for (int t = 0; t < nkt; ++t) {
        const int kb = 32 * t;
        const bool more = t + 1 < nkt;
        if (more) {
            const int nr = min(32, T - kb - 32);
            kt.load(base + (size_t)(kb + 32) * rs + C, rs, nr, tid);
            vt.load(base + (size_t)(kb + 32) * rs + 2 * C, rs, nr, tid);
        }
        if (t < my_nkt) {
            const float *ks = smem + (t & 1) * S::BUF;
            if (kb + 32 > q0w || kb + 32 > T)  // diagonal or ragged
                q_tile<HS, true>(ks, qf, df, L2, Dq, dq, kb, qi, qv, T, l32, hf);
            else
                q_tile<HS, false>(ks, qf, df, L2, Dq, dq, kb, qi, qv, T, l32, hf);
        }
        if (more) {
            float *nb = smem + ((t + 1) & 1) * S::BUF;
            kt.store_rows(nb, S::LD, tid);
            vt.store_rows(nb + 32 * S::LD, S::LD, tid);
        }
        __syncthreads();
    }

    if (active && qv) {
        float *dst = dqkv + ((size_t)b * T + qi) * rs + h * HS;
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                bmb::st4(dst + d * 32 + 8 * r4 + 4 * hf,
                         make_float4(dq[d][4 * r4 + 0] * scale, dq[d][4 * r4 + 1] * scale,
                                     dq[d][4 * r4 + 2] * scale, dq[d][4 * r4 + 3] * scale));
    }
}

// MODE 0: dK/dV and dQ workgroups interleaved in one launch.
// MODE 1: dK/dV only.  MODE 2: dQ only (recomputing S and dP).
// MODE 3: dK/dV, also storing dS in ws.  MODE 4: dQ from the dS in ws.
template <int HS, int WPB, int MODE, int MINW>
__global__ __launch_bounds__(WPB * 64) __attribute__((amdgpu_waves_per_eu(MINW))) void
flash_bwd_k(float *__restrict__ dqkv, const float *__restrict__ qkv,
            const float *__restrict__ dout, const float *__restrict__ lse,
            const float *__restrict__ dsum, int T, int NH, int BH, float scale, float qscale,
            float *__restrict__ ws, const Items items, const int *__restrict__ sched_off,
            const unsigned *__restrict__ sched_ent) {
    extern __shared__ float smem[];
    constexpr int RB = 32 * WPB;
    const int nblk = (T + RB - 1) / RB;
    int role, bid = blockIdx.x;
    if (MODE == 0) {
        // Pairs (dK/dV item, dQ item) of equal rank in their longest-first
        // orders. With B*NH a multiple of 8 the grid is a multiple of 16 and
        // ids x, x+8, ... (one XCD) keep to one set of heads in both roles.
        if (BH % NXCD == 0) {
            const int xcd = bid % NXCD, w = bid / NXCD;
            role = w & 1;
            bid = (w >> 1) * NXCD + xcd;
        } else {
            role = bid & 1;
            bid >>= 1;
        }
    } else {
        role = MODE == 3 ? 0 : MODE == 4 ? 2 : MODE - 1;
    }
    const int ntiles = (T + 31) / 32;
    int blk, bh;
    if (MODE == 3 || MODE == 4) {
        // Persistent workgroup: the (item, head) entries the host assigned
        // to it, one after the other.
        const int e0 = sched_off[bid], e1 = sched_off[bid + 1];
        for (int e = e0; e < e1; ++e) {
            const unsigned ent = sched_ent[e];
            const int it = (int)(ent & 0xffffu);
            bh = (int)(ent >> 16);
            if (e > e0) __syncthreads();  // the previous item's last LDS reads
            if (MODE == 3)
                bwd_kv_block<HS, WPB>(smem, dqkv, qkv, dout, lse, dsum, T, NH, items.blk[it],
                                      bh, scale, qscale, ws, items.t0[it], items.t1[it],
                                      items.split[it]);
            else
                bwd_dq_from_ds_block<HS, WPB>(smem, dqkv, qkv, ws, T, NH, items.blk[it], bh,
                                              scale, items.t0[it], items.t1[it],
                                              items.split[it]);
        }
    } else if (role == 0) {
        work_item<false>(bid, BH, nblk, false, 0, blk, bh);
        bwd_kv_block<HS, WPB>(smem, dqkv, qkv, dout, lse, dsum, T, NH, blk, bh, scale, qscale,
                              nullptr, blk * WPB, ntiles, false);
    } else {
        work_item<false>(bid, BH, nblk, true, 0, blk, bh);
        bwd_q_block<HS, WPB>(smem, dqkv, qkv, dout, lse, dsum, T, NH, blk, bh, scale, qscale);
    }
}

// ------------------------------------------------------ backward, fp16x3
//
// The default backward on v_mfma_f32_32x32x16_f16 with fp16 hi/lo operands,
// as the fp16x3 forward above: three passes.
//  1. flash_dsum_h_k: D = rowsum(dO * O), and per 32-row tile the largest
//     |Q|, |dO| and |K|, from which the other passes take the tiles'
//     power-of-two scales (no cross-wave reduction there).
//  2. dK/dV (kv_tile_h): per key block, streaming query tiles. S = Q K^T and
//     dP = dO V^T contract over head dims (A: Q / dO rows in LDS, B: the
//     wave's own K / V rows in registers, per-key scaled); P and dS as in the
//     fp32 pass; dV += P^T dO and dK += dS^T Q contract over the tile's 32
//     queries, so Q and dO are also staged transposed (Q^T, dO^T: 8 queries
//     of one dim per 128-bit read, in the slot order of the forward's V^T).
//     P^T and dS^T are already A operands (lanes hold keys). dS is stored, in
//     fp32 with its tile's exponent, for pass 3.
//  3. dQ (bwd_dq_h_block): dQ = scale dS K from the stored tiles (A: dS rows
//     from HBM, split on the fly; B: K^T staged in LDS).
// Scaling: every staged tile and the register operands carry powers of two
// that put their largest magnitude in [2^13, 2^14); accumulators are kept at
// the scale of the largest product exponent seen so far (dV: dO's, dK and dQ:
// dS's times Q's or K's), rescaled when it grows, so no operand exceeds 2^15.

// Per (head, 32-row tile): D rows as flash_dsum_k, and tmax = (max |Q|,
// max |dO|, 0, max |D|). The dK/dV pass fills in the third component, max |K|,
// from the key rows it loads anyway, for the dQ pass. A workgroup is one
// tile: 32 rows x HS/4 lanes.
template <int HS>
__global__ __launch_bounds__(8 * HS) void flash_dsum_h_k(
    float *__restrict__ dsum, float4 *__restrict__ tmax, const float *__restrict__ dout,
    const float *__restrict__ out, const float *__restrict__ qkv, int T, int NH,
    float *__restrict__ dqkv, int blk_rows, unsigned long long kv_zero,
    unsigned long long q_zero) {
    constexpr int LPR = HS / 4, NT = 32 * LPR, NW = NT / 64;
    __shared__ float red[3][NW];  // per wave: max |Q|, max |dO|, max |D|
    const int ntiles = (T + 31) / 32;
    const int tile = blockIdx.x % ntiles, bh = blockIdx.x / ntiles;
    const int tid = threadIdx.x, sub = tid % LPR;
    const int t = tile * 32 + tid / LPR;
    const int h = bh % NH, b = bh / NH;
    const size_t C = (size_t)NH * HS;
    float s = 0.0f, mq = 0.0f, mo = 0.0f;
    if (t < T) {
        const size_t off = ((size_t)b * T + t) * C + (size_t)h * HS + sub * 4;
        const float4 a = bmb::ld4(dout + off), c = bmb::ld4(out + off);
        s = a.x * c.x + a.y * c.y + a.z * c.z + a.w * c.w;
        mo = absmax4(a);
        const float *qr = qkv + ((size_t)b * T + t) * 3 * C + (size_t)h * HS + sub * 4;
        mq = absmax4(bmb::ld4(qr));
    }
#pragma unroll
    for (int w = 1; w < LPR; w <<= 1) s += __shfl_xor(s, w);
    if (t < T && sub == 0) dsum[(size_t)bh * T + t] = s;
    mq = wave_max_nonneg(mq);
    mo = wave_max_nonneg(mo);
    float md = wave_max_nonneg(fabsf(s));
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = mq;
        red[1][tid >> 6] = mo;
        red[2][tid >> 6] = md;
    }
    __syncthreads();
    if (tid == 0) {
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            mq = fmaxf(mq, red[0][w]);
            mo = fmaxf(mo, red[1][w]);
            md = fmaxf(md, red[2][w]);
        }
        tmax[(size_t)bh * ntiles + tile] = make_float4(mq, mo, 0.0f, md);
    }
    if (t < T && (kv_zero | q_zero) != 0) {
        const int blk = t / blk_rows;
        float *r = dqkv + ((size_t)b * T + t) * 3 * C + (size_t)h * HS + sub * 4;
        if (blk < 64 && ((q_zero >> blk) & 1)) bmb::st4(r, zero4());
        if (blk < 64 && ((kv_zero >> blk) & 1)) {
            bmb::st4(r + C, zero4());
            bmb::st4(r + 2 * C, zero4());
        }
    }
}

template <int HS>
struct BwdSmemH {
    static constexpr int LDR = HS + 8;  // halves per row-major row (+16 bytes)
    static constexpr int LDT = 32 + 8;  // halves per transposed row (+16 bytes)
    static constexpr int RPLANE = 32 * LDR * 2;  // bytes
    static constexpr int TPLANE = HS * LDT * 2;
    // dK/dV pass: Q hi/lo, dO hi/lo (row-major), Q^T hi/lo, dO^T hi/lo,
    // lse * log2 e, D (32 floats each).
    static constexpr int OFF_QL = RPLANE, OFF_OH = 2 * RPLANE, OFF_OL = 3 * RPLANE;
    static constexpr int OFF_QTH = 4 * RPLANE, OFF_QTL = OFF_QTH + TPLANE;
    static constexpr int OFF_OTH = OFF_QTH + 2 * TPLANE, OFF_OTL = OFF_QTH + 3 * TPLANE;
    static constexpr int OFF_L = OFF_QTH + 4 * TPLANE, OFF_D = OFF_L + 128;
    static constexpr int KV_BUF = OFF_D + 128;
    // dQ pass: K^T hi/lo.
    static constexpr int Q_BUF = 2 * TPLANE;
    static constexpr size_t KV_BYTES = 2 * (size_t)KV_BUF, Q_BYTES = 2 * (size_t)Q_BUF;
};

// Split a scaled pair and store it in two planes (hi at off, lo at off + dlo).
__device__ __forceinline__ void put2(char *buf, int off, int dlo, float a, float b) {
    unsigned hi, lo;
    split2(a, b, hi, lo);
    *reinterpret_cast<unsigned *>(buf + off) = hi;
    *reinterpret_cast<unsigned *>(buf + off + dlo) = lo;
}

// A 32-row tile of Q and dO (and its lse, D) for the dK/dV pass, in flight to
// LDS. Thread mapping as KVTileH: float4 column c of rows 2p, 2p+1.
template <int HS, int NT>
struct QOTileH {
    static constexpr int G = HS / 4;
    static constexpr int PAIRS = NT / G;
    static constexpr int PASSES = (16 + PAIRS - 1) / PAIRS;
    float4 q[PASSES][2], o[PASSES][2];
    float lv;

    __device__ __forceinline__ static bool has(int p) { return PAIRS * PASSES <= 16 || p < 16; }

    __device__ __forceinline__ void load(const float *qb, const float *ob, size_t rs, size_t os,
                                         int nrows, int tid, const float *lrow,
                                         const float *drow, int q0, int T) {
        const int c = (tid % G) * 4;
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int p = tid / G + ps * PAIRS;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (!has(p)) {
                    q[ps][j] = o[ps][j] = zero4();
                    continue;
                }
                const int r = min(2 * p + j, nrows - 1);
                q[ps][j] = ld4_at(qb, 4u * ((unsigned)r * (unsigned)rs + c));
                o[ps][j] = ld4_at(ob, 4u * ((unsigned)r * (unsigned)os + c));
            }
        }
        if (tid < 64) {
            const int qq = q0 + (tid & 31);
            lv = qq < T ? (tid < 32 ? lrow[qq] : drow[qq]) : 0.0f;
        }
    }

    // Scale by 2^(14 - eq) and 2^(14 - eo), split, store row-major and
    // transposed planes; lse (log2 units) and D.
    __device__ __forceinline__ void store(char *buf, int eq, int eo, int tid) const {
        using S = BwdSmemH<HS>;
        const int sq = eq == NOEXP ? 0 : 14 - eq, so = eo == NOEXP ? 0 : 14 - eo;
        const int c = (tid % G) * 4;
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int p = tid / G + ps * PAIRS;
            if (!has(p)) continue;
            // Row j, dims c..c+3 of Q and dO: hi/lo words (dims c, c+1) and
            // (c+2, c+3), stored row-major; the transposed words (row 0, row 1)
            // of each dim are the same halves regrouped.
            uint2 qh[2], ql[2], oh[2], ol[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float4 a = q[ps][j], bo = o[ps][j];
                split2(ldexpf(a.x, sq), ldexpf(a.y, sq), qh[j].x, ql[j].x);
                split2(ldexpf(a.z, sq), ldexpf(a.w, sq), qh[j].y, ql[j].y);
                split2(ldexpf(bo.x, so), ldexpf(bo.y, so), oh[j].x, ol[j].x);
                split2(ldexpf(bo.z, so), ldexpf(bo.w, so), oh[j].y, ol[j].y);
                const int ro = (2 * p + j) * S::LDR * 2 + c * 2;
                *reinterpret_cast<uint2 *>(buf + ro) = qh[j];
                *reinterpret_cast<uint2 *>(buf + S::OFF_QL + ro) = ql[j];
                *reinterpret_cast<uint2 *>(buf + S::OFF_OH + ro) = oh[j];
                *reinterpret_cast<uint2 *>(buf + S::OFF_OL + ro) = ol[j];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int to = (t_row(c + i) * S::LDT + vt_pos(2 * p)) * 2;
                const unsigned sel = (i & 1) ? 0x07060302u : 0x05040100u;  // high / low halves
                const unsigned w0 = (i < 2) ? 0 : 1;
                auto pick = [&](const uint2 (&x)[2]) {
                    return __builtin_amdgcn_perm(w0 ? x[1].y : x[1].x, w0 ? x[0].y : x[0].x, sel);
                };
                *reinterpret_cast<unsigned *>(buf + S::OFF_QTH + to) = pick(qh);
                *reinterpret_cast<unsigned *>(buf + S::OFF_QTL + to) = pick(ql);
                *reinterpret_cast<unsigned *>(buf + S::OFF_OTH + to) = pick(oh);
                *reinterpret_cast<unsigned *>(buf + S::OFF_OTL + to) = pick(ol);
            }
        }
        if (tid < 64) reinterpret_cast<float *>(buf + S::OFF_L)[tid] = tid < 32 ? lv * LOG2E : lv;
    }
};

// One 32-query tile of the dK/dV pass for this wave's 32 keys (lane = key
// l32; register r of S, dP, P, dS holds query qb + res_row(r, hf)).
// cS, cD: per-lane factors that turn the MFMA sums into log2-unit scores and
// dP. eq, eo: the tile's exponents of Q and dO; eds: an exponent bounding
// |dS| over the tile (|dS| <= |dP| + |D| <= HS max|dO| max|V| + max|D|).
// Ev, Ek: current scales of dv and dk (see the section comment).
template <int HS, bool MASK>
__device__ __forceinline__ void kv_tile_h(const char *buf, const h8 (&kh)[HS / 16],
                                          const h8 (&kl)[HS / 16], const h8 (&vh)[HS / 16],
                                          const h8 (&vl)[HS / 16], float cS, float cD, int eq,
                                          int eo, int eds, f32x16 (&dv)[HS / 32],
                                          f32x16 (&dk)[HS / 32], int &Ev, int &Ek, int qb,
                                          int key, int T, int l32, int hf,
                                          float *__restrict__ ds_out) {
    constexpr int NS = HS / 16, DT = HS / 32;
    using S = BwdSmemH<HS>;
    f32x16 s = zero16(), dp = zero16();
    const char *qr = buf + l32 * S::LDR * 2 + hf * HS;
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        const h8 qh = *reinterpret_cast<const h8 *>(qr + 16 * st);
        const h8 ql = *reinterpret_cast<const h8 *>(qr + S::OFF_QL + 16 * st);
        const h8 oh = *reinterpret_cast<const h8 *>(qr + S::OFF_OH + 16 * st);
        const h8 ol = *reinterpret_cast<const h8 *>(qr + S::OFF_OL + 16 * st);
        s = mfma_h(qh, kh[st], s);
        dp = mfma_h(oh, vh[st], dp);
        s = mfma_h(qh, kl[st], s);
        dp = mfma_h(oh, vl[st], dp);
        s = mfma_h(ql, kh[st], s);
        dp = mfma_h(ol, vh[st], dp);
    }
    // Scales: dv holds sum P dO 2^(29 - Ev), dk holds sum dS Q 2^(14 - Ek).
    // (Uniform; decided while the score MFMAs run.)
    const int nv = max(Ev, eo), nk = max(Ek, eq + eds - 15);
    if (nv > Ev || nk > Ek) {
        const float av = ldexpf(1.0f, Ev - nv), ak = ldexpf(1.0f, Ek - nk);
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                dv[d][r] *= av;
                dk[d][r] *= ak;
            }
        Ev = nv;
        Ek = nk;
    }
    const int gp = eo - Ev + 15, gd = eq - Ek;  // P'' = P 2^gp <= 2^15, dS'' = dS 2^gd <= 2^15
    float p[16], ds[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 L4 = *reinterpret_cast<const float4 *>(buf + S::OFF_L + 4 * (8 * j + 4 * hf));
        const float4 D4 = *reinterpret_cast<const float4 *>(buf + S::OFF_D + 4 * (8 * j + 4 * hf));
        const float Lr[4] = {L4.x, L4.y, L4.z, L4.w};
        const float Dr[4] = {D4.x, D4.y, D4.z, D4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * j + i;
            float x = fmaf(s[r], cS, -Lr[i]);
            if (MASK) {
                const int q = qb + res_row(r, hf);
                x = ((key > q) | (q >= T)) ? -INFINITY : x;  // exp2(-inf) = 0
            }
            p[r] = exp2_hw(x);
            ds[r] = p[r] * fmaf(dp[r], cD, -Dr[i]);
        }
    }
    // dS tile for the dQ pass, float4-major: float4 j = 2 (k >> 4) + ((k >> 2)
    // & 1) of query q and half h = (k >> 3) & 1 holds keys k..k+3 of that row
    // at float (j * 64 + 2 q + h) * 4. Each of the dQ pass's four loads per
    // tile then reads 1 KB contiguous (a wave's 64 lanes, 16 bytes each)
    // instead of 32 bytes from each of 32 rows: that pass ran 11% faster,
    // this one 2-4% slower (its stores write 32-byte pieces of 8 lines per
    // instruction instead of 2 whole rows).
    float *dsl = ds_out + (2 * (l32 >> 4) + ((l32 >> 2) & 1)) * 256 + ((l32 >> 3) & 1) * 4 +
                 (l32 & 3) + 32 * hf;
#pragma unroll
    for (int r = 0; r < 16; ++r) dsl[8 * (8 * (r >> 2) + (r & 3))] = ds[r];
    h8 ph[2], pl[2], dh[2], dl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        unsigned a[4], b[4], c[4], e[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = 8 * ks + 2 * u;
            split2(ldexpf(p[r], gp), ldexpf(p[r + 1], gp), a[u], b[u]);
            split2(ldexpf(ds[r], gd), ldexpf(ds[r + 1], gd), c[u], e[u]);
        }
        ph[ks] = __builtin_bit_cast(h8, make_uint4(a[0], a[1], a[2], a[3]));
        pl[ks] = __builtin_bit_cast(h8, make_uint4(b[0], b[1], b[2], b[3]));
        dh[ks] = __builtin_bit_cast(h8, make_uint4(c[0], c[1], c[2], c[3]));
        dl[ks] = __builtin_bit_cast(h8, make_uint4(e[0], e[1], e[2], e[3]));
    }
    // dV += P^T dO, dK += dS^T Q: B operands dO^T / Q^T rows (dim d*32 + l32).
#pragma unroll
    for (int d = 0; d < DT; ++d) {
        const int row = d * 32 + l32;
        const char *orow = buf + S::OFF_OTH + t_row(row) * S::LDT * 2;
        const char *qrow = buf + S::OFF_QTH + t_row(row) * S::LDT * 2;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int off = 32 * ks + 16 * hf;
            const h8 oh = *reinterpret_cast<const h8 *>(orow + off);
            const h8 ol = *reinterpret_cast<const h8 *>(orow + S::TPLANE + off);
            const h8 qh = *reinterpret_cast<const h8 *>(qrow + off);
            const h8 ql = *reinterpret_cast<const h8 *>(qrow + S::TPLANE + off);
            dv[d] = mfma_h(ph[ks], oh, dv[d]);
            dk[d] = mfma_h(dh[ks], qh, dk[d]);
            dv[d] = mfma_h(ph[ks], ol, dv[d]);
            dk[d] = mfma_h(dh[ks], ql, dk[d]);
            dv[d] = mfma_h(pl[ks], oh, dv[d]);
            dk[d] = mfma_h(dl[ks], qh, dk[d]);
        }
    }
}

// Loads of per-tile values at a uniform address through the vector memory
// path: a scalar load would share its wait counter with LDS accesses, so the
// first LDS wait after it would also wait for its global-memory latency.
template <typename V>
__device__ __forceinline__ V vload(const V *p, size_t i) {
    unsigned lo = (unsigned)i;
    asm volatile("" : "+v"(lo));  // a VGPR index: the compiler emits a vector load
    return p[((i >> 32) << 32) | lo];
}

// Exponent of the largest magnitude of a tile from the dsum pass's maxima
// (component c: 0 Q, 1 dO, 2 K, 3 D).
__device__ __forceinline__ int tile_exp(const float4 *tmax, int bh, int ntiles, int tile, int c) {
    const float4 v = vload(tmax, (size_t)bh * ntiles + tile);
    return max_exp(c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w);
}

// dK, dV for the WPB*32 keys of key block kblk of head bh (fp16x3), storing
// the dS tiles in ws and the exponent bounding each in ws_exp.
template <int HS, int WPB>
__device__ __forceinline__ void bwd_kv_h_block(char *smem, float *__restrict__ dqkv,
                                               const float *__restrict__ qkv,
                                               const float *__restrict__ dout,
                                               const float *__restrict__ lse,
                                               const float *__restrict__ dsum,
                                               float4 *tmax, int T, int NH,
                                               int kblk, int bh, float scale, float qscale,
                                               float *__restrict__ ws, int *__restrict__ ws_exp,
                                               int tq0, int tq1, bool accumulate) {
    constexpr int NT = WPB * 64, KB = 32 * WPB, HH = HS / 2, NS = HS / 16, DT = HS / 32;
    using S = BwdSmemH<HS>;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;
    const float *dob = dout + (size_t)b * T * C + h * HS;
    const float *lrow = lse + (size_t)bh * T;
    const float *drow = dsum + (size_t)bh * T;
    const int ntiles = (T + 31) / 32;

    const int k0w = kblk * KB + wave * 32, key = k0w + l32;
    const bool active = k0w < T;
    // B operands: this lane's key row of K (times qscale) and V, each scaled
    // by the key's power of two and split. evw: exponent of the wave's max |V|.
    h8 kh[NS], kl[NS], vh[NS], vl[NS];
    float fk, fv;
    int evw;
    {
        float kq[HH], vq[HH];
        float ak = 0.0f, av = 0.0f, araw = 0.0f;
#pragma unroll
        for (int j = 0; j < HH; j += 4) {
            float4 kv = zero4(), vv = zero4();
            if (key < T) {
                kv = bmb::ld4(base + (size_t)key * rs + C + hf * HH + j);
                vv = bmb::ld4(base + (size_t)key * rs + 2 * C + hf * HH + j);
            }
            kq[j + 0] = kv.x * qscale; kq[j + 1] = kv.y * qscale;
            kq[j + 2] = kv.z * qscale; kq[j + 3] = kv.w * qscale;
            vq[j + 0] = vv.x; vq[j + 1] = vv.y; vq[j + 2] = vv.z; vq[j + 3] = vv.w;
            ak = fmaxf(ak, absmax4(make_float4(kq[j], kq[j + 1], kq[j + 2], kq[j + 3])));
            av = fmaxf(av, absmax4(vv));
            araw = fmaxf(araw, absmax4(kv));
        }
        evw = max_exp(wave_max_nonneg(av));
        // max |K| of this wave's key tile (its 32 rows): the dQ pass scales
        // its K^T tiles by it. Both halves of a split block store the same
        // value.
        araw = wave_max_nonneg(araw);
        if (active && lane == 0) tmax[(size_t)bh * ntiles + k0w / 32].z = araw;
        const int ek = max_exp(pair_max(ak)), ev = max_exp(pair_max(av));
        fk = ek == NOEXP ? 0.0f : ldexpf(1.0f, ek - 14);
        fv = ev == NOEXP ? 0.0f : ldexpf(1.0f, ev - 14);
        const int sk = ek == NOEXP ? 0 : 14 - ek, sv = ev == NOEXP ? 0 : 14 - ev;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            unsigned a[4], bb[4], c[4], e[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = 8 * st + 2 * u;
                split2(ldexpf(kq[j], sk), ldexpf(kq[j + 1], sk), a[u], bb[u]);
                split2(ldexpf(vq[j], sv), ldexpf(vq[j + 1], sv), c[u], e[u]);
            }
            kh[st] = __builtin_bit_cast(h8, make_uint4(a[0], a[1], a[2], a[3]));
            kl[st] = __builtin_bit_cast(h8, make_uint4(bb[0], bb[1], bb[2], bb[3]));
            vh[st] = __builtin_bit_cast(h8, make_uint4(c[0], c[1], c[2], c[3]));
            vl[st] = __builtin_bit_cast(h8, make_uint4(e[0], e[1], e[2], e[3]));
        }
    }

    f32x16 dv[DT], dk[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) { dv[d] = zero16(); dk[d] = zero16(); }
    int Ev = -2000, Ek = -2000;  // below every product exponent

    const int nqt = tq1 - tq0;
    QOTileH<HS, NT> qo;
    // Tile t (clamped to the last) of Q and dO, and its exponents.
    auto load_tile = [&](int t) {
        const int q0 = (tq0 + min(t, nqt - 1)) * 32;
        qo.load(base + (size_t)q0 * rs, dob + (size_t)q0 * C, rs, C, min(32, T - q0), tid, lrow,
                drow, q0, T);
    };
    // (kept in scalar registers: the values are uniform)
    auto uni = [](float x) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x))); };
    auto tile_max = [&](int t) {
        const float4 v = vload(tmax, (size_t)bh * ntiles + tq0 + min(t, nqt - 1));
        return make_float4(uni(v.x), uni(v.y), uni(v.z), uni(v.w));
    };
    // The tile maxima are read one tile ahead (their loads would otherwise sit
    // right before their first use).
    float4 m_cur = tile_max(0);
    load_tile(0);
    qo.store(smem, max_exp(m_cur.x), max_exp(m_cur.y), tid);
    float4 m_next = tile_max(1);
    __syncthreads();

    for (int t = 0; t < nqt; ++t) {
        const int qb = (tq0 + t) * 32;
        const float4 m_after = tile_max(t + 2);
        if (active && qb >= k0w) {
            const char *buf = smem + (t & 1) * S::KV_BUF;
            const int eq = max_exp(m_cur.x), eo = max_exp(m_cur.y);
            const float cS = ldexpf(fk, eq == NOEXP ? -2000 : eq - 14);
            const float cD = ldexpf(fv, eo == NOEXP ? -2000 : eo - 14);
            // |dS| < HS 2^(eo + evw) + max|D|
            const int eds = (eo == NOEXP || evw == NOEXP)
                                ? max_exp(m_cur.w)
                                : max_exp(ldexpf((float)HS, eo + evw) + m_cur.w);
            const size_t dti = (size_t)bh * ds_tiles_per_head(T) +
                               (size_t)(qb >> 5) * ((qb >> 5) + 1) / 2 + (k0w >> 5);
            float *dso = ws + dti * 1024;
            if (l32 == 0 && hf == 0) ws_exp[dti] = eds;
            if (qb == k0w || qb + 32 > T || k0w + 32 > T)  // diagonal or ragged
                kv_tile_h<HS, true>(buf, kh, kl, vh, vl, cS, cD, eq, eo, eds, dv, dk, Ev, Ek, qb,
                                    key, T, l32, hf, dso);
            else
                kv_tile_h<HS, false>(buf, kh, kl, vh, vl, cS, cD, eq, eo, eds, dv, dk, Ev, Ek,
                                     qb, key, T, l32, hf, dso);
        }
        // Stage tile t+1 (past the last tile: the last again, into the buffer
        // nobody reads). Its loads are issued only now: held across the tile's
        // work their registers would push the kernel past 256 VGPRs, and the
        // other workgroup's wave on the SIMD covers their latency.
        load_tile(t + 1);
        qo.store(smem + ((t + 1) & 1) * S::KV_BUF, max_exp(m_next.x), max_exp(m_next.y), tid);
        m_cur = m_next;
        m_next = m_after;
        __syncthreads();
    }

    if (!active) return;
    const int sv = Ev - 29, sk = Ek - 14;
    float *dkb = dqkv + ((size_t)b * T + k0w) * rs + C + h * HS + l32;
    auto out = [&](auto &&put) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float *dkp = dkb + (size_t)res_row(r, hf) * rs;
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                put(dkp + d * 32, ldexpf(dk[d][r], sk) * scale);
                put(dkp + C + d * 32, ldexpf(dv[d][r], sv));
            }
        }
    };
    if (k0w + 32 <= T) {
        if (accumulate) out([](float *a, float v) { atomicAdd(a, v); });
        else out([](float *a, float v) { *a = v; });
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if (k0w + res_row(r, hf) >= T) continue;
            float *dkp = dkb + (size_t)res_row(r, hf) * rs;
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                const float vk = ldexpf(dk[d][r], sk) * scale, vv = ldexpf(dv[d][r], sv);
                if (accumulate) {
                    atomicAdd(dkp + d * 32, vk);
                    atomicAdd(dkp + C + d * 32, vv);
                } else {
                    dkp[d * 32] = vk;
                    dkp[C + d * 32] = vv;
                }
            }
        }
    }
}

// dQ for the WPB*32 queries of query block qblk of head bh from the stored dS
// tiles (fp16x3): dQ = scale dS K. A operand: dS row l32 of the wave's tile,
// keys 16 ks + 8 hf + 0..7 (step ks), read from HBM PF tiles ahead; B operand:
// K^T rows from LDS (the same keys). dq holds sum dS K 2^(14 - F), F the
// largest exponent of dS times K seen so far minus 15.
template <int HS, int WPB>
__device__ __forceinline__ void bwd_dq_h_block(char *smem, float *__restrict__ dqkv,
                                               const float *__restrict__ qkv,
                                               const float *__restrict__ ws,
                                               const int *__restrict__ ws_exp,
                                               const float4 *__restrict__ tmax, int T, int NH,
                                               int qblk, int bh, float scale, int tk0, int tk1,
                                               bool accumulate) {
    constexpr int NT = WPB * 64, DT = HS / 32;
    constexpr int G = HS / 4, PAIRS = NT / G, PASSES = (16 + PAIRS - 1) / PAIRS;
    using S = BwdSmemH<HS>;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;
    const int ntiles = (T + 31) / 32;

    const int qtw = qblk * WPB + wave, q0w = qtw * 32;
    const bool active = q0w < T;
    const int nkt = tk1 - tk0;
    const int my_nkt = active ? max(0, min(tk1, qtw + 1) - tk0) : 0;

    f32x16 dq[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) dq[d] = zero16();
    int F = -2000;

    // dS ring, PF tiles ahead (see bwd_dq_from_ds_block); every load issued.
    constexpr int PF = 3;
    const int last = max(my_nkt - 1, 0);
    const size_t tile0 = (size_t)bh * ds_tiles_per_head(T) +
                         (my_nkt > 0 ? (size_t)qtw * (qtw + 1) / 2 + tk0 : 0);
    const float *wsw = ws + tile0 * 1024;
    const int *wse = ws_exp + tile0;
    // keys 8hf..8hf+7 and 16+8hf..16+8hf+7 of query row l32: float4s 0-3 of
    // (row, half) in the float4-major tile (kv_tile_h), 1 KB apart
    const unsigned lane_off = 16u * (2 * l32 + hf);
    float4 ring[PF][4];
    auto ds_load = [&](float4 (&r)[4], int j) {
        const unsigned tb = 4096u * min(j, last) + lane_off;
        r[0] = ld4_at(wsw, tb);
        r[1] = ld4_at(wsw, tb + 1024u);
        r[2] = ld4_at(wsw, tb + 2048u);
        r[3] = ld4_at(wsw, tb + 3072u);
    };
    // K tile loads one tile ahead: thread holds float4 column c of keys 2p, 2p+1.
    float4 kr[PASSES][2];
    auto k_load = [&](int j) {
        const int k0 = (tk0 + min(j, nkt - 1)) * 32, nr = min(32, T - k0);
        const int c = (tid % G) * 4;
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int p = tid / G + ps * PAIRS;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                if (PAIRS * PASSES > 16 && p >= 16) { kr[ps][jj] = zero4(); continue; }
                const int r = min(2 * p + jj, nr - 1);
                kr[ps][jj] = ld4_at(base + (size_t)k0 * rs + C, 4u * ((unsigned)r * (unsigned)rs + c));
            }
        }
    };
    auto k_store = [&](char *buf, int e) {
        const int sk = e == NOEXP ? 0 : 14 - e;
        const int c = (tid % G) * 4;
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int p = tid / G + ps * PAIRS;
            if (PAIRS * PASSES > 16 && p >= 16) continue;
            const float a0[4] = {kr[ps][0].x, kr[ps][0].y, kr[ps][0].z, kr[ps][0].w};
            const float a1[4] = {kr[ps][1].x, kr[ps][1].y, kr[ps][1].z, kr[ps][1].w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                put2(buf, (t_row(c + i) * S::LDT + 2 * p) * 2, S::TPLANE,
                     ldexpf(a0[i], sk), ldexpf(a1[i], sk));
        }
    };
    // Exponents of K tile j and of the wave's dS tile j, read ahead of use.
    auto kexp = [&](int j) { return tile_exp(tmax, bh, ntiles, tk0 + min(j, nkt - 1), 2); };
    int eds_ring[PF];
    k_load(0);
#pragma unroll
    for (int j = 0; j < PF; ++j) {
        ds_load(ring[j], j);
        eds_ring[j] = vload(wse, (size_t)min(j, last));
    }
    int ek_cur = kexp(0), ek_next = kexp(1);
    k_store(smem, ek_cur);
    k_load(1);
    __syncthreads();

    for (int t0 = 0; t0 < nkt; t0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int t = t0 + u;
            if (t >= nkt) break;
            const int ek_after = kexp(t + 2);
            if (t < my_nkt) {
                const char *buf = smem + (t & 1) * S::Q_BUF;
                const int eds = __builtin_amdgcn_readfirstlane(eds_ring[u]);
                const int ek = ek_cur;
                const int G2 = (eds == NOEXP || ek == NOEXP) ? -2000 : eds + ek - 15;
                if (G2 > F) {
                    const float a = ldexpf(1.0f, F - G2);
#pragma unroll
                    for (int d = 0; d < DT; ++d)
#pragma unroll
                        for (int r = 0; r < 16; ++r) dq[d][r] *= a;
                    F = G2;
                }
                const int sh = ek == NOEXP ? -2000 : ek - F;  // dS'' = dS 2^sh <= 2^15
                const float v[16] = {ring[u][0].x, ring[u][0].y, ring[u][0].z, ring[u][0].w,
                                     ring[u][1].x, ring[u][1].y, ring[u][1].z, ring[u][1].w,
                                     ring[u][2].x, ring[u][2].y, ring[u][2].z, ring[u][2].w,
                                     ring[u][3].x, ring[u][3].y, ring[u][3].z, ring[u][3].w};
                h8 ah[2], al[2];
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    unsigned x[4], y[4];
#pragma unroll
                    for (int w = 0; w < 4; ++w)
                        split2(ldexpf(v[8 * ks + 2 * w], sh), ldexpf(v[8 * ks + 2 * w + 1], sh),
                               x[w], y[w]);
                    ah[ks] = __builtin_bit_cast(h8, make_uint4(x[0], x[1], x[2], x[3]));
                    al[ks] = __builtin_bit_cast(h8, make_uint4(y[0], y[1], y[2], y[3]));
                }
#pragma unroll
                for (int d = 0; d < DT; ++d) {
                    const int row = d * 32 + l32;
                    const char *kt = buf + t_row(row) * S::LDT * 2;
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const int off = 32 * ks + 16 * hf;
                        const h8 bh8 = *reinterpret_cast<const h8 *>(kt + off);
                        const h8 bl8 = *reinterpret_cast<const h8 *>(kt + S::TPLANE + off);
                        dq[d] = mfma_h(ah[ks], bh8, dq[d]);
                        dq[d] = mfma_h(ah[ks], bl8, dq[d]);
                        dq[d] = mfma_h(al[ks], bh8, dq[d]);
                    }
                }
            }
            ds_load(ring[u], t + PF);
            eds_ring[u] = vload(wse, (size_t)min(t + PF, last));
            k_store(smem + ((t + 1) & 1) * S::Q_BUF, ek_next);
            k_load(t + 2);
            ek_cur = ek_next;
            ek_next = ek_after;
            __syncthreads();
        }
    }

    if (!active) return;
    const int sq = F - 14;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int q = q0w + res_row(r, hf);
        if (q >= T) continue;
        float *dst = dqkv + ((size_t)b * T + q) * rs + h * HS;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            const float val = ldexpf(dq[d][r], sq) * scale;
            if (accumulate) atomicAdd(dst + d * 32 + l32, val);
            else dst[d * 32 + l32] = val;
        }
    }
}

// MODE 0: dK/dV (storing dS), MODE 1: dQ from dS; persistent workgroups as
// flash_bwd_k's MODE 3 / 4.
template <int HS, int WPB, int MODE, int MINW>
__global__ __launch_bounds__(WPB * 64) __attribute__((amdgpu_waves_per_eu(MINW))) void
flash_bwd_h_k(float *__restrict__ dqkv, const float *__restrict__ qkv,
              const float *__restrict__ dout, const float *__restrict__ lse,
              const float *__restrict__ dsum, float4 *tmax, int T, int NH,
              float scale, float qscale, float *__restrict__ ws, int *__restrict__ ws_exp,
              const Items items, const int *__restrict__ sched_off,
              const unsigned *__restrict__ sched_ent) {
    extern __shared__ float smem[];
    char *sm = reinterpret_cast<char *>(smem);
    const int bid = blockIdx.x;
    const int e0 = sched_off[bid], e1 = sched_off[bid + 1];
    for (int e = e0; e < e1; ++e) {
        const unsigned ent = sched_ent[e];
        const int it = (int)(ent & 0xffffu);
        const int bh = (int)(ent >> 16);
        if (e > e0) __syncthreads();  // the previous item's last LDS reads
        if (MODE == 0)
            bwd_kv_h_block<HS, WPB>(sm, dqkv, qkv, dout, lse, dsum, tmax, T, NH, items.blk[it],
                                    bh, scale, qscale, ws, ws_exp, items.t0[it], items.t1[it],
                                    items.split[it]);
        else
            bwd_dq_h_block<HS, WPB>(sm, dqkv, qkv, ws, ws_exp, tmax, T, NH, items.blk[it], bh,
                                    scale, items.t0[it], items.t1[it], items.split[it]);
    }
}

// ------------------------------------------------------------- host side

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Per device, read once; concurrent first calls store the same value.
int cus_per_xcd() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 32;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess || cus < NXCD)
            cus = 256;
        v = cus / NXCD;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Forward tile configs. wpb: 32-query waves per workgroup (they share every
// staged K/V tile); snake: snake work order (see work_item); minw: minimum
// waves per SIMD the register allocation must allow; h16: the fp16x3 kernel.
struct FwdCfg {
    const char *name;
    int wpb;
    bool snake;
    int minw;
    bool h16;
};
const FwdCfg FWD_CFGS[] = {
    {"q128/wg lds-kv mfma32 snake", 4, true, 1, false},
    {"q64/wg lds-kv mfma32 snake", 2, true, 1, false},
    {"q128/wg lds-kv mfma32", 4, false, 1, false},
    {"q128/wg lds-kv mfma32 snake 4w/simd", 4, true, 4, false},
    {"q64/wg lds-kv mfma32 snake 4w/simd", 2, true, 4, false},
    {"q128/wg lds-kv fp16x3 mfma16 snake", 4, true, 1, true},
    {"q128/wg lds-kv fp16x3 mfma16 snake 2w/simd", 4, true, 2, true},
};
constexpr int N_FWD = sizeof(FWD_CFGS) / sizeof(FWD_CFGS[0]);
constexpr int FWD_DEFAULT = 5;

// Backward configs. fused: dK/dV and dQ workgroups in one launch; ds_ws:
// the dK/dV pass stores dS in a library-owned workspace and dQ = scale dS K
// is a separate light pass (5 matmul passes instead of 7).
struct BwdCfg {
    const char *name;
    int wpb;
    bool fused;
    int minw;
    bool ds_ws;
    bool h16;  // the fp16x3 kernels (dS stored)
};
const BwdCfg BWD_CFGS[] = {
    {"kv128+q128/wg fused lds mfma32 2w/simd", 4, true, 2, false, false},
    {"kv64+q64/wg fused lds mfma32 2w/simd", 2, true, 2, false, false},
    {"kv128/wg then q128/wg lds mfma32 2w/simd", 4, false, 2, false, false},
    {"kv64/wg then q64/wg lds mfma32 2w/simd", 2, false, 2, false, false},
    {"kv128+q128/wg fused lds mfma32", 4, true, 1, false, false},
    {"kv128/wg storing dS, then dQ=dS.K q128/wg, mfma32 2w/simd", 4, false, 2, true, false},
    {"kv64/wg storing dS, then dQ=dS.K q64/wg, mfma32 2w/simd", 2, false, 2, true, false},
    {"kv128/wg storing dS, then dQ=dS.K q128/wg, mfma32", 4, false, 1, true, false},
    {"kv128/wg storing dS, then dQ=dS.K q128/wg, fp16x3 mfma16 2w/simd", 4, false, 2, true, true},
};
constexpr int N_BWD = sizeof(BWD_CFGS) / sizeof(BWD_CFGS[0]);
constexpr int BWD_DEFAULT = 8;  // the fp16x3 backward

// dS workspace: leased from the library's per-device pool for one backward
// call (workspace.hpp). Both passes that use it are queued on the null stream
// within the call, so a buffer that goes back to the pool is only reused by
// launches that run after them; concurrent calls from several host threads
// hold buffers of their own.

int grid_blocks(int BH, int T, int rows_per_block) {
    return BH * ((T + rows_per_block - 1) / rows_per_block);
}

// Workgroups of `kern` that fit on one CU at once (0 if unknown).
template <typename K>
int wgs_per_cu(K kern, int threads, size_t smem) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, smem) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return per_cu;
}

// Placement of the forward's (query block, head) items when the whole grid is
// resident at once. The dispatcher then puts block b on XCD b % 8 and, within
// an XCD, its local blocks w, w + c, w + 2c, ... (c = CUs per XCD) on the
// same CU, and the workgroups sharing a CU run side by side until the last
// one ends: a CU's run time tracks the sum of its items' work (measured
// correlation 0.93), which the formula order (work_item) left 174-222 key
// tiles per CU at B=8 H=12 T=1024. Here the items of each XCD's heads (the
// same heads per XCD as work_item, for L2 reuse) go longest first to the
// least loaded CU of the XCD that has a free slot; work of an item = the key
// tiles its waves stream. Entry b = (head << 16) | query block. Built once per
// (device, shape, occupancy), uploaded (a few KB) and kept until the process
// ends. nullptr (use the formula order): the grid does not fit at once, B*NH
// is not a multiple of 8 or above 65535, or the upload fails.
std::mutex g_fwd_mu;
std::map<std::tuple<int, int, int, int, int>, unsigned *> g_fwd_order;

const unsigned *fwd_order(int T, int wpb, int BH, int per_cu) {
    const int QB = 32 * wpb, nqb = (T + QB - 1) / QB, cpx = cus_per_xcd();
    if (per_cu <= 0 || BH % NXCD != 0 || BH > 65535 || nqb > 65535) return nullptr;
    const long long nblocks = (long long)nqb * BH;
    if (nblocks > (long long)cpx * NXCD * per_cu) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    const auto key = std::make_tuple(dev, T, wpb, BH, per_cu);
    std::lock_guard<std::mutex> lock(g_fwd_mu);
    const auto found = g_fwd_order.find(key);
    if (found != g_fwd_order.end()) return found->second;

    const int hpx = BH / NXCD, nx = hpx * nqb;  // heads and items per XCD
    std::vector<int> cost(nqb);
    for (int qb = 0; qb < nqb; ++qb) {
        cost[qb] = 0;
        for (int w = 0; w < wpb; ++w) {
            const int q0 = qb * QB + 32 * w;
            if (q0 < T) cost[qb] += (std::min(T, q0 + 32) + 31) / 32;
        }
    }
    std::vector<unsigned> ent((size_t)nblocks);
    std::vector<int> order_items(nx), load(cpx), used(cpx), cap(cpx);
    for (int x = 0; x < NXCD; ++x) {
        for (int i = 0; i < nx; ++i) order_items[i] = i;  // i = qb * hpx + h
        std::stable_sort(order_items.begin(), order_items.end(),
                         [&](int a, int b) { return cost[a / hpx] > cost[b / hpx]; });
        for (int c = 0; c < cpx; ++c) {
            load[c] = used[c] = 0;
            cap[c] = (nx - c + cpx - 1) / cpx;  // local blocks w < nx with w % cpx == c
        }
        for (const int i : order_items) {
            const int qb = i / hpx, h = i % hpx;
            int best = -1;
            for (int c = 0; c < cpx; ++c)
                if (used[c] < cap[c] && (best < 0 || load[c] < load[best])) best = c;
            const int w = best + used[best] * cpx;
            ++used[best];
            load[best] += cost[qb];
            const int bh = h * NXCD + x;
            ent[(size_t)w * NXCD + x] = ((unsigned)bh << 16) | (unsigned)qb;
        }
    }
    unsigned *d = nullptr;
    if (hipMalloc(&d, ent.size() * sizeof(unsigned)) != hipSuccess ||
        hipMemcpy(d, ent.data(), ent.size() * sizeof(unsigned), hipMemcpyHostToDevice) !=
            hipSuccess) {
        (void)hipGetLastError();
        if (d) (void)hipFree(d);
        return nullptr;
    }
    g_fwd_order[key] = d;
    return d;
}

template <int HS, int WPB, bool SNAKE, int MINW>
void run_fwd(float *out, float *lse, const float *qkv, int B, int T, int NH) {
    const int BH = B * NH;
    const float qscale = (1.0f / sqrtf((float)HS)) * LOG2E;
    const size_t smem = FwdSmem<HS>::BYTES;
    auto kern = flash_fwd_k<HS, WPB, SNAKE, MINW>;
    bmb::allow_smem(kern, smem);
    const unsigned *order =
        SNAKE ? fwd_order(T, WPB, BH, wgs_per_cu(kern, WPB * 64, smem)) : nullptr;
    bmb::launch(kern, dim3(grid_blocks(BH, T, 32 * WPB)), dim3(WPB * 64), smem, nullptr, out,
                lse, qkv, T, NH, BH, qscale, cus_per_xcd(), order);
}

template <int HS, int WPB, int MINW>
void run_fwd_h(float *out, float *lse, const float *qkv, int B, int T, int NH) {
    const int BH = B * NH;
    const float qscale = (1.0f / sqrtf((float)HS)) * LOG2E;
    const size_t smem = FwdSmemH<HS>::bytes(WPB);
    auto kern = flash_fwd_h_k<HS, WPB, MINW>;
    bmb::allow_smem(kern, smem);
    const unsigned *order = fwd_order(T, WPB, BH, wgs_per_cu(kern, WPB * 64, smem));
    bmb::launch(kern, dim3(grid_blocks(BH, T, 32 * WPB)), dim3(WPB * 64), smem, nullptr, out,
                lse, qkv, T, NH, BH, qscale, cus_per_xcd(), order);
}

template <int HS>
bool fwd_hs(int cfg, float *out, float *lse, const float *qkv, int B, int T, int NH) {
    const FwdCfg &c = FWD_CFGS[cfg];
    if (c.h16) {
        if (c.wpb == 4 && c.minw == 1) run_fwd_h<HS, 4, 1>(out, lse, qkv, B, T, NH);
        else if (c.wpb == 4 && c.minw == 2) run_fwd_h<HS, 4, 2>(out, lse, qkv, B, T, NH);
        else return false;
        return true;
    }
#define BMB_FWD(W, S, M)                                                       \
    if (c.wpb == W && c.snake == S && c.minw == M) {                           \
        run_fwd<HS, W, S, M>(out, lse, qkv, B, T, NH);                         \
        return true;                                                           \
    }
    BMB_FWD(4, true, 1)
    BMB_FWD(2, true, 1)
    BMB_FWD(4, false, 1)
    BMB_FWD(4, true, 4)
    BMB_FWD(2, true, 4)
#undef BMB_FWD
    return false;
}

// Per-head work list of the dK/dV pass (kv = true: block = WPB*32 keys,
// streaming query tiles from its diagonal to the end) or of the dQ-from-dS
// pass (block = WPB*32 queries, streaming key tiles from 0 to its diagonal).
// A block longer than `target` tiles is split into two halves; the bit of a
// split block is set in *zero_mask. Returns false if T has more blocks than
// the list (or the zero mask) can hold.
bool build_items(bool kv, int T, int wpb, int target, Items &it, unsigned long long &zero_mask) {
    const int ntiles = (T + 31) / 32;
    const int nblk = (ntiles + wpb - 1) / wpb;
    zero_mask = 0;
    if (nblk > MAX_ITEMS) return false;
    struct Item { int blk, t0, t1, split; };
    std::vector<Item> v;
    for (int k = 0; k < nblk; ++k) {
        const int t0 = kv ? k * wpb : 0, t1 = kv ? ntiles : std::min(ntiles, (k + 1) * wpb);
        const int len = t1 - t0;
        if (nblk <= 64 && len > target && len >= 4 && (int)v.size() + 2 <= MAX_ITEMS) {
            const int mid = t0 + len / 2;
            v.push_back({k, t0, mid, 1});
            v.push_back({k, mid, t1, 1});
            zero_mask |= 1ULL << k;
        } else {
            v.push_back({k, t0, t1, 0});
        }
    }
    std::stable_sort(v.begin(), v.end(),
                     [](const Item &a, const Item &b) { return a.t1 - a.t0 > b.t1 - b.t0; });
    it.n = (int)v.size();
    for (int i = 0; i < it.n; ++i) {
        it.blk[i] = (unsigned short)v[i].blk;
        it.t0[i] = (unsigned short)v[i].t0;
        it.t1[i] = (unsigned short)v[i].t1;
        it.split[i] = (unsigned char)v[i].split;
    }
    return true;
}

// Relative cost of an item: 2 per streamed tile, plus 1 for each tile that
// holds a wave's diagonal (masked, and some waves of the workgroup idle),
// plus 2 for a split half (its results are atomic adds).
int item_cost(const Items &it, int i, int wpb) {
    const int d0 = it.blk[i] * wpb, d1 = d0 + wpb;
    const int diag = std::max(0, std::min((int)it.t1[i], d1) - std::max((int)it.t0[i], d0));
    return 2 * (it.t1[i] - it.t0[i]) + diag + 2 * it.split[i];
}

// Longest-first placement of weighted entries onto `nbins` bins, each entry
// going to the least loaded bin (lowest index on ties). Entries are (cost,
// payload) and are given in the order they should be considered.
void lpt(const std::vector<std::pair<int, unsigned>> &entries, int nbins,
         std::vector<std::vector<std::pair<int, unsigned>>> &bins, std::vector<long long> &load) {
    bins.assign(nbins, {});
    load.assign(nbins, 0);
    std::vector<std::pair<long long, int>> heap;
    for (int b = 0; b < nbins; ++b) heap.push_back({0, b});
    auto cmp = [](const std::pair<long long, int> &x, const std::pair<long long, int> &y) {
        return x > y;
    };
    std::make_heap(heap.begin(), heap.end(), cmp);
    for (const auto &e : entries) {
        std::pop_heap(heap.begin(), heap.end(), cmp);
        auto &top = heap.back();
        bins[top.second].push_back(e);
        top.first += e.first;
        load[top.second] = top.first;
        std::push_heap(heap.begin(), heap.end(), cmp);
    }
}

// Static schedule of a backward pass over persistent workgroups, all
// resident at once: per_cu of them on each of the ncu CUs of every XCD.
// Workgroup g runs entries [off[g], off[g+1]) of ent, each (item index |
// bh << 16). With B*NH a multiple of 8, workgroup g runs on XCD g % 8 (the
// hardware hands ids round robin to the XCDs) and takes only heads bh = g
// (mod 8), so a head's tiles are read through one L2. Within an XCD the
// workgroups with local index w = g / 8 and w + ncu, w + 2 ncu, ... share a CU
// (the dispatcher fills each CU once before it places a second workgroup on
// any, as measured on MI355X), and the workgroups of a CU share its SIMDs,
// so the run time is set by the work per CU: the (item, head) pairs are
// placed longest first onto the least loaded CU, then each CU's pairs onto
// its workgroups the same way. Returns the modelled run time: per CU the
// larger of (its work / per_cu) and (its longest workgroup / 1.5), a
// workgroup left alone on a CU running about 1.5x faster.
double plan_schedule(const Items &it, int wpb, int BH, int ncu, int per_cu, std::vector<int> &off,
                     std::vector<unsigned> &ent) {
    const int nx = (BH % NXCD == 0) ? NXCD : 1;
    if (nx == 1) ncu *= NXCD;  // one group: the CUs of all XCDs, ids still dealt round robin
    // no more workgroups per CU than there are entries to fill them
    const long long per_group = (long long)it.n * (BH / nx);
    per_cu = (int)std::max(1LL, std::min<long long>(per_cu, (per_group + ncu - 1) / ncu));
    const int wg_per_x = ncu * per_cu;
    std::vector<std::vector<unsigned>> wg_list((size_t)wg_per_x * nx);
    double model = 0.0;
    for (int x = 0; x < nx; ++x) {
        std::vector<std::pair<int, unsigned>> entries;
        for (int i = 0; i < it.n; ++i)
            for (int h = x; h < BH; h += nx)
                entries.push_back({item_cost(it, i, wpb), (unsigned)i | ((unsigned)h << 16)});
        std::stable_sort(entries.begin(), entries.end(),
                         [](const std::pair<int, unsigned> &a, const std::pair<int, unsigned> &b) {
                             return a.first > b.first;
                         });
        std::vector<std::vector<std::pair<int, unsigned>>> cu_bins, wg_bins;
        std::vector<long long> cu_load, wg_load;
        lpt(entries, ncu, cu_bins, cu_load);
        for (int c = 0; c < ncu; ++c) {
            lpt(cu_bins[c], per_cu, wg_bins, wg_load);
            long long wmax = 0;
            for (int k = 0; k < per_cu; ++k) {
                wmax = std::max(wmax, wg_load[k]);
                const int w = c + k * ncu;  // local index of the k-th workgroup on CU c
                auto &dst = wg_list[(size_t)w * nx + x];
                for (const auto &e : wg_bins[k]) dst.push_back(e.second);
            }
            model = std::max(model, std::max((double)cu_load[c] / per_cu, wmax / 1.5));
        }
    }
    off.assign(1, 0);
    ent.clear();
    for (const auto &l : wg_list) {
        ent.insert(ent.end(), l.begin(), l.end());
        off.push_back((int)ent.size());
    }
    return model;
}

struct Sched {
    Items items;
    unsigned long long zero_mask = 0;
    int wgs = 0;                  // workgroups to launch
    int *off = nullptr;           // device, wgs + 1 entries
    unsigned *ent = nullptr;      // device
};

// Schedules are built once per (device, pass, shape, resident workgroups) and
// kept until the process ends.
std::mutex g_sched_mu;
std::map<std::tuple<int, int, int, int, int, int>, Sched> g_sched;

// Work list and persistent schedule of a backward pass. The split target is
// the one (of the block lengths minus one, or none) whose schedule has the
// smallest modelled run time; ties keep fewer splits. per_cu = 0 (occupancy
// unknown) gives one item per workgroup. Returns false (the caller then tries another
// config) if BH > 65535 (the entry encoding) or the schedule cannot be
// uploaded.
bool get_sched(bool kv, int T, int wpb, int BH, int per_cu, Sched &out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    const auto key = std::make_tuple(dev, (int)kv, T, wpb, BH, per_cu);
    std::lock_guard<std::mutex> lock(g_sched_mu);
    auto found = g_sched.find(key);
    if (found != g_sched.end()) {
        out = found->second;
        return true;
    }
    if (BH > 65535) return false;
    // occupancy unknown: as many workgroups as (item, head) pairs
    if (per_cu <= 0) per_cu = 1 << 20;
    Sched s;
    {
        const int ntiles = (T + 31) / 32, nblk = (ntiles + wpb - 1) / wpb;
        std::vector<int> targets = {ntiles + 1};
        for (int k = 0; k < nblk; ++k) {
            const int len = kv ? ntiles - k * wpb : std::min(ntiles, (k + 1) * wpb);
            if (len >= 4) targets.push_back(len - 1);
        }
        std::sort(targets.begin(), targets.end(), std::greater<int>());
        targets.erase(std::unique(targets.begin(), targets.end()), targets.end());
        double best = -1.0;
        std::vector<int> off, best_off;
        std::vector<unsigned> ent, best_ent;
        for (int target : targets) {
            Items it;
            unsigned long long zm = 0;
            if (!build_items(kv, T, wpb, target, it, zm)) continue;
            const double mk = plan_schedule(it, wpb, BH, cus_per_xcd(), per_cu, off, ent);
            if (best < 0 || mk < best) {
                best = mk;
                s.items = it;
                s.zero_mask = zm;
                best_off.swap(off);
                best_ent.swap(ent);
            }
        }
        if (best >= 0) {
            int *doff = nullptr;
            unsigned *dent = nullptr;
            const size_t nent = std::max<size_t>(1, best_ent.size());
            if (hipMalloc(&doff, best_off.size() * sizeof(int)) == hipSuccess &&
                hipMalloc(&dent, nent * sizeof(unsigned)) == hipSuccess &&
                hipMemcpy(doff, best_off.data(), best_off.size() * sizeof(int),
                          hipMemcpyHostToDevice) == hipSuccess &&
                (best_ent.empty() ||
                 hipMemcpy(dent, best_ent.data(), best_ent.size() * sizeof(unsigned),
                           hipMemcpyHostToDevice) == hipSuccess)) {
                s.wgs = (int)best_off.size() - 1;
                s.off = doff;
                s.ent = dent;
            } else {
                (void)hipGetLastError();
                if (doff) (void)hipFree(doff);
                if (dent) (void)hipFree(dent);
            }
        }
    }
    if (s.wgs == 0) return false;
    g_sched[key] = s;
    out = s;
    return true;
}

// Kernel of a backward launch mode, with its LDS size allowed.
template <int HS, int WPB, int MODE, int MINW>
auto bwd_kernel() {
    auto kern = flash_bwd_k<HS, WPB, MODE, MINW>;
    bmb::allow_smem(kern, BwdSmem<HS>::BYTES);
    return kern;
}

template <int HS, int WPB, int MODE, int MINW>
void run_bwd_mode(float *dqkv, const float *dout, const float *qkv, const float *lse,
                  const float *dsum, int B, int T, int NH, float *ws, const Sched &sc) {
    const int BH = B * NH;
    const int blocks = (MODE == 3 || MODE == 4) ? sc.wgs
                                                : grid_blocks(BH, T, 32 * WPB) * (MODE == 0 ? 2 : 1);
    const float scale = 1.0f / sqrtf((float)HS);
    auto kern = bwd_kernel<HS, WPB, MODE, MINW>();
    bmb::launch(kern, dim3(blocks), dim3(WPB * 64), BwdSmem<HS>::BYTES, nullptr, dqkv, qkv,
                dout, lse, dsum, T, NH, BH, scale, scale * LOG2E, ws, sc.items,
                (const int *)sc.off, (const unsigned *)sc.ent);
}

template <int HS, int WPB, int MINW>
bool run_bwd(const BwdCfg &c, float *dqkv, float *dsum, const float *dout, const float *qkv,
             const float *out, const float *lse, int B, int T, int NH) {
    float *ws = nullptr;
    std::optional<bmb::ScratchLease> lease;
    Sched kv_sc, q_sc;
    kv_sc.items.n = q_sc.items.n = 0;
    const int BH = B * NH;
    if (c.ds_ws) {
        const int threads = WPB * 64;
        const size_t smem = BwdSmem<HS>::BYTES;
        if (!get_sched(true, T, WPB, BH,
                       wgs_per_cu(bwd_kernel<HS, WPB, 3, MINW>(), threads, smem), kv_sc) ||
            !get_sched(false, T, WPB, BH,
                       wgs_per_cu(bwd_kernel<HS, WPB, 4, MINW>(), threads, smem), q_sc))
            return false;
        lease.emplace(bmb::SCRATCH_FLASH_DS,
                      (size_t)B * NH * ds_tiles_per_head(T) * 1024 * sizeof(float));
        ws = static_cast<float *>(lease->get());
        if (ws == nullptr) return false;  // no workspace: the caller tries another config
    }
    const unsigned long long kv_zero = kv_sc.zero_mask, q_zero = q_sc.zero_mask;
    const long long rows = (long long)B * T * NH;
    const long long threads = rows * (HS / 4);
    bmb::launch(flash_dsum_k<HS>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                nullptr, dsum, dout, out, T, NH, rows, dqkv, 32 * WPB, kv_zero, q_zero);
    if (c.ds_ws) {
        run_bwd_mode<HS, WPB, 3, MINW>(dqkv, dout, qkv, lse, dsum, B, T, NH, ws, kv_sc);
        run_bwd_mode<HS, WPB, 4, MINW>(dqkv, dout, qkv, lse, dsum, B, T, NH, ws, q_sc);
    } else if (c.fused) {
        run_bwd_mode<HS, WPB, 0, MINW>(dqkv, dout, qkv, lse, dsum, B, T, NH, nullptr, kv_sc);
    } else {
        run_bwd_mode<HS, WPB, 1, MINW>(dqkv, dout, qkv, lse, dsum, B, T, NH, nullptr, kv_sc);
        run_bwd_mode<HS, WPB, 2, MINW>(dqkv, dout, qkv, lse, dsum, B, T, NH, nullptr, kv_sc);
    }
    return true;
}

// The fp16x3 backward: dsum + tile maxima, dK/dV storing dS, dQ from dS.
// Workspace (one lease): the dS tiles (fp32), their exponents, the tile
// maxima.
template <int HS, int WPB, int MINW>
bool run_bwd_h(float *dqkv, float *dsum, const float *dout, const float *qkv, const float *out,
               const float *lse, int B, int T, int NH) {
    using S = BwdSmemH<HS>;
    const int BH = B * NH, threads = WPB * 64, ntiles = (T + 31) / 32;
    auto kkv = flash_bwd_h_k<HS, WPB, 0, MINW>;
    auto kq = flash_bwd_h_k<HS, WPB, 1, MINW>;
    bmb::allow_smem(kkv, S::KV_BYTES);
    bmb::allow_smem(kq, S::Q_BYTES);
    Sched kv_sc, q_sc;
    if (!get_sched(true, T, WPB, BH, wgs_per_cu(kkv, threads, S::KV_BYTES), kv_sc) ||
        !get_sched(false, T, WPB, BH, wgs_per_cu(kq, threads, S::Q_BYTES), q_sc))
        return false;
    const size_t nds = (size_t)BH * ds_tiles_per_head(T);
    const size_t off_exp = nds * 4096, off_max = off_exp + ((nds * 4 + 15) & ~(size_t)15);
    std::optional<bmb::ScratchLease> lease;
    lease.emplace(bmb::SCRATCH_FLASH_DS, off_max + (size_t)BH * ntiles * sizeof(float4));
    char *w = static_cast<char *>(lease->get());
    if (w == nullptr) return false;  // no workspace: the caller tries another config
    float *ws = reinterpret_cast<float *>(w);
    int *ws_exp = reinterpret_cast<int *>(w + off_exp);
    float4 *tmax = reinterpret_cast<float4 *>(w + off_max);
    bmb::launch(flash_dsum_h_k<HS>, dim3((unsigned)(BH * ntiles)), dim3(8 * HS), 0, nullptr,
                dsum, tmax, dout, out, qkv, T, NH, dqkv, 32 * WPB, kv_sc.zero_mask,
                q_sc.zero_mask);
    const float scale = 1.0f / sqrtf((float)HS);
    bmb::launch(kkv, dim3(kv_sc.wgs), dim3(threads), S::KV_BYTES, nullptr, dqkv, qkv, dout, lse,
                dsum, tmax, T, NH, scale, scale * LOG2E, ws, ws_exp,
                kv_sc.items, (const int *)kv_sc.off, (const unsigned *)kv_sc.ent);
    bmb::launch(kq, dim3(q_sc.wgs), dim3(threads), S::Q_BYTES, nullptr, dqkv, qkv, dout, lse,
                dsum, tmax, T, NH, scale, scale * LOG2E, ws, ws_exp,
                q_sc.items, (const int *)q_sc.off, (const unsigned *)q_sc.ent);
    return true;
}

template <int HS>
bool bwd_hs(int cfg, float *dqkv, float *dsum, const float *dout, const float *qkv,
            const float *out, const float *lse, int B, int T, int NH) {
    const BwdCfg &c = BWD_CFGS[cfg];
    if (c.h16) {
        // (head size 128 needs the whole register file: one wave per SIMD)
        if (c.wpb == 4 && c.minw == 2)
            return run_bwd_h<HS, 4, HS == 128 ? 1 : 2>(dqkv, dsum, dout, qkv, out, lse, B, T, NH);
        return false;
    }
#define BMB_BWD(W, M)                                                              \
    if (c.wpb == W && c.minw == M)                                                 \
        return run_bwd<HS, W, M>(c, dqkv, dsum, dout, qkv, out, lse, B, T, NH);
    BMB_BWD(4, 2)
    BMB_BWD(2, 2)
    BMB_BWD(4, 1)
#undef BMB_BWD
    return false;
}

// Shape legality shared by forward and backward: a supported head size.
bool shape_ok(int B, int T, int C, int NH, int &hs) {
    if (B < 0 || T < 0 || NH <= 0 || C <= 0 || C % NH != 0) return false;
    // Tile loads address a 32-row tile of qkv by 32-bit byte offsets.
    if (32LL * 3 * C * (long long)sizeof(float) >= (1LL << 31)) return false;
    hs = C / NH;
    return hs == 32 || hs == 64 || hs == 128;
}

}  // namespace

extern "C" {

int flash_num_configs(void) { return N_FWD; }

const char *flash_config_name(int cfg) {
    return (cfg >= 0 && cfg < N_FWD) ? FWD_CFGS[cfg].name : "?";
}

int flash_default_config(void) { return FWD_DEFAULT; }

bool flash_attention_forward_cfg(int cfg, float *out, float *lse, const float *qkv, int B,
                                 int T, int C, int NH) {
    int hs;
    if (cfg < 0 || cfg >= N_FWD || !shape_ok(B, T, C, NH, hs)) return false;
    // Every row segment is a run of 128-bit loads and stores.
    if (!aligned16(qkv) || !aligned16(out)) return false;
    if (B == 0 || T == 0) return true;
    switch (hs) {
    case 32: return fwd_hs<32>(cfg, out, lse, qkv, B, T, NH);
    case 64: return fwd_hs<64>(cfg, out, lse, qkv, B, T, NH);
    case 128: return fwd_hs<128>(cfg, out, lse, qkv, B, T, NH);
    default: return false;
    }
}

void flash_attention_forward(float *out, float *lse, const float *qkv, int B, int T, int C,
                             int NH) {
    if (flash_attention_forward_cfg(flash_default_config(), out, lse, qkv, B, T, C, NH)) return;
    for (int cfg = 0; cfg < N_FWD; ++cfg)
        if (flash_attention_forward_cfg(cfg, out, lse, qkv, B, T, C, NH)) return;
    fprintf(stderr, "flash: no tile config for head size %d (C=%d, NH=%d)\n",
            NH > 0 ? C / NH : -1, C, NH);
    exit(1);
}

int flash_num_bwd_configs(void) { return N_BWD; }

const char *flash_bwd_config_name(int cfg) {
    return (cfg >= 0 && cfg < N_BWD) ? BWD_CFGS[cfg].name : "?";
}

int flash_default_bwd_config(void) { return BWD_DEFAULT; }

bool flash_attention_backward_cfg(int cfg, float *dqkv, float *dsum, const float *dout,
                                  const float *qkv, const float *out, const float *lse, int B,
                                  int T, int C, int NH) {
    int hs;
    if (cfg < 0 || cfg >= N_BWD || !shape_ok(B, T, C, NH, hs)) return false;
    if (!aligned16(qkv) || !aligned16(dqkv) || !aligned16(dout) || !aligned16(out))
        return false;
    if (B == 0 || T == 0) return true;
    switch (hs) {
    case 32: return bwd_hs<32>(cfg, dqkv, dsum, dout, qkv, out, lse, B, T, NH);
    case 64: return bwd_hs<64>(cfg, dqkv, dsum, dout, qkv, out, lse, B, T, NH);
    case 128: return bwd_hs<128>(cfg, dqkv, dsum, dout, qkv, out, lse, B, T, NH);
    default: return false;
    }
}

void flash_attention_backward(float *dqkv, float *dsum, const float *dout, const float *qkv,
                              const float *out, const float *lse, int B, int T, int C, int NH) {
    if (flash_attention_backward_cfg(flash_default_bwd_config(), dqkv, dsum, dout, qkv, out,
                                     lse, B, T, C, NH))
        return;
    for (int cfg = 0; cfg < N_BWD; ++cfg)
        if (flash_attention_backward_cfg(cfg, dqkv, dsum, dout, qkv, out, lse, B, T, C, NH))
            return;
    fprintf(stderr, "flash: no backward tile config for head size %d (C=%d, NH=%d)\n",
            NH > 0 ? C / NH : -1, C, NH);
    exit(1);
}

}  // extern "C"
