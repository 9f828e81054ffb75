// Fused causal attention, forward and backward, for gfx950 -- the
// counterpart of bare-metal-bard's src/flash.cu (API: src/flash.h).
//
// Design: one wave64 owns a 32-row tile and keeps everything in registers.
//
// Every contraction is a chain of v_mfma_f32_32x32x2_f32 (fp32 in, exact fp32
// products, fp32 accumulate). In that instruction lane l supplies
// A[m = l%32][kk = l/32] and B[kk = l/32][n = l%32], and the 32x32 result
// leaves lane l holding column n = l%32, register r holding row
// 8*(r/4) + 4*(l/32) + r%4. Two consequences drive the whole layout:
//
//  * If the score tile is computed TRANSPOSED, S^T = K Q^T (keys x queries),
//    each lane holds one query's scores for 16 of the 32 keys and its partner
//    lane (l ^ 32) the other 16. Row max / row sum are then an in-register
//    reduction plus one cross-half exchange, the online-softmax rescale
//    touches only the lane's own O^T registers, and the probabilities are
//    ALREADY in the B-operand layout of O^T += V^T P^T: MFMA step s takes
//    register s, i.e. key 8*(s/4) + 4*(l/32) + s%4. No LDS round trip, no
//    barrier. (The reference stages P through shared memory, flash.cu:262-276.)
//  * The contraction over head dims uses dd = (l/32) * hs/2 + s for step s, so
//    each lane's q/k/v/dO fragment is hs/2 contiguous floats: 128-bit loads.
//
// Scores are kept in log2 units: q is pre-multiplied by scale*log2(e), so
// p = exp2(s - m) uses the hardware v_exp_f32. lse is stored in natural-log
// units (lse = m*ln2 + ln l), exactly the quantity src/flash.cu:309 stores,
// so forward and backward stay interchangeable with the reference's.
//
// Causality is a loop bound (a query tile visits key tiles up to its
// diagonal; a key tile visits query tiles from its diagonal on); only the
// diagonal tile and a ragged last tile are masked. Tiles are handed out
// longest-first so the causal triangle does not leave a long tail.
//
// Backward (src/flash.cu:434-466 for the maths): a dsum kernel
// D = rowsum(dO * O), then ONE launch in which half of the waves compute dK/dV
// for a 32-key tile (S = Q K^T so that P^T and dS^T are in A-operand layout
// for dV += P^T dO and dK += dS^T Q) and the other half compute dQ for a
// 32-query tile (S^T layout as in the forward, dQ^T += K^T dS^T). dQ and dK/dV
// are disjoint slices of dqkv, so no atomics are needed and both halves share
// the machine: the long dK/dV tiles are interleaved with the long dQ tiles.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "common.hpp"
#include "../../include/flash.h"
#include "launch.hpp"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

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

__device__ __forceinline__ float xhalf(float v) {  // value of lane l ^ 32
    return __shfl_xor(v, 32);
}

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

// Loads N contiguous floats (N % 4 == 0, 16-byte aligned) times `mul`, or
// zeros when !valid.
template <int N>
__device__ __forceinline__ void load_frag(float (&f)[N], const float *p,
                                          bool valid, float mul) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (valid) v = bmb::ld4(p + i);
        f[i + 0] = v.x * mul; f[i + 1] = v.y * mul;
        f[i + 2] = v.z * mul; f[i + 3] = v.w * mul;
    }
}

// ------------------------------------------------------------------ forward
//
// Wave g of the launch owns query tile qt of head bh. qkv row t of (b, h):
// q at +0, k at +C, v at +2C, each hs floats (src/flash.cu:151-152).
template <int HS, int WPB>
__global__ __launch_bounds__(WPB * 64) void flash_fwd_k(
    float *__restrict__ out, float *__restrict__ lse,
    const float *__restrict__ qkv, int T, int NH, int BH, float qscale) {
    constexpr int HH = HS / 2, DT = HS / 32;
    const int lane = threadIdx.x & 63, l32 = lane & 31, hf = lane >> 5;
    const int nqt = (T + 31) / 32;
    const int g = blockIdx.x * WPB + (threadIdx.x >> 6);
    if (g >= BH * nqt) return;
    const int qt = nqt - 1 - g / BH;  // longest (most keys) first
    const int bh = g % BH, b = bh / NH, h = bh % NH;
    const int C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;

    const int q0 = qt * 32, qi = q0 + l32;
    float qf[HH];
    load_frag<HH>(qf, base + (size_t)qi * rs + hf * HH, qi < T, qscale);

    f32x16 o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = zero16();
    float m = -INFINITY, l = 0.0f;

    const int kend = min(T, q0 + 32);
    float kf[HH];
    load_frag<HH>(kf, base + (size_t)l32 * rs + C + hf * HH, l32 < T, 1.0f);

    for (int kb = 0; kb < kend; kb += 32) {
        // V^T operand for this tile: step s uses key kb + res_row(s, hf).
        float vf[16][DT];
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int key = kb + res_row(s, hf);
#pragma unroll
            for (int d = 0; d < DT; ++d)
                vf[s][d] = key < T ? base[(size_t)key * rs + 2 * C + d * 32 + l32] : 0.0f;
        }

        // S^T = K Q^T, 32 keys x 32 queries, log2 units.
        f32x16 s = zero16();
#pragma unroll
        for (int st = 0; st < HH; ++st) s = mfma(kf[st], qf[st], s);

        // Next tile's K while this one's softmax and PV run.
        if (kb + 32 < kend) {
            const int nk = kb + 32 + l32;
            load_frag<HH>(kf, base + (size_t)nk * rs + C + hf * HH, nk < T, 1.0f);
        }

        if (kb + 32 > q0 || kb + 32 > T) {  // diagonal or ragged tile
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kb + res_row(r, hf);
                if (key > qi || key >= T) s[r] = -INFINITY;
            }
        }
        float mb = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mb = fmaxf(mb, s[r]);
        mb = fmaxf(mb, xhalf(mb));
        const float mn = fmaxf(m, mb);
        float p[16], ls = 0.0f, alpha = 1.0f;
        if (mn == -INFINITY) {
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = 0.0f;
        } else {
            alpha = fast_exp2(m - mn);  // 0 when m was -inf
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                p[r] = fast_exp2(s[r] - mn);
                ls += p[r];
            }
        }
        ls += xhalf(ls);
        l = l * alpha + ls;
        m = mn;
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[d][r] *= alpha;

        // O^T += V^T P^T
#pragma unroll
        for (int st = 0; st < 16; ++st)
#pragma unroll
            for (int d = 0; d < DT; ++d) o[d] = mfma(vf[st][d], p[st], o[d]);
    }

    if (qi < T) {
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

// --------------------------------------------------------------- backward

// D[b,h,t] = sum_i dO[b,t,h*hs+i] * O[b,t,h*hs+i] (src/flash.cu:471-487).
// HS/4 lanes per row, one float4 each, reduced with cross-lane xor shuffles.
template <int HS>
__global__ __launch_bounds__(256) void flash_dsum_k(float *__restrict__ dsum,
                                                    const float *__restrict__ dout,
                                                    const float *__restrict__ out,
                                                    int T, int NH, long long rows) {
    constexpr int LPR = HS / 4;  // lanes per row
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long row = gid / LPR;  // row = (b*T + t)*NH + h: memory order
    const int sub = (int)(gid % LPR);
    float s = 0.0f;
    if (row < rows) {
        const size_t off = (size_t)row * HS + sub * 4;
        const float4 a = bmb::ld4(dout + off), c = bmb::ld4(out + off);
        s = a.x * c.x + a.y * c.y + a.z * c.z + a.w * c.w;
    }
#pragma unroll
    for (int w = 1; w < LPR; w <<= 1) s += __shfl_xor(s, w);
    if (row < rows && sub == 0) {
        const int h = (int)(row % NH);
        const long long bt = row / NH;
        const int t = (int)(bt % T);
        const long long b = bt / T;
        dsum[((size_t)b * NH + h) * T + t] = s;
    }
}

// dK, dV for key tile kt of head bh.
template <int HS>
__device__ __forceinline__ void bwd_kv_tile(float *__restrict__ dqkv,
                                            const float *__restrict__ qkv,
                                            const float *__restrict__ dout,
                                            const float *__restrict__ lse,
                                            const float *__restrict__ dsum,
                                            int T, int NH, int kt, int bh,
                                            float scale, float qscale) {
    constexpr int HH = HS / 2, DT = HS / 32;
    const int lane = threadIdx.x & 63, l32 = lane & 31, hf = lane >> 5;
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;
    const float *dob = dout + (size_t)b * T * C + h * HS;
    const float *lrow = lse + (size_t)bh * T;
    const float *drow = dsum + (size_t)bh * T;

    const int k0 = kt * 32, key = k0 + l32;
    // B operands of S = Q K^T and dP = dO V^T: K (log2-scaled) and V.
    float kf[HH], vf[HH];
    load_frag<HH>(kf, base + (size_t)key * rs + C + hf * HH, key < T, qscale);
    load_frag<HH>(vf, base + (size_t)key * rs + 2 * C + hf * HH, key < T, 1.0f);

    f32x16 dv[DT], dk[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) { dv[d] = zero16(); dk[d] = zero16(); }

    for (int qb = k0; qb < T; qb += 32) {
        const int qa_row = qb + l32;
        float qa[HH], da[HH];
        load_frag<HH>(qa, base + (size_t)qa_row * rs + hf * HH, qa_row < T, 1.0f);
        load_frag<HH>(da, dob + (size_t)qa_row * C + hf * HH, qa_row < T, 1.0f);
        // lse (as log2) and D of the 16 query rows this lane's results hold.
        float L2[16], Dv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int q = qb + res_row(r, hf);
            L2[r] = q < T ? lrow[q] * LOG2E : 0.0f;
            Dv[r] = q < T ? drow[q] : 0.0f;
        }

        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int st = 0; st < HH; ++st) {
            s = mfma(qa[st], kf[st], s);
            dp = mfma(da[st], vf[st], dp);
        }

        // B operands of dV += P^T dO and dK += dS^T Q: rows q(st) of dO, Q.
        float dob_f[16][DT], qb_f[16][DT];
#pragma unroll
        for (int st = 0; st < 16; ++st) {
            const int q = qb + res_row(st, hf);
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                dob_f[st][d] = q < T ? dob[(size_t)q * C + d * 32 + l32] : 0.0f;
                qb_f[st][d] = q < T ? base[(size_t)q * rs + d * 32 + l32] : 0.0f;
            }
        }

        const bool edge = (qb < k0 + 32) || (qb + 32 > T);
        float p[16], ds[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int q = qb + res_row(r, hf);
            const bool live = !edge || (q < T && key < T && key <= q);
            p[r] = live ? fast_exp2(s[r] - L2[r]) : 0.0f;
            ds[r] = p[r] * (dp[r] - Dv[r]);
        }

#pragma unroll
        for (int st = 0; st < 16; ++st)
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                dv[d] = mfma(p[st], dob_f[st][d], dv[d]);
                dk[d] = mfma(ds[st], qb_f[st][d], dk[d]);
            }
    }

    // Lane holds column d*32 + l32 of rows key k0 + res_row(r, hf).
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int kr = k0 + res_row(r, hf);
        if (kr >= T) continue;
        float *dkp = dqkv + ((size_t)b * T + kr) * rs + C + h * HS;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            dkp[d * 32 + l32] = dk[d][r] * scale;
            dkp[C + d * 32 + l32] = dv[d][r];
        }
    }
}

// dQ for query tile qt of head bh.
template <int HS>
__device__ __forceinline__ void bwd_q_tile(float *__restrict__ dqkv,
                                           const float *__restrict__ qkv,
                                           const float *__restrict__ dout,
                                           const float *__restrict__ lse,
                                           const float *__restrict__ dsum,
                                           int T, int NH, int qt, int bh,
                                           float scale, float qscale) {
    constexpr int HH = HS / 2, DT = HS / 32;
    const int lane = threadIdx.x & 63, l32 = lane & 31, hf = lane >> 5;
    const int b = bh / NH, h = bh % NH, C = NH * HS;
    const size_t rs = 3 * (size_t)C;
    const float *base = qkv + (size_t)b * T * rs + h * HS;
    const float *dob = dout + (size_t)b * T * C + h * HS;

    const int q0 = qt * 32, qi = q0 + l32;
    const bool qv = qi < T;
    float qf[HH], df[HH];
    load_frag<HH>(qf, base + (size_t)qi * rs + hf * HH, qv, qscale);
    load_frag<HH>(df, dob + (size_t)qi * C + hf * HH, qv, 1.0f);
    const float L2 = qv ? lse[(size_t)bh * T + qi] * LOG2E : 0.0f;
    const float Dq = qv ? dsum[(size_t)bh * T + qi] : 0.0f;

    f32x16 dq[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) dq[d] = zero16();

    const int kend = min(T, q0 + 32);
    for (int kb = 0; kb < kend; kb += 32) {
        const int ka_row = kb + l32;
        float ka[HH], va[HH];
        load_frag<HH>(ka, base + (size_t)ka_row * rs + C + hf * HH, ka_row < T, 1.0f);
        load_frag<HH>(va, base + (size_t)ka_row * rs + 2 * C + hf * HH, ka_row < T, 1.0f);

        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int st = 0; st < HH; ++st) {
            s = mfma(ka[st], qf[st], s);
            dp = mfma(va[st], df[st], dp);
        }

        // A operand of dQ^T += K^T dS^T: rows key(st) of K.
        float kb_f[16][DT];
#pragma unroll
        for (int st = 0; st < 16; ++st) {
            const int kr = kb + res_row(st, hf);
#pragma unroll
            for (int d = 0; d < DT; ++d)
                kb_f[st][d] = kr < T ? base[(size_t)kr * rs + C + d * 32 + l32] : 0.0f;
        }

        const bool edge = (kb + 32 > q0) || (kb + 32 > T);
        float ds[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int kr = kb + res_row(r, hf);
            const bool live = !edge || (qv && kr < T && kr <= qi);
            const float p = live ? fast_exp2(s[r] - L2) : 0.0f;
            ds[r] = p * (dp[r] - Dq);
        }

#pragma unroll
        for (int st = 0; st < 16; ++st)
#pragma unroll
            for (int d = 0; d < DT; ++d) dq[d] = mfma(kb_f[st][d], ds[st], dq[d]);
    }

    if (qv) {
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

// MODE 0: waves alternate dK/dV and dQ work, both longest-first.
// MODE 1: dK/dV only.  MODE 2: dQ only.
template <int HS, int WPB, int MODE>
__global__ __launch_bounds__(WPB * 64) void flash_bwd_k(
    float *__restrict__ dqkv, const float *__restrict__ qkv,
    const float *__restrict__ dout, const float *__restrict__ lse,
    const float *__restrict__ dsum, int T, int NH, int BH, float scale,
    float qscale) {
    const int nt = (T + 31) / 32;
    const int items = BH * nt;
    const int g = blockIdx.x * WPB + (threadIdx.x >> 6);
    int kind, u;
    if (MODE == 0) { kind = g & 1; u = g >> 1; }
    else           { kind = MODE - 1; u = g; }
    if (u >= items) return;
    const int tile = u / BH, bh = u % BH;
    if (kind == 0)
        bwd_kv_tile<HS>(dqkv, qkv, dout, lse, dsum, T, NH, tile, bh, scale, qscale);
    else
        bwd_q_tile<HS>(dqkv, qkv, dout, lse, dsum, T, NH, nt - 1 - tile, bh, scale, qscale);
}

// ------------------------------------------------------------- host side

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

struct FwdCfg {
    const char *name;
    int wpb;
};
// Waves per workgroup only changes how many independent 32-query waves share
// a workgroup slot; the per-wave work is identical.
const FwdCfg FWD_CFGS[] = {
    {"q32/wave mfma32 wg4", 4},
    {"q32/wave mfma32 wg1", 1},
    {"q32/wave mfma32 wg2", 2},
    {"q32/wave mfma32 wg8", 8},
};
constexpr int N_FWD = sizeof(FWD_CFGS) / sizeof(FWD_CFGS[0]);
constexpr int FWD_DEFAULT = 0;

struct BwdCfg {
    const char *name;
    int wpb;
    bool fused;
};
const BwdCfg BWD_CFGS[] = {
    {"kv32+q32 fused mfma32 wg4", 4, true},
    {"kv32+q32 fused mfma32 wg2", 2, true},
    {"kv32 then q32 mfma32 wg4", 4, false},
    {"kv32+q32 fused mfma32 wg1", 1, true},
};
constexpr int N_BWD = sizeof(BWD_CFGS) / sizeof(BWD_CFGS[0]);
constexpr int BWD_DEFAULT = 0;

template <int HS, int WPB>
void run_fwd(float *out, float *lse, const float *qkv, int B, int T, int NH) {
    const int BH = B * NH, nqt = (T + 31) / 32;
    const long long waves = (long long)BH * nqt;
    const float qscale = (1.0f / sqrtf((float)HS)) * LOG2E;
    bmb::launch(flash_fwd_k<HS, WPB>, dim3((unsigned)((waves + WPB - 1) / WPB)),
                dim3(WPB * 64), 0, nullptr, out, lse, qkv, T, NH, BH, qscale);
}

template <int HS>
bool fwd_hs(int cfg, float *out, float *lse, const float *qkv, int B, int T, int NH) {
    switch (FWD_CFGS[cfg].wpb) {
    case 1: run_fwd<HS, 1>(out, lse, qkv, B, T, NH); return true;
    case 2: run_fwd<HS, 2>(out, lse, qkv, B, T, NH); return true;
    case 4: run_fwd<HS, 4>(out, lse, qkv, B, T, NH); return true;
    case 8: run_fwd<HS, 8>(out, lse, qkv, B, T, NH); return true;
    default: return false;
    }
}

template <int HS, int WPB, int MODE>
void run_bwd_mode(float *dqkv, const float *dout, const float *qkv,
                  const float *lse, const float *dsum, int B, int T, int NH) {
    const int BH = B * NH, nt = (T + 31) / 32;
    const long long waves = (long long)BH * nt * (MODE == 0 ? 2 : 1);
    const float scale = 1.0f / sqrtf((float)HS);
    bmb::launch(flash_bwd_k<HS, WPB, MODE>, dim3((unsigned)((waves + WPB - 1) / WPB)),
                dim3(WPB * 64), 0, nullptr, dqkv, qkv, dout, lse, dsum, T, NH, BH,
                scale, scale * LOG2E);
}

template <int HS, int WPB>
void run_bwd(bool fused, float *dqkv, float *dsum, const float *dout,
             const float *qkv, const float *out, const float *lse, int B, int T,
             int NH) {
    const long long rows = (long long)B * T * NH;
    const long long threads = rows * (HS / 4);
    bmb::launch(flash_dsum_k<HS>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                nullptr, dsum, dout, out, T, NH, rows);
    if (fused) {
        run_bwd_mode<HS, WPB, 0>(dqkv, dout, qkv, lse, dsum, B, T, NH);
    } else {
        run_bwd_mode<HS, WPB, 1>(dqkv, dout, qkv, lse, dsum, B, T, NH);
        run_bwd_mode<HS, WPB, 2>(dqkv, dout, qkv, lse, dsum, B, T, NH);
    }
}

template <int HS>
bool bwd_hs(int cfg, float *dqkv, float *dsum, const float *dout, const float *qkv,
            const float *out, const float *lse, int B, int T, int NH) {
    const BwdCfg &c = BWD_CFGS[cfg];
    switch (c.wpb) {
    case 1: run_bwd<HS, 1>(c.fused, dqkv, dsum, dout, qkv, out, lse, B, T, NH); return true;
    case 2: run_bwd<HS, 2>(c.fused, dqkv, dsum, dout, qkv, out, lse, B, T, NH); return true;
    case 4: run_bwd<HS, 4>(c.fused, dqkv, dsum, dout, qkv, out, lse, B, T, NH); return true;
    default: return false;
    }
}

// Shape legality shared by forward and backward: a supported head size and
// 16-byte aligned rows (every fragment is a run of 128-bit loads).
bool shape_ok(int B, int T, int C, int NH, int &hs) {
    if (B < 0 || T < 0 || NH <= 0 || C <= 0 || C % NH != 0) return false;
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

bool flash_attention_forward_cfg(int cfg, float *out, float *lse,
                                 const float *qkv, int B, int T, int C, int NH) {
    int hs;
    if (cfg < 0 || cfg >= N_FWD || !shape_ok(B, T, C, NH, hs)) return false;
    if (!aligned16(qkv) || !aligned16(out)) return false;
    if (B == 0 || T == 0) return true;
    switch (hs) {
    case 32: return fwd_hs<32>(cfg, out, lse, qkv, B, T, NH);
    case 64: return fwd_hs<64>(cfg, out, lse, qkv, B, T, NH);
    case 128: return fwd_hs<128>(cfg, out, lse, qkv, B, T, NH);
    default: return false;
    }
}

void flash_attention_forward(float *out, float *lse, const float *qkv, int B,
                             int T, int C, int NH) {
    if (flash_attention_forward_cfg(flash_default_config(), out, lse, qkv, B, T, C, NH))
        return;
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

bool flash_attention_backward_cfg(int cfg, float *dqkv, float *dsum,
                                  const float *dout, const float *qkv,
                                  const float *out, const float *lse, int B,
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

void flash_attention_backward(float *dqkv, float *dsum, const float *dout,
                              const float *qkv, const float *out,
                              const float *lse, int B, int T, int C, int NH) {
    if (flash_attention_backward_cfg(flash_default_bwd_config(), dqkv, dsum, dout,
                                     qkv, out, lse, B, T, C, NH))
        return;
    for (int cfg = 0; cfg < N_BWD; ++cfg)
        if (flash_attention_backward_cfg(cfg, dqkv, dsum, dout, qkv, out, lse, B, T,
                                         C, NH))
            return;
    fprintf(stderr, "flash: no backward tile config for head size %d (C=%d, NH=%d)\n",
            NH > 0 ? C / NH : -1, C, NH);
    exit(1);
}

}  // extern "C"
