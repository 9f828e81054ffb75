// Unfused causal attention for gfx950 -- the counterpart of bare-metal-bard's
// src/attention.cu (API: src/attention.h).
//
// This path materialises the (B, NH, T, T) probabilities, which is what makes
// it the independent check of the fused kernels and the trainer's --unfused
// mode. Its four contractions are the library's MFMA batched GEMM, one
// problem per (batch, head); what is written here are the HBM-bound pieces:
//   * head permutes between the (B, T, 3C) / (B, T, C) activations and the
//     head-contiguous (B, NH, T, hs) layout the batched GEMM needs, one float4
//     per lane (hs % 4 == 0) so both sides move in 128-bit accesses;
//   * the causal softmax and its backward, one wave64 per score row with the
//     row held in registers: positions past the diagonal are never read and
//     are written as exact zeros, so the following att @ v reads no stale
//     memory (src/attention.cu:86-129).
#include <math.h>

#include "common.hpp"
#include "launch.hpp"
#include "../../include/attention.h"
#include "../../include/gemm.h"

using bmb::ceil_div;

namespace {

constexpr int NT = 256;
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float4 ldu4(const float *p) {
    float4 v;
    __builtin_memcpy(&v, p, sizeof(v));
    return v;
}
__device__ __forceinline__ void stu4(float *p, float4 v) { __builtin_memcpy(p, &v, sizeof(v)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Work item e of a head-major tensor (B, NH, T, hs) in chunks of W floats
// (W = 4 when hs % 4 == 0, else 1): element offset e*W there, and the offset
// of the same (b, t, h, i) in a row-major (B, T, rowC) tensor whose head h
// starts at column h*hs.
struct HeadMap {
    int T, NH, hs, W;
    __device__ __forceinline__ size_t row_offset(long long e, int rowC) const {
        const int per_row = hs / W;
        const int i = (int)(e % per_row) * W;
        const long long bht = e / per_row;
        const int t = (int)(bht % T);
        const long long bh = bht / T;
        const int h = (int)(bh % NH);
        const long long b = bh / NH;
        return (size_t)(b * T + t) * rowC + (size_t)h * hs + i;
    }
};

template <int W>
__device__ __forceinline__ void copy_w(float *dst, const float *src) {
    if (W == 4)
        stu4(dst, ldu4(src));
    else
        *dst = *src;
}

// qkv (B,T,3C) -> qkvr slots 0..2 (src/attention.cu:19-38)
template <int W>
__global__ __launch_bounds__(NT) void permute_qkv_k(float *qkvr, const float *qkv, HeadMap m,
                                                     long long total, long long items) {
    const long long e = (long long)blockIdx.x * NT + threadIdx.x;
    if (e >= items) return;
    const int C = m.NH * m.hs;
    const size_t src = m.row_offset(e, 3 * C);
    const size_t dst = (size_t)e * W;
    copy_w<W>(qkvr + dst, qkv + src);
    copy_w<W>(qkvr + total + dst, qkv + src + C);
    copy_w<W>(qkvr + 2 * total + dst, qkv + src + 2 * C);
}

// dqkvr slots 0..2 -> dqkv (B,T,3C) (src/attention.cu:41-56)
template <int W>
__global__ __launch_bounds__(NT) void unpermute_qkv_k(float *dqkv, const float *dqkvr,
                                                       HeadMap m, long long total,
                                                       long long items) {
    const long long e = (long long)blockIdx.x * NT + threadIdx.x;
    if (e >= items) return;
    const int C = m.NH * m.hs;
    const size_t dst = m.row_offset(e, 3 * C);
    const size_t src = (size_t)e * W;
    copy_w<W>(dqkv + dst, dqkvr + src);
    copy_w<W>(dqkv + dst + C, dqkvr + total + src);
    copy_w<W>(dqkv + dst + 2 * C, dqkvr + 2 * total + src);
}

// (B,NH,T,hs) <-> (B,T,C) (src/attention.cu:59-83). TO_ROWS: head-major in.
template <int W, bool TO_ROWS>
__global__ __launch_bounds__(NT) void permute_out_k(float *dst, const float *src, HeadMap m,
                                                     long long items) {
    const long long e = (long long)blockIdx.x * NT + threadIdx.x;
    if (e >= items) return;
    const size_t r = m.row_offset(e, m.NH * m.hs);
    const size_t h = (size_t)e * W;
    if (TO_ROWS)
        copy_w<W>(dst + r, src + h);
    else
        copy_w<W>(dst + h, src + r);
}

// Causal softmax in place, one wave per row (b, h, t1); the row's first
// t1 + 1 entries are live. NCH float4 per lane hold the row (T <= 256*NCH,
// T % 4 == 0); NCH == 0 is the scalar path for any T.
template <int NCH>
__global__ __launch_bounds__(NT) void softmax_causal_k(float *att, int T, long long rows) {
    const long long row = (long long)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int len = (int)(row % T) + 1;
    float *x = att + (size_t)row * T;
    if (NCH > 0) {
        float4 v[NCH > 0 ? NCH : 1];
        float m = -INFINITY;
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int c = (k * 64 + lane) * 4;
            v[k] = c < len ? ldu4(x + c) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            if (c + 1 >= len) v[k].y = -INFINITY;
            if (c + 2 >= len) v[k].z = -INFINITY;
            if (c + 3 >= len) v[k].w = -INFINITY;
            m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
        }
        const float ml = wave_max(m) * LOG2E;
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            v[k].x = __builtin_amdgcn_exp2f(v[k].x * LOG2E - ml);
            v[k].y = __builtin_amdgcn_exp2f(v[k].y * LOG2E - ml);
            v[k].z = __builtin_amdgcn_exp2f(v[k].z * LOG2E - ml);
            v[k].w = __builtin_amdgcn_exp2f(v[k].w * LOG2E - ml);
            s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
        }
        const float inv = 1.0f / wave_sum(s);
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int c = (k * 64 + lane) * 4;
            if (c < T)
                stu4(x + c, make_float4(v[k].x * inv, v[k].y * inv, v[k].z * inv, v[k].w * inv));
        }
    } else {
        float m = -INFINITY;
        for (int c = lane; c < len; c += 64) m = fmaxf(m, x[c]);
        const float ml = wave_max(m) * LOG2E;
        float s = 0.0f;
        for (int c = lane; c < len; c += 64) s += __builtin_amdgcn_exp2f(x[c] * LOG2E - ml);
        const float inv = 1.0f / wave_sum(s);
        for (int c = lane; c < T; c += 64)
            x[c] = c < len ? __builtin_amdgcn_exp2f(x[c] * LOG2E - ml) * inv : 0.0f;
    }
}

// dpre = att * (datt - rowsum(att * datt)) on the live part, 0 beyond
// (src/attention.cu:113-129). dpre may alias datt: each lane reads its
// entries before the wave's reduction and writes only those entries after it.
template <int NCH>
__global__ __launch_bounds__(NT) void softmax_causal_bwd_k(float *dpre, const float *datt,
                                                            const float *att, int T,
                                                            long long rows) {
    const long long row = (long long)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int len = (int)(row % T) + 1;
    const float *y = att + (size_t)row * T;
    const float *dy = datt + (size_t)row * T;
    float *dx = dpre + (size_t)row * T;
    if (NCH > 0) {
        float4 a[NCH > 0 ? NCH : 1], g[NCH > 0 ? NCH : 1];
        float dot = 0.0f;
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int c = (k * 64 + lane) * 4;
            a[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            g[k] = a[k];
            if (c < len) {
                a[k] = ldu4(y + c);
                g[k] = ldu4(dy + c);
                if (c + 1 >= len) a[k].y = 0.0f;
                if (c + 2 >= len) a[k].z = 0.0f;
                if (c + 3 >= len) a[k].w = 0.0f;
            }
            dot += (a[k].x * g[k].x + a[k].y * g[k].y) + (a[k].z * g[k].z + a[k].w * g[k].w);
        }
        dot = wave_sum(dot);
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int c = (k * 64 + lane) * 4;
            if (c < T)
                stu4(dx + c, make_float4(a[k].x * (g[k].x - dot), a[k].y * (g[k].y - dot),
                                         a[k].z * (g[k].z - dot), a[k].w * (g[k].w - dot)));
        }
    } else {
        float dot = 0.0f;
        for (int c = lane; c < len; c += 64) dot += y[c] * dy[c];
        dot = wave_sum(dot);
        // A lane's reads of entry c all happen before its write of entry c.
        for (int c = lane; c < T; c += 64) dx[c] = c < len ? y[c] * (dy[c] - dot) : 0.0f;
    }
}

int softmax_chunks(int T) {
    if (T % 4 != 0) return 0;
    const int n = ceil_div(T, 256);
    return n <= 4 ? n : 0;
}

void softmax_fwd(float *att, int T, long long rows) {
    const dim3 grid((unsigned)((rows + NT / 64 - 1) / (NT / 64)));
    switch (softmax_chunks(T)) {
        case 1: bmb::launch(softmax_causal_k<1>, grid, dim3(NT), 0, nullptr, att, T, rows); break;
        case 2: bmb::launch(softmax_causal_k<2>, grid, dim3(NT), 0, nullptr, att, T, rows); break;
        case 3: bmb::launch(softmax_causal_k<3>, grid, dim3(NT), 0, nullptr, att, T, rows); break;
        case 4: bmb::launch(softmax_causal_k<4>, grid, dim3(NT), 0, nullptr, att, T, rows); break;
        default: bmb::launch(softmax_causal_k<0>, grid, dim3(NT), 0, nullptr, att, T, rows);
    }
}

void softmax_bwd(float *dpre, const float *datt, const float *att, int T, long long rows) {
    const dim3 grid((unsigned)((rows + NT / 64 - 1) / (NT / 64)));
    switch (softmax_chunks(T)) {
        case 1: bmb::launch(softmax_causal_bwd_k<1>, grid, dim3(NT), 0, nullptr, dpre, datt, att, T, rows); break;
        case 2: bmb::launch(softmax_causal_bwd_k<2>, grid, dim3(NT), 0, nullptr, dpre, datt, att, T, rows); break;
        case 3: bmb::launch(softmax_causal_bwd_k<3>, grid, dim3(NT), 0, nullptr, dpre, datt, att, T, rows); break;
        case 4: bmb::launch(softmax_causal_bwd_k<4>, grid, dim3(NT), 0, nullptr, dpre, datt, att, T, rows); break;
        default: bmb::launch(softmax_causal_bwd_k<0>, grid, dim3(NT), 0, nullptr, dpre, datt, att, T, rows);
    }
}

struct Shape {
    HeadMap m;
    long long total, items;
    unsigned grid;
    bool vec;
    Shape(int B, int T, int C, int NH) {
        const int hs = C / NH;
        vec = hs % 4 == 0;
        m = HeadMap{T, NH, hs, vec ? 4 : 1};
        total = (long long)B * T * C;
        items = total / m.W;
        grid = (unsigned)((items + NT - 1) / NT);
    }
};

}  // namespace

extern "C" {

void attention_forward(float *out, float *qkvr, float *att, const float *qkv, int B, int T,
                       int C, int NH) {
    if (B <= 0 || T <= 0 || C <= 0 || NH <= 0 || C % NH != 0) return;
    const Shape s(B, T, C, NH);
    const int hs = C / NH;
    const float scale = 1.0f / sqrtf((float)hs);
    const long long sHead = (long long)T * hs, sAtt = (long long)T * T;
    if (s.vec)
        bmb::launch(permute_qkv_k<4>, dim3(s.grid), dim3(NT), 0, nullptr, qkvr, qkv, s.m,
                    s.total, s.items);
    else
        bmb::launch(permute_qkv_k<1>, dim3(s.grid), dim3(NT), 0, nullptr, qkvr, qkv, s.m,
                    s.total, s.items);
    const float *q = qkvr, *k = qkvr + s.total, *v = qkvr + 2 * s.total;
    float *vacc = qkvr + 3 * s.total;
    // scores = scale * q k^T (k stored T x hs: the transB case), softmax in
    // place, then att @ v (src/attention.cu:144-166).
    batched_gemm(false, true, B * NH, T, T, hs, scale, q, sHead, k, sHead, 0.0f, att, sAtt,
                 nullptr);
    softmax_fwd(att, T, (long long)B * NH * T);
    batched_gemm(false, false, B * NH, T, hs, T, 1.0f, att, sAtt, v, sHead, 0.0f, vacc, sHead,
                 nullptr);
    if (s.vec)
        bmb::launch(permute_out_k<4, true>, dim3(s.grid), dim3(NT), 0, nullptr, out,
                    (const float *)vacc, s.m, s.items);
    else
        bmb::launch(permute_out_k<1, true>, dim3(s.grid), dim3(NT), 0, nullptr, out,
                    (const float *)vacc, s.m, s.items);
}

void attention_backward(float *dqkv, float *dqkvr, float *datt, float *dpreatt,
                        const float *dout, const float *qkvr, const float *att, int B, int T,
                        int C, int NH) {
    if (B <= 0 || T <= 0 || C <= 0 || NH <= 0 || C % NH != 0) return;
    const Shape s(B, T, C, NH);
    const int hs = C / NH;
    const float scale = 1.0f / sqrtf((float)hs);
    const long long sHead = (long long)T * hs, sAtt = (long long)T * T;
    const float *q = qkvr, *k = qkvr + s.total, *v = qkvr + 2 * s.total;
    float *dq = dqkvr, *dk = dqkvr + s.total, *dv = dqkvr + 2 * s.total;
    float *dvacc = dqkvr + 3 * s.total;
    if (s.vec)
        bmb::launch(permute_out_k<4, false>, dim3(s.grid), dim3(NT), 0, nullptr, dvacc, dout,
                    s.m, s.items);
    else
        bmb::launch(permute_out_k<1, false>, dim3(s.grid), dim3(NT), 0, nullptr, dvacc, dout,
                    s.m, s.items);
    // datt = dvacc v^T, dv = att^T dvacc, dpre = softmax backward,
    // dq = scale dpre k, dk = scale dpre^T q (src/attention.cu:183-197).
    batched_gemm(false, true, B * NH, T, T, hs, 1.0f, dvacc, sHead, v, sHead, 0.0f, datt, sAtt,
                 nullptr);
    batched_gemm(true, false, B * NH, T, hs, T, 1.0f, att, sAtt, dvacc, sHead, 0.0f, dv, sHead,
                 nullptr);
    softmax_bwd(dpreatt, datt, att, T, (long long)B * NH * T);
    batched_gemm(false, false, B * NH, T, hs, T, scale, dpreatt, sAtt, k, sHead, 0.0f, dq,
                 sHead, nullptr);
    batched_gemm(true, false, B * NH, T, hs, T, scale, dpreatt, sAtt, q, sHead, 0.0f, dk,
                 sHead, nullptr);
    if (s.vec)
        bmb::launch(unpermute_qkv_k<4>, dim3(s.grid), dim3(NT), 0, nullptr, dqkv,
                    (const float *)dqkvr, s.m, s.total, s.items);
    else
        bmb::launch(unpermute_qkv_k<1>, dim3(s.grid), dim3(NT), 0, nullptr, dqkv,
                    (const float *)dqkvr, s.m, s.total, s.items);
}

}  // extern "C"
