// Transformer building blocks of the GPT trainer for gfx950 -- the
// counterpart of bare-metal-bard's src/nn.cu (API: src/nn.h).
//
// Everything here is HBM-bound: arithmetic intensity below one flop per byte.
// The design rules are therefore about bytes, not flops:
//   * each tensor is read and written once, with 128-bit accesses (gfx950
//     global loads and stores need only 4-byte alignment, so rows of any
//     width C % 4 == 0 use them; other widths fall back to 32-bit accesses);
//   * a row-wise reduction (layernorm, softmax) gives a row to one wave64 (or,
//     for the 50k-wide vocabulary rows, one 1024-lane workgroup) that keeps the
//     whole row in registers between its passes, so the row is fetched once;
//   * reductions across rows (the layernorm weight/bias gradients, the bias
//     gradient, the gradient norm) never use floating-point atomics: blocks
//     write partial sums to a library-owned scratch buffer and a second kernel
//     adds them in a fixed order. The grid shapes depend only on the problem
//     shape, so every result is the same bit pattern on every call.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "common.hpp"
#include "launch.hpp"
#include "nn_fused.hpp"
#include "workspace.hpp"
#include "../../include/nn.h"

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
__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Grid size for a flat launch of `n` work items of NT lanes each.
inline unsigned grid_for(long long items) {
    return (unsigned)((items + NT - 1) / NT);
}

// ------------------------------------------------------------ row/column maps
// Row-structured elementwise kernels split each row of width C into float4
// chunks (the last one may be partial): work item i is row i / C4, columns
// 4*(i % C4) .. +3, with C4 = ceil(C/4). VEC: C % 4 == 0, so every chunk is
// whole and rows are 4-byte aligned for the 128-bit accesses.

// out[r, c] = wte[tok[r], c] + wpe[r % T, c]   (src/nn.cu:23-36)
template <bool VEC>
__global__ __launch_bounds__(NT) void encoder_fwd_k(float *out, const int *tokens,
                                                     const float *wte, const float *wpe,
                                                     int T, int C, int C4, long long items) {
    const long long i = (long long)blockIdx.x * NT + threadIdx.x;
    if (i >= items) return;
    const int r = (int)(i / C4), c = (int)(i % C4) * 4;
    const int t = r % T;
    const float *e = wte + (size_t)tokens[r] * C + c;
    const float *p = wpe + (size_t)t * C + c;
    float *o = out + (size_t)r * C + c;
    if (VEC) {
        const float4 a = ldu4(e), b = ldu4(p);
        stu4(o, make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w));
    } else {
        for (int k = 0; k < 4 && c + k < C; ++k) o[k] = e[k] + p[k];
    }
}

// dwpe[t, c] += sum_b dout[b, t, c], b ascending.
template <bool VEC>
__global__ __launch_bounds__(NT) void encoder_bwd_wpe_k(float *dwpe, const float *dout, int B,
                                                         int T, int C, int C4, long long items) {
    const long long i = (long long)blockIdx.x * NT + threadIdx.x;
    if (i >= items) return;
    const int t = (int)(i / C4), c = (int)(i % C4) * 4;
    const size_t bstride = (size_t)T * C;
    const float *src = dout + (size_t)t * C + c;
    float *dst = dwpe + (size_t)t * C + c;
    if (VEC) {
        float4 s = zero4();
        for (int b = 0; b < B; ++b) {
            const float4 v = ldu4(src + b * bstride);
            s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
        }
        float4 d = ldu4(dst);
        d.x += s.x; d.y += s.y; d.z += s.z; d.w += s.w;
        stu4(dst, d);
    } else {
        for (int k = 0; k < 4 && c + k < C; ++k) {
            float s = 0.0f;
            for (int b = 0; b < B; ++b) s += src[b * bstride + k];
            dst[k] += s;
        }
    }
}

// dwte[tok, :] += sum over positions j with tokens[j] == tok, j ascending.
// One wave per position i. A position that is not the first occurrence of
// its token leaves; the first one gathers every later occurrence in order and
// owns the update of that wte row, so no two waves touch the same row.
__global__ __launch_bounds__(NT) void encoder_bwd_wte_k(float *dwte, const float *dout,
                                                         const int *tokens, int N, int C) {
    const int i = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= N) return;
    const int tok = tokens[i];
    for (int j0 = 0; j0 < i; j0 += 64) {
        const int j = j0 + lane;
        if (__ballot(j < i && tokens[j] == tok) != 0) return;
    }
    const bool vec = (C & 3) == 0;
    float *dst = dwte + (size_t)tok * C;
    for (int c0 = 0; c0 < C; c0 += 256) {
        const int c = c0 + lane * 4;
        float4 s = zero4();
        for (int j0 = i; j0 < N; j0 += 64) {
            const int j = j0 + lane;
            unsigned long long m = __ballot(j < N && tokens[j] == tok);
            while (m != 0) {
                const int jj = j0 + __ffsll((long long)m) - 1;
                m &= m - 1;
                const float *src = dout + (size_t)jj * C + c;
                if (vec && c < C) {
                    const float4 v = ldu4(src);
                    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
                } else if (!vec) {
                    if (c + 0 < C) s.x += src[0];
                    if (c + 1 < C) s.y += src[1];
                    if (c + 2 < C) s.z += src[2];
                    if (c + 3 < C) s.w += src[3];
                }
            }
        }
        if (vec && c < C) {
            float4 d = ldu4(dst + c);
            d.x += s.x; d.y += s.y; d.z += s.z; d.w += s.w;
            stu4(dst + c, d);
        } else if (!vec) {
            if (c + 0 < C) dst[c + 0] += s.x;
            if (c + 1 < C) dst[c + 1] += s.y;
            if (c + 2 < C) dst[c + 2] += s.z;
            if (c + 3 < C) dst[c + 3] += s.w;
        }
    }
}

// ------------------------------------------------------------------ layernorm
// One wave per row, the row held in NCH float4 registers per lane
// (C <= 256*NCH, C % 4 == 0). Mean first, then the variance about it
// (src/nn.cu:54-82): biased, eps 1e-5. RES: the row is first formed as
// res_a + res_b and stored to res_out (residual_forward fused in front: the
// same one rounding per element, then the same layernorm of the stored sum).
template <int NCH, bool RES>
__global__ __launch_bounds__(NT) void ln_fwd_k(float *out, float *mean, float *rstd,
                                                const float *inp, const float *weight,
                                                const float *bias, int N, int C,
                                                float *res_out, const float *res_b) {
    const int row = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;
    const float *x = inp + (size_t)row * C;
    float4 v[NCH];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c = (k * 64 + lane) * 4;
        v[k] = c < C ? ldu4(x + c) : zero4();
        if (RES && c < C) {
            const float4 y = ldu4(res_b + (size_t)row * C + c);
            v[k] = make_float4(v[k].x + y.x, v[k].y + y.y, v[k].z + y.z, v[k].w + y.w);
            stu4(res_out + (size_t)row * C + c, v[k]);
        }
        s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    const float mu = wave_sum(s) / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c = (k * 64 + lane) * 4;
        if (c < C) {
            const float a = v[k].x - mu, b = v[k].y - mu, d = v[k].z - mu, e = v[k].w - mu;
            q += (a * a + b * b) + (d * d + e * e);
        }
    }
    const float var = wave_sum(q) / (float)C;
    const float rs = rsqrtf(var + 1e-5f);
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = rs;
    }
    float *y = out + (size_t)row * C;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c = (k * 64 + lane) * 4;
        if (c < C) {
            const float4 w = ldu4(weight + c), b = ldu4(bias + c);
            float4 o;
            o.x = ((v[k].x - mu) * rs) * w.x + b.x;
            o.y = ((v[k].y - mu) * rs) * w.y + b.y;
            o.z = ((v[k].z - mu) * rs) * w.z + b.z;
            o.w = ((v[k].w - mu) * rs) * w.w + b.w;
            stu4(y + c, o);
        }
    }
}

// Any C: one wave per row, three passes over the row.
__global__ __launch_bounds__(NT) void ln_fwd_generic_k(float *out, float *mean, float *rstd,
                                                        const float *inp, const float *weight,
                                                        const float *bias, int N, int C) {
    const int row = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;
    const float *x = inp + (size_t)row * C;
    float s = 0.0f;
    for (int c = lane; c < C; c += 64) s += x[c];
    const float mu = wave_sum(s) / (float)C;
    float q = 0.0f;
    for (int c = lane; c < C; c += 64) {
        const float d = x[c] - mu;
        q += d * d;
    }
    const float rs = rsqrtf(wave_sum(q) / (float)C + 1e-5f);
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = rs;
    }
    float *y = out + (size_t)row * C;
    for (int c = lane; c < C; c += 64) y[c] = ((x[c] - mu) * rs) * weight[c] + bias[c];
}

// Layernorm backward, fused (C % 4 == 0, C <= 256*NCH). A workgroup of
// LN_WAVES waves owns rows [blk*rpb, (blk+1)*rpb); each wave takes every
// LN_WAVES-th of them. Per row (src/nn.cu:85-111):
//   dinp += rstd * (dxhat - mean(dxhat) - xhat * mean(dxhat * xhat)),
//   dxhat = dout * w, xhat = (x - mean) * rstd.
// The weight and bias gradients of the workgroup's rows are summed in
// registers, combined across its waves through LDS in wave order, and written
// as partial[blk][0:C] (dweight) and partial[blk][C:2C] (dbias).
constexpr int LN_WAVES = 8;

template <int NCH>
__global__ __launch_bounds__(LN_WAVES * 64) void ln_bwd_k(
    float *dinp, float *partial, const float *dout, const float *inp, const float *weight,
    const float *mean, const float *rstd, int N, int C, int rpb) {
    extern __shared__ float red[];  // [LN_WAVES][2C]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float4 w[NCH], dw[NCH], db[NCH];
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c = (k * 64 + lane) * 4;
        w[k] = c < C ? ldu4(weight + c) : zero4();
        dw[k] = zero4();
        db[k] = zero4();
    }
    const int r0 = blockIdx.x * rpb;
    const int r1 = min(N, r0 + rpb);
    for (int r = r0 + wave; r < r1; r += LN_WAVES) {
        const float mu = mean[r], rs = rstd[r];
        const float *x = inp + (size_t)r * C;
        const float *dy = dout + (size_t)r * C;
        float4 xh[NCH], g[NCH];
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int c = (k * 64 + lane) * 4;
            float4 xv = zero4();
            g[k] = zero4();
            if (c < C) {
                xv = ldu4(x + c);
                g[k] = ldu4(dy + c);
            }
            xh[k] = make_float4((xv.x - mu) * rs, (xv.y - mu) * rs, (xv.z - mu) * rs,
                                (xv.w - mu) * rs);
            const float4 d = make_float4(g[k].x * w[k].x, g[k].y * w[k].y, g[k].z * w[k].z,
                                         g[k].w * w[k].w);
            s1 += (d.x + d.y) + (d.z + d.w);
            s2 += (d.x * xh[k].x + d.y * xh[k].y) + (d.z * xh[k].z + d.w * xh[k].w);
        }
        const float m1 = wave_sum(s1) / (float)C;
        const float m2 = wave_sum(s2) / (float)C;
        float *dx = dinp + (size_t)r * C;
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int c = (k * 64 + lane) * 4;
            if (c < C) {
                float4 o = ldu4(dx + c);
                o.x += rs * (g[k].x * w[k].x - m1 - xh[k].x * m2);
                o.y += rs * (g[k].y * w[k].y - m1 - xh[k].y * m2);
                o.z += rs * (g[k].z * w[k].z - m1 - xh[k].z * m2);
                o.w += rs * (g[k].w * w[k].w - m1 - xh[k].w * m2);
                stu4(dx + c, o);
                dw[k].x += g[k].x * xh[k].x; dw[k].y += g[k].y * xh[k].y;
                dw[k].z += g[k].z * xh[k].z; dw[k].w += g[k].w * xh[k].w;
                db[k].x += g[k].x; db[k].y += g[k].y; db[k].z += g[k].z; db[k].w += g[k].w;
            }
        }
    }
    float *mine = red + wave * 2 * C;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c = (k * 64 + lane) * 4;
        if (c < C) {
            bmb::st4(mine + c, dw[k]);
            bmb::st4(mine + C + c, db[k]);
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < 2 * C; j += LN_WAVES * 64) {
        float s = red[j];
#pragma unroll
        for (int q = 1; q < LN_WAVES; ++q) s += red[q * 2 * C + j];
        partial[(size_t)blockIdx.x * 2 * C + j] = s;
    }
}

// Any C: dinp only, one wave per row, scalar passes. The weight and bias
// gradients come from colsum_k<true> below.
__global__ __launch_bounds__(NT) void ln_bwd_dx_generic_k(float *dinp, const float *dout,
                                                           const float *inp, const float *weight,
                                                           const float *mean, const float *rstd,
                                                           int N, int C) {
    const int r = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= N) return;
    const float mu = mean[r], rs = rstd[r];
    const float *x = inp + (size_t)r * C;
    const float *dy = dout + (size_t)r * C;
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = lane; c < C; c += 64) {
        const float xh = (x[c] - mu) * rs, d = dy[c] * weight[c];
        s1 += d;
        s2 += d * xh;
    }
    const float m1 = wave_sum(s1) / (float)C, m2 = wave_sum(s2) / (float)C;
    float *dx = dinp + (size_t)r * C;
    for (int c = lane; c < C; c += 64) {
        const float xh = (x[c] - mu) * rs, d = dy[c] * weight[c];
        dx[c] += rs * (d - m1 - xh * m2);
    }
}

// Column sums over row chunks: block (strip, chunk) sums rows
// [chunk*rpc, (chunk+1)*rpc) of columns [strip*NT, strip*NT + NT), one column
// per lane, rows in ascending order.
//   LN == false: partial[chunk][c] = sum dout[r, c]                 (width C)
//   LN == true:  partial[chunk][c] = sum dout * xhat, [C + c] = sum dout (2C)
template <bool LN>
__global__ __launch_bounds__(NT) void colsum_k(float *partial, const float *dout,
                                                const float *inp, const float *mean,
                                                const float *rstd, int N, int C, int rpc) {
    const int c = blockIdx.x * NT + threadIdx.x;
    const int r0 = blockIdx.y * rpc;
    const int r1 = min(N, r0 + rpc);
    if (c >= C) return;
    float s0 = 0.0f, s1 = 0.0f;
    for (int r = r0; r < r1; ++r) {
        const float g = dout[(size_t)r * C + c];
        if (LN) s0 += g * ((inp[(size_t)r * C + c] - mean[r]) * rstd[r]);
        s1 += g;
    }
    const int width = LN ? 2 * C : C;
    float *p = partial + (size_t)blockIdx.y * width;
    if (LN) {
        p[c] = s0;
        p[C + c] = s1;
    } else {
        p[c] = s1;
    }
}

// The bias case of colsum_k with 128-bit loads (C % 4 == 0, dout 16-byte
// aligned): each lane owns 4 adjacent columns and adds its rows in the same
// order, so every column's partial sum is the same fp32 value as colsum_k's.
// Four times fewer load instructions; the row loop is unrolled so that
// several rows' loads are in flight at once.
__global__ __launch_bounds__(NT) void colsum4_k(float *partial, const float *dout, int N, int C,
                                                 int rpc) {
    const int C4 = C / 4;
    const int c4 = blockIdx.x * NT + threadIdx.x;
    const int r0 = blockIdx.y * rpc;
    const int r1 = min(N, r0 + rpc);
    if (c4 >= C4) return;
    const float4 *p = reinterpret_cast<const float4 *>(dout) + c4;
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
    for (int r = r0; r < r1; ++r) {
        const float4 g = p[(size_t)r * C4];
        s.x += g.x;
        s.y += g.y;
        s.z += g.z;
        s.w += g.w;
    }
    reinterpret_cast<float4 *>(partial + (size_t)blockIdx.y * C)[c4] = s;
}

// dst0[c] += sum_g partial[g][c] for c < C0, dst1[c - C0] += ... for the rest
// (width columns in all). A workgroup covers FIN_COLS columns with
// NT / FIN_COLS slices of lanes: slice q sums g = q, q + slices, ... in order,
// then the slice sums are added in slice order. Few columns per workgroup
// and many slices keep each lane's chain of dependent adds short (the
// partials are a few hundred rows and sit in L2; this kernel is latency-
// bound, not bandwidth-bound).
constexpr int FIN_COLS = 8;
__global__ __launch_bounds__(NT) void colsum_finish_k(float *dst0, float *dst1, int C0,
                                                       const float *partial, int G, int width) {
    constexpr int SL = NT / FIN_COLS;
    __shared__ float sl[SL][FIN_COLS];
    const int col = threadIdx.x % FIN_COLS, q = threadIdx.x / FIN_COLS;
    const int c = blockIdx.x * FIN_COLS + col;
    float s = 0.0f;
    if (c < width)
        for (int g = q; g < G; g += SL) s += partial[(size_t)g * width + c];
    sl[q][col] = s;
    __syncthreads();
    if (q == 0 && c < width) {
        float t = sl[0][col];
        for (int k = 1; k < SL; ++k) t += sl[k][col];
        if (c < C0)
            dst0[c] += t;
        else
            dst1[c - C0] += t;
    }
}

// ------------------------------------------------------------ elementwise ops
__device__ __forceinline__ float gelu1(float x) { return bmb::gelu(x); }
__device__ __forceinline__ float dgelu1(float x, float g) { return bmb::gelu_grad(x, g); }

// Flat elementwise map: work item i covers elements 4i .. 4i+3 (the last one
// may be partial); a grid-stride loop keeps the launch under the 2^32
// work-item limit of one dispatch for any n. OP is a functor with vec(base)
// and one(index).
constexpr long long MAP_MAX_BLOCKS = 1 << 20;

template <class OP>
__global__ __launch_bounds__(NT) void map_k(OP op, long long n) {
    const long long items = (n + 3) / 4;
    for (long long i = (long long)blockIdx.x * NT + threadIdx.x; i < items;
         i += (long long)gridDim.x * NT) {
        const long long base = i * 4;
        if (base + 3 < n)
            op.vec(base);
        else
            for (long long j = base; j < n; ++j) op.one(j);
    }
}

struct GeluFwd {
    float *out;
    const float *inp;
    __device__ void vec(long long i) const {
        const float4 x = ldu4(inp + i);
        stu4(out + i, make_float4(gelu1(x.x), gelu1(x.y), gelu1(x.z), gelu1(x.w)));
    }
    __device__ void one(long long i) const { out[i] = gelu1(inp[i]); }
};
struct GeluBwd {
    float *dinp;
    const float *inp, *dout;
    __device__ void vec(long long i) const {
        const float4 x = ldu4(inp + i), g = ldu4(dout + i);
        stu4(dinp + i, make_float4(dgelu1(x.x, g.x), dgelu1(x.y, g.y), dgelu1(x.z, g.z),
                                   dgelu1(x.w, g.w)));
    }
    __device__ void one(long long i) const { dinp[i] = dgelu1(inp[i], dout[i]); }
};
struct Residual {
    float *out;
    const float *a, *b;
    __device__ void vec(long long i) const {
        const float4 x = ldu4(a + i), y = ldu4(b + i);
        stu4(out + i, make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w));
    }
    __device__ void one(long long i) const { out[i] = a[i] + b[i]; }
};
struct AddInplace {
    float *dst;
    const float *src;
    __device__ void vec(long long i) const {
        const float4 x = ldu4(dst + i), y = ldu4(src + i);
        stu4(dst + i, make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w));
    }
    __device__ void one(long long i) const { dst[i] += src[i]; }
};
struct Zero {
    float *p;
    __device__ void vec(long long i) const { stu4(p + i, zero4()); }
    __device__ void one(long long i) const { p[i] = 0.0f; }
};

// AdamW (src/nn.cu:240-255, 336-343) with the reference's fp32 operation order. FP
// contraction is off here so that each product and sum rounds separately, as
// written; the result is then a function of the inputs alone.
__device__ __forceinline__ void adam1(float &p, float &m, float &v, float grad, float lr,
                                      float beta1, float beta2, float eps, float wd, float bc1,
                                      float bc2, float gscale) {
#pragma clang fp contract(off)
    const float g = grad * gscale;
    const float mi = beta1 * m + (1.0f - beta1) * g;
    const float vi = beta2 * v + (1.0f - beta2) * g * g;
    m = mi;
    v = vi;
    const float mhat = mi / bc1;
    const float vhat = vi / bc2;
    p = p - lr * (mhat / (sqrtf(vhat) + eps) + wd * p);
}

struct AdamW {
    float *params;
    const float *grads;
    float *m, *v;
    float lr, beta1, beta2, eps, wd, bc1, bc2, gscale;
    __device__ void one(long long i) const {
        float p = params[i], mi = m[i], vi = v[i];
        adam1(p, mi, vi, grads[i], lr, beta1, beta2, eps, wd, bc1, bc2, gscale);
        params[i] = p;
        m[i] = mi;
        v[i] = vi;
    }
    __device__ void vec(long long i) const {
        float4 p = ldu4(params + i), mi = ldu4(m + i), vi = ldu4(v + i);
        const float4 g = ldu4(grads + i);
        adam1(p.x, mi.x, vi.x, g.x, lr, beta1, beta2, eps, wd, bc1, bc2, gscale);
        adam1(p.y, mi.y, vi.y, g.y, lr, beta1, beta2, eps, wd, bc1, bc2, gscale);
        adam1(p.z, mi.z, vi.z, g.z, lr, beta1, beta2, eps, wd, bc1, bc2, gscale);
        adam1(p.w, mi.w, vi.w, g.w, lr, beta1, beta2, eps, wd, bc1, bc2, gscale);
        stu4(params + i, p);
        stu4(m + i, mi);
        stu4(v + i, vi);
    }
};

template <class OP>
void run_map(const OP &op, long long n) {
    if (n <= 0) return;
    const long long blocks = std::min(MAP_MAX_BLOCKS, ((n + 3) / 4 + NT - 1) / NT);
    bmb::launch(map_k<OP>, dim3((unsigned)blocks), dim3(NT), 0, nullptr, op, n);
}

// out[r, c] += bias[c]
template <bool VEC>
__global__ __launch_bounds__(NT) void bias_fwd_k(float *out, const float *bias, int C, int C4,
                                                  long long items) {
    const long long i = (long long)blockIdx.x * NT + threadIdx.x;
    if (i >= items) return;
    const int r = (int)(i / C4), c = (int)(i % C4) * 4;
    float *o = out + (size_t)r * C + c;
    if (VEC) {
        float4 v = ldu4(o);
        const float4 b = ldu4(bias + c);
        v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
        stu4(o, v);
    } else {
        for (int k = 0; k < 4 && c + k < C; ++k) o[k] += bias[c + k];
    }
}

// dlogits[r, i] = (probs[r, i] - [i == target]) * scale for i < V, 0 beyond.
template <bool VEC>
__global__ __launch_bounds__(NT) void xent_bwd_k(float *dlogits, const float *probs,
                                                  const int *targets, int V, int Vp, int C4,
                                                  long long items, float scale) {
    const long long i = (long long)blockIdx.x * NT + threadIdx.x;
    if (i >= items) return;
    const int r = (int)(i / C4), c = (int)(i % C4) * 4;
    const int tgt = targets[r];
    const float *p = probs + (size_t)r * Vp + c;
    float *d = dlogits + (size_t)r * Vp + c;
    if (VEC) {
        const float4 pv = ldu4(p);
        float4 o;
        o.x = c + 0 < V ? (pv.x - (c + 0 == tgt ? 1.0f : 0.0f)) * scale : 0.0f;
        o.y = c + 1 < V ? (pv.y - (c + 1 == tgt ? 1.0f : 0.0f)) * scale : 0.0f;
        o.z = c + 2 < V ? (pv.z - (c + 2 == tgt ? 1.0f : 0.0f)) * scale : 0.0f;
        o.w = c + 3 < V ? (pv.w - (c + 3 == tgt ? 1.0f : 0.0f)) * scale : 0.0f;
        stu4(d, o);
    } else {
        for (int k = 0; k < 4 && c + k < Vp; ++k)
            d[k] = c + k < V ? (p[k] - (c + k == tgt ? 1.0f : 0.0f)) * scale : 0.0f;
    }
}

// ------------------------------------------------------- softmax + cross-entropy
// One workgroup of NTHR lanes per row, the row's first V logits held in NCH
// float4 registers per lane (V <= 4*NTHR*NCH, Vp % 4 == 0): max, then
// exp(x - max) and its sum, then the normalised probabilities -- one read of
// the logits and one write of the probabilities (src/nn.cu:197-221).
// exp(x - m) is exp2((x - m) * log2 e) on v_exp_f32.
template <int NTHR>
__device__ __forceinline__ float block_reduce(float v, float *sh, bool is_max) {
    constexpr int NW = NTHR / 64;
    v = is_max ? wave_max(v) : wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();  // sh may still be read by a previous reduction
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float r = sh[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) r = is_max ? fmaxf(r, sh[k]) : r + sh[k];
    return r;
}

__device__ __forceinline__ float xent_loss(float p) { return -logf(fmaxf(p, 1e-30f)); }

template <int NTHR, int NCH>
__global__ __launch_bounds__(NTHR) void softmax_xent_k(float *probs, float *losses,
                                                        const float *logits, const int *targets,
                                                        int V, int Vp) {
    __shared__ float sh[NTHR / 64];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *x = logits + (size_t)row * Vp;
    float *p = probs + (size_t)row * Vp;
    float4 v[NCH];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c = (k * NTHR + tid) * 4;
        v[k] = c < V ? ldu4(x + c) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (c + 1 >= V) v[k].y = -INFINITY;
        if (c + 2 >= V) v[k].z = -INFINITY;
        if (c + 3 >= V) v[k].w = -INFINITY;
        m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
    }
    m = block_reduce<NTHR>(m, sh, true);
    const float ml = m * LOG2E;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        v[k].x = __builtin_amdgcn_exp2f(v[k].x * LOG2E - ml);
        v[k].y = __builtin_amdgcn_exp2f(v[k].y * LOG2E - ml);
        v[k].z = __builtin_amdgcn_exp2f(v[k].z * LOG2E - ml);
        v[k].w = __builtin_amdgcn_exp2f(v[k].w * LOG2E - ml);
        s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    s = block_reduce<NTHR>(s, sh, false);
    const float inv = 1.0f / s;
    const int tgt = targets[row];
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int c = (k * NTHR + tid) * 4;
        const float4 o = make_float4(v[k].x * inv, v[k].y * inv, v[k].z * inv, v[k].w * inv);
        if (c < Vp) stu4(p + c, o);  // columns in [V, Vp) come out as exp2(-inf) = 0
        if (tgt >= c && tgt < c + 4 && tgt < V) {
            const int j = tgt - c;
            const float pt = j == 0 ? o.x : j == 1 ? o.y : j == 2 ? o.z : o.w;
            losses[row] = xent_loss(pt);
        }
    }
    for (int c = (NCH * NTHR + tid) * 4; c < Vp; c += NTHR * 4) stu4(p + c, zero4());
    if (tid == 0) {
        if (tgt >= V && tgt < Vp) losses[row] = xent_loss(0.0f);
        if (tgt < 0 || tgt >= Vp) losses[row] = NAN;
    }
}

// Any V, Vp: three passes over the row with scalar accesses.
__global__ __launch_bounds__(NT) void softmax_xent_generic_k(float *probs, float *losses,
                                                              const float *logits,
                                                              const int *targets, int V, int Vp) {
    __shared__ float sh[NT / 64];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *x = logits + (size_t)row * Vp;
    float *p = probs + (size_t)row * Vp;
    float m = -INFINITY;
    for (int i = tid; i < V; i += NT) m = fmaxf(m, x[i]);
    m = block_reduce<NT>(m, sh, true);
    const float ml = m * LOG2E;
    float s = 0.0f;
    for (int i = tid; i < V; i += NT) {
        const float e = __builtin_amdgcn_exp2f(x[i] * LOG2E - ml);
        p[i] = e;
        s += e;
    }
    s = block_reduce<NT>(s, sh, false);
    const float inv = 1.0f / s;
    // Each lane rescales exactly the entries it wrote, so no barrier is needed.
    for (int i = tid; i < V; i += NT) p[i] *= inv;
    for (int i = V + tid; i < Vp; i += NT) p[i] = 0.0f;
    const int tgt = targets[row];
    if (tgt >= 0 && tgt < V && (tgt % NT) == tid) losses[row] = xent_loss(p[tgt]);
    if (tid == 0) {
        if (tgt >= V && tgt < Vp) losses[row] = xent_loss(0.0f);
        if (tgt < 0 || tgt >= Vp) losses[row] = NAN;
    }
}

// ------------------------------------------------------------- scalar results
// sum of squares in fp64: NORM_BLOCKS partials, then one workgroup adds them.
constexpr int NORM_BLOCKS = 1024;

__global__ __launch_bounds__(NT) void sumsq_k(double *partial, const float *g, long long n) {
    __shared__ double sh[NT / 64];
    double acc = 0.0;
    const long long n4 = n / 4;
    for (long long i = (long long)blockIdx.x * NT + threadIdx.x; i < n4;
         i += (long long)gridDim.x * NT) {
        const float4 v = ldu4(g + 4 * i);
        acc += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const double v = g[4 * n4 + threadIdx.x];
        acc += v * v;
    }
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// out = sqrt(sum partial) (SQRT) or sum(partial) / n, one workgroup.
template <bool SQRT>
__global__ __launch_bounds__(NT) void finish_scalar_k(float *out, const double *partial,
                                                       int count, long long n) {
    __shared__ double sh[NT / 64];
    double acc = 0.0;
    for (int i = threadIdx.x; i < count; i += NT) acc += partial[i];
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        const double s = (sh[0] + sh[1]) + (sh[2] + sh[3]);
        *out = SQRT ? (float)sqrt(s) : (float)(s / (double)n);
    }
}

// Sum of n floats in fp64 into partial[blockIdx.x] (grid-stride, scalar).
__global__ __launch_bounds__(NT) void sum_k(double *partial, const float *x, long long n) {
    __shared__ double sh[NT / 64];
    double acc = 0.0;
    for (long long i = (long long)blockIdx.x * NT + threadIdx.x; i < n;
         i += (long long)gridDim.x * NT)
        acc += x[i];
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// ------------------------------------------------------------------ host side
// The partial sums of a reduction live in a buffer leased for the call
// (workspace.hpp). A void op that cannot get one stops the process, as the
// reference's CUDA_CHECK does on any CUDA error (src/gpt.cu:18-26): returning
// would leave its gradients unwritten with nothing to tell the caller.
[[noreturn]] void scratch_failure(const char *what) {
    fprintf(stderr, "bmb: %s: cannot allocate the reduction scratch buffer\n", what);
    exit(1);
}

// Number of float4 chunks per lane for the register-resident row kernels.
int row_chunks(int C) {
    if (C % 4 != 0) return 0;
    const int n = ceil_div(C, 256);
    return n <= 4 ? n : 0;
}

// Column-sum launch for dout (N, C): G row chunks of rpc rows, chosen from the
// shape alone so that strips * G is about 1024 workgroups.
void colsum_shape(int N, int C, int &rpc, int &G) {
    const int strips = ceil_div(C, NT);
    int g = std::max(1, std::min(ceil_div(N, 16), ceil_div(1024, strips)));
    rpc = ceil_div(N, g);
    G = ceil_div(N, rpc);
}

void colsum_finish(float *d0, float *d1, int C0, const float *partial, int G, int width) {
    bmb::launch(colsum_finish_k, dim3(ceil_div(width, FIN_COLS)), dim3(NT), 0, nullptr, d0, d1,
                C0, partial, G, width);
}

template <int NCH, bool RES = false>
void ln_fwd_launch(float *out, float *mean, float *rstd, const float *inp, const float *w,
                   const float *b, int N, int C, float *res_out = nullptr,
                   const float *res_b = nullptr) {
    bmb::launch(ln_fwd_k<NCH, RES>, dim3(ceil_div(N, NT / 64)), dim3(NT), 0, nullptr, out, mean,
                rstd, inp, w, b, N, C, res_out, res_b);
}

template <int NCH>
void ln_bwd_launch(float *dinp, float *partial, const float *dout, const float *inp,
                   const float *w, const float *mean, const float *rstd, int N, int C, int rpb,
                   int G) {
    const size_t smem = (size_t)LN_WAVES * 2 * C * sizeof(float);
    bmb::allow_smem(ln_bwd_k<NCH>, smem);
    bmb::launch(ln_bwd_k<NCH>, dim3(G), dim3(LN_WAVES * 64), smem, nullptr, dinp, partial,
                dout, inp, w, mean, rstd, N, C, rpb);
}

template <int NTHR, int NCH>
void xent_launch(float *probs, float *losses, const float *logits, const int *targets, int N,
                 int V, int Vp) {
    bmb::launch(softmax_xent_k<NTHR, NCH>, dim3(N), dim3(NTHR), 0, nullptr, probs, losses,
                logits, targets, V, Vp);
}

float scalar_result(const float *dptr) {
    float h = NAN;
    const hipError_t e = hipMemcpy(&h, dptr, sizeof(float), hipMemcpyDeviceToHost);
    bmb::note_launch_status(e);
    return e == hipSuccess ? h : NAN;
}

}  // namespace

void bmb::residual_layernorm_forward(float *res_out, float *ln_out, float *mean, float *rstd,
                                     const float *a, const float *b, const float *weight,
                                     const float *bias, int N, int C) {
    if (N <= 0 || C <= 0) return;
    switch (row_chunks(C)) {
        case 1: return ln_fwd_launch<1, true>(ln_out, mean, rstd, a, weight, bias, N, C, res_out, b);
        case 2: return ln_fwd_launch<2, true>(ln_out, mean, rstd, a, weight, bias, N, C, res_out, b);
        case 3: return ln_fwd_launch<3, true>(ln_out, mean, rstd, a, weight, bias, N, C, res_out, b);
        case 4: return ln_fwd_launch<4, true>(ln_out, mean, rstd, a, weight, bias, N, C, res_out, b);
        default:
            residual_forward(res_out, a, b, N * C);
            layernorm_forward(ln_out, mean, rstd, res_out, weight, bias, N, C);
    }
}

extern "C" {

void encoder_forward(float *out, const int *tokens, const float *wte, const float *wpe, int B,
                     int T, int C) {
    if (B <= 0 || T <= 0 || C <= 0) return;
    const int C4 = ceil_div(C, 4);
    const long long items = (long long)B * T * C4;
    if (C % 4 == 0)
        bmb::launch(encoder_fwd_k<true>, dim3(grid_for(items)), dim3(NT), 0, nullptr, out,
                    tokens, wte, wpe, T, C, C4, items);
    else
        bmb::launch(encoder_fwd_k<false>, dim3(grid_for(items)), dim3(NT), 0, nullptr, out,
                    tokens, wte, wpe, T, C, C4, items);
}

void encoder_backward(float *dwte, float *dwpe, const float *dout, const int *tokens, int B,
                      int T, int C) {
    if (B <= 0 || T <= 0 || C <= 0) return;
    const int C4 = ceil_div(C, 4);
    const long long items = (long long)T * C4;
    if (C % 4 == 0)
        bmb::launch(encoder_bwd_wpe_k<true>, dim3(grid_for(items)), dim3(NT), 0, nullptr, dwpe,
                    dout, B, T, C, C4, items);
    else
        bmb::launch(encoder_bwd_wpe_k<false>, dim3(grid_for(items)), dim3(NT), 0, nullptr,
                    dwpe, dout, B, T, C, C4, items);
    const int N = B * T;
    bmb::launch(encoder_bwd_wte_k, dim3(ceil_div(N, NT / 64)), dim3(NT), 0, nullptr, dwte, dout,
                tokens, N, C);
}

void layernorm_forward(float *out, float *mean, float *rstd, const float *inp,
                       const float *weight, const float *bias, int N, int C) {
    if (N <= 0 || C <= 0) return;
    switch (row_chunks(C)) {
        case 1: ln_fwd_launch<1>(out, mean, rstd, inp, weight, bias, N, C); break;
        case 2: ln_fwd_launch<2>(out, mean, rstd, inp, weight, bias, N, C); break;
        case 3: ln_fwd_launch<3>(out, mean, rstd, inp, weight, bias, N, C); break;
        case 4: ln_fwd_launch<4>(out, mean, rstd, inp, weight, bias, N, C); break;
        default:
            bmb::launch(ln_fwd_generic_k, dim3(ceil_div(N, NT / 64)), dim3(NT), 0, nullptr, out,
                        mean, rstd, inp, weight, bias, N, C);
    }
}

void layernorm_backward(float *dinp, float *dweight, float *dbias, const float *dout,
                        const float *inp, const float *weight, const float *mean,
                        const float *rstd, int N, int C) {
    if (N <= 0 || C <= 0) return;
    const int nch = row_chunks(C);
    if (nch > 0) {
        // Workgroups of LN_WAVES waves, about 256 of them, whole waves of rows.
        const int G0 = std::max(1, std::min(256, ceil_div(N, LN_WAVES)));
        const int rpb = ceil_div(ceil_div(N, G0), LN_WAVES) * LN_WAVES;
        const int G = ceil_div(N, rpb);
        bmb::ScratchLease ws(bmb::SCRATCH_NN, (size_t)G * 2 * C * sizeof(float));
        if (!ws) scratch_failure("layernorm_backward");
        float *partial = static_cast<float *>(ws.get());
        switch (nch) {
            case 1: ln_bwd_launch<1>(dinp, partial, dout, inp, weight, mean, rstd, N, C, rpb, G); break;
            case 2: ln_bwd_launch<2>(dinp, partial, dout, inp, weight, mean, rstd, N, C, rpb, G); break;
            case 3: ln_bwd_launch<3>(dinp, partial, dout, inp, weight, mean, rstd, N, C, rpb, G); break;
            default: ln_bwd_launch<4>(dinp, partial, dout, inp, weight, mean, rstd, N, C, rpb, G); break;
        }
        colsum_finish(dweight, dbias, C, partial, G, 2 * C);
        return;
    }
    int rpc, G;
    colsum_shape(N, C, rpc, G);
    bmb::ScratchLease ws(bmb::SCRATCH_NN, (size_t)G * 2 * C * sizeof(float));
    if (!ws) scratch_failure("layernorm_backward");
    float *partial = static_cast<float *>(ws.get());
    bmb::launch(ln_bwd_dx_generic_k, dim3(ceil_div(N, NT / 64)), dim3(NT), 0, nullptr, dinp,
                dout, inp, weight, mean, rstd, N, C);
    bmb::launch(colsum_k<true>, dim3(ceil_div(C, NT), G), dim3(NT), 0, nullptr, partial, dout,
                inp, mean, rstd, N, C, rpc);
    colsum_finish(dweight, dbias, C, partial, G, 2 * C);
}

void gelu_forward(float *out, const float *inp, int n) { run_map(GeluFwd{out, inp}, n); }

void gelu_backward(float *dinp, const float *inp, const float *dout, int n) {
    run_map(GeluBwd{dinp, inp, dout}, n);
}

void residual_forward(float *out, const float *a, const float *b, int n) {
    run_map(Residual{out, a, b}, n);
}

void add_inplace(float *dst, const float *src, int n) { run_map(AddInplace{dst, src}, n); }

void bias_forward(float *out, const float *bias, int N, int C) {
    if (N <= 0 || C <= 0) return;
    const int C4 = ceil_div(C, 4);
    const long long items = (long long)N * C4;
    if (C % 4 == 0)
        bmb::launch(bias_fwd_k<true>, dim3(grid_for(items)), dim3(NT), 0, nullptr, out, bias, C,
                    C4, items);
    else
        bmb::launch(bias_fwd_k<false>, dim3(grid_for(items)), dim3(NT), 0, nullptr, out, bias,
                    C, C4, items);
}

void bias_backward(float *dbias, const float *dout, int N, int C) {
    if (N <= 0 || C <= 0) return;
    int rpc, G;
    colsum_shape(N, C, rpc, G);
    bmb::ScratchLease ws(bmb::SCRATCH_NN, (size_t)G * C * sizeof(float));
    if (!ws) scratch_failure("bias_backward");
    float *partial = static_cast<float *>(ws.get());
    if (C % 4 == 0 && ((uintptr_t)dout & 15u) == 0)
        bmb::launch(colsum4_k, dim3(ceil_div(C / 4, NT), G), dim3(NT), 0, nullptr, partial, dout,
                    N, C, rpc);
    else
        bmb::launch(colsum_k<false>, dim3(ceil_div(C, NT), G), dim3(NT), 0, nullptr, partial,
                    dout, nullptr, nullptr, nullptr, N, C, rpc);
    colsum_finish(dbias, dbias, C, partial, G, C);
}

void softmax_crossentropy_forward(float *probs, float *losses, const float *logits,
                                  const int *targets, int N, int V, int Vp) {
    if (N <= 0 || V <= 0 || Vp < V) return;
    if (Vp % 4 == 0) {
        if (V <= 1024) return xent_launch<256, 1>(probs, losses, logits, targets, N, V, Vp);
        if (V <= 4096) return xent_launch<256, 4>(probs, losses, logits, targets, N, V, Vp);
        if (V <= 16384) return xent_launch<1024, 4>(probs, losses, logits, targets, N, V, Vp);
        if (V <= 32768) return xent_launch<1024, 8>(probs, losses, logits, targets, N, V, Vp);
        if (V <= 65536) return xent_launch<1024, 16>(probs, losses, logits, targets, N, V, Vp);
    }
    bmb::launch(softmax_xent_generic_k, dim3(N), dim3(NT), 0, nullptr, probs, losses, logits,
                targets, V, Vp);
}

void crossentropy_softmax_backward(float *dlogits, const float *probs, const int *targets,
                                   int N, int V, int Vp, float dloss_scale) {
    if (N <= 0 || Vp <= 0) return;
    const int C4 = ceil_div(Vp, 4);
    const long long items = (long long)N * C4;
    if (Vp % 4 == 0)
        bmb::launch(xent_bwd_k<true>, dim3(grid_for(items)), dim3(NT), 0, nullptr, dlogits,
                    probs, targets, V, Vp, C4, items, dloss_scale);
    else
        bmb::launch(xent_bwd_k<false>, dim3(grid_for(items)), dim3(NT), 0, nullptr, dlogits,
                    probs, targets, V, Vp, C4, items, dloss_scale);
}

void adamw_update(float *params, float *grads, float *m, float *v, int n, float lr, float beta1,
                  float beta2, float eps, float weight_decay, int step, float grad_scale) {
    const float bc1 = 1.0f - powf(beta1, (float)step);
    const float bc2 = 1.0f - powf(beta2, (float)step);
    run_map(AdamW{params, grads, m, v, lr, beta1, beta2, eps, weight_decay, bc1, bc2, grad_scale},
            n);
}

float grad_global_norm(const float *grads, int n) {
    if (n <= 0) return 0.0f;
    bmb::ScratchLease ws(bmb::SCRATCH_NN, NORM_BLOCKS * sizeof(double) + 256);
    if (!ws) {
        fprintf(stderr, "bmb: grad_global_norm: cannot allocate the reduction scratch buffer\n");
        bmb::note_launch_status(hipErrorOutOfMemory);
        return NAN;
    }
    double *partial = static_cast<double *>(ws.get());
    float *out = reinterpret_cast<float *>(partial + NORM_BLOCKS);
    const int blocks = (int)std::max(1LL, std::min<long long>(NORM_BLOCKS, (n / 4 + NT - 1) / NT));
    bmb::launch(sumsq_k, dim3(blocks), dim3(NT), 0, nullptr, partial, grads, (long long)n);
    bmb::launch(finish_scalar_k<true>, dim3(1), dim3(NT), 0, nullptr, out,
                (const double *)partial, blocks, (long long)n);
    return scalar_result(out);
}

void zero_buffer(float *p, size_t n) { run_map(Zero{p}, (long long)n); }

float reduce_mean(const float *d_values, int n) {
    if (n <= 0) return NAN;
    bmb::ScratchLease ws(bmb::SCRATCH_NN, NORM_BLOCKS * sizeof(double) + 256);
    if (!ws) {
        fprintf(stderr, "bmb: reduce_mean: cannot allocate the reduction scratch buffer\n");
        bmb::note_launch_status(hipErrorOutOfMemory);
        return NAN;
    }
    double *partial = static_cast<double *>(ws.get());
    float *out = reinterpret_cast<float *>(partial + NORM_BLOCKS);
    const int blocks = (int)std::max(1LL, std::min<long long>(NORM_BLOCKS, ((long long)n + NT - 1) / NT));
    bmb::launch(sum_k, dim3(blocks), dim3(NT), 0, nullptr, partial, d_values, (long long)n);
    bmb::launch(finish_scalar_k<false>, dim3(1), dim3(NT), 0, nullptr, out,
                (const double *)partial, blocks, (long long)n);
    return scalar_result(out);
}

}  // extern "C"
