/*
 * CPU oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h). Not linked into, or
 * called by, the shipped HIP library. Loaded by tests/, by
 * __graft_entry__.smoke() as its checker, and by bench.py for the CPU
 * baseline measurement.
 *
 * Built with -ffp-contract=off so that every fused multiply-add below is an
 * explicit fmaf()/fma() and no other expression is silently contracted.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fills */

static inline uint32_t xs32(uint32_t s) {
    /* Marsaglia's xorshift32, triple (13, 17, 5): src/bench.cu:62. */
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}

void orc_xorshift_stream(uint32_t *out, size_t n, uint32_t seed) {
    uint32_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        s = xs32(s);
        out[i] = s;
    }
}

void orc_fill_xorshift(float *v, size_t n, uint32_t seed) {
    /* src/bench.cu:59-66: v = (float)((int)(s % 2000) - 1000) / 1000.0f */
    uint32_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        s = xs32(s);
        v[i] = (float)((int)(s % 2000u) - 1000) / 1000.0f;
    }
}

void orc_fill_normal(float *v, size_t n, uint32_t seed, float stddev) {
    const double two_pi = 6.283185307179586476925286766559;
    uint32_t s = seed;
    size_t i = 0;
    while (i < n) {
        s = xs32(s);
        const double u1 = ((double)s + 1.0) / 4294967296.0; /* (0, 1] */
        s = xs32(s);
        const double u2 = (double)s / 4294967296.0; /* [0, 1) */
        const double r = sqrt(-2.0 * log(u1));
        v[i++] = (float)(stddev * r * cos(two_pi * u2));
        if (i < n) v[i++] = (float)(stddev * r * sin(two_pi * u2));
    }
}

/* ------------------------------------------------------------------- GEMM */

static inline float elemA(int ta, const float *A, int M, int K, int i, int k) {
    return ta ? A[(size_t)k * M + i] : A[(size_t)i * K + k];
}
static inline float elemB(int tb, const float *B, int N, int K, int k, int j) {
    return tb ? B[(size_t)j * K + k] : B[(size_t)k * N + j];
}

/* One output row i, k-sequential fmaf per output (see oracle.h). */
static void gemm_row_f32seq(int ta, int tb, int M, int N, int K, float alpha,
                            const float *A, const float *B, float beta,
                            float *C, int i, float *acc) {
    for (int j = 0; j < N; ++j) acc[j] = 0.0f;
    for (int k = 0; k < K; ++k) {
        const float a = elemA(ta, A, M, K, i, k);
        if (!tb) {
            const float *brow = B + (size_t)k * N;
            for (int j = 0; j < N; ++j) acc[j] = fmaf(a, brow[j], acc[j]);
        } else {
            for (int j = 0; j < N; ++j)
                acc[j] = fmaf(a, B[(size_t)j * K + k], acc[j]);
        }
    }
    float *crow = C + (size_t)i * N;
    if (beta == 0.0f) {
        for (int j = 0; j < N; ++j) crow[j] = alpha * acc[j];
    } else {
        for (int j = 0; j < N; ++j) crow[j] = fmaf(alpha, acc[j], beta * crow[j]);
    }
}

void orc_gemm_f32seq(int ta, int tb, int M, int N, int K, float alpha,
                     const float *A, const float *B, float beta, float *C) {
    float *acc = (float *)malloc(sizeof(float) * (size_t)(N > 0 ? N : 1));
    for (int i = 0; i < M; ++i)
        gemm_row_f32seq(ta, tb, M, N, K, alpha, A, B, beta, C, i, acc);
    free(acc);
}

void orc_gemm_f32seq_mt(int ta, int tb, int M, int N, int K, float alpha,
                        const float *A, const float *B, float beta, float *C,
                        int threads) {
#ifdef _OPENMP
    if (threads < 1) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)(N > 0 ? N : 1));
#pragma omp for schedule(static)
        for (int i = 0; i < M; ++i)
            gemm_row_f32seq(ta, tb, M, N, K, alpha, A, B, beta, C, i, acc);
        free(acc);
    }
#else
    (void)threads;
    orc_gemm_f32seq(ta, tb, M, N, K, alpha, A, B, beta, C);
#endif
}

void orc_gemm_f64(int ta, int tb, int M, int N, int K, double alpha,
                  const float *A, const float *B, double beta, const float *C0,
                  double *Cout) {
    /* Rows are independent: OpenMP over i (each row is computed by one
     * thread, so the result does not depend on the thread count). Row i of
     * op(A) is widened into a contiguous buffer; with transB the j-th output
     * is then a dot product of two k-contiguous rows, otherwise the k loop
     * streams rows of B -- both cache friendly whatever the transposes. */
#pragma omp parallel
    {
        double *acc = (double *)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
        double *arow = (double *)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(dynamic, 4)
        for (int i = 0; i < M; ++i) {
            for (int k = 0; k < K; ++k) arow[k] = (double)elemA(ta, A, M, K, i, k);
            if (tb) {
                for (int j = 0; j < N; ++j) {
                    const float *brow = B + (size_t)j * K;
                    double d = 0.0;
                    for (int k = 0; k < K; ++k) d += arow[k] * (double)brow[k];
                    acc[j] = d;
                }
            } else {
                for (int j = 0; j < N; ++j) acc[j] = 0.0;
                for (int k = 0; k < K; ++k) {
                    const double a = arow[k];
                    const float *brow = B + (size_t)k * N;
                    for (int j = 0; j < N; ++j) acc[j] += a * (double)brow[j];
                }
            }
            for (int j = 0; j < N; ++j) {
                const size_t idx = (size_t)i * N + j;
                double c = alpha * acc[j];
                if (beta != 0.0) c += beta * (double)C0[idx];
                Cout[idx] = c;
            }
        }
        free(acc);
        free(arow);
    }
}

void orc_batched_gemm_f32seq(int ta, int tb, int batch, int M, int N, int K,
                             float alpha, const float *A, long long sA,
                             const float *B, long long sB, float beta, float *C,
                             long long sC) {
    for (int z = 0; z < batch; ++z)
        orc_gemm_f32seq(ta, tb, M, N, K, alpha, A + z * sA, B + z * sB, beta,
                        C + z * sC);
}

void orc_batched_gemm_f64(int ta, int tb, int batch, int M, int N, int K,
                          double alpha, const float *A, long long sA,
                          const float *B, long long sB, double beta,
                          const float *C0, long long sC, double *Cout) {
    for (int z = 0; z < batch; ++z)
        orc_gemm_f64(ta, tb, M, N, K, alpha, A + z * sA, B + z * sB, beta,
                     C0 ? C0 + z * sC : NULL, Cout + z * sC);
}

/* ----------------------------------------------------------------- metric */

double orc_normwise_f32(const float *got, const float *ref, size_t n,
                        size_t *nonfinite) {
    double maxabs = 0.0, refinf = 0.0;
    size_t bad = 0;
    for (size_t i = 0; i < n; ++i) {
        const double g = (double)got[i], r = (double)ref[i];
        if (!isfinite(g)) { ++bad; continue; }
        const double d = fabs(g - r);
        if (d > maxabs) maxabs = d;
        if (fabs(r) > refinf) refinf = fabs(r);
    }
    if (nonfinite) *nonfinite = bad;
    return maxabs / (refinf > 1e-30 ? refinf : 1e-30);
}

double orc_normwise_f64(const float *got, const double *ref, size_t n,
                        size_t *nonfinite) {
    double maxabs = 0.0, refinf = 0.0;
    size_t bad = 0;
    for (size_t i = 0; i < n; ++i) {
        const double g = (double)got[i], r = ref[i];
        if (!isfinite(g)) { ++bad; continue; }
        const double d = fabs(g - r);
        if (d > maxabs) maxabs = d;
        if (fabs(r) > refinf) refinf = fabs(r);
    }
    if (nonfinite) *nonfinite = bad;
    return maxabs / (refinf > 1e-30 ? refinf : 1e-30);
}

/* -------------------------------------------------------------- attention */

void orc_attn_fwd_f64(const float *qkv, int B, int T, int C, int NH,
                      double *out, double *lse) {
    const int hs = C / NH;
    const double scale = 1.0 / sqrt((double)hs);
    double *s = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < NH; ++h)
            for (int i = 0; i < T; ++i) {
                const float *q = qkv + ((size_t)b * T + i) * 3 * C + h * hs;
                double m = -INFINITY;
                for (int j = 0; j <= i; ++j) { /* causal: j <= i */
                    const float *k = qkv + ((size_t)b * T + j) * 3 * C + C + h * hs;
                    double d = 0.0;
                    for (int x = 0; x < hs; ++x) d += (double)q[x] * (double)k[x];
                    s[j] = scale * d;
                    if (s[j] > m) m = s[j];
                }
                double l = 0.0;
                for (int j = 0; j <= i; ++j) {
                    s[j] = exp(s[j] - m);
                    l += s[j];
                }
                double *o = out + ((size_t)b * T + i) * C + h * hs;
                for (int x = 0; x < hs; ++x) o[x] = 0.0;
                for (int j = 0; j <= i; ++j) {
                    const float *v = qkv + ((size_t)b * T + j) * 3 * C + 2 * C + h * hs;
                    const double p = s[j] / l;
                    for (int x = 0; x < hs; ++x) o[x] += p * (double)v[x];
                }
                lse[((size_t)b * NH + h) * T + i] = m + log(l);
            }
    free(s);
}

void orc_dsum_f64(const float *dout, const float *out, int B, int T, int C,
                  int NH, double *dsum) {
    const int hs = C / NH;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < NH; ++h)
            for (int t = 0; t < T; ++t) {
                const size_t off = ((size_t)b * T + t) * C + (size_t)h * hs;
                double d = 0.0;
                for (int x = 0; x < hs; ++x)
                    d += (double)dout[off + x] * (double)out[off + x];
                dsum[((size_t)b * NH + h) * T + t] = d;
            }
}

void orc_attn_bwd_f64(const float *qkv, const float *dout, int B, int T, int C,
                      int NH, double *dqkv) {
    const int hs = C / NH;
    const double scale = 1.0 / sqrt((double)hs);
    const size_t TT = (size_t)T * T;
    double *P = (double *)malloc(sizeof(double) * (TT > 0 ? TT : 1));
    double *dS = (double *)malloc(sizeof(double) * (TT > 0 ? TT : 1));
    memset(dqkv, 0, sizeof(double) * (size_t)B * T * 3 * C);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < NH; ++h) {
            const float *base = qkv + (size_t)b * T * 3 * C + h * hs;
            const float *dob = dout + (size_t)b * T * C + h * hs;
            double *dbase = dqkv + (size_t)b * T * 3 * C + h * hs;
            /* P row by row (causal), then dP, D and dS */
            for (int i = 0; i < T; ++i) {
                const float *q = base + (size_t)i * 3 * C;
                double m = -INFINITY;
                for (int j = 0; j <= i; ++j) {
                    const float *k = base + (size_t)j * 3 * C + C;
                    double d = 0.0;
                    for (int x = 0; x < hs; ++x) d += (double)q[x] * (double)k[x];
                    P[(size_t)i * T + j] = scale * d;
                    if (P[(size_t)i * T + j] > m) m = P[(size_t)i * T + j];
                }
                double l = 0.0;
                for (int j = 0; j <= i; ++j) {
                    P[(size_t)i * T + j] = exp(P[(size_t)i * T + j] - m);
                    l += P[(size_t)i * T + j];
                }
                for (int j = 0; j <= i; ++j) P[(size_t)i * T + j] /= l;
                const float *g = dob + (size_t)i * C;
                double D = 0.0;
                for (int j = 0; j <= i; ++j) {
                    const float *v = base + (size_t)j * 3 * C + 2 * C;
                    double dp = 0.0;
                    for (int x = 0; x < hs; ++x) dp += (double)g[x] * (double)v[x];
                    dS[(size_t)i * T + j] = dp;
                    D += P[(size_t)i * T + j] * dp;
                }
                for (int j = 0; j <= i; ++j)
                    dS[(size_t)i * T + j] = P[(size_t)i * T + j] * (dS[(size_t)i * T + j] - D);
            }
            for (int i = 0; i < T; ++i) {
                double *dq = dbase + (size_t)i * 3 * C;
                const float *g = dob + (size_t)i * C;
                const float *q = base + (size_t)i * 3 * C;
                for (int j = 0; j <= i; ++j) {
                    const float *k = base + (size_t)j * 3 * C + C;
                    double *dk = dbase + (size_t)j * 3 * C + C;
                    double *dv = dbase + (size_t)j * 3 * C + 2 * C;
                    const double ds = dS[(size_t)i * T + j], p = P[(size_t)i * T + j];
                    for (int x = 0; x < hs; ++x) {
                        dq[x] += scale * ds * (double)k[x];
                        dk[x] += scale * ds * (double)q[x];
                        dv[x] += p * (double)g[x];
                    }
                }
            }
        }
    free(P);
    free(dS);
}

/* fp32 unfused attention (src/attention.cu:132-200) for one (b, h). */
static void attn_head_f32(const float *qkv, const float *dout, int T, int C,
                          int hs, int b, int h, float scale, float *out,
                          float *dqkv, float *att, float *datt) {
    const float *base = qkv + (size_t)b * T * 3 * C + h * hs;
    const float *dob = dout + (size_t)b * T * C + h * hs;
    float *ob = out + (size_t)b * T * C + h * hs;
    float *db = dqkv + (size_t)b * T * 3 * C + h * hs;
    /* preatt = scale * q @ k^T over the full T x T (bgemm NT, alpha=scale) */
    for (int i = 0; i < T; ++i) {
        const float *q = base + (size_t)i * 3 * C;
        for (int j = 0; j < T; ++j) {
            const float *k = base + (size_t)j * 3 * C + C;
            float acc = 0.0f;
            for (int x = 0; x < hs; ++x) acc = fmaf(q[x], k[x], acc);
            att[(size_t)i * T + j] = scale * acc;
        }
    }
    /* causal softmax with explicit zeros (attention.cu:86-110) */
    for (int i = 0; i < T; ++i) {
        float *y = att + (size_t)i * T;
        float m = -INFINITY;
        for (int j = 0; j <= i; ++j) m = fmaxf(m, y[j]);
        float s = 0.0f;
        for (int j = 0; j <= i; ++j) { y[j] = expf(y[j] - m); s += y[j]; }
        const float inv = 1.0f / s;
        for (int j = 0; j <= i; ++j) y[j] *= inv;
        for (int j = i + 1; j < T; ++j) y[j] = 0.0f;
    }
    /* out = att @ v */
    for (int i = 0; i < T; ++i) {
        float *o = ob + (size_t)i * C;
        for (int x = 0; x < hs; ++x) o[x] = 0.0f;
        for (int j = 0; j < T; ++j) {
            const float p = att[(size_t)i * T + j];
            const float *v = base + (size_t)j * 3 * C + 2 * C;
            for (int x = 0; x < hs; ++x) o[x] = fmaf(p, v[x], o[x]);
        }
    }
    /* datt = dout @ v^T ; dv = att^T @ dout */
    for (int i = 0; i < T; ++i) {
        const float *g = dob + (size_t)i * C;
        for (int j = 0; j < T; ++j) {
            const float *v = base + (size_t)j * 3 * C + 2 * C;
            float acc = 0.0f;
            for (int x = 0; x < hs; ++x) acc = fmaf(g[x], v[x], acc);
            datt[(size_t)i * T + j] = acc;
        }
    }
    for (int j = 0; j < T; ++j) {
        float *dv = db + (size_t)j * 3 * C + 2 * C;
        for (int x = 0; x < hs; ++x) dv[x] = 0.0f;
    }
    for (int i = 0; i < T; ++i) {
        const float *g = dob + (size_t)i * C;
        for (int j = 0; j < T; ++j) {
            const float p = att[(size_t)i * T + j];
            float *dv = db + (size_t)j * 3 * C + 2 * C;
            for (int x = 0; x < hs; ++x) dv[x] = fmaf(p, g[x], dv[x]);
        }
    }
    /* softmax backward (attention.cu:113-129), in place in datt */
    for (int i = 0; i < T; ++i) {
        const float *y = att + (size_t)i * T;
        float *dy = datt + (size_t)i * T;
        float dot = 0.0f;
        for (int j = 0; j <= i; ++j) dot = fmaf(dy[j], y[j], dot);
        for (int j = 0; j <= i; ++j) dy[j] = y[j] * (dy[j] - dot);
        for (int j = i + 1; j < T; ++j) dy[j] = 0.0f;
    }
    /* dq = scale * dpreatt @ k ; dk = scale * dpreatt^T @ q */
    for (int i = 0; i < T; ++i) {
        float *dq = db + (size_t)i * 3 * C;
        float acc[256];
        for (int x = 0; x < hs; ++x) acc[x] = 0.0f;
        for (int j = 0; j < T; ++j) {
            const float d = datt[(size_t)i * T + j];
            const float *k = base + (size_t)j * 3 * C + C;
            for (int x = 0; x < hs; ++x) acc[x] = fmaf(d, k[x], acc[x]);
        }
        for (int x = 0; x < hs; ++x) dq[x] = scale * acc[x];
    }
    for (int j = 0; j < T; ++j) {
        float *dk = db + (size_t)j * 3 * C + C;
        float acc[256];
        for (int x = 0; x < hs; ++x) acc[x] = 0.0f;
        for (int i = 0; i < T; ++i) {
            const float d = datt[(size_t)i * T + j];
            const float *q = base + (size_t)i * 3 * C;
            for (int x = 0; x < hs; ++x) acc[x] = fmaf(d, q[x], acc[x]);
        }
        for (int x = 0; x < hs; ++x) dk[x] = scale * acc[x];
    }
}

void orc_attn_fwdbwd_f32(const float *qkv, const float *dout, int B, int T,
                         int C, int NH, float *out, float *dqkv, int threads) {
    const int hs = C / NH;
    const float scale = 1.0f / sqrtf((float)hs);
    if (hs > 256) return;
#ifdef _OPENMP
    if (threads < 1) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
    {
        float *att = (float *)malloc(sizeof(float) * (size_t)T * T);
        float *datt = (float *)malloc(sizeof(float) * (size_t)T * T);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int bh = 0; bh < B * NH; ++bh)
            attn_head_f32(qkv, dout, T, C, hs, bh / NH, bh % NH, scale, out,
                          dqkv, att, datt);
        free(att);
        free(datt);
    }
    (void)threads;
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
