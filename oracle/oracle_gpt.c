/*
 * CPU oracle for the transformer building blocks (src/nn.cu) and the GPT
 * model (src/gpt.cu) -- TEST INFRASTRUCTURE ONLY (see oracle.h). Not linked
 * into, or called by, the shipped HIP library.
 *
 * Everything is computed in fp64 from fp64 inputs (the fp32 values the GPU
 * sees, widened exactly), except orc_adamw_f32, which restates the
 * reference's fp32 AdamW operation by operation so that the GPU update can be
 * compared bit for bit. Built with -ffp-contract=off like oracle.c.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- nn ops */

void orc_encoder_fwd(double *out, const int *tokens, const double *wte,
                     const double *wpe, int B, int T, int C) {
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t) {
            const size_t r = (size_t)b * T + t;
            const double *e = wte + (size_t)tokens[r] * C;
            const double *p = wpe + (size_t)t * C;
            for (int c = 0; c < C; ++c) out[r * C + c] = e[c] + p[c];
        }
}

void orc_encoder_bwd(double *dwte, double *dwpe, const double *dout,
                     const int *tokens, int B, int T, int C) {
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t) {
            const size_t r = (size_t)b * T + t;
            for (int c = 0; c < C; ++c) {
                dwte[(size_t)tokens[r] * C + c] += dout[r * C + c];
                dwpe[(size_t)t * C + c] += dout[r * C + c];
            }
        }
}

void orc_layernorm_fwd(double *out, double *mean, double *rstd,
                       const double *inp, const double *w, const double *b,
                       int N, int C) {
    for (int r = 0; r < N; ++r) {
        const double *x = inp + (size_t)r * C;
        double mu = 0.0;
        for (int c = 0; c < C; ++c) mu += x[c];
        mu /= C;
        double var = 0.0;
        for (int c = 0; c < C; ++c) var += (x[c] - mu) * (x[c] - mu);
        var /= C;
        const double rs = 1.0 / sqrt(var + 1e-5);
        mean[r] = mu;
        rstd[r] = rs;
        for (int c = 0; c < C; ++c)
            out[(size_t)r * C + c] = (x[c] - mu) * rs * w[c] + b[c];
    }
}

void orc_layernorm_bwd(double *dinp, double *dw, double *db,
                       const double *dout, const double *inp, const double *w,
                       const double *mean, const double *rstd, int N, int C) {
    for (int r = 0; r < N; ++r) {
        const double *x = inp + (size_t)r * C;
        const double *dy = dout + (size_t)r * C;
        const double mu = mean[r], rs = rstd[r];
        double m1 = 0.0, m2 = 0.0;
        for (int c = 0; c < C; ++c) {
            const double xh = (x[c] - mu) * rs, d = dy[c] * w[c];
            m1 += d;
            m2 += d * xh;
        }
        m1 /= C;
        m2 /= C;
        for (int c = 0; c < C; ++c) {
            const double xh = (x[c] - mu) * rs, d = dy[c] * w[c];
            dinp[(size_t)r * C + c] += rs * (d - m1 - xh * m2);
            dw[c] += dy[c] * xh;
            db[c] += dy[c];
        }
    }
}

#define GELU_S 0.7978845608028654 /* sqrt(2/pi) */
#define GELU_C 0.044715

void orc_gelu_fwd(double *out, const double *inp, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const double x = inp[i];
        out[i] = 0.5 * x * (1.0 + tanh(GELU_S * (x + GELU_C * x * x * x)));
    }
}

void orc_gelu_bwd(double *dinp, const double *inp, const double *dout, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const double x = inp[i];
        const double t = tanh(GELU_S * (x + GELU_C * x * x * x));
        const double dinner = GELU_S * (1.0 + 3.0 * GELU_C * x * x);
        dinp[i] = dout[i] * (0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * dinner);
    }
}

void orc_bias_bwd(double *dbias, const double *dout, int N, int C) {
    for (int r = 0; r < N; ++r)
        for (int c = 0; c < C; ++c) dbias[c] += dout[(size_t)r * C + c];
}

void orc_softmax_xent_fwd(double *probs, double *losses, const double *logits,
                          const int *targets, int N, int V, int Vp) {
    for (int r = 0; r < N; ++r) {
        const double *x = logits + (size_t)r * Vp;
        double *p = probs + (size_t)r * Vp;
        double m = -INFINITY;
        for (int i = 0; i < V; ++i) m = x[i] > m ? x[i] : m;
        double s = 0.0;
        for (int i = 0; i < V; ++i) {
            p[i] = exp(x[i] - m);
            s += p[i];
        }
        for (int i = 0; i < V; ++i) p[i] /= s;
        for (int i = V; i < Vp; ++i) p[i] = 0.0;
        if (losses) {
            const int t = targets[r];
            if (t < 0 || t >= Vp) {
                losses[r] = NAN;
            } else {
                const double pt = p[t] > 1e-30 ? p[t] : 1e-30;
                losses[r] = -log(pt);
            }
        }
    }
}

void orc_xent_bwd(double *dlogits, const double *probs, const int *targets,
                  int N, int V, int Vp, double scale) {
    for (int r = 0; r < N; ++r)
        for (int i = 0; i < Vp; ++i) {
            const double ind = (i == targets[r]) ? 1.0 : 0.0;
            dlogits[(size_t)r * Vp + i] =
                i < V ? (probs[(size_t)r * Vp + i] - ind) * scale : 0.0;
        }
}

void orc_adamw_f32(float *params, const float *grads, float *m, float *v,
                   size_t n, float lr, float beta1, float beta2, float eps,
                   float wd, int step, float grad_scale) {
    const float bc1 = 1.0f - powf(beta1, (float)step);
    const float bc2 = 1.0f - powf(beta2, (float)step);
    for (size_t i = 0; i < n; ++i) {
        const float g = grads[i] * grad_scale;
        const float mi = beta1 * m[i] + (1.0f - beta1) * g;
        const float vi = beta2 * v[i] + (1.0f - beta2) * g * g;
        m[i] = mi;
        v[i] = vi;
        const float mhat = mi / bc1;
        const float vhat = vi / bc2;
        params[i] = params[i] - lr * (mhat / (sqrtf(vhat) + eps) + wd * params[i]);
    }
}

/* ------------------------------------------------- attention (fp64, saved P) */

/* out = causal softmax(q k^T * scale) v per (b, h); att (B,NH,T,T) keeps the
 * post-softmax weights with explicit zeros above the diagonal
 * (src/attention.cu:86-110). */
static void attn_fwd_d(double *out, double *att, const double *qkv, int B,
                       int T, int C, int NH) {
    const int hs = C / NH;
    const double scale = 1.0 / sqrt((double)hs);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < NH; ++h) {
            double *A = att + ((size_t)b * NH + h) * T * T;
            for (int i = 0; i < T; ++i) {
                const double *q = qkv + ((size_t)b * T + i) * 3 * C + h * hs;
                double *row = A + (size_t)i * T;
                double m = -INFINITY;
                for (int j = 0; j <= i; ++j) {
                    const double *k = qkv + ((size_t)b * T + j) * 3 * C + C + h * hs;
                    double d = 0.0;
                    for (int x = 0; x < hs; ++x) d += q[x] * k[x];
                    row[j] = d * scale;
                    if (row[j] > m) m = row[j];
                }
                double s = 0.0;
                for (int j = 0; j <= i; ++j) {
                    row[j] = exp(row[j] - m);
                    s += row[j];
                }
                for (int j = 0; j <= i; ++j) row[j] /= s;
                for (int j = i + 1; j < T; ++j) row[j] = 0.0;
                double *o = out + ((size_t)b * T + i) * C + h * hs;
                for (int x = 0; x < hs; ++x) o[x] = 0.0;
                for (int j = 0; j <= i; ++j) {
                    const double *v = qkv + ((size_t)b * T + j) * 3 * C + 2 * C + h * hs;
                    for (int x = 0; x < hs; ++x) o[x] += row[j] * v[x];
                }
            }
        }
}

/* dqkv (written) from dout, qkv and the saved att (src/attention.cu:113-200):
 * datt = dout v^T, dpre = att * (datt - rowsum(att * datt)),
 * dq = scale dpre k, dk = scale dpre^T q, dv = att^T dout. */
static void attn_bwd_d(double *dqkv, const double *dout, const double *qkv,
                       const double *att, int B, int T, int C, int NH) {
    const int hs = C / NH;
    const double scale = 1.0 / sqrt((double)hs);
    double *dpre = (double *)malloc(sizeof(double) * (size_t)T);
    memset(dqkv, 0, sizeof(double) * (size_t)B * T * 3 * C);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < NH; ++h) {
            const double *A = att + ((size_t)b * NH + h) * T * T;
            for (int i = 0; i < T; ++i) {
                const double *row = A + (size_t)i * T;
                const double *g = dout + ((size_t)b * T + i) * C + h * hs;
                double D = 0.0;
                for (int j = 0; j <= i; ++j) {
                    const double *v = qkv + ((size_t)b * T + j) * 3 * C + 2 * C + h * hs;
                    double d = 0.0;
                    for (int x = 0; x < hs; ++x) d += g[x] * v[x];
                    dpre[j] = d;
                    D += row[j] * d;
                }
                const double *q = qkv + ((size_t)b * T + i) * 3 * C + h * hs;
                double *dq = dqkv + ((size_t)b * T + i) * 3 * C + h * hs;
                for (int j = 0; j <= i; ++j) {
                    const double ds = row[j] * (dpre[j] - D);
                    const double *k = qkv + ((size_t)b * T + j) * 3 * C + C + h * hs;
                    double *dk = dqkv + ((size_t)b * T + j) * 3 * C + C + h * hs;
                    double *dv = dqkv + ((size_t)b * T + j) * 3 * C + 2 * C + h * hs;
                    for (int x = 0; x < hs; ++x) {
                        dq[x] += scale * ds * k[x];
                        dk[x] += scale * ds * q[x];
                        dv[x] += row[j] * g[x];
                    }
                }
            }
        }
    free(dpre);
}

/* ------------------------------------------------------------ GPT (fp64) */

/* src/gpt.cu:32-50 */
void orc_gpt_param_sizes(size_t *s, const int cfg[6]) {
    const size_t maxT = cfg[0], Vp = cfg[2], L = cfg[3], C = cfg[5];
    s[0] = Vp * C;
    s[1] = maxT * C;
    s[2] = L * C;
    s[3] = L * C;
    s[4] = L * 3 * C * C;
    s[5] = L * 3 * C;
    s[6] = L * C * C;
    s[7] = L * C;
    s[8] = L * C;
    s[9] = L * C;
    s[10] = L * 4 * C * C;
    s[11] = L * 4 * C;
    s[12] = L * C * 4 * C;
    s[13] = L * C;
    s[14] = C;
    s[15] = C;
}

/* y[n, o] = sum_i x[n, i] w[o, i] + (bias ? bias[o] : 0): forward of a
 * (out, in) weight (gemm(false, true, ...), src/gpt.cu:256). */
static void linear_fwd(double *y, const double *x, const double *w,
                       const double *bias, int N, int I, int O) {
    for (int n = 0; n < N; ++n)
        for (int o = 0; o < O; ++o) {
            double s = bias ? bias[o] : 0.0;
            const double *xr = x + (size_t)n * I, *wr = w + (size_t)o * I;
            for (int i = 0; i < I; ++i) s += xr[i] * wr[i];
            y[(size_t)n * O + o] = s;
        }
}

/* dx = dy w (written), dw += dy^T x, dbias += column sums of dy
 * (src/gpt.cu:330-333: gemm NN, gemm TN beta 1, bias_backward). */
static void linear_bwd(double *dx, double *dw, double *dbias, const double *dy,
                       const double *x, const double *w, int N, int I, int O) {
    for (int n = 0; n < N; ++n) {
        const double *g = dy + (size_t)n * O;
        double *dxr = dx + (size_t)n * I;
        for (int i = 0; i < I; ++i) dxr[i] = 0.0;
        for (int o = 0; o < O; ++o) {
            const double *wr = w + (size_t)o * I;
            for (int i = 0; i < I; ++i) dxr[i] += g[o] * wr[i];
        }
        const double *xr = x + (size_t)n * I;
        for (int o = 0; o < O; ++o) {
            double *dwr = dw + (size_t)o * I;
            for (int i = 0; i < I; ++i) dwr[i] += g[o] * xr[i];
            if (dbias) dbias[o] += g[o];
        }
    }
}

typedef struct {
    double *ln1, *ln1_mean, *ln1_rstd, *qkv, *att, *atty, *residual2;
    double *ln2, *ln2_mean, *ln2_rstd, *fch, *fch_gelu, *residual3;
} LayerActs;

double orc_gpt_forward_backward(const int cfg[6], int B, int T,
                                const double *params, const int *tokens,
                                const int *targets, double *losses_out,
                                double *grads, double *logits_out) {
    const int V = cfg[1], Vp = cfg[2], L = cfg[3], NH = cfg[4], C = cfg[5];
    const int N = B * T;
    const size_t BTC = (size_t)N * C;
    size_t s[16], off[16], total = 0;
    orc_gpt_param_sizes(s, cfg);
    for (int i = 0; i < 16; ++i) {
        off[i] = total;
        total += s[i];
    }
    const double *wte = params + off[0], *wpe = params + off[1];
    const double *lnfw = params + off[14], *lnfb = params + off[15];

    double *encoded = (double *)calloc(BTC, sizeof(double));
    LayerActs *la = (LayerActs *)calloc((size_t)L, sizeof(LayerActs));
    for (int l = 0; l < L; ++l) {
        la[l].ln1 = (double *)calloc(BTC, sizeof(double));
        la[l].ln1_mean = (double *)calloc(N, sizeof(double));
        la[l].ln1_rstd = (double *)calloc(N, sizeof(double));
        la[l].qkv = (double *)calloc(3 * BTC, sizeof(double));
        la[l].att = (double *)calloc((size_t)B * NH * T * T, sizeof(double));
        la[l].atty = (double *)calloc(BTC, sizeof(double));
        la[l].residual2 = (double *)calloc(BTC, sizeof(double));
        la[l].ln2 = (double *)calloc(BTC, sizeof(double));
        la[l].ln2_mean = (double *)calloc(N, sizeof(double));
        la[l].ln2_rstd = (double *)calloc(N, sizeof(double));
        la[l].fch = (double *)calloc(4 * BTC, sizeof(double));
        la[l].fch_gelu = (double *)calloc(4 * BTC, sizeof(double));
        la[l].residual3 = (double *)calloc(BTC, sizeof(double));
    }
    double *tmp = (double *)calloc(BTC, sizeof(double));
    double *lnf = (double *)calloc(BTC, sizeof(double));
    double *lnf_mean = (double *)calloc(N, sizeof(double));
    double *lnf_rstd = (double *)calloc(N, sizeof(double));
    double *logits = (double *)calloc((size_t)N * Vp, sizeof(double));
    double *probs = (double *)calloc((size_t)N * Vp, sizeof(double));
    double *losses = (double *)calloc(N, sizeof(double));

    /* forward: src/gpt.cu:228-300 */
    orc_encoder_fwd(encoded, tokens, wte, wpe, B, T, C);
    const double *residual = encoded;
    for (int l = 0; l < L; ++l) {
        LayerActs *a = &la[l];
        const double *ln1w = params + off[2] + (size_t)l * C, *ln1b = params + off[3] + (size_t)l * C;
        const double *qkvw = params + off[4] + (size_t)l * 3 * C * C, *qkvb = params + off[5] + (size_t)l * 3 * C;
        const double *apw = params + off[6] + (size_t)l * C * C, *apb = params + off[7] + (size_t)l * C;
        const double *ln2w = params + off[8] + (size_t)l * C, *ln2b = params + off[9] + (size_t)l * C;
        const double *fcw = params + off[10] + (size_t)l * 4 * C * C, *fcb = params + off[11] + (size_t)l * 4 * C;
        const double *fpw = params + off[12] + (size_t)l * 4 * C * C, *fpb = params + off[13] + (size_t)l * C;
        orc_layernorm_fwd(a->ln1, a->ln1_mean, a->ln1_rstd, residual, ln1w, ln1b, N, C);
        linear_fwd(a->qkv, a->ln1, qkvw, qkvb, N, C, 3 * C);
        attn_fwd_d(a->atty, a->att, a->qkv, B, T, C, NH);
        linear_fwd(tmp, a->atty, apw, apb, N, C, C);
        for (size_t i = 0; i < BTC; ++i) a->residual2[i] = residual[i] + tmp[i];
        orc_layernorm_fwd(a->ln2, a->ln2_mean, a->ln2_rstd, a->residual2, ln2w, ln2b, N, C);
        linear_fwd(a->fch, a->ln2, fcw, fcb, N, C, 4 * C);
        orc_gelu_fwd(a->fch_gelu, a->fch, 4 * BTC);
        linear_fwd(tmp, a->fch_gelu, fpw, fpb, N, 4 * C, C);
        for (size_t i = 0; i < BTC; ++i) a->residual3[i] = a->residual2[i] + tmp[i];
        residual = a->residual3;
    }
    orc_layernorm_fwd(lnf, lnf_mean, lnf_rstd, residual, lnfw, lnfb, N, C);
    linear_fwd(logits, lnf, wte, NULL, N, C, Vp);
    orc_softmax_xent_fwd(probs, losses, logits, targets, N, V, Vp);
    double loss = 0.0;
    for (int r = 0; r < N; ++r) loss += losses[r];
    loss /= N;
    if (losses_out) memcpy(losses_out, losses, sizeof(double) * N);
    if (logits_out) memcpy(logits_out, logits, sizeof(double) * (size_t)N * Vp);

    if (grads) {
        /* backward: src/gpt.cu:303-386 */
        memset(grads, 0, sizeof(double) * total);
        double *d = grads;
        double *dlogits = (double *)calloc((size_t)N * Vp, sizeof(double));
        double *dres = (double *)calloc(BTC, sizeof(double));
        double *dx = (double *)calloc(BTC, sizeof(double));
        double *dfch = (double *)calloc(4 * BTC, sizeof(double));
        double *dfch_gelu = (double *)calloc(4 * BTC, sizeof(double));
        double *dqkv = (double *)calloc(3 * BTC, sizeof(double));
        double *dln = (double *)calloc(BTC, sizeof(double));

        orc_xent_bwd(dlogits, probs, targets, N, V, Vp, 1.0 / N);
        linear_bwd(dx, d + off[0], NULL, dlogits, lnf, wte, N, C, Vp);
        orc_layernorm_bwd(dres, d + off[14], d + off[15], dx, residual, lnfw,
                          lnf_mean, lnf_rstd, N, C);
        for (int l = L - 1; l >= 0; --l) {
            LayerActs *a = &la[l];
            const double *lin = (l == 0) ? encoded : la[l - 1].residual3;
            const double *ln1w = params + off[2] + (size_t)l * C;
            const double *qkvw = params + off[4] + (size_t)l * 3 * C * C;
            const double *apw = params + off[6] + (size_t)l * C * C;
            const double *ln2w = params + off[8] + (size_t)l * C;
            const double *fcw = params + off[10] + (size_t)l * 4 * C * C;
            const double *fpw = params + off[12] + (size_t)l * 4 * C * C;
            linear_bwd(dfch_gelu, d + off[12] + (size_t)l * 4 * C * C, d + off[13] + (size_t)l * C,
                       dres, a->fch_gelu, fpw, N, 4 * C, C);
            orc_gelu_bwd(dfch, a->fch, dfch_gelu, 4 * BTC);
            linear_bwd(dln, d + off[10] + (size_t)l * 4 * C * C, d + off[11] + (size_t)l * 4 * C,
                       dfch, a->ln2, fcw, N, C, 4 * C);
            orc_layernorm_bwd(dres, d + off[8] + (size_t)l * C, d + off[9] + (size_t)l * C, dln,
                              a->residual2, ln2w, a->ln2_mean, a->ln2_rstd, N, C);
            linear_bwd(dx, d + off[6] + (size_t)l * C * C, d + off[7] + (size_t)l * C, dres,
                       a->atty, apw, N, C, C);
            attn_bwd_d(dqkv, dx, a->qkv, a->att, B, T, C, NH);
            linear_bwd(dln, d + off[4] + (size_t)l * 3 * C * C, d + off[5] + (size_t)l * 3 * C,
                       dqkv, a->ln1, qkvw, N, C, 3 * C);
            orc_layernorm_bwd(dres, d + off[2] + (size_t)l * C, d + off[3] + (size_t)l * C, dln,
                              lin, ln1w, a->ln1_mean, a->ln1_rstd, N, C);
        }
        orc_encoder_bwd(d + off[0], d + off[1], dres, tokens, B, T, C);
        free(dlogits);
        free(dres);
        free(dx);
        free(dfch);
        free(dfch_gelu);
        free(dqkv);
        free(dln);
    }

    for (int l = 0; l < L; ++l) {
        free(la[l].ln1); free(la[l].ln1_mean); free(la[l].ln1_rstd); free(la[l].qkv);
        free(la[l].att); free(la[l].atty); free(la[l].residual2); free(la[l].ln2);
        free(la[l].ln2_mean); free(la[l].ln2_rstd); free(la[l].fch); free(la[l].fch_gelu);
        free(la[l].residual3);
    }
    free(la);
    free(encoded);
    free(tmp);
    free(lnf);
    free(lnf_mean);
    free(lnf_rstd);
    free(logits);
    free(probs);
    free(losses);
    return loss;
}
