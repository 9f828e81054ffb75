/*
 * Transformer building blocks of the GPT trainer -- C-ABI drop-in for
 * bare-metal-bard's src/nn.h (the launchers of src/nn.cu).
 *
 * Every activation is row-major (B, T, C) and fp32; (b, t) is one flat row,
 * so N = B*T. Weights are (out_features, in_features). All pointers are
 * caller-owned device pointers; launches go to the null stream. Names,
 * argument order and meaning follow src/nn.h:10-60. Where the reference
 * silently relies on n % 4 == 0 or C % 4 == 0 (src/nn.cu:304-322) these
 * entry points also handle the remainder.
 *
 * Determinism: every reduction here runs in a fixed order that depends only
 * on the shape, so repeated calls on the same inputs give the same bits. The
 * reference uses atomics for the layernorm weight/bias and the embedding
 * gradients (src/nn.cu:44-45,108-109); this library reduces the layernorm and
 * bias gradients through per-block partial sums in a scratch buffer that the
 * call leases from a library-owned pool of the device (a few MB at GPT-2
 * sizes; the pool keeps one buffer per concurrently calling host thread until
 * the process ends; a void op that cannot allocate it prints an error and
 * exits, as any CUDA error does in the reference) and the token-embedding
 * gradient by letting the first position of each token id sum all its
 * positions in order.
 */
#ifndef BMB_NN_H
#define BMB_NN_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif
/* Only the declarations below are exported from libbmb.so (built with -fvisibility=hidden). */
#pragma GCC visibility push(default)

/* ---- embeddings (src/nn.h:10-14) ----
 * out[b,t,:] = wte[tokens[b,t],:] + wpe[t,:]. Token ids must lie in the
 * rows of wte. */
void encoder_forward(float *out, const int *tokens, const float *wte,
                     const float *wpe, int B, int T, int C);
/* dwte[tok,:] += sum of dout rows with that token; dwpe[t,:] += sum over b. */
void encoder_backward(float *dwte, float *dwpe, const float *dout,
                      const int *tokens, int B, int T, int C);

/* ---- layernorm (src/nn.h:19-25) ----
 * y = (x - mean) * rstd * w + b, biased variance, eps 1e-5; mean and rstd
 * (N floats each) are saved for the backward. */
void layernorm_forward(float *out, float *mean, float *rstd, const float *inp,
                       const float *weight, const float *bias, int N, int C);
/* dinp += rstd * (dxhat - mean(dxhat) - xhat * mean(dxhat * xhat)) with
 * dxhat = dout * w; dweight += sum_rows dout * xhat; dbias += sum_rows dout. */
void layernorm_backward(float *dinp, float *dweight, float *dbias,
                        const float *dout, const float *inp,
                        const float *weight, const float *mean,
                        const float *rstd, int N, int C);

/* ---- activations and residuals (src/nn.h:28-31) ----
 * GELU is GPT-2's tanh form 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
 * gelu_backward writes (not accumulates) dinp. */
void gelu_forward(float *out, const float *inp, int n);
void gelu_backward(float *dinp, const float *inp, const float *dout, int n);
void residual_forward(float *out, const float *a, const float *b, int n);
void add_inplace(float *dst, const float *src, int n);

/* ---- bias (src/nn.h:36-37) ----
 * out[r,c] += bias[c]; dbias[c] += sum_r dout[r,c]. */
void bias_forward(float *out, const float *bias, int N, int C);
void bias_backward(float *dbias, const float *dout, int N, int C);

/* ---- loss (src/nn.h:43-48) ----
 * logits/probs/dlogits are (N, Vp); columns [V, Vp) are excluded from the
 * softmax and get probability 0 and gradient 0. losses[r] =
 * -ln(max(probs[r, targets[r]], 1e-30)); a target outside [0, Vp) gives a
 * NaN loss (and contributes no indicator to the backward) instead of an
 * out-of-bounds read. */
void softmax_crossentropy_forward(float *probs, float *losses,
                                  const float *logits, const int *targets,
                                  int N, int V, int Vp);
/* dlogits[r,i] = (probs[r,i] - [i == targets[r]]) * dloss_scale for i < V,
 * 0 for i >= V. */
void crossentropy_softmax_backward(float *dlogits, const float *probs,
                                   const int *targets, int N, int V, int Vp,
                                   float dloss_scale);

/* ---- optimizer (src/nn.h:53-57) ----
 * AdamW with bias correction (1 - beta^step, computed on the host in fp32)
 * and decoupled weight decay; every gradient is multiplied by grad_scale on
 * the way in. Same fp32 operation order as src/nn.cu:240-255. */
void adamw_update(float *params, float *grads, float *m, float *v, int n,
                  float lr, float beta1, float beta2, float eps,
                  float weight_decay, int step, float grad_scale);
/* sqrt(sum g^2), accumulated in fp64; blocks until the result is on the
 * host. */
float grad_global_norm(const float *grads, int n);

/* ---- utility (src/nn.h:59-60) ---- */
/* Zero-fill with a kernel (no memset node, so the call is safe inside a
 * captured graph). */
void zero_buffer(float *p, size_t n);
/* Mean of n device floats, accumulated in fp64; blocks until the result is
 * on the host. */
float reduce_mean(const float *d_values, int n);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
