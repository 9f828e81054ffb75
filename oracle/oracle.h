/*
 * CPU oracle for the SGEMM ladder, the transpose-aware / batched GEMM, the
 * fused causal attention, and the transformer building blocks and GPT model
 * built on them, of bare-metal-bard.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links or calls this
 * code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it, and only as the checker (or, for the CPU baseline, as the timed CPU
 * restatement).
 *
 * Every function cites the reference file:line whose semantics it restates.
 * Reference paths are relative to the bare-metal-bard source tree.
 */
#ifndef BMB_ORACLE_H
#define BMB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic fills -------------------------------------------------
 * xorshift32 (Marsaglia 2003, shift triple 13/17/5), mapped to the 1e-3 grid
 * (int)(s % 2000) - 1000) / 1000 in [-1, 0.999]: src/bench.cu:59-66,
 * tools/test_gemm.cu:40-45, tools/test_flash.cu:33-39. */
void orc_fill_xorshift(float *v, size_t n, uint32_t seed);
/* Raw xorshift32 stream (for the known-answer test of the generator). */
void orc_xorshift_stream(uint32_t *out, size_t n, uint32_t seed);
/* N(0,1) by Box-Muller (Box & Muller 1958) over the same xorshift32 stream:
 * u1 = (s1 + 1) / 2^32, u2 = s2 / 2^32, z0 = sqrt(-2 ln u1) cos(2 pi u2),
 * z1 = sqrt(-2 ln u1) sin(2 pi u2). Computed in double, rounded to float. */
void orc_fill_normal(float *v, size_t n, uint32_t seed, float stddev);

/* ---- SGEMM / GEMM ---------------------------------------------------------
 * Row-major C[M,N] = alpha * op(A) @ op(B) + beta * C (src/gemm.h:4-19,
 * src/kernels.h:1-11). op(A) = A^T means A is stored K x M.
 *
 * f32seq: per output, acc starts at +0 and takes acc = fmaf(a_k, b_k, acc)
 * for k = 0..K-1 in order -- the summation every fp32 ladder kernel performs
 * (src/kernels/k01_naive.cu:25-27, k08_doublebuffer.cu:138-147 accumulate
 * acc += a*b, contracted to one fused multiply-add per term). The epilogue
 * is BLAS-style: beta == 0 writes alpha*acc without reading C; otherwise
 * C = fmaf(alpha, acc, beta * C). (The reference always reads C,
 * src/gemm.cu:154-159; the two agree whenever C is finite.)
 * The loop order is i, k, j with j innermost, which keeps each output's
 * k-order sequential, so it is bit-identical to the literal i-j-k loop. */
void orc_gemm_f32seq(int transA, int transB, int M, int N, int K, float alpha,
                     const float *A, const float *B, float beta, float *C);
/* Same result, rows split over `threads` OpenMP threads (order preserving). */
void orc_gemm_f32seq_mt(int transA, int transB, int M, int N, int K,
                        float alpha, const float *A, const float *B,
                        float beta, float *C, int threads);
/* Exact-ish reference: fp64 products and sums, fp64 epilogue.
 * Cout[i*N+j] = alpha * sum_k A*B + beta * C0[i*N+j] (C0 may be NULL when
 * beta == 0). */
void orc_gemm_f64(int transA, int transB, int M, int N, int K, double alpha,
                  const float *A, const float *B, double beta, const float *C0,
                  double *Cout);
/* Batched form (src/bgemm.cu:25-27): problem z uses A + z*strideA, etc. */
void orc_batched_gemm_f32seq(int transA, int transB, int batch, int M, int N,
                             int K, float alpha, const float *A,
                             long long strideA, const float *B,
                             long long strideB, float beta, float *C,
                             long long strideC);
void orc_batched_gemm_f64(int transA, int transB, int batch, int M, int N,
                          int K, double alpha, const float *A,
                          long long strideA, const float *B, long long strideB,
                          double beta, const float *C0, long long strideC,
                          double *Cout);

/* ---- accuracy metric ------------------------------------------------------
 * Normwise relative error max|got - ref| / max|ref| (src/bench.cu:133-147).
 * *nonfinite is set to the number of non-finite entries of got (any one of
 * which fails a check regardless of the norm, bench.cu:142). */
double orc_normwise_f32(const float *got, const float *ref, size_t n,
                        size_t *nonfinite);
double orc_normwise_f64(const float *got, const double *ref, size_t n,
                        size_t *nonfinite);

/* ---- causal attention -----------------------------------------------------
 * Layout (src/flash.h:29-35): qkv (B,T,3C) with [q|k|v] along 3C and head h
 * at column offset h*hs; out (B,T,C); lse (B,NH,T); dqkv (B,T,3C).
 * scale = 1/sqrt(hs) (src/flash.cu:406).
 *
 * fp64 textbook form: S = scale * q k^T over keys j <= i, P = softmax(S),
 * O = P v, lse = ln sum_j exp(S_ij) (src/flash.cu:10-24,293-310;
 * src/attention.cu:86-110). */
void orc_attn_fwd_f64(const float *qkv, int B, int T, int C, int NH,
                      double *out, double *lse);
/* D[b,h,t] = sum_i dO[b,t,h*hs+i] * O[b,t,h*hs+i] (src/flash.cu:471-487). */
void orc_dsum_f64(const float *dout, const float *out, int B, int T, int C,
                  int NH, double *dsum);
/* Analytic fp64 backward (src/flash.cu:447-458, src/attention.cu:165-200):
 * dV_j = sum_i P_ij dO_i; dP_ij = dO_i . v_j; dS_ij = P_ij (dP_ij - D_i) with
 * D_i = sum_j P_ij dP_ij; dQ_i = scale sum_j dS_ij k_j; dK_j = scale sum_i
 * dS_ij q_i. Writes all of dqkv. */
void orc_attn_bwd_f64(const float *qkv, const float *dout, int B, int T, int C,
                      int NH, double *dqkv);
/* fp32 materialised attention, forward then backward, in the unfused
 * reference's order of operations (src/attention.cu:132-200: scores, causal
 * softmax with explicit zeros, P@V, then the Jacobian backward). Used as the
 * CPU baseline's timed work; parallel over (b,h) with `threads` threads.
 * Writes out (B,T,C) and dqkv (B,T,3C). */
void orc_attn_fwdbwd_f32(const float *qkv, const float *dout, int B, int T,
                         int C, int NH, float *out, float *dqkv, int threads);

/* ---- transformer building blocks (oracle_gpt.c) ---------------------------
 * fp64 in, fp64 out; the fp32 values the GPU sees are widened exactly.
 * Gradient outputs marked "+=" accumulate, as the reference's do. */
/* out[b,t,:] = wte[tokens[b,t],:] + wpe[t,:]  (src/nn.cu:23-36) */
void orc_encoder_fwd(double *out, const int *tokens, const double *wte,
                     const double *wpe, int B, int T, int C);
/* dwte[tok,:] += dout[b,t,:], dwpe[t,:] += dout[b,t,:]  (src/nn.cu:38-46) */
void orc_encoder_bwd(double *dwte, double *dwpe, const double *dout,
                     const int *tokens, int B, int T, int C);
/* biased variance, eps 1e-5, rstd = 1/sqrt(var + eps)  (src/nn.cu:54-82) */
void orc_layernorm_fwd(double *out, double *mean, double *rstd,
                       const double *inp, const double *w, const double *b,
                       int N, int C);
/* dinp += rstd (dxhat - mean(dxhat) - xhat mean(dxhat xhat)), dw += dy xhat,
 * db += dy  (src/nn.cu:85-111) */
void orc_layernorm_bwd(double *dinp, double *dw, double *db,
                       const double *dout, const double *inp, const double *w,
                       const double *mean, const double *rstd, int N, int C);
/* GPT-2 tanh GELU and its derivative (src/nn.cu:116-151); dinp written */
void orc_gelu_fwd(double *out, const double *inp, size_t n);
void orc_gelu_bwd(double *dinp, const double *inp, const double *dout, size_t n);
/* dbias[c] += sum_r dout[r,c]  (src/nn.cu:184-192) */
void orc_bias_bwd(double *dbias, const double *dout, int N, int C);
/* softmax over the first V of Vp columns, probs[V:Vp] = 0, loss =
 * -ln(max(p[target], 1e-30)) (src/nn.cu:197-221); a target outside [0,Vp)
 * gives NaN. losses may be NULL. */
void orc_softmax_xent_fwd(double *probs, double *losses, const double *logits,
                          const int *targets, int N, int V, int Vp);
/* dlogits = (p - [i == target]) * scale for i < V, 0 beyond
 * (src/nn.cu:226-236) */
void orc_xent_bwd(double *dlogits, const double *probs, const int *targets,
                  int N, int V, int Vp, double scale);
/* fp32 AdamW restated operation by operation (src/nn.cu:240-255, bias
 * corrections 1 - powf(beta, step) as at src/nn.cu:336-343). */
void orc_adamw_f32(float *params, const float *grads, float *m, float *v,
                   size_t n, float lr, float beta1, float beta2, float eps,
                   float wd, int step, float grad_scale);

/* ---- GPT model (oracle_gpt.c) ----------------------------------------------
 * cfg = {max_seq_len, vocab_size, padded_vocab, n_layer, n_head, n_embd}, the
 * field order of GPTConfig (src/gpt.h:10-17). */
/* The 16 parameter tensor sizes in PARAM_NAMES order (src/gpt.cu:32-50). */
void orc_gpt_param_sizes(size_t *s, const int cfg[6]);
/* Forward of src/gpt.cu:228-300 and, when grads != NULL, the backward of
 * src/gpt.cu:303-386 (grads written, fp64, flat in parameter order), with
 * the unfused attention of src/attention.cu as the attention. params is the
 * flat parameter vector in fp64. Returns the mean loss; losses_out (N) and
 * logits_out (N x Vp) are filled when not NULL. */
double orc_gpt_forward_backward(const int cfg[6], int B, int T,
                                const double *params, const int *tokens,
                                const int *targets, double *losses_out,
                                double *grads, double *logits_out);

/* Number of threads OpenMP would use by default (for reporting). */
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
