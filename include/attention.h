/*
 * Unfused causal multi-head self-attention -- C-ABI drop-in for
 * bare-metal-bard's src/attention.h (the three-kernel path the trainer uses
 * with --unfused, and the materialised-softmax check for the fused kernels).
 *
 * Buffer shapes (src/attention.h:5-16), fp32, caller-owned device memory,
 * hs = C / NH:
 *   qkv   (B, T, 3C)         [q|k|v] along 3C
 *   qkvr  (4, B, NH, T, hs)  q, k, v head-contiguous, then the head-major
 *                            attention output (4*B*T*C floats)
 *   att   (B, NH, T, T)      post-softmax weights, exact zeros above the
 *                            diagonal
 *   out   (B, T, C)
 * The four contractions run on the library's batched GEMM; permutes and the
 * causal softmax are separate HBM-bound kernels. Launches go to the null
 * stream.
 */
#ifndef BMB_ATTENTION_H
#define BMB_ATTENTION_H

#ifdef __cplusplus
extern "C" {
#endif
/* Only the declarations below are exported from libbmb.so (built with -fvisibility=hidden). */
#pragma GCC visibility push(default)

/* src/attention.h:19-20 */
void attention_forward(float *out, float *qkvr, float *att, const float *qkv,
                       int B, int T, int C, int NH);

/* src/attention.h:23-25. dqkv is written; dqkvr (4*B*T*C floats) and datt
 * are scratch; dpreatt may alias datt. */
void attention_backward(float *dqkv, float *dqkvr, float *datt, float *dpreatt,
                        const float *dout, const float *qkvr, const float *att,
                        int B, int T, int C, int NH);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
