// Library-internal GEMM entries with fused epilogues, for the GPT model.
#pragma once

#include <hip/hip_runtime_api.h>

namespace bmb {

// C[M,N] = A[M,K] @ W[N,K]^T + bias[N] (row broadcast), the linear layer of
// src/gpt.cu (gemm(false, true, ...) then bias_forward); when gelu_out is not
// null it also stores gelu(C) there (the FC layer's gelu_forward). Same fp32
// results as the three separate passes; null stream, like the reference.
void gemm_bias_nt(int M, int N, int K, const float *A, const float *W, const float *bias,
                  float *C, float *gelu_out);

// C[M,N] = gelu_grad(pre, A[M,K] @ B[K,N]) elementwise: the dX GEMM of the
// FC projection (gemm(false, false, ...)) followed by gelu_backward
// (src/gpt.cu:331-337), without storing the product. Same fp32 results.
void gemm_gelu_grad_nn(int M, int N, int K, const float *A, const float *B, const float *pre,
                       float *C);

// C = alpha * sum_{s < splits} P[s] + beta * C over mn = M * N floats (P is
// splits x M x N), the splits added in ascending order: the reduce of every
// split-K GEMM in the library (one kernel, so the result depends only on the
// shape and the split count).
void splitk_reduce(float *C, const float *P, int splits, long long mn, int N, float alpha,
                   float beta, hipStream_t stream);

}  // namespace bmb
