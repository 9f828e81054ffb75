// Library-internal GEMM entries with fused epilogues, for the GPT model.
#pragma once

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

}  // namespace bmb
