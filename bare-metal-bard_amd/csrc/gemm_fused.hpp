// Library-internal GEMM entry with a fused epilogue, for the GPT forward.
#pragma once

namespace bmb {

// C[M,N] = A[M,K] @ W[N,K]^T + bias[N] (row broadcast), the linear layer of
// src/gpt.cu (gemm(false, true, ...) then bias_forward); when gelu_out is not
// null it also stores gelu(C) there (the FC layer's gelu_forward). Same fp32
// results as the three separate passes; null stream, like the reference.
void gemm_bias_nt(int M, int N, int K, const float *A, const float *W, const float *bias,
                  float *C, float *gelu_out);

}  // namespace bmb
