// Library-internal GEMM entries with fused epilogues, for the GPT model.
#pragma once

#include <hip/hip_runtime_api.h>

namespace bmb {

// C[M,N] = A[M,K] @ W[N,K]^T + bias[N] (row broadcast), the linear layer of
// src/gpt.cu (gemm(false, true, ...) then bias_forward); when gelu_out is not
// null it also stores gelu(C) there (the FC layer's gelu_forward). The product
// is gemm()'s (bf16x3); bias and GELU are applied in fp32 as the separate
// passes do; null stream, like the reference.
void gemm_bias_nt(int M, int N, int K, const float *A, const float *W, const float *bias,
                  float *C, float *gelu_out);

// C[M,N] = gelu_grad(pre, A[M,K] @ B[K,N]) elementwise: the dX GEMM of the
// FC projection (gemm(false, false, ...)) followed by gelu_backward
// (src/gpt.cu:331-337), without storing the product.
void gemm_gelu_grad_nn(int M, int N, int K, const float *A, const float *B, const float *pre,
                       float *C);

// C = alpha * sum_{s < splits} P[s] + beta * C over mn = M * N floats (P is
// splits x M x N), the splits added in ascending order: the reduce of every
// split-K GEMM in the library (one kernel, so the result depends only on the
// shape and the split count).
void splitk_reduce(float *C, const float *P, int splits, long long mn, int N, float alpha,
                   float beta, hipStream_t stream);

// The same reduce ending in epilogue `epi` (an Epi of mfma_gemm.hpp: bias[N],
// act = gelu(C) output, pre = the GELU input, as the GEMM epilogues), C's
// rows (and those of act, pre) ldc floats apart.
void splitk_reduce_epi(int epi, float *C, const float *P, int splits, long long mn, int N,
                       int ldc, float alpha, float beta, hipStream_t stream, const float *bias,
                       float *act, const float *pre);

// Row-major C[M,N] = epilogue(op(A) @ op(B)) on bf16x3 matrix-core products
// (sgemm_bf16x3.hip): each fp32 operand split into bf16 hi + lo, three bf16
// products per term, fp32 accumulation. epi: EPI_BLAS (C = alpha acc +
// beta C, any transposes), EPI_BIAS / EPI_BIAS_GELU (transB only), or
// EPI_GELU_GRAD (no transposes). Split-K partials go to `fixed` (at most
// fixed_floats floats) on any stream, or to leased scratch on the null stream
// only. Returns false, launching nothing, for an unsupported combination.
bool bf16x3_gemm(bool ta, bool tb, int M, int N, int K, float alpha, const float *A,
                 const float *B, float beta, float *C, hipStream_t stream, int epi,
                 const float *bias, float *act, const float *pre, float *fixed,
                 long long fixed_floats);

// Thin edges of a corner plan (edge_gemm.hip): of an M x N x K problem with
// row-major A (lda), B (ldb) and C (ldc), C = alpha A B + beta C over rows
// [0, m1) x columns [n1, N) and rows [m1, M) x all columns, where N - n1 and
// M - m1 are at most EDGE_MAX. bf16x3: products as the bf16x3 kernels form
// them (hi*hi + hi*lo + lo*hi of their split), else exact fp32 products. P:
// edge_partial_floats(M - m1, N - n1, N, K) floats of scratch (the bottom
// edge's partials and a packed copy of B's right edge).
constexpr int EDGE_MAX = 8;
int edge_ranges(int N, int K);
long long edge_partial_floats(int rm, int rn, int N, int K);
// Modelled time of the edges (seconds), for the planners.
double edge_model_s(long long m1, long long rn, long long rm, long long N, long long K);
void gemm_edges(bool bf16x3, int M, int N, int K, int m1, int n1, float alpha, const float *A,
                int lda, const float *B, int ldb, float beta, float *C, int ldc, float *P,
                hipStream_t stream);

}  // namespace bmb
