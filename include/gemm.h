/*
 * Transpose-aware and batched GEMM -- C-ABI drop-in for bare-metal-bard's
 * src/gemm.h.
 *
 * Row-major throughout (src/gemm.h:4-11):
 *     C[M,N] = alpha * op(A) @ op(B) + beta * C
 *     op(A) = A   with A stored M x K (lda = K)   when transA == false
 *           = A^T with A stored K x M (lda = M)   when transA == true
 *     op(B) = B   with B stored K x N (ldb = N)   when transB == false
 *           = B^T with B stored N x K (ldb = K)   when transB == true
 * Pointers are caller-owned device pointers. beta == 0 means C is write-only.
 * gemm() (and gemm_noalloc()) computes on bf16x3 matrix-core products: each
 * fp32 operand is split into bfloat16 hi + lo (x - hi is exact in fp32),
 * every product term is hi*hi + hi*lo + lo*hi (each bf16 x bf16 product exact
 * in fp32) and accumulation is fp32. What is dropped (lo*lo and the rounding
 * of lo) is a few 2^-17 of |a b| per product, so the normwise error against
 * the exact product is ~1e-6, a hundred times inside the reference's 1e-4 bar
 * (tools/test_gemm.cu:107). batched_gemm() uses fp32 matrix-core products
 * (fp32 rounding level).
 */
#ifndef BMB_GEMM_H
#define BMB_GEMM_H

#include <hip/hip_runtime_api.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
#define BMB_DEFAULT_STREAM = 0
extern "C" {
#else
#define BMB_DEFAULT_STREAM
#endif
/* Only the declarations below are exported from libbmb.so (built with -fvisibility=hidden). */
#pragma GCC visibility push(default)

/* src/gemm.h:17-19 (cudaStream_t becomes hipStream_t; 0 = null stream). */
void gemm(bool transA, bool transB, int M, int N, int K, float alpha,
          const float *A, const float *B, float beta, float *C,
          hipStream_t stream BMB_DEFAULT_STREAM);

/* src/gemm.h:26-29: `batch` independent problems; problem z reads
 * A + z*strideA, B + z*strideB and updates C + z*strideC. */
void batched_gemm(bool transA, bool transB, int batch, int M, int N, int K,
                  float alpha, const float *A, long long strideA,
                  const float *B, long long strideB, float beta, float *C,
                  long long strideC, hipStream_t stream BMB_DEFAULT_STREAM);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc): gemm() that allocates nothing. Its split-K partial sums
 * live in a fixed 64 MiB array of the library's device memory (one per GPU,
 * held until the process ends) instead of leased scratch, so unlike gemm()
 * it also splits K on non-null streams. The planner only considers splits
 * whose partials (splits * M * N floats) fit the array; shapes that would
 * need more run with fewer K ranges or none, so no size is refused for its
 * scratch. The first call on a device resolves the array's address (do it
 * once outside any graph capture). Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (two streams, or host threads on
 * different streams) race on it and must be ordered by the caller. Nothing
 * in the array needs to start at zero (every partial is written before it
 * is read). Returns 0 once the work is queued, -1 with a message on stderr
 * if the array cannot be resolved or a plan would not fit it. */
int gemm_noalloc(bool transA, bool transB, int M, int N, int K, float alpha,
                 const float *A, const float *B, float beta, float *C,
                 hipStream_t stream BMB_DEFAULT_STREAM);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
