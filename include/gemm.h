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
 * By default gemm() (and gemm_noalloc()) computes on bf16x3 matrix-core
 * products: each fp32 operand is split into bfloat16 hi + lo (x - hi is exact
 * in fp32), every product term is hi*hi + hi*lo + lo*hi (each bf16 x bf16
 * product exact in fp32) and accumulation is fp32. What is dropped (lo*lo and
 * the rounding of lo) is a few 2^-17 of |a b| per product, so the normwise
 * error against the exact product is 1e-6 to 4e-6: well inside the
 * reference's 1e-4 bar (tools/test_gemm.cu:107), but ten to thirty times the
 * ~1e-7 of an fp32 FMA GEMM such as the reference's (src/gemm.cu:33-162).
 * gemm_set_math(GEMM_MATH_FP32) switches them to fp32 matrix-core products
 * (exact fp32 products, fp32 accumulation: the reference's rounding level) at
 * about a third of the bf16x3 rate. batched_gemm() always uses fp32
 * matrix-core products.
 *
 * Split-K: gemm() may split K over ranges whose fp32 partial sums it adds in
 * range order (deterministic: the same bits for a shape on any stream). The
 * partials live in library scratch leased per call; its reuse is ordered on
 * the device by an event recorded on the caller's stream, so every stream
 * may split. Under HIP graph capture gemm() does not split (a lease could
 * allocate): capture gemm_noalloc() instead.
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
 * forbid hipMalloc): gemm() that allocates nothing, in the arithmetic
 * gemm_set_math() selects. Its split-K partial sums live in a fixed 64 MiB
 * array of the library's device memory (one per GPU, held until the process
 * ends) instead of leased scratch, also under graph capture. The planner only
 * considers splits whose partials (splits * M * N floats) fit the array;
 * shapes that would need more run with fewer K ranges or none, so no size is
 * refused for its scratch (their result can then differ from gemm()'s in the
 * last bits, within the same bound). The first call on a device resolves the
 * array's address (do it once outside any graph capture). Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (two streams, or
 * host threads on different streams) race on it and must be ordered by the
 * caller. Nothing in the array needs to start at zero (every partial is
 * written before it is read). Returns 0 once the work is queued, -1 with a
 * message on stderr if the array's address cannot be resolved. */
int gemm_noalloc(bool transA, bool transB, int M, int N, int K, float alpha,
                 const float *A, const float *B, float beta, float *C,
                 hipStream_t stream BMB_DEFAULT_STREAM);

/* No counterpart in the reference. Selects the arithmetic of gemm(),
 * gemm_noalloc() and the GPT model's linear layers (gpt_forward,
 * gpt_backward) for the whole process, for calls made after it returns:
 *   GEMM_MATH_BF16X3 (the default): bf16x3 matrix-core products, 1e-6 to
 *     4e-6 normwise from the exact product;
 *   GEMM_MATH_FP32: fp32 matrix-core products (the KERNELS id 9 kernels:
 *     exact fp32 products, fp32 accumulation), the fp32 rounding level of the
 *     reference's gemm() (~1e-7 normwise).
 * Allocates nothing and launches nothing. Returns the previous mode, or -1
 * (with a message on stderr, nothing changed) for an unknown one. */
#define GEMM_MATH_BF16X3 0
#define GEMM_MATH_FP32 1
int gemm_set_math(int math);

/* The mode gemm_set_math() last set (GEMM_MATH_BF16X3 before any call). */
int gemm_get_math(void);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
