/*
 * SGEMM kernel table -- C-ABI drop-in for bare-metal-bard's src/kernels.h and
 * src/registry.cu.
 *
 * Contract (src/kernels.h:1-11), row-major throughout:
 *     C = alpha * A @ B + beta * C,  A: M x K (lda = K), B: K x N, C: M x N.
 * All pointers are caller-owned device pointers; launches go to the null
 * stream and are asynchronous. beta == 0 means C is write-only (BLAS
 * semantics); for finite C this equals the reference's alpha*acc + beta*C.
 */
#ifndef BMB_KERNELS_H
#define BMB_KERNELS_H

#ifdef __cplusplus
extern "C" {
#endif
/* Only the declarations below are exported from libbmb.so (built with -fvisibility=hidden). */
#pragma GCC visibility push(default)

/* src/kernels.h:10-11 */
typedef void (*sgemm_fn)(int M, int N, int K, float alpha, const float *A,
                         const float *B, float beta, float *C);

/* src/kernels.h:13-25. tol is the normwise bound max|got-ref|/max|ref| the
 * kernel is held to against an fp32 reference. */
typedef struct KernelEntry {
    int id;
    const char *name;
    sgemm_fn fn;
    const char *note;
    double tol;
} KernelEntry;

/* src/registry.cu:4-16 */
extern const KernelEntry KERNELS[];
extern const int NUM_KERNELS;

/* src/registry.cu:18-23: NULL when no kernel has that id. */
const KernelEntry *find_kernel(int id);

/* One launcher per ladder stage, src/kernels.h:34-42. Every fp32 VALU stage
 * (ids 1-8) accumulates each output as acc = fma(a_k, b_k, acc) for
 * k = 0..K-1 in order, so all of them are bit-identical to one another and to
 * a sequential fmaf loop on the CPU. Every stage handles any M, N, K >= 0. */
void sgemm_naive(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
void sgemm_coalesced(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
void sgemm_smem(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
void sgemm_tile1d(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
void sgemm_tile2d(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
void sgemm_vectorized(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
void sgemm_warptile(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
void sgemm_doublebuffer(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
/* id 9 keeps the reference's name (src/kernels.h:42) but is the matrix-core
 * stage of this build: fp32 in, fp32 products, fp32 accumulate on
 * v_mfma_f32_32x32x2_f32 (gfx950 has no TF32/XF32 MFMA). */
void sgemm_tensorcore(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);
/* id 10, no counterpart in the reference: each fp32 operand split as
 * hi + lo in bf16, three bf16 MFMA products (hi*hi + hi*lo + lo*hi) with
 * fp32 accumulation. Stands where the reference's TF32 stage stood: a
 * deliberately lower-precision answer with its own tolerance. */
void sgemm_mfma_bf16x3(int M, int N, int K, float alpha, const float *A, const float *B, float beta, float *C);

/* Status of the last launch made by this library on the calling host thread
 * (0 = success; otherwise a hipError_t value). No counterpart in the
 * reference, whose harnesses call cudaGetLastError themselves
 * (src/bench.cu:267). */
int bmb_last_error(void);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
