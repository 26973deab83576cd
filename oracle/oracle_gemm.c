/*
 * TEST INFRASTRUCTURE ONLY — part of the CPU oracle.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this code,
 * and only as the checker / the timed CPU baseline.  The product path
 * (foundry-trainer_amd/) never links it.
 *
 * Row-major f32 GEMMs for the attention restatement.  They stand in for the
 * f32 matmuls that Candle's CPU backend runs through the gemm 0.19.0 crate
 * (Cargo.lock:94-142; matmuls at crates/foundry-spike/src/lib.rs:145,148,
 * 243-244,252-257).  Every output element is accumulated in f32 over k in
 * ascending order (FMA contraction allowed), so results are deterministic for
 * any thread count.  Parallelism: OpenMP over blocks of output rows.
 */
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define JB 128 /* output columns held in the accumulator block */
#define IB 4   /* output rows per micro-block */

static inline int imin(int a, int b) { return a < b ? a : b; }

/* C[M][N] = A[M][K] * B[K][N] */
void og_gemm_nn(int M, int N, int K, const float *A, long lda, const float *B, long ldb,
                float *C, long ldc, int nthreads)
{
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int i0 = 0; i0 < M; i0 += IB) {
        const int ib = imin(IB, M - i0);
        float acc[IB][JB];
        for (int j0 = 0; j0 < N; j0 += JB) {
            const int jb = imin(JB, N - j0);
            memset(acc, 0, sizeof(acc));
            for (int k = 0; k < K; ++k) {
                const float *b = B + (long)k * ldb + j0;
                for (int r = 0; r < ib; ++r) {
                    const float a = A[(long)(i0 + r) * lda + k];
                    float *c = acc[r];
                    for (int j = 0; j < jb; ++j) c[j] += a * b[j];
                }
            }
            for (int r = 0; r < ib; ++r)
                memcpy(C + (long)(i0 + r) * ldc + j0, acc[r], sizeof(float) * jb);
        }
    }
}

/* C[M][N] = A^T * B with A stored [K][M] and B stored [K][N] */
void og_gemm_tn(int M, int N, int K, const float *A, long lda, const float *B, long ldb,
                float *C, long ldc, int nthreads)
{
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int i0 = 0; i0 < M; i0 += IB) {
        const int ib = imin(IB, M - i0);
        float acc[IB][JB];
        for (int j0 = 0; j0 < N; j0 += JB) {
            const int jb = imin(JB, N - j0);
            memset(acc, 0, sizeof(acc));
            for (int k = 0; k < K; ++k) {
                const float *b = B + (long)k * ldb + j0;
                const float *a = A + (long)k * lda + i0;
                for (int r = 0; r < ib; ++r) {
                    const float ar = a[r];
                    float *c = acc[r];
                    for (int j = 0; j < jb; ++j) c[j] += ar * b[j];
                }
            }
            for (int r = 0; r < ib; ++r)
                memcpy(C + (long)(i0 + r) * ldc + j0, acc[r], sizeof(float) * jb);
        }
    }
}

/* dst[c][r] = src[r][c] for an R x C block */
void og_transpose(int R, int C, const float *src, long lds, float *dst, long ldd, int nthreads)
{
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int c0 = 0; c0 < C; c0 += 32)
        for (int r = 0; r < R; ++r)
            for (int c = c0; c < imin(c0 + 32, C); ++c) dst[(long)c * ldd + r] = src[(long)r * lds + c];
}
