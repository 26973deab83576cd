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
 * any thread count.  Parallelism: OpenMP over 48 x 256 tiles of the output.
 */
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* Register-blocked 6 x 16 output tiles: 12 AVX2 accumulators stay in
 * registers over a block of k, which runs in ascending order with one FMA per
 * output element and k -- the same arithmetic, element for element, as the
 * plain triple loop.  Blocks of k after the first reload the partial sums from
 * C (an exact f32 round trip), so blocking k does not change any result.
 * Rows and columns past the last whole tile take the plain loop (fmaf, k
 * ascending). */
#define MR 6
#define NR 16
#define MC 48  /* rows of C per parallel task */
#define NC 256 /* columns of C per parallel task (B block of KC x NC in L2) */
#define KC 256 /* depth of one k block */

static inline int imin(int a, int b) { return a < b ? a : b; }

/* A_AT(r, k): address of the A element of tile row r at depth k */
#define MICRO_KERNEL(NAME, A_AT)                                                                  \
    static void NAME(int k0, int k1, const float *A, long lda, const float *B, long ldb, float *C,  \
                     long ldc)                                                                    \
    {                                                                                             \
        __m256 c00, c01, c10, c11, c20, c21, c30, c31, c40, c41, c50, c51;                        \
        if (k0 == 0) {                                                                            \
            c00 = c01 = c10 = c11 = c20 = c21 = _mm256_setzero_ps();                              \
            c30 = c31 = c40 = c41 = c50 = c51 = _mm256_setzero_ps();                              \
        } else {                                                                                  \
            c00 = _mm256_loadu_ps(C + 0 * ldc); c01 = _mm256_loadu_ps(C + 0 * ldc + 8);           \
            c10 = _mm256_loadu_ps(C + 1 * ldc); c11 = _mm256_loadu_ps(C + 1 * ldc + 8);           \
            c20 = _mm256_loadu_ps(C + 2 * ldc); c21 = _mm256_loadu_ps(C + 2 * ldc + 8);           \
            c30 = _mm256_loadu_ps(C + 3 * ldc); c31 = _mm256_loadu_ps(C + 3 * ldc + 8);           \
            c40 = _mm256_loadu_ps(C + 4 * ldc); c41 = _mm256_loadu_ps(C + 4 * ldc + 8);           \
            c50 = _mm256_loadu_ps(C + 5 * ldc); c51 = _mm256_loadu_ps(C + 5 * ldc + 8);           \
        }                                                                                         \
        for (int k = k0; k < k1; ++k) {                                                           \
            const float *b = B + (long)k * ldb;                                                   \
            const __m256 b0 = _mm256_loadu_ps(b), b1 = _mm256_loadu_ps(b + 8);                    \
            __m256 a;                                                                             \
            a = _mm256_broadcast_ss(A_AT(0, k)); c00 = _mm256_fmadd_ps(a, b0, c00); c01 = _mm256_fmadd_ps(a, b1, c01); \
            a = _mm256_broadcast_ss(A_AT(1, k)); c10 = _mm256_fmadd_ps(a, b0, c10); c11 = _mm256_fmadd_ps(a, b1, c11); \
            a = _mm256_broadcast_ss(A_AT(2, k)); c20 = _mm256_fmadd_ps(a, b0, c20); c21 = _mm256_fmadd_ps(a, b1, c21); \
            a = _mm256_broadcast_ss(A_AT(3, k)); c30 = _mm256_fmadd_ps(a, b0, c30); c31 = _mm256_fmadd_ps(a, b1, c31); \
            a = _mm256_broadcast_ss(A_AT(4, k)); c40 = _mm256_fmadd_ps(a, b0, c40); c41 = _mm256_fmadd_ps(a, b1, c41); \
            a = _mm256_broadcast_ss(A_AT(5, k)); c50 = _mm256_fmadd_ps(a, b0, c50); c51 = _mm256_fmadd_ps(a, b1, c51); \
        }                                                                                         \
        _mm256_storeu_ps(C + 0 * ldc, c00); _mm256_storeu_ps(C + 0 * ldc + 8, c01);               \
        _mm256_storeu_ps(C + 1 * ldc, c10); _mm256_storeu_ps(C + 1 * ldc + 8, c11);               \
        _mm256_storeu_ps(C + 2 * ldc, c20); _mm256_storeu_ps(C + 2 * ldc + 8, c21);               \
        _mm256_storeu_ps(C + 3 * ldc, c30); _mm256_storeu_ps(C + 3 * ldc + 8, c31);               \
        _mm256_storeu_ps(C + 4 * ldc, c40); _mm256_storeu_ps(C + 4 * ldc + 8, c41);               \
        _mm256_storeu_ps(C + 5 * ldc, c50); _mm256_storeu_ps(C + 5 * ldc + 8, c51);               \
    }

#define NN_AT(r, k) (A + (long)(r) * lda + (k)) /* A stored [M][K] */
#define TN_AT(r, k) (A + (long)(k) * lda + (r)) /* A stored [K][M] */
MICRO_KERNEL(micro_nn, NN_AT)
MICRO_KERNEL(micro_tn, TN_AT)

/* Plain loop over rows [i0, i1) x columns [j0, j1) (the edge tiles). */
static void plain_block(int tn, int i0, int i1, int j0, int j1, int K, const float *A, long lda,
                        const float *B, long ldb, float *C, long ldc)
{
    for (int i = i0; i < i1; ++i)
        for (int j = j0; j < j1; ++j) {
            float acc = 0.f;
            for (int k = 0; k < K; ++k) {
                const float a = tn ? A[(long)k * lda + i] : A[(long)i * lda + k];
                acc = fmaf(a, B[(long)k * ldb + j], acc);
            }
            C[(long)i * ldc + j] = acc;
        }
}

static void gemm(int tn, int M, int N, int K, const float *A, long lda, const float *B, long ldb, float *C,
                 long ldc, int nthreads)
{
    const int mfull = M / MR * MR, nfull = N / NR * NR;
    const int tiles_m = (mfull + MC - 1) / MC, tiles_n = (nfull + NC - 1) / NC;
    if (K == 0) {
        for (int i = 0; i < M; ++i) memset(C + (long)i * ldc, 0, sizeof(float) * (size_t)N);
        return;
    }
#pragma omp parallel num_threads(nthreads)
    {
#pragma omp for schedule(static) nowait
        for (long t = 0; t < (long)tiles_m * tiles_n; ++t) {
            const int im = (int)(t / tiles_n) * MC, jn = (int)(t % tiles_n) * NC;
            const int ie = imin(im + MC, mfull), je = imin(jn + NC, nfull);
            for (int k0 = 0; k0 < K; k0 += KC) {
                const int k1 = imin(k0 + KC, K);
                for (int i0 = im; i0 < ie; i0 += MR) {
                    const float *a = tn ? A + i0 : A + (long)i0 * lda;
                    for (int j0 = jn; j0 < je; j0 += NR) {
                        if (tn)
                            micro_tn(k0, k1, a, lda, B + j0, ldb, C + (long)i0 * ldc + j0, ldc);
                        else
                            micro_nn(k0, k1, a, lda, B + j0, ldb, C + (long)i0 * ldc + j0, ldc);
                    }
                }
            }
        }
        /* edges: the last N % 16 columns of the whole rows, then the last M % 6 rows */
#pragma omp for schedule(static)
        for (int i0 = 0; i0 < M; i0 += MR) {
            if (i0 < mfull) {
                if (nfull < N) plain_block(tn, i0, i0 + MR, nfull, N, K, A, lda, B, ldb, C, ldc);
            } else {
                plain_block(tn, i0, M, 0, N, K, A, lda, B, ldb, C, ldc);
            }
        }
    }
}

/* C[M][N] = A[M][K] * B[K][N] */
void og_gemm_nn(int M, int N, int K, const float *A, long lda, const float *B, long ldb,
                float *C, long ldc, int nthreads)
{
    gemm(0, M, N, K, A, lda, B, ldb, C, ldc, nthreads);
}

/* C[M][N] = A^T * B with A stored [K][M] and B stored [K][N] */
void og_gemm_tn(int M, int N, int K, const float *A, long lda, const float *B, long ldb,
                float *C, long ldc, int nthreads)
{
    gemm(1, M, N, K, A, lda, B, ldb, C, ldc, nthreads);
}

/* dst[c][r] = src[r][c] for an R x C block */
void og_transpose(int R, int C, const float *src, long lds, float *dst, long ldd, int nthreads)
{
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int c0 = 0; c0 < C; c0 += 32)
        for (int r = 0; r < R; ++r)
            for (int c = c0; c < imin(c0 + 32, C); ++c) dst[(long)c * ldd + r] = src[(long)r * lds + c];
}
