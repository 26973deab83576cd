/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the attention hot path.
 *
 * A plain-C restatement of erikerikerik/foundry-trainer's `foundry-spike`
 * Candle CPU path (crates/foundry-spike/src/lib.rs):
 *   rms_norm            lib.rs:45-58
 *   rope_tables_dtype   lib.rs:77-105
 *   apply_rope          lib.rs:107-129
 *   attn_fwd            lib.rs:131-149   (AttnBwd::cpu_fwd, lib.rs:158-187)
 *   AttnBwd::bwd        lib.rs:216-263
 *   linear_scaled       lib.rs:270-287
 * extended only where the MI355X boundary needs more than the reference
 * offers: a batch dimension, a runtime softmax scale, the natural-log row
 * logsumexp (LSE) of the scaled scores, and an optional key-keep mask.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library.  The product (foundry-trainer_amd/) never does.
 *
 * Conventions
 *   - q, k, v, o, dO, dq, dk, dv: f32 arrays laid out [B][S][H][D]
 *     (B = 1 gives the reference's per-sample (S, H, D)).
 *   - lse: f32 [B][H][S]; -INFINITY for a row whose keys are all masked.
 *   - key_keep: NULL or uint8 [B][S], nonzero = key takes part.
 *   - bf16 != 0 emulates the reference's bf16 run: inputs are taken to be
 *     bf16-valued already, arithmetic is f32, and results are rounded to bf16
 *     (round-to-nearest-even) exactly where the reference casts back to the
 *     compute dtype.  bf16 == 0 is the reference's f32 run (no rounding).
 *   - [h_begin, h_end) restricts work to a subset of heads (all batch items);
 *     outputs for other heads are left untouched.  nthreads = OpenMP threads.
 */
#ifndef FOUNDRY_ORACLE_H
#define FOUNDRY_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float oracle_bf16_round(float x);
void oracle_round_bf16_inplace(float *x, long n);

int oracle_attn_fwd(const float *q, const float *k, const float *v, float *o, float *lse,
                    int B, int S, int H, int D, float scale, const uint8_t *key_keep, int bf16,
                    int h_begin, int h_end, int nthreads);

int oracle_attn_bwd(const float *q, const float *k, const float *v, const float *dout,
                    float *dq, float *dk, float *dv, int B, int S, int H, int D, float scale,
                    const uint8_t *key_keep, int bf16, int h_begin, int h_end, int nthreads);

void oracle_rms_norm(const float *x, const float *w, float *y, long rows, int D, float eps, int bf16);

int oracle_rope_tables(const float *positions, int n_pos, int n_axes, const int *axes,
                       float theta, float *cos_out, float *sin_out, int bf16);

int oracle_apply_rope(const float *x, const float *cos_t, const float *sin_t, float *y, long S,
                      int H, int n_axes, const int *axes, int bf16);

int oracle_qk_prologue_bwd(const float *x, const float *w, const float *cos_t,
                           const float *sin_t, const float *dy, float *dx, long S, int H,
                           int n_axes, const int *axes, float eps);

void oracle_linear_lora(const float *x, const float *W, const float *bias, const float *A,
                        const float *Bm, float *y, int N, int in_f, int out_f, int r,
                        float scale, int bf16, int nthreads);

void oracle_linear_lora_bwd(const float *x, const float *W, const float *A, const float *Bm,
                            const float *dy, float *dx, float *dA, float *dB, int N, int in_f,
                            int out_f, int r, float scale, int bf16, int nthreads);

/* GEMM helpers (oracle_gemm.c) */
void og_gemm_nn(int M, int N, int K, const float *A, long lda, const float *B, long ldb,
                float *C, long ldc, int nthreads);
void og_gemm_tn(int M, int N, int K, const float *A, long lda, const float *B, long ldb,
                float *C, long ldc, int nthreads);
void og_transpose(int R, int C, const float *src, long lds, float *dst, long ldd, int nthreads);

/* Double-stream block ops (block_oracle.c): rows are [N][C] contiguous. */
void oracle_ln_mod_fwd(const float *x, long N, int C, const float *shift, const float *scale, float eps,
                       int bf16, float *y, float *mean, float *rstd);
void oracle_ln_mod_bwd(const float *x, const float *dy, long N, int C, const float *scale, const float *mean,
                       const float *rstd, const float *dres, int bf16, float *dx);
void oracle_gated_residual(const float *x, const float *g, const float *b, long N, int C, int bf16, float *y);
void oracle_gelu_fwd(const float *b, long n, int bf16, float *y);
void oracle_gelu_bwd(const float *dy, const float *b, long n, int bf16, float *y);
void oracle_silu(const float *b, long n, int bf16, float *y);
void oracle_swiglu_fwd(const float *gate, const float *up, long n, int bf16, float *y);
void oracle_swiglu_bwd(const float *dy, const float *gate, const float *up, long n, int bf16, float *dgate,
                       float *dup);
void oracle_adamw_step(float *param, const float *grad, float *m, float *v, long n, double lr, double beta1,
                       double beta2, double eps, int step, int bf16);

#ifdef __cplusplus
}
#endif
#endif
