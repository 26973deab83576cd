/*
 * TEST INFRASTRUCTURE ONLY — CPU oracle for the attention hot path.
 * See oracle.h for the contract and the reference lines each function follows.
 * Compiled with -ffp-contract=off so elementwise steps round exactly as the
 * reference's separate Candle ops do (one rounding per op); the GEMMs live in
 * oracle_gemm.c.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* Round an f32 to the nearest bf16 (ties to even), returned as f32.  This is
 * the cast the reference performs with `to_dtype(DType::BF16)`. */
float oracle_bf16_round(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x; /* NaN stays NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    memcpy(&x, &u, 4);
    return x;
}

void oracle_round_bf16_inplace(float *x, long n)
{
    for (long i = 0; i < n; ++i) x[i] = oracle_bf16_round(x[i]);
}

static inline float rnd(float x, int bf16) { return bf16 ? oracle_bf16_round(x) : x; }

/* ---- per-head gather/scatter between [B][S][H][D] and a dense [S][D] ---- */
static void gather_head(const float *src, float *dst, int b, int h, int S, int H, int D)
{
    for (int s = 0; s < S; ++s)
        memcpy(dst + (long)s * D, src + (((long)b * S + s) * H + h) * D, sizeof(float) * D);
}

static void scatter_head(const float *src, float *dst, int b, int h, int S, int H, int D)
{
    for (int s = 0; s < S; ++s)
        memcpy(dst + (((long)b * S + s) * H + h) * D, src + (long)s * D, sizeof(float) * D);
}

/*
 * Softmax of one row of raw scores, lib.rs:146-147: scores.affine(scale, 0)
 * then candle_nn::ops::softmax (max, exp(x - max), sum, divide), all f32.
 * Masked keys (keep[j] == 0) take no part: p = 0.  Returns the natural-log
 * LSE of the scaled scores (-INFINITY when every key is masked).
 */
static float softmax_row(float *row, int S, float scale, const uint8_t *keep, float *cast, int bf16)
{
    float m = -INFINITY;
    for (int j = 0; j < S; ++j) {
        row[j] = row[j] * scale;
        if ((!keep || keep[j]) && row[j] > m) m = row[j];
    }
    if (m == -INFINITY) {
        for (int j = 0; j < S; ++j) row[j] = 0.0f;
        if (cast)
            for (int j = 0; j < S; ++j) cast[j] = 0.0f;
        return -INFINITY;
    }
    float sum = 0.0f;
    for (int j = 0; j < S; ++j) {
        const float e = (!keep || keep[j]) ? expf(row[j] - m) : 0.0f;
        row[j] = e;
        sum += e;
    }
    if (cast) {
        for (int j = 0; j < S; ++j) {
            const float p = row[j] / sum;
            row[j] = p;
            cast[j] = rnd(p, bf16);
        }
    } else {
        for (int j = 0; j < S; ++j) row[j] = row[j] / sum;
    }
    return m + logf(sum);
}

/* P32 [S][S] = softmax(Qh Kh^T * scale), lse[S]; lib.rs:138-147 / 222-239.
 * With P16 (which may be P itself), also P16 = P32 cast to the compute dtype
 * (`probs.to_dtype(q.dtype())`, lib.rs:147 / 239), elementwise. */
static void probs_f32(const float *Qh, const float *Kh, float *KT, float *P, float *lse, int S,
                      int D, float scale, const uint8_t *keep, float *P16, int bf16, int nthreads)
{
    og_transpose(S, D, Kh, D, KT, S, nthreads);
    og_gemm_nn(S, S, D, Qh, D, KT, S, P, S, nthreads);
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int i = 0; i < S; ++i) {
        const float l = softmax_row(P + (long)i * S, S, scale, keep, P16 ? P16 + (long)i * S : NULL, bf16);
        if (lse) lse[i] = l;
    }
}

/* Score-sized [S][S] buffers, kept per thread from one call to the next so
 * that a run over many heads does not map and fault in fresh pages each time
 * (held until the thread ends). */
#define N_SCORE_BUFS 3
static _Thread_local float *score_buf[N_SCORE_BUFS];
static _Thread_local size_t score_cap[N_SCORE_BUFS];

static float *score_buffer(int slot, size_t n)
{
    if (score_cap[slot] < n) {
        free(score_buf[slot]);
        score_buf[slot] = malloc(sizeof(float) * n);
        score_cap[slot] = score_buf[slot] ? n : 0;
    }
    return score_buf[slot];
}

static int check_dims(int B, int S, int H, int D, int h_begin, int h_end)
{
    if (B < 0 || S < 0 || H <= 0 || D <= 0) return -1;
    if (h_begin < 0 || h_end > H || h_begin > h_end) return -1;
    return 0;
}

int oracle_attn_fwd(const float *q, const float *k, const float *v, float *o, float *lse,
                    int B, int S, int H, int D, float scale, const uint8_t *key_keep, int bf16,
                    int h_begin, int h_end, int nthreads)
{
    if (check_dims(B, S, H, D, h_begin, h_end)) return -1;
    if (S == 0 || B == 0) return 0;
    float *Qh = malloc(sizeof(float) * S * D), *Kh = malloc(sizeof(float) * S * D);
    float *Vh = malloc(sizeof(float) * S * D), *KT = malloc(sizeof(float) * S * D);
    float *Oh = malloc(sizeof(float) * S * D), *L = malloc(sizeof(float) * S);
    float *P = score_buffer(0, (size_t)S * S);
    if (!Qh || !Kh || !Vh || !KT || !Oh || !L || !P) {
        free(Qh); free(Kh); free(Vh); free(KT); free(Oh); free(L);
        return -2;
    }
    for (int b = 0; b < B; ++b) {
        const uint8_t *keep = key_keep ? key_keep + (long)b * S : NULL;
        for (int h = h_begin; h < h_end; ++h) {
            gather_head(q, Qh, b, h, S, H, D);
            gather_head(k, Kh, b, h, S, H, D);
            gather_head(v, Vh, b, h, S, H, D);
            /* softmax, then probs.to_dtype(q.dtype()) in place — lib.rs:146-147 */
            probs_f32(Qh, Kh, KT, P, L, S, D, scale, keep, P, bf16, nthreads);
            /* probs.matmul(vt) in the compute dtype — lib.rs:148 */
            og_gemm_nn(S, D, S, P, S, Vh, D, Oh, D, nthreads);
            if (bf16) oracle_round_bf16_inplace(Oh, (long)S * D);
            scatter_head(Oh, o, b, h, S, H, D);
            if (lse) memcpy(lse + ((long)b * H + h) * S, L, sizeof(float) * S);
        }
    }
    free(Qh); free(Kh); free(Vh); free(KT); free(Oh); free(L);
    return 0;
}

int oracle_attn_bwd(const float *q, const float *k, const float *v, const float *dout,
                    float *dq, float *dk, float *dv, int B, int S, int H, int D, float scale,
                    const uint8_t *key_keep, int bf16, int h_begin, int h_end, int nthreads)
{
    if (check_dims(B, S, H, D, h_begin, h_end)) return -1;
    if (S == 0 || B == 0) return 0;
    const long SD = (long)S * D, SS = (long)S * S;
    float *Qh = malloc(sizeof(float) * SD), *Kh = malloc(sizeof(float) * SD);
    float *Vh = malloc(sizeof(float) * SD), *dOh = malloc(sizeof(float) * SD);
    float *T = malloc(sizeof(float) * SD), *R = malloc(sizeof(float) * SD);
    float *P32 = score_buffer(0, (size_t)SS), *P16 = score_buffer(1, (size_t)SS);
    float *dP = score_buffer(2, (size_t)SS);
    if (!Qh || !Kh || !Vh || !dOh || !T || !R || !P32 || !P16 || !dP) {
        free(Qh); free(Kh); free(Vh); free(dOh); free(T); free(R);
        return -2;
    }
    for (int b = 0; b < B; ++b) {
        const uint8_t *keep = key_keep ? key_keep + (long)b * S : NULL;
        for (int h = h_begin; h < h_end; ++h) {
            gather_head(q, Qh, b, h, S, H, D);
            gather_head(k, Kh, b, h, S, H, D);
            gather_head(v, Vh, b, h, S, H, D);
            gather_head(dout, dOh, b, h, S, H, D);
            /* recompute the f32 probabilities — lib.rs:227-238 — and
             * probs = probs32.to_dtype(q.dtype()) — lib.rs:239 */
            probs_f32(Qh, Kh, T, P32, NULL, S, D, scale, keep, P16, bf16, nthreads);
            /* dprobs = dout @ vt^T in the compute dtype — lib.rs:243 */
            og_transpose(S, D, Vh, D, T, S, nthreads);
            og_gemm_nn(S, S, D, dOh, D, T, S, dP, S, nthreads);
            /* (its cast to the compute dtype is taken in the softmax-backward
             * loop below, which is dP's next reader) */
            /* dV = probs^T @ dout — lib.rs:244 */
            og_gemm_tn(S, D, S, P16, S, dOh, D, R, D, nthreads);
            if (bf16) oracle_round_bf16_inplace(R, SD);
            scatter_head(R, dv, b, h, S, H, D);
            /* softmax backward in f32 — lib.rs:246-250:
             * rowsum = sum_j dP*P32; dS = P32 * (dP - rowsum) * scale */
#pragma omp parallel for num_threads(nthreads) schedule(static)
            for (int i = 0; i < S; ++i) {
                float *dpr = dP + (long)i * S;
                const float *pr = P32 + (long)i * S;
                float rs = 0.0f;
                for (int j = 0; j < S; ++j) {
                    dpr[j] = rnd(dpr[j], bf16);
                    rs += dpr[j] * pr[j];
                }
                for (int j = 0; j < S; ++j) dpr[j] = (pr[j] * (dpr[j] - rs)) * scale;
            }
            /* dQ = dS @ K_f32, dK = dS^T @ Q_f32, f32 matmuls cast back — lib.rs:251-257 */
            og_gemm_nn(S, D, S, dP, S, Kh, D, R, D, nthreads);
            if (bf16) oracle_round_bf16_inplace(R, SD);
            scatter_head(R, dq, b, h, S, H, D);
            og_gemm_tn(S, D, S, dP, S, Qh, D, R, D, nthreads);
            if (bf16) oracle_round_bf16_inplace(R, SD);
            scatter_head(R, dk, b, h, S, H, D);
        }
    }
    free(Qh); free(Kh); free(Vh); free(dOh); free(T); free(R);
    return 0;
}

/*
 * rms_norm — lib.rs:45-58: stats in f32, y = (x / sqrt(mean(x^2) + eps)),
 * cast to the compute dtype, then * weight in the compute dtype.
 * x, y: [rows][D]; w: [D].
 */
void oracle_rms_norm(const float *x, const float *w, float *y, long rows, int D, float eps, int bf16)
{
    for (long r = 0; r < rows; ++r) {
        const float *xr = x + r * D;
        float ss = 0.0f;
        for (int d = 0; d < D; ++d) ss += xr[d] * xr[d];
        const float sc = sqrtf(ss / (float)D + eps);
        for (int d = 0; d < D; ++d) y[r * D + d] = rnd(rnd(xr[d] / sc, bf16) * w[d], bf16);
    }
}

/*
 * rope_tables_dtype — lib.rs:77-105: for each position and axis a of width
 * dim_a, inv_j = theta^(-2j/dim_a) and f = pos[a] * inv_j in f32; cos/sin are
 * laid out [f_0..f_{half-1}, f_0..f_{half-1}] per axis segment and cast to the
 * compute dtype.  positions: [n_pos][n_axes]; cos_out/sin_out: [n_pos][sum(axes)].
 */
int oracle_rope_tables(const float *positions, int n_pos, int n_axes, const int *axes,
                       float theta, float *cos_out, float *sin_out, int bf16)
{
    int D = 0;
    for (int a = 0; a < n_axes; ++a) {
        if (axes[a] <= 0 || axes[a] % 2) return -1;
        D += axes[a];
    }
    for (int p = 0; p < n_pos; ++p) {
        int off = 0;
        for (int a = 0; a < n_axes; ++a) {
            const int dim_a = axes[a], half = dim_a / 2;
            for (int j = 0; j < half; ++j) {
                const float inv = powf(theta, -2.0f * (float)j / (float)dim_a);
                const float f = positions[(long)p * n_axes + a] * inv;
                const float c = rnd(cosf(f), bf16), s = rnd(sinf(f), bf16);
                cos_out[(long)p * D + off + j] = c;
                cos_out[(long)p * D + off + half + j] = c;
                sin_out[(long)p * D + off + j] = s;
                sin_out[(long)p * D + off + half + j] = s;
            }
            off += dim_a;
        }
    }
    return 0;
}

/* rotate-half per axis segment: [x1 | x2] -> [-x2 | x1] — lib.rs:107-120 */
static void rotate_half(const float *x, float *out, int n_axes, const int *axes)
{
    int off = 0;
    for (int a = 0; a < n_axes; ++a) {
        const int half = axes[a] / 2;
        for (int j = 0; j < half; ++j) {
            out[off + j] = -x[off + half + j];
            out[off + half + j] = x[off + j];
        }
        off += axes[a];
    }
}

/* transpose of rotate_half: [a1 | a2] -> [a2 | -a1] */
static void rotate_half_t(const float *x, float *out, int n_axes, const int *axes)
{
    int off = 0;
    for (int a = 0; a < n_axes; ++a) {
        const int half = axes[a] / 2;
        for (int j = 0; j < half; ++j) {
            out[off + j] = x[off + half + j];
            out[off + half + j] = -x[off + j];
        }
        off += axes[a];
    }
}

/*
 * apply_rope — lib.rs:122-129: out = x*cos + rot(x)*sin in f32 (tables upcast
 * from the compute dtype), cast back.  x, y: [S][H][D]; cos/sin: [S][D].
 */
int oracle_apply_rope(const float *x, const float *cos_t, const float *sin_t, float *y, long S,
                      int H, int n_axes, const int *axes, int bf16)
{
    int D = 0;
    for (int a = 0; a < n_axes; ++a) D += axes[a];
    if (D > 1024) return -1;
    float rot[1024];
    for (long s = 0; s < S; ++s)
        for (int h = 0; h < H; ++h) {
            const float *xr = x + (s * H + h) * D;
            rotate_half(xr, rot, n_axes, axes);
            for (int d = 0; d < D; ++d) {
                const float a = xr[d] * cos_t[s * D + d];
                const float b = rot[d] * sin_t[s * D + d];
                y[(s * H + h) * D + d] = rnd(a + b, bf16);
            }
        }
    return 0;
}

/*
 * Backward of apply_rope(rms_norm(x, w)) in f32 (the chain rule through
 * lib.rs:45-58 and 122-129, rounding casts treated as identity):
 *   g  = dy*cos + rot^T(dy*sin)            (RoPE is linear in its input)
 *   n  = x / sigma, sigma = sqrt(mean(x^2) + eps)
 *   dn = g * w
 *   dx = (dn - n * mean(dn * n)) / sigma
 * x, dy, dx: [S][H][D]; w: [D]; cos/sin: [S][D].
 */
int oracle_qk_prologue_bwd(const float *x, const float *w, const float *cos_t,
                           const float *sin_t, const float *dy, float *dx, long S, int H,
                           int n_axes, const int *axes, float eps)
{
    int D = 0;
    for (int a = 0; a < n_axes; ++a) D += axes[a];
    if (D > 1024) return -1;
    float t[1024], g[1024];
    for (long s = 0; s < S; ++s)
        for (int h = 0; h < H; ++h) {
            const float *xr = x + (s * H + h) * D, *dyr = dy + (s * H + h) * D;
            for (int d = 0; d < D; ++d) t[d] = dyr[d] * sin_t[s * D + d];
            rotate_half_t(t, g, n_axes, axes);
            for (int d = 0; d < D; ++d) g[d] = dyr[d] * cos_t[s * D + d] + g[d];
            float ss = 0.0f;
            for (int d = 0; d < D; ++d) ss += xr[d] * xr[d];
            const float sigma = sqrtf(ss / (float)D + eps);
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += (g[d] * w[d]) * (xr[d] / sigma);
            const float mdot = dot / (float)D;
            for (int d = 0; d < D; ++d)
                dx[(s * H + h) * D + d] = (g[d] * w[d] - (xr[d] / sigma) * mdot) / sigma;
        }
    return 0;
}

/*
 * linear_scaled — lib.rs:270-287:
 *   y = x W^T (+ bias) + scale * ((x A^T) B^T)
 * with x [N][in], W [out][in], A [r][in], B [out][r]; bias may be NULL, and
 * A == NULL or B == NULL disables the LoRA term.  In bf16 mode every Candle op
 * result is rounded to bf16 (matmul, bias add, both LoRA matmuls, the affine
 * and the final add), as in the reference's bf16 run.
 */
void oracle_linear_lora(const float *x, const float *W, const float *bias, const float *A,
                        const float *Bm, float *y, int N, int in_f, int out_f, int r,
                        float scale, int bf16, int nthreads)
{
    float *WT = malloc(sizeof(float) * (long)in_f * out_f);
    og_transpose(out_f, in_f, W, in_f, WT, out_f, nthreads);
    og_gemm_nn(N, out_f, in_f, x, in_f, WT, out_f, y, out_f, nthreads);
    free(WT);
    const long NO = (long)N * out_f;
    for (long i = 0; i < NO; ++i) {
        float t = rnd(y[i], bf16);
        if (bias) t = rnd(t + bias[i % out_f], bf16);
        y[i] = t;
    }
    if (!A || !Bm || r <= 0) return;
    float *AT = malloc(sizeof(float) * (long)in_f * r), *u = malloc(sizeof(float) * (long)N * r);
    float *BT = malloc(sizeof(float) * (long)r * out_f), *lo = malloc(sizeof(float) * NO);
    og_transpose(r, in_f, A, in_f, AT, r, nthreads);
    og_gemm_nn(N, r, in_f, x, in_f, AT, r, u, r, nthreads);
    for (long i = 0; i < (long)N * r; ++i) u[i] = rnd(u[i], bf16);
    og_transpose(out_f, r, Bm, r, BT, out_f, nthreads);
    og_gemm_nn(N, out_f, r, u, r, BT, out_f, lo, out_f, nthreads);
    for (long i = 0; i < NO; ++i) {
        const float l = rnd(rnd(lo[i], bf16) * scale, bf16);
        y[i] = rnd(y[i] + l, bf16);
    }
    free(AT); free(u); free(BT); free(lo);
}

/*
 * Backward of linear_scaled (chain rule through lib.rs:276-285, the steps
 * Candle's autograd takes):
 *   g  = scale * dy              (affine backward)
 *   u  = x A^T
 *   dB = g^T u                   [out][r]
 *   du = g B                     [N][r]
 *   dA = du^T x                  [r][in]
 *   dx = dy W + du A             [N][in]   (dx may be NULL)
 * In bf16 mode each op's result is rounded to bf16.
 */
void oracle_linear_lora_bwd(const float *x, const float *W, const float *A, const float *Bm,
                            const float *dy, float *dx, float *dA, float *dB, int N, int in_f,
                            int out_f, int r, float scale, int bf16, int nthreads)
{
    const long NO = (long)N * out_f, NR = (long)N * r;
    float *g = malloc(sizeof(float) * NO), *AT = malloc(sizeof(float) * (long)in_f * r);
    float *u = malloc(sizeof(float) * NR), *du = malloc(sizeof(float) * NR);
    for (long i = 0; i < NO; ++i) g[i] = rnd(dy[i] * scale, bf16);
    og_transpose(r, in_f, A, in_f, AT, r, nthreads);
    og_gemm_nn(N, r, in_f, x, in_f, AT, r, u, r, nthreads);
    for (long i = 0; i < NR; ++i) u[i] = rnd(u[i], bf16);
    og_gemm_tn(out_f, r, N, g, out_f, u, r, dB, r, nthreads);
    for (long i = 0; i < (long)out_f * r; ++i) dB[i] = rnd(dB[i], bf16);
    og_gemm_nn(N, r, out_f, g, out_f, Bm, r, du, r, nthreads);
    for (long i = 0; i < NR; ++i) du[i] = rnd(du[i], bf16);
    og_gemm_tn(r, in_f, N, du, r, x, in_f, dA, in_f, nthreads);
    for (long i = 0; i < (long)r * in_f; ++i) dA[i] = rnd(dA[i], bf16);
    if (dx) {
        float *t = malloc(sizeof(float) * (long)N * in_f);
        og_gemm_nn(N, in_f, out_f, dy, out_f, W, in_f, dx, in_f, nthreads);
        og_gemm_nn(N, in_f, r, du, r, A, in_f, t, in_f, nthreads);
        for (long i = 0; i < (long)N * in_f; ++i) dx[i] = rnd(rnd(dx[i], bf16) + rnd(t[i], bf16), bf16);
        free(t);
    }
    free(g); free(AT); free(u); free(du);
}
