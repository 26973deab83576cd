/*
 * TEST INFRASTRUCTURE ONLY — CPU restatement of the memory-bound ops of
 * foundry-spike's double-stream LoRA block.
 *   layer_norm_mod       lib.rs:60-71 (and its autograd gradient)
 *   gated residual       bin/throughput.rs:552-572   (x + g * branch)
 *   tanh-GELU            c4's MLP activation: no reference counterpart (the
 *                        reference block uses SwiGLU, lib.rs:293-297); the
 *                        closed form u/2 (1 + tanh(sqrt(2/pi)(u + 0.044715 u^3)))
 *   silu                 bin/throughput.rs:297-324 (modulation input)
 *   adamw_step           lib.rs:477-510, operation for operation
 * f32 arithmetic throughout; bf16 != 0 rounds results to bf16 where the
 * reference casts back to the compute dtype.  Only tests/ load this.
 */
#include <math.h>
#include <stddef.h>

#include "oracle.h"

static float rnd(float x, int bf16) { return bf16 ? oracle_bf16_round(x) : x; }

/* lib.rs:60-71: xf = f32(x); mean; centered; var = mean(centered^2);
 * normed = centered / sqrt(var + eps); m = normed * (scale + 1) + shift. */
void oracle_ln_mod_fwd(const float *x, long N, int C, const float *shift, const float *scale, float eps,
                       int bf16, float *y, float *mean, float *rstd) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < N; ++r) {
        const float *xr = x + r * C;
        float s = 0.f;
        for (int c = 0; c < C; ++c) s += xr[c];
        const float mu = s / (float)C;
        float q = 0.f;
        for (int c = 0; c < C; ++c) {
            const float d = xr[c] - mu;
            q += d * d;
        }
        const float var = q / (float)C;
        const float den = sqrtf(var + eps);
        for (int c = 0; c < C; ++c) {
            const float normed = (xr[c] - mu) / den;
            y[r * C + c] = rnd(normed * (scale[c] + 1.f) + shift[c], bf16);
        }
        if (mean) mean[r] = mu;
        if (rstd) rstd[r] = 1.f / den;
    }
}

/* Gradient of layer_norm_mod w.r.t. x (shift and scale frozen):
 * n = (x - mean) * rstd, dn = dy * (1 + scale),
 * dx = dres + rstd * (dn - mean(dn) - n * mean(dn * n)). */
void oracle_ln_mod_bwd(const float *x, const float *dy, long N, int C, const float *scale, const float *mean,
                       const float *rstd, const float *dres, int bf16, float *dx) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < N; ++r) {
        const float *xr = x + r * C, *gr = dy + r * C;
        double a = 0.0, b = 0.0;
        for (int c = 0; c < C; ++c) {
            const float n = (xr[c] - mean[r]) * rstd[r];
            const float dn = gr[c] * (scale[c] + 1.f);
            a += dn;
            b += (double)dn * n;
        }
        const float ma = (float)(a / C), mb = (float)(b / C);
        for (int c = 0; c < C; ++c) {
            const float n = (xr[c] - mean[r]) * rstd[r];
            const float dn = gr[c] * (scale[c] + 1.f);
            const float v = (dres ? dres[r * C + c] : 0.f) + rstd[r] * (dn - ma - n * mb);
            dx[r * C + c] = rnd(v, bf16);
        }
    }
}

/* x + g * b per row (x may be NULL), g broadcast over rows. */
void oracle_gated_residual(const float *x, const float *g, const float *b, long N, int C, int bf16, float *y) {
    for (long r = 0; r < N; ++r)
        for (int c = 0; c < C; ++c)
            y[r * C + c] = rnd((x ? x[r * C + c] : 0.f) + g[c] * b[r * C + c], bf16);
}

static const double kK0 = 0.79788456080286535588; /* sqrt(2/pi) */
static const double kK1 = 0.044715;

void oracle_gelu_fwd(const float *b, long n, int bf16, float *y) {
    for (long i = 0; i < n; ++i) {
        const double u = b[i];
        y[i] = rnd((float)(0.5 * u * (1.0 + tanh(kK0 * (u + kK1 * u * u * u)))), bf16);
    }
}

/* y = dy * d/du gelu(u) = dy * (0.5 (1 + t) + 0.5 u (1 - t^2) k0 (1 + 3 k1 u^2)) */
void oracle_gelu_bwd(const float *dy, const float *b, long n, int bf16, float *y) {
    for (long i = 0; i < n; ++i) {
        const double u = b[i];
        const double t = tanh(kK0 * (u + kK1 * u * u * u));
        const double d = 0.5 * (1.0 + t) + 0.5 * u * (1.0 - t * t) * kK0 * (1.0 + 3.0 * kK1 * u * u);
        y[i] = rnd((float)(dy[i] * d), bf16);
    }
}

void oracle_silu(const float *b, long n, int bf16, float *y) {
    for (long i = 0; i < n; ++i) y[i] = rnd((float)(b[i] / (1.0 + exp(-(double)b[i]))), bf16);
}

/* swiglu activation, lib.rs:293-297 (and gen_block.py:167, throughput.rs:620):
 * y = silu(gate) * up, the silu op's result rounded to the tensor dtype
 * before the mul.  Computed in f64, rounded at the two op results. */
void oracle_swiglu_fwd(const float *gate, const float *up, long n, int bf16, float *y) {
    for (long i = 0; i < n; ++i) {
        const double g = gate[i];
        const float s = rnd((float)(g / (1.0 + exp(-g))), bf16);
        y[i] = rnd((float)((double)s * up[i]), bf16);
    }
}

/* Backward of the above by the chain rule (the autograd of mul, then silu):
 *   dup   = dy * silu(gate)                     (mul backward, one product)
 *   dgate = (dy * up) * sig(g) (1 + g (1 - sig(g)))
 * dy * up and each result rounded to the tensor dtype. */
void oracle_swiglu_bwd(const float *dy, const float *gate, const float *up, long n, int bf16, float *dgate,
                       float *dup) {
    for (long i = 0; i < n; ++i) {
        const double g = gate[i];
        const double sg = 1.0 / (1.0 + exp(-g));
        const float s = rnd((float)(g * sg), bf16);
        dup[i] = rnd((float)((double)dy[i] * s), bf16);
        const float dgu = rnd((float)((double)dy[i] * up[i]), bf16);
        dgate[i] = rnd((float)((double)dgu * sg * (1.0 + g * (1.0 - sg))), bf16);
    }
}

/* lib.rs:477-510 with f32 tensors: the AdamW constants are f64, and
 * affine(mul, add) multiplies / adds them cast to f32; 1 - beta and
 * bc = 1 - beta^step are formed in f64.  bf16 != 0 rounds the updated
 * parameter (the Var's dtype) to bf16. */
void oracle_adamw_step(float *param, const float *grad, float *m, float *v, long n, double lr, double beta1,
                       double beta2, double eps, int step, int bf16) {
    const float b1 = (float)beta1, b2 = (float)beta2;
    const float omb1 = (float)(1.0 - beta1), omb2 = (float)(1.0 - beta2);
    const float ibc1 = (float)(1.0 / (1.0 - pow(beta1, step)));
    const float ibc2 = (float)(1.0 / (1.0 - pow(beta2, step)));
    const float lrf = (float)lr, epsf = (float)eps;
    for (long i = 0; i < n; ++i) {
        const float g = grad[i];
        const float mn = m[i] * b1 + g * omb1;
        const float gg = g * g;
        const float vn = v[i] * b2 + gg * omb2;
        const float mhat = mn * ibc1;
        const float den = sqrtf(vn * ibc2) + epsf;
        const float delta = (mhat / den) * lrf;
        param[i] = rnd(param[i] - delta, bf16);
        m[i] = mn;
        v[i] = vn;
    }
}
