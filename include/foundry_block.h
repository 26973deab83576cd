/*
 * foundry_block.h — C ABI of the memory-bound ops of the double-stream LoRA
 * block (libfoundry_attn.so, same library and conventions as foundry_attn.h).
 *
 * These replace the Candle op chains the reference's block runs between its
 * linears and its attention (crates/foundry-spike/src/bin/throughput.rs:
 * 480-574, the fixture-sized lib.rs:301-392):
 *   layer_norm_mod   lib.rs:60-71        fa_ln_mod_fwd / fa_ln_mod_bwd
 *   gated residual + layer_norm_mod   throughput.rs:552-566
 *                                        fa_gated_ln_mod_fwd / fa_ln_mod_bwd_gate
 *   gated residual   throughput.rs:552-572   fa_gated_residual
 *   MLP activation   (c4 block: tanh-GELU; the reference block's SwiGLU,
 *                    lib.rs:293-297, has no tanh-GELU counterpart)
 *                                        fa_gelu_fwd / fa_gelu_bwd
 *   swiglu           lib.rs:293-297 (the activation between its linears;
 *                    single block throughput.rs:620)
 *                                        fa_swiglu_fwd / fa_swiglu_bwd
 *   modulation input silu(temb)  throughput.rs:297-324     fa_silu
 *   adamw_step       lib.rs:477-510      fa_adamw_step, fa_adamw_step_many
 *   MLP linear + activation  linear_scaled's base product lib.rs:270-287
 *                    at throughput.rs:254-256, fused with the GELU that
 *                    follows W1 or the GELU gradient after W2's dX
 *                                        fa_gemm_bf16
 *
 * Row views: `rows` x `cols` elements, row r starting at base + r * ld
 * elements; cols % 8 == 0, ld >= cols, and base and ld keep every row
 * 16-byte aligned (ld % 8 == 0 for bf16, % 4 for f32).  Per-column vectors
 * ([cols]: shift, scale, gate) are contiguous and 16-byte aligned.
 * Arithmetic is f32; results are rounded once to the storage dtype.
 */
#ifndef FOUNDRY_BLOCK_H
#define FOUNDRY_BLOCK_H

#include "foundry_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fa_ln_mod_args {
    int32_t dtype;        /* fa_dtype of x, shift, scale, y (and dy, dres, dx)   */
    int32_t rows, cols;   /* N >= 1; 8 <= C <= 4096                              */
    float eps;            /* > 0 (the reference's NORM_EPS is 1e-6)              */
    const void *x;        /* [N, C]                                              */
    int64_t ldx;
    const void *shift;    /* [C] */
    const void *scale;    /* [C]: y = (1 + scale) * LN(x) + shift                */
    void *y;              /* [N, C] output (fwd)                                 */
    int64_t ldy;
    float *mean, *rstd;   /* [N] f32: written by fwd when non-NULL (rstd =
                             1/sqrt(var + eps)); required by bwd                 */
} fa_ln_mod_args;

/* y = (1 + scale) * (x - mean) / sqrt(var + eps) + shift per row, mean and
 * (biased) variance in f32.  Replaces layer_norm_mod (lib.rs:60-71). */
fa_status fa_ln_mod_fwd(const fa_ln_mod_args *args, void *stream);

typedef struct fa_ln_mod_bwd_args {
    fa_ln_mod_args fwd;   /* x, scale, mean, rstd as in the forward; y unused    */
    const void *dy;       /* [N, C] gradient of y                                */
    int64_t lddy;
    const void *dres;     /* [N, C] or NULL: added to dx (the residual path)     */
    int64_t ldres;
    void *dx;             /* [N, C] output                                       */
    int64_t lddx;
} fa_ln_mod_bwd_args;

/* dx = dres + rstd * (dn - mean(dn) - n * mean(dn * n)), n = (x - mean) * rstd,
 * dn = dy * (1 + scale): the gradient Candle's autograd forms through
 * layer_norm_mod (shift and scale are frozen, so no gradient for them). */
fa_status fa_ln_mod_bwd(const fa_ln_mod_bwd_args *args, void *stream);

typedef struct fa_gated_ln_mod_args {
    fa_ln_mod_args ln;    /* x: the residual stream; y, mean, rstd: layer_norm_mod
                             of the sum below (ln.x is not normalised itself)   */
    const void *g;        /* [C] gate                                            */
    const void *b;        /* [N, C] gated branch                                 */
    int64_t ldb;
    void *sum;            /* [N, C] output: x + g * b, the norm's input          */
    int64_t ldsum;
    void *sum2;           /* [N, C] or NULL: a second copy of the sum            */
    int64_t ldsum2;
} fa_gated_ln_mod_args;

/* sum = x + g * b (as fa_gated_residual), then y = layer_norm_mod(sum), in one
 * pass: the gated residual and the layer_norm_mod that follows it in the
 * double block (throughput.rs:552-566, lib.rs:60-71), with the bits of
 * fa_gated_residual followed by fa_ln_mod_fwd on its output.  sum may alias
 * x or b element for element; y, sum2 and the statistics must not overlap
 * any other view. */
fa_status fa_gated_ln_mod_fwd(const fa_gated_ln_mod_args *args, void *stream);

typedef struct fa_ln_mod_bwd_gate_args {
    fa_ln_mod_bwd_args bwd; /* as for fa_ln_mod_bwd                              */
    const void *g;        /* [C] gate                                            */
    void *gdx;            /* [N, C] output: g * dx                               */
    int64_t ldgdx;
} fa_ln_mod_bwd_gate_args;

/* dx as fa_ln_mod_bwd, and gdx = g * dx (dx as rounded to the dtype) in the
 * same pass: the gradient through the gated branch whose sum fed the norm
 * (Candle's autograd through throughput.rs:552-566), with the bits of
 * fa_ln_mod_bwd followed by fa_gated_residual (x NULL) on its dx.  gdx must
 * not overlap dx. */
fa_status fa_ln_mod_bwd_gate(const fa_ln_mod_bwd_gate_args *args, void *stream);

typedef struct fa_rows_args {
    int32_t dtype;        /* fa_dtype of every view                              */
    int32_t rows, cols;
    const void *x;        /* [N, C] (see each op)                                */
    int64_t ldx;
    const void *g;        /* [C] gate (fa_gated_residual only)                   */
    const void *b;        /* [N, C] input                                        */
    int64_t ldb;
    void *y;              /* [N, C] output; may alias x or b element for element */
    int64_t ldy;
} fa_rows_args;

/* y = x + g * b with g broadcast over rows; x may be NULL (y = g * b, the
 * gradient of the gated branch).  Replaces the broadcast_mul + add of
 * throughput.rs:552-572. */
fa_status fa_gated_residual(const fa_rows_args *args, void *stream);

/* y = b/2 * (1 + tanh(sqrt(2/pi) * (b + 0.044715 b^3))) (x unused).  The c4
 * block's MLP activation; no reference counterpart (the reference block uses
 * SwiGLU, lib.rs:293-297). */
fa_status fa_gelu_fwd(const fa_rows_args *args, void *stream);

/* y = x * gelu'(b): x is the gradient of gelu(b). */
fa_status fa_gelu_bwd(const fa_rows_args *args, void *stream);

/* y = b / (1 + exp(-b)) (x unused): the SiLU of the conditioning vector that
 * feeds the frozen modulation linear (throughput.rs:297-324). */
fa_status fa_silu(const fa_rows_args *args, void *stream);

typedef struct fa_swiglu_args {
    int32_t dtype;        /* fa_dtype of every view                              */
    int32_t rows, cols;   /* N >= 1; C % 8 == 0                                  */
    const void *gate;     /* [N, C] gate projection (pre-activation)             */
    int64_t ldgate;
    const void *up;       /* [N, C] up projection                                */
    int64_t ldup;
    void *y;              /* [N, C] output (fwd)                                 */
    int64_t ldy;
} fa_swiglu_args;

/* y = silu(gate) * up, silu(g) = g / (1 + exp(-g)) rounded to the storage
 * dtype before the product (Candle's silu op result, then its mul):
 * replaces the silu + mul of swiglu (lib.rs:293-297) and of the single block
 * (throughput.rs:620). */
fa_status fa_swiglu_fwd(const fa_swiglu_args *args, void *stream);

typedef struct fa_swiglu_bwd_args {
    fa_swiglu_args fwd;   /* gate, up as in the forward; y unused                */
    const void *dy;       /* [N, C] gradient of y                                */
    int64_t lddy;
    void *dgate;          /* [N, C] output: (dy * up) * silu'(gate)              */
    int64_t lddgate;
    void *dup;            /* [N, C] output: dy * silu(gate)                      */
    int64_t lddup;
} fa_swiglu_bwd_args;

/* The gradients Candle's autograd forms through silu(gate) * up, with
 * silu'(g) = s(g) (1 + g (1 - s(g))), s = sigmoid; dy*up and dy*silu(gate) are
 * rounded to the storage dtype as the mul's backward products. */
fa_status fa_swiglu_bwd(const fa_swiglu_bwd_args *args, void *stream);

typedef struct fa_adamw_args {
    int32_t dtype;        /* fa_dtype of param                                   */
    int64_t n;            /* elements, >= 1                                      */
    void *param;          /* [n], updated in place                               */
    const float *grad;    /* [n] f32                                             */
    float *m, *v;         /* [n] f32 moments, updated in place (zero at step 1)  */
    double lr, beta1, beta2, eps; /* f64, as the reference's AdamW fields; each is
                             rounded to f32 where the reference's f32 affine
                             uses it, 1 - beta and the bias corrections are
                             formed in f64                                       */
    int32_t step;         /* >= 1: bias corrections 1 - beta^step (in double)   */
} fa_adamw_args;

/* One AdamW step, weight decay 0, in adamw_step's operation order
 * (lib.rs:477-510): m' = m*b1 + g*(1-b1); v' = v*b2 + g^2*(1-b2);
 * p' = p - ((m'/bc1) / (sqrt(v'/bc2) + eps)) * lr, every f32 product or sum
 * rounded separately. */
fa_status fa_adamw_step(const fa_adamw_args *args, void *stream);

/* fa_adamw_step over `count` tensors of one optimiser step (one adapter
 * stack's LoRA factors) in as few launches as possible (up to 32 tensors
 * each): every tensor gets the same bits as its own fa_adamw_step call.
 * dtype, lr, betas, eps and step must be equal across the array.  The
 * reference steps each parameter in turn (lib.rs:477-510 inside the loop of
 * throughput.rs:787-803). */
fa_status fa_adamw_step_many(const fa_adamw_args *args, int32_t count, void *stream);

typedef struct fa_copy2d_args {
    int32_t dtype;            /* fa_dtype of src and dst                         */
    int32_t rows, cols;       /* >= 1                                            */
    const void *src;          /* element (r, c) at src[r * src_rs + c * src_cs]  */
    int64_t src_rs, src_cs;   /* strides in elements, >= 0                       */
    void *dst;                /* element (r, c) at dst[r * dst_rs + c * dst_cs]  */
    int64_t dst_rs, dst_cs;
} fa_copy2d_args;

/* dst[r, c] = src[r, c] over each of `count` 2D views, in as few launches as
 * possible (up to 32 views each).  No view's destination may overlap another
 * view's source or destination.  No counterpart in the reference, which
 * applies each LoRA factor where it is stored (lib.rs:270-287): the blocks
 * here keep copies of the factors inside the frozen GEMMs' operands and
 * transposed, and refresh them after each AdamW step with one such call. */
fa_status fa_copy2d_many(const fa_copy2d_args *args, int32_t count, void *stream);

/* Epilogues of fa_gemm_bf16. */
typedef enum fa_gemm_epilogue {
    FA_GEMM_PLAIN = 0,  /* c = bf16(acc)                                         */
    FA_GEMM_GELU = 1,   /* c = pre = bf16(acc), c2 = bf16(gelu(pre))             */
    FA_GEMM_DGELU = 2   /* c = bf16(bf16(acc) * gelu'(aux)), aux = the saved pre */
} fa_gemm_epilogue;

typedef struct fa_gemm_args {
    int32_t epilogue;     /* fa_gemm_epilogue                                    */
    int32_t m, n, k;      /* m, n multiples of 256; k a multiple of 64, >= 64    */
    const void *a;        /* [m, k] bf16 (x), row stride lda                     */
    int64_t lda;
    const void *b;        /* [n, k] bf16 (W as stored by a linear), stride ldb   */
    int64_t ldb;
    void *c;              /* [m, n] bf16 output, stride ldc                      */
    int64_t ldc;
    void *c2;             /* FA_GEMM_GELU: [m, n] bf16 gelu(c), stride ldc2      */
    int64_t ldc2;
    const void *aux;      /* FA_GEMM_DGELU: [m, n] bf16 pre-activation, ldaux    */
    int64_t ldaux;
} fa_gemm_args;

/* c = a b^T (bf16 in, f32 accumulation) with the epilogue, one launch.  The
 * base product of linear_scaled (lib.rs:270-287) for the c4 block's MLP
 * linears (throughput.rs:480-574), fused with the elementwise op after it:
 * W1's forward with its GELU (FA_GEMM_GELU, c holds the pre-activation the
 * backward needs), and W2's dX product with the GELU gradient (FA_GEMM_DGELU:
 * the result is the gradient at W1's output).  The product is rounded to bf16
 * before the epilogue, as the reference's bf16 matmul output is; gelu is the
 * tanh form of fa_gelu_fwd / fa_gelu_bwd.  Views: 16-byte aligned bases, row
 * strides multiples of 8 elements and >= k (a, b) or >= n (c, c2, aux);
 * c and c2 must not overlap a, b or aux; a 256-row block of a or b must span
 * fewer than 2^31 bytes. */
fa_status fa_gemm_bf16(const fa_gemm_args *args, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FOUNDRY_BLOCK_H */
