/*
 * foundry_attn.h — C ABI of the MI355X (gfx950) attention hot path.
 *
 * Drop-in boundary for erikerikerik/foundry-trainer's `foundry-spike` crate:
 * the Candle `CustomOp3` `AttnBwd` (crates/foundry-spike/src/lib.rs:151-264)
 * and the memory-bound ops around it (rms_norm lib.rs:45-58, rope_tables_dtype
 * lib.rs:77-105, apply_rope lib.rs:122-129, linear_scaled lib.rs:270-287).
 * Each entry point below names the reference interface it replaces.
 *
 * Conventions
 *   - Every device buffer is owned by the caller; nothing on the hot path
 *     allocates.  Scratch memory comes in through a caller workspace.
 *   - Launches go on the caller's HIP stream (`stream`, a hipStream_t, NULL =
 *     the null stream) and are asynchronous.
 *   - Attention tensors are [B, S, H, D] views given by element strides for
 *     b, s and h; the head-dim stride is 1.  B = 1 with contiguous strides is
 *     the reference's per-sample (S, H, D) layout.  Base pointers and strides
 *     must keep every row 16-byte aligned.
 *   - The joint sequence is txt first, then img (lib.rs:363-365).
 *   - No exception or C++ type crosses this boundary.  On failure a call
 *     returns a non-zero fa_status and fa_last_error() (thread-local) says why.
 *     Arguments are validated before any device work.
 *   - Calls on distinct streams may run concurrently.
 */
#ifndef FOUNDRY_ATTN_H
#define FOUNDRY_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 2

typedef enum fa_status {
    FA_OK = 0,
    FA_ERR_INVALID_ARG = 1, /* bad shape, stride, pointer, scale or workspace      */
    FA_ERR_UNSUPPORTED = 2, /* valid request this build does not implement          */
    FA_ERR_NO_DEVICE = 3,   /* no HIP device visible                                */
    FA_ERR_LOAD_FAILED = 4, /* device is not gfx950 / code object cannot be used    */
    FA_ERR_HIP = 5          /* a HIP runtime call or kernel launch failed           */
} fa_status;

typedef enum fa_dtype {
    FA_DTYPE_BF16 = 0, /* bf16 storage, f32 arithmetic and accumulation */
    FA_DTYPE_F32 = 1   /* f32 storage and arithmetic (the reference's CPU dtype) */
} fa_dtype;

/* Element strides of a [B, S, H, D] view; the D stride is 1. */
typedef struct fa_strides {
    int64_t b, s, h;
} fa_strides;

/* ------------------------------------------------------------------------- */
/* Library                                                                   */
/* ------------------------------------------------------------------------- */

/* ABI version (FA_ABI_VERSION). */
int fa_version(void);

/* Reason for the last failure on this thread ("" if none). */
const char *fa_last_error(void);

/* Name of the op, as CustomOp3::name returns it (lib.rs:154-156):
 * "foundry-attn-bwd". */
const char *fa_op_name(void);

/* Checks that `device` is a gfx950 GPU and prepares the kernels for it
 * (LDS limits), and looks up the device address of fa_attn_bwd_noalloc's
 * scratch on it.  Idempotent and thread-safe; the attention entry points call
 * the device part for the current device on first use.  Replaces the CUDA
 * device/NVRTC setup the reference does through cudarc (src/main.rs:16-38). */
fa_status fa_init(int device);

/* ------------------------------------------------------------------------- */
/* Attention (AttnBwd)                                                       */
/* ------------------------------------------------------------------------- */

typedef struct fa_attn_fwd_args {
    int32_t dtype;           /* fa_dtype of q, k, v and o                          */
    int32_t batch;           /* B >= 1                                            */
    int32_t seq;             /* S >= 1 (queries and keys: joint self-attention)   */
    int32_t heads;           /* H >= 1                                            */
    int32_t head_dim;        /* D: 64 or 128                                      */
    float scale;             /* softmax scale, finite and > 0; the reference
                                hard-codes 1/sqrt(128) (lib.rs:138)               */
    const void *q, *k, *v;   /* [B,S,H,D]                                         */
    void *o;                 /* [B,S,H,D] output                                  */
    float *lse;              /* [B,H,S] contiguous f32 output: natural-log
                                logsumexp of the scaled scores of each query row;
                                -inf for a row whose keys are all masked          */
    const uint8_t *key_keep; /* NULL (no mask) or [B,S] contiguous: 0 = key is
                                excluded from every row's softmax                 */
    fa_strides q_stride, k_stride, v_stride, o_stride;
    void *workspace;         /* NULL, or device scratch (256-B aligned) of at
                                least fa_attn_fwd_workspace_size bytes: lets a
                                small bf16 grid split each tile's keys         */
    size_t workspace_bytes;
} fa_attn_fwd_args;

/* Bytes of workspace a split forward needs for these shapes: nonzero for bf16
 * when B x H x ceil(S/256) workgroups would leave at least half of the
 * current device's CUs idle and S >= 1024 (for example 3 or 6 heads at
 * S = 4608: one GPU's share of 24 heads over 8 or 4 GPUs).  Each query tile's
 * keys are then cut into up to 16 ranges of >= 512 keys on separate
 * workgroups, whose f32 partials are merged through their LSEs.  0 means
 * the forward never splits these shapes.  No reference counterpart. */
size_t fa_attn_fwd_workspace_size(const fa_attn_fwd_args *args);

/* O = softmax(Q K^T * scale) V per (b, h), scores and softmax in f32, P cast to
 * the storage dtype before P V (lib.rs:131-149), plus the per-row LSE that the
 * backward uses to recompute P.  A fully masked row gives O = 0, LSE = -inf.
 * With workspace NULL the call never splits; with a workspace of at least
 * fa_attn_fwd_workspace_size bytes it splits the shapes that size covers (a
 * smaller non-NULL workspace is FA_ERR_INVALID_ARG).  Results are
 * deterministic either way.  Replaces AttnBwd::cuda_fwd (lib.rs:189-214) and
 * AttnBwd::cpu_fwd (lib.rs:158-187). */
fa_status fa_attn_fwd(const fa_attn_fwd_args *args, void *stream);

typedef struct fa_attn_bwd_args {
    int32_t dtype, batch, seq, heads, head_dim; /* as in fa_attn_fwd_args        */
    float scale;                                /* the forward's scale           */
    const void *q, *k, *v;                      /* forward inputs                */
    const void *o;                              /* forward output (`res`)        */
    const void *dout;                           /* upstream gradient dL/dO       */
    const float *lse;                           /* forward LSE [B,H,S]           */
    const uint8_t *key_keep;                    /* the forward's mask or NULL    */
    void *dq, *dk, *dv;                         /* [B,S,H,D] outputs             */
    void *workspace;                            /* device scratch, 256-B aligned */
    size_t workspace_bytes;                     /* >= fa_attn_bwd_workspace_size */
    fa_strides q_stride, k_stride, v_stride, o_stride, do_stride;
    fa_strides dq_stride, dk_stride, dv_stride;
} fa_attn_bwd_args;

/* Bytes of workspace fa_attn_bwd takes for these shapes (0 on bad args): the
 * pre-pass rows, plus, for the shapes fa_attn_fwd_workspace_size splits, f32
 * partial sums of dQ, dK and dV (dQ's key range and dK/dV's query range are
 * split the same way, and a reduce pass adds the partials in a fixed order),
 * plus, for unsplit bf16 calls with 8-wave workgroups, the bf16 dS of every
 * (key, query) pair ([B*H][seq rounded up to 32][seq rounded up to 256]),
 * through which dQ reads the dK/dV kernel's dS instead of recomputing S and
 * dP (about 1 GB at B1 H24 S4608; shapes whose dS would exceed
 * FA_BWD_DS_MAX_BYTES keep the recomputing path and ask for no dS).  No
 * reference counterpart: AttnBwd::bwd (lib.rs:216-263) allocates its own
 * tensors. */
#define FA_BWD_DS_MAX_BYTES (16ull << 30)
size_t fa_attn_bwd_workspace_size(const fa_attn_bwd_args *args);

/* The least workspace fa_attn_bwd accepts (0 on bad args): without the dS^T
 * rows, so dQ recomputes S and dP.  A workspace of at least
 * fa_attn_bwd_workspace_size bytes takes the stored-dS path, a smaller one
 * (of at least this size) the recomputing one.  Both multiply the same bf16
 * dS by K in the same key order, so they give the same bits.  No reference
 * counterpart. */
size_t fa_attn_bwd_min_workspace_size(const fa_attn_bwd_args *args);

/* dQ, dK, dV of the forward above: P is recomputed from Q, K and the saved
 * LSE; dS = P * (dP - rowsum(dO * O)) * scale; dQ = dS K, dK = dS^T Q,
 * dV = P^T dO, f32 accumulation, deterministic (no atomics).  For bf16 with
 * 4-wave (128-row) workgroups -- seq < 512, or an 8-wave grid whose last
 * round would be under half full -- the dQ kernel runs on a library-owned
 * side stream (one per host thread and device, default priority) beside
 * dK/dV, joined back to `stream` by events before the call returns.  With
 * 8-wave workgroups the launches run in order on `stream`: with the full
 * workspace the pre-pass, dK/dV (also storing dS), then dQ = dS K * scale
 * read from the stored dS; with the minimum one dQ (which also forms the
 * pre-pass for its queries, recomputing S and dP), then dK/dV; a split call
 * adds one reduce of the partials.  Either way everything queued on `stream`
 * afterwards sees the results.  Replaces AttnBwd::bwd (lib.rs:216-263). */
fa_status fa_attn_bwd(const fa_attn_bwd_args *args, void *stream);

/* The backward in its three launches, for callers that time them or run the
 * two independent gradient kernels on separate streams:
 *   FA_BWD_PREPASS  rowsum(dO * O) and LSE*log2(e) into the workspace
 *   FA_BWD_DKDV     dK and dV (needs the pre-pass)
 *   FA_BWD_DQ       dQ        (needs the pre-pass; through the stored dS,
 *                             also dK/dV, whose dS it reads)
 * FA_BWD_ALL runs all three, as fa_attn_bwd.  The caller orders the pre-pass
 * before the other two (same stream, or an event), and with a workspace of
 * fa_attn_bwd_workspace_size bytes (the stored-dS path, see above) dK/dV
 * before dQ; with fa_attn_bwd_min_workspace_size bytes dK/dV and dQ are
 * independent.  No reference counterpart: AttnBwd::bwd (lib.rs:216-263) is
 * one call. */
typedef enum fa_bwd_phase {
    FA_BWD_ALL = 0,
    FA_BWD_PREPASS = 1,
    FA_BWD_DKDV = 2,
    FA_BWD_DQ = 3
} fa_bwd_phase;
fa_status fa_attn_bwd_phase(const fa_attn_bwd_args *args, int32_t phase, void *stream);

/* Largest B * heads * seq that fa_attn_bwd_noalloc accepts, and the scratch
 * it holds per device for them (delta and LSE*log2(e) rows, f32 each). */
#define FA_BWD_NOALLOC_MAX_ROWS (1 << 21)
#define FA_BWD_NOALLOC_SCRATCH_BYTES (2 * FA_BWD_NOALLOC_MAX_ROWS * 4)

/* fa_attn_bwd without a workspace and without any allocation: no counterpart
 * in the reference.  It is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  `workspace` must be NULL and `workspace_bytes` 0; the scratch
 * is a fixed array of FA_BWD_NOALLOC_SCRATCH_BYTES (16 MiB) in the library's
 * device code, one per GPU, held until the process ends, so calls with
 * B * heads * seq > FA_BWD_NOALLOC_MAX_ROWS fail with FA_ERR_INVALID_ARG.
 * The call never splits key or query ranges (the split partials would not
 * fit), runs every launch in order on `stream` (no side stream), and calls no
 * allocating routine.  For shapes fa_attn_bwd does not split the results are
 * bit-identical to fa_attn_bwd's; for shapes it splits they are the unsplit
 * kernels' results (deterministic, within the same tolerance of the exact
 * gradients).  All calls on one GPU share its scratch, and every call
 * overwrites all the scratch rows it reads before reading them, so nothing
 * carries over from an earlier call; calls that overlap on one GPU (two
 * streams, or two host threads, at once) race on it.
 * Graph capture: the first call on a device queries the device and looks up
 * its scratch address, which must not happen inside a capture.  Call
 * fa_init(device) (or this function once, eagerly) before capturing; the
 * calls captured afterwards make only kernel launches on `stream`. */
fa_status fa_attn_bwd_noalloc(const fa_attn_bwd_args *args, void *stream);

/* ------------------------------------------------------------------------- */
/* QK prologue: RMSNorm -> axial RoPE -> joint buffer                        */
/* ------------------------------------------------------------------------- */

#define FA_MAX_ROPE_AXES 8

typedef struct fa_qk_prologue_args {
    int32_t dtype;          /* fa_dtype of x, y, weight, cos, sin             */
    int32_t batch;          /* B                                              */
    int32_t tokens;         /* tokens of this stream (txt or img)             */
    int32_t heads;          /* H                                              */
    int32_t head_dim;       /* D: 64 or 128, == sum(axes)                     */
    float eps;              /* RMSNorm epsilon (reference: 1e-6, lib.rs:26)   */
    const void *x;          /* [B,tokens,H,D] view: q or k linear output      */
    fa_strides x_stride;
    const void *weight;     /* [D] learned RMSNorm scale                      */
    const void *cos, *sin;  /* [tokens, D] tables, contiguous                 */
    int32_t n_axes;         /* rotate-half segments, 1..FA_MAX_ROPE_AXES      */
    int32_t axes[FA_MAX_ROPE_AXES]; /* even widths summing to D               */
    void *y;                /* joint [B,S,H,D] buffer                         */
    fa_strides y_stride;
    int32_t y_seq_offset;   /* first joint row this stream writes (txt: 0,
                               img: txt_len)                                  */
} fa_qk_prologue_args;

/* y[:, off:off+tokens] = apply_rope(rms_norm(x, weight, eps), cos, sin), with
 * the reference's cast points (stats f32; normalised value cast to dtype, then
 * * weight in dtype; rotation in f32, cast back).  Fuses lib.rs:45-58,
 * lib.rs:122-129 and the txt||img concatenation lib.rs:363-365.
 * Views of x, y (and dx): token and head strides below 2^24 elements, and a
 * batch item's rows within 2^31 elements of its first; tokens < 2^24 and
 * heads <= 1024 (FA_ERR_UNSUPPORTED otherwise). */
fa_status fa_qk_prologue_fwd(const fa_qk_prologue_args *args, void *stream);

typedef struct fa_qk_prologue_bwd_args {
    fa_qk_prologue_args fwd; /* the forward's arguments (x, weight, tables)    */
    const void *dy;          /* gradient wrt the joint buffer, fwd.y_stride,
                                read at rows fwd.y_seq_offset..+tokens        */
    void *dx;                /* [B,tokens,H,D] output, dx_stride              */
    fa_strides dx_stride;
} fa_qk_prologue_bwd_args;

/* dx of the fused prologue (chain rule through RoPE then RMSNorm, f32).
 * The norm weight is frozen, so no weight gradient is produced. */
fa_status fa_qk_prologue_bwd(const fa_qk_prologue_bwd_args *args, void *stream);

/* Up to FA_MAX_PROLOGUE_SEGS prologues in one launch: args[0..count) are
 * independent calls of fa_qk_prologue_fwd (or _bwd) that share dtype and
 * head_dim -- typically Q and K of the txt and img streams of one block
 * (lib.rs:322-357), each writing its rows of the joint Q or K buffer.  One
 * launch amortises the launch ramp and each workgroup's setup over all of
 * them; results are those of the separate calls, bit for bit.  Segments
 * that write the same buffer (same y, or dx, and strides) must write
 * disjoint rows; arguments are validated as the single calls validate them.
 * No reference counterpart: the reference runs these as separate Candle op
 * chains. */
#define FA_MAX_PROLOGUE_SEGS 4
fa_status fa_qk_prologue_fwd_multi(const fa_qk_prologue_args *args, int32_t count, void *stream);
fa_status fa_qk_prologue_bwd_multi(const fa_qk_prologue_bwd_args *args, int32_t count, void *stream);

/* Host helper: RoPE tables exactly as rope_tables_dtype (lib.rs:77-105):
 * inv_j = theta^(-2j/d_a), f = pos[a]*inv_j in f32, cos/sin duplicated per
 * axis segment, then cast to `dtype` (bf16 tables are written as uint16 bf16
 * bits).  positions: [n_pos, n_axes] host f32; cos_out/sin_out: host buffers
 * of n_pos * sum(axes) elements of `dtype`.  No device work. */
fa_status fa_rope_tables_host(const float *positions, int32_t n_pos, int32_t n_axes,
                              const int32_t *axes, float theta, int32_t dtype, void *cos_out,
                              void *sin_out);

/* ------------------------------------------------------------------------- */
/* LoRA down/up (linear_scaled's adapter term)                               */
/* ------------------------------------------------------------------------- */

typedef struct fa_lora_args {
    int32_t dtype;        /* fa_dtype of x, a, b, y, dy, dx                    */
    int32_t tokens;       /* N rows of x and y                                 */
    int32_t in_features;  /* K                                                 */
    int32_t out_features; /* M                                                 */
    int32_t rank;         /* r: 1..32                                          */
    float scale;          /* alpha / r (reference fixture 2.0, harness 1.0)    */
    const void *x;        /* [N, K] rows of stride ldx                         */
    int64_t ldx;
    const void *a;        /* [r, K] contiguous (LoRA down, `lora_a`)           */
    const void *b;        /* [M, r] contiguous (LoRA up, `lora_b`)             */
    float *u;             /* [N, r] f32: x A^T (written by fwd, read by bwd)   */
    void *y;              /* [N, M] rows of stride ldy (fwd: in/out)           */
    int64_t ldy;
} fa_lora_args;

/* y += scale * (x A^T) B^T, with u = x A^T kept in f32 for the backward.
 * y holds the base linear x W^T (+ bias) on entry.  Replaces the adapter
 * term of linear_scaled (lib.rs:280-285). */
fa_status fa_lora_fwd(const fa_lora_args *args, void *stream);

typedef struct fa_lora_bwd_args {
    fa_lora_args fwd;  /* the forward's arguments (x, a, b, u; y unused)       */
    const void *dy;    /* [N, M] rows of stride ldy                            */
    int64_t ldy;
    float *da;         /* [r, K] f32 output: scale * (dy B)^T x                */
    float *db;         /* [M, r] f32 output: scale * dy^T u                    */
    void *dx;          /* NULL, or [N, K] rows of stride ldx: dx += scale *
                          (dy B) A (the adapter's share of the input grad)     */
    int64_t ldx;
    void *workspace;   /* device scratch, 256-B aligned                        */
    size_t workspace_bytes;
} fa_lora_bwd_args;

size_t fa_lora_bwd_workspace_size(const fa_lora_bwd_args *args);

/* LoRA gradients of linear_scaled's adapter term (Candle autograd through
 * lib.rs:280-285): dB = s dy^T u, dA = s (dy B)^T x, optional dx += s (dy B) A.
 * Deterministic. */
fa_status fa_lora_bwd(const fa_lora_bwd_args *args, void *stream);

/* ---- adapter pieces for a base GEMM that carries the adapter ------------- */
/* The adapter term s (x A^T) B^T can ride in the frozen GEMM: appending s*u
 * (u = x A^T) as r extra K-columns of the GEMM's left operand and B as r
 * extra columns of its weight gives x W^T + s u B^T in one product, and
 * appending A as r extra rows of W makes the product also output u (or, in
 * a backward, dy B).  These three calls are the pieces around such a GEMM,
 * bf16 only, reading and writing the rank columns as row views (u + n*ldu),
 * ldu*2 % 16 == 0 for the 16-byte paths, rank 1..64 (so the adapters of
 * several projections that share x -- q, k, v -- can run as one stacked
 * rank).  They restate the adapter term of linear_scaled (lib.rs:280-285)
 * and its autograd. */

typedef struct fa_lora_down_args {
    int32_t dtype;        /* FA_DTYPE_BF16                                     */
    int32_t tokens;       /* N                                                 */
    int32_t in_features;  /* K (% 16 == 0)                                     */
    int32_t rank;         /* r                                                 */
    float scale;
    const void *x;        /* [N, K] rows of stride ldx, 16-byte aligned        */
    int64_t ldx;
    const void *a;        /* [r, K] contiguous (lora_a), 16-byte aligned       */
    void *u;              /* [N, r] output rows of stride ldu: scale * x A^T   */
    int64_t ldu;
} fa_lora_down_args;

/* u = scale * x A^T, rounded to bf16 (the reference's bf16 matmul result). */
fa_status fa_lora_down(const fa_lora_down_args *args, void *stream);

typedef struct fa_lora_up_args {
    int32_t dtype;        /* FA_DTYPE_BF16                                     */
    int32_t tokens;       /* N                                                 */
    int32_t out_features; /* M (% 16 == 0)                                     */
    int32_t rank;         /* r                                                 */
    float scale;
    const void *u;        /* [N, r] rows of stride ldu                         */
    int64_t ldu;
    const void *b;        /* [M, r] contiguous (lora_b layout)                 */
    void *y;              /* [N, M] rows of stride ldy, updated in place       */
    int64_t ldy;
} fa_lora_up_args;

/* y += scale * u B^T. */
fa_status fa_lora_up(const fa_lora_up_args *args, void *stream);

typedef struct fa_lora_grad_args {
    int32_t dtype;        /* FA_DTYPE_BF16                                     */
    int32_t tokens;       /* N                                                 */
    int32_t features;     /* C (% 16 == 0)                                     */
    int32_t rank;         /* r                                                 */
    float scale;
    const void *u;        /* [N, r] rows of stride ldu                         */
    int64_t ldu;
    const void *x;        /* [N, C] rows of stride ldx, 16-byte aligned        */
    int64_t ldx;
    float *grad;          /* f32 output: scale * u^T x                         */
    int32_t transpose;    /* 0: grad is [r, C] (lora_a layout, dA = du^T x);
                             1: grad is [C, r] (lora_b layout, dB = dy^T u)    */
    void *workspace;      /* device scratch, 256-B aligned                     */
    size_t workspace_bytes;
} fa_lora_grad_args;

size_t fa_lora_grad_workspace_size(const fa_lora_grad_args *args);

/* grad = scale * u^T x (or its transpose), deterministic split-K reduction. */
fa_status fa_lora_grad(const fa_lora_grad_args *args, void *stream);

/* Several fa_lora_grad products, each of its own token count, in one set of
 * launches (up to 16 products per set; count <= 64): each grad gets the bits of its own
 * fa_lora_grad call.  The products' own workspace fields are ignored; the
 * call takes one workspace of fa_lora_grad_many_workspace_size bytes (0 for
 * invalid arguments).  The reference forms each adapter's dA and dB through
 * autograd, one matmul each (linear_scaled, lib.rs:270-287, applied by
 * throughput.rs:254-256 and differentiated by the backward at
 * throughput.rs:799); the double block calls this once per step for the q,
 * k, v and out adapters of both streams. */
size_t fa_lora_grad_many_workspace_size(const fa_lora_grad_args *args, int32_t count);
fa_status fa_lora_grad_many(const fa_lora_grad_args *args, int32_t count, void *workspace,
                            size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FOUNDRY_ATTN_H */
