// Kernel parameter blocks and host-side launchers (defined next to each
// kernel).  The C ABI layer (fa_abi.cpp) validates arguments, fills these
// blocks and calls the launchers; nothing here is exported.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

struct AttnFwdParams {
    const void *q, *k, *v;
    void *o;
    float *lse;
    const uint8_t *keep;  // [B,S] or nullptr
    int64_t q_sb, q_ss, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_ss, o_sh;
    int B, S, H;
    float scale;       // softmax scale
    float scale_log2;  // scale * log2(e)
    // Key-range split (split > 1, bf16 only): `split` workgroups per query
    // tile each cover a range of keys and leave O / l (f32, [split][B*H*S][D])
    // and the range's LSE ([split][B*H*S]) here; a combine pass writes o, lse.
    int split;
    float *part_o, *part_lse;
};

struct AttnBwdParams {
    const void *q, *k, *v, *o, *dout;
    const float *lse;
    const uint8_t *keep;
    void *dq, *dk, *dv;
    float *delta;  // workspace: [B,H,S] rowsum(dO * O)
    float *lse2;   // workspace: [B,H,S] LSE * log2(e), +inf for fully masked rows
    int64_t q_sb, q_ss, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_ss, o_sh;
    int64_t do_sb, do_ss, do_sh;
    int64_t dq_sb, dq_ss, dq_sh;
    int64_t dk_sb, dk_ss, dk_sh;
    int64_t dv_sb, dv_ss, dv_sh;
    int B, S, H;
    float scale, scale_log2;
    // Split (split > 1, bf16 only): dQ workgroups cover a range of keys, dK/dV
    // workgroups a range of queries; each leaves unscaled f32 partial sums
    // ([split][B*H*S][D] per gradient) here and a reduce pass writes dq, dk, dv.
    int split;
    float *part_dq, *part_dk, *part_dv;
    // dS through the workspace (ds != nullptr, unsplit bf16 only): dK/dV also
    // stores the unscaled bf16 dS^T = (P * (dP - delta))^T of every (key,
    // query) as [B*H][S keys][ds_ld queries], and dQ = scale * dS K is a
    // streaming product over it instead of recomputing S and dP.
    void *ds;
    int ds_ld;  // queries per dS^T row: S rounded up to a multiple of 256
};

// Returns hipSuccess or the launch error.  `D` is 64 or 128.
hipError_t launch_attn_fwd_bf16(const AttnFwdParams &p, int D, hipStream_t s);
hipError_t launch_attn_fwd_f32(const AttnFwdParams &p, int D, hipStream_t s);
// phase: 0 all, 1 pre-pass, 2 dK/dV, 3 dQ
hipError_t launch_attn_bwd_bf16(const AttnBwdParams &p, int D, int phase, hipStream_t s);
// Waves per workgroup (4 or 8, i.e. 128- or 256-row tiles) of the bf16
// forward, dK/dV and D = 128 dQ kernels for B x H sequences of S tokens on
// the current device (see attn_fwd.hip).
int attn_waves(int B, int H, int S);
// Range split factor (1 = none) of the bf16 kernels for B x H sequences of S
// tokens on the current device: > 1 when even 8-wave workgroups would leave
// most CUs idle (e.g. one GPU's share of heads under sequence parallelism).
int attn_split(int B, int H, int S);
// f32 elements of the split partials per gradient or O (split * B*H*S*D).
size_t attn_split_elems(int B, int H, int S, int D, int split);
hipError_t launch_attn_bwd_f32(const AttnBwdParams &p, int D, int phase, hipStream_t s);

// CU count of the current device (cached per device; 256 if unknown).
int device_cu_count();

// One-time per-process kernel attribute setup (dynamic LDS limits).
hipError_t prepare_attn_kernels();

struct QkPrologueParams {
    const void *x;
    int64_t x_sb, x_ss, x_sh;
    const void *w, *cos, *sin;
    void *y;
    int64_t y_sb, y_ss, y_sh;
    int y_off;
    const void *dy;  // bwd only (y strides)
    void *dx;        // bwd only
    int64_t dx_sb, dx_ss, dx_sh;
    int B, T, H, D;
    float eps;
    int n_axes;
    int axes[8];
    float inv_h;  // 1 / H, set by the launcher
};

// n segments (1..kMaxPrologueSegs) of one dtype and head_dim in one launch.
constexpr int kMaxPrologueSegs = 4;
hipError_t launch_qk_prologue_fwd(const QkPrologueParams *ps, int n, int dtype, hipStream_t s);
hipError_t launch_qk_prologue_bwd(const QkPrologueParams *ps, int n, int dtype, hipStream_t s);

struct LoraParams {
    const void *x;
    int64_t ldx;
    const void *a, *b;
    float *u;
    void *y;
    int64_t ldy;
    const void *dy;
    int64_t lddy;
    float *da, *db;
    void *dx;
    int64_t lddx;
    float *work;  // bwd: [N, r] f32 (dy B)
    int N, K, M, r;
    float scale;
};

hipError_t launch_lora_fwd(const LoraParams &p, int dtype, hipStream_t s);
hipError_t launch_lora_bwd(const LoraParams &p, int dtype, hipStream_t s);
hipError_t launch_lora_down_bf16(const void *x, int64_t ldx, const void *a, int N, int K, int R, float scale,
                                 void *u, int64_t ldu, hipStream_t st);
hipError_t launch_lora_up_bf16(const void *u, int64_t ldu, const void *b, int N, int M, int R, float scale, void *y,
                               int64_t ldy, hipStream_t st);
// grad = scale * u^T x ([R, C]) or its transpose ([C, R]); u bf16 [N, R <= 64]
struct LoraGradItem {
    const void *u;
    int64_t ldu;
    const void *x;
    int64_t ldx;
    int N, C, R;
    float scale;
    float *grad;
    bool transpose;
};
size_t lora_grad_many_workspace_bytes(const LoraGradItem *items, int count);
hipError_t launch_lora_grad_many_bf16(const LoraGradItem *items, int count, void *work, hipStream_t st);

// LayerNorm-modulation over [N, C] rows (C % 8 == 0, C <= 4096).
struct LnModParams {
    const void *x;
    int64_t ldx;
    const void *shift, *scale;  // [C]
    void *y;
    int64_t ldy;
    float *mean, *rstd;  // [N]: written by fwd (optional), read by bwd
    const void *dy;      // bwd
    int64_t lddy;
    const void *dres;  // bwd: residual gradient added to dx (optional)
    int64_t ldres;
    void *dx;
    int64_t lddx;
    int N, C;
    float eps;
    const void *g;  // [C] gate: fwd with b, the gated residual x + g * b in
                    // front of the norm; bwd with gdx, g * dx after it
    const void *b;  // fwd: [N, C] gated branch, or null (plain layer norm)
    int64_t ldb;
    void *sum;      // fwd with b: [N, C] output x + g * b (the norm's input)
    int64_t ldsum;
    void *sum2;     // fwd with b: optional second copy of the sum
    int64_t ldsum2;
    void *gdx;      // bwd: [N, C] output g * dx, or null
    int64_t ldgdx;
};
hipError_t launch_ln_mod_fwd(const LnModParams &p, int dtype, hipStream_t s);
hipError_t launch_ln_mod_bwd(const LnModParams &p, int dtype, hipStream_t s);

// Elementwise ops over an [N, C] view (C % 8 == 0): 0 gated residual
// y = x + g*b, 1 y = gelu(b), 2 y = x * gelu'(b), 3 y = silu(b).
struct EltParams {
    const void *x;
    int64_t ldx;
    const void *g;  // [C]
    const void *b;
    int64_t ldb;
    void *y;
    int64_t ldy;
    int N, C;
};
hipError_t launch_elementwise(const EltParams &p, int op, int dtype, hipStream_t s);

struct SwigluParams {
    const void *gate;
    int64_t ldg;
    const void *up;
    int64_t ldu;
    const void *dy;  // backward only
    int64_t lddy;
    void *y;         // forward output, or dgate in the backward
    int64_t ldy;
    void *dup;       // backward only
    int64_t lddup;
    int N, C;
};
hipError_t launch_swiglu(const SwigluParams &p, bool bwd, int dtype, hipStream_t s);

struct AdamwParams {
    void *param;        // dtype of the op
    const float *grad;  // f32
    float *m, *v;       // f32 moments
    int64_t n;
    float lr, b1, b2, one_m_b1, one_m_b2, eps, ibc1, ibc2;
};
hipError_t launch_adamw(const AdamwParams &p, int dtype, hipStream_t s);

// Up to kCopyMany strided 2D views copied in one launch (strides in
// elements); block0 is filled by the launcher.
constexpr int kCopyMany = 32;
struct Copy2dMany {
    const void *src[kCopyMany];
    void *dst[kCopyMany];
    int64_t src_rs[kCopyMany], src_cs[kCopyMany], dst_rs[kCopyMany], dst_cs[kCopyMany];
    int rows[kCopyMany], cols[kCopyMany];
    int block0[kCopyMany + 1];
    int count;
};
hipError_t launch_copy2d_many(Copy2dMany p, int elt_bytes, hipStream_t s);

// Up to kAdamwMany tensors of one step (shared hyperparameters); block0 is
// filled by the launcher.
constexpr int kAdamwMany = 32;
struct AdamwMany {
    void *param[kAdamwMany];
    const float *grad[kAdamwMany];
    float *m[kAdamwMany], *v[kAdamwMany];
    int64_t n[kAdamwMany];
    int block0[kAdamwMany + 1];
    int count;
    float lr, b1, b2, one_m_b1, one_m_b2, eps, ibc1, ibc2;
};
hipError_t launch_adamw_many(AdamwMany p, int dtype, hipStream_t s);

}  // namespace fa

namespace fa {
// C[M, N] = A[M, K] B[N, K]^T, bf16, with a fused epilogue (gemm.hip).
// M and N multiples of 256, K a multiple of 64; rows 16-byte aligned.
constexpr int kGemmNone = 0, kGemmGelu = 1, kGemmDgelu = 2;
struct GemmParams {
    const void *a, *b;  // A [M, K] (lda), B [N, K] (ldb)
    void *c;            // C [M, N] (ldc): T(acc), pre (GELU) or the GELU gradient (DGELU)
    void *c2;           // GELU: gelu(pre) [M, N] (ldc2)
    const void *aux;    // DGELU: the saved pre-activation [M, N] (ldaux)
    int64_t lda, ldb, ldc, ldc2, ldaux;
    int M, N, K, epi;
    int group_m;  // set by the launcher: M tiles per band of the tile order
};
hipError_t launch_gemm_tn_bf16(const GemmParams &p, hipStream_t s);
}  // namespace fa
