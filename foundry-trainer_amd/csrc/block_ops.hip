// Memory-bound kernels of foundry-spike's double-stream LoRA block (the
// pieces around the attention and the frozen linears):
//   LayerNorm-modulation   y = (1 + scale) * LN(x) + shift    (lib.rs:60-71)
//   its backward           dx = dres + rstd*(dn - mean(dn) - n*mean(dn*n)),
//                          dn = dy * (1 + scale)
//   gated residual         y = x + g * b, g broadcast over rows
//                          (throughput.rs:552-572)
//   tanh-GELU and its derivative (the c4 block's MLP activation; the
//                          reference block uses SwiGLU, lib.rs:293-297)
//   SiLU                   of the conditioning vector (throughput.rs:297-324)
//   AdamW step             lib.rs:477-510, operation for operation
// All are HBM-bound: rows move with 16-byte vector accesses, statistics are
// f32, results are rounded once to the storage type.
#include <math.h>

#include "fa_device.hpp"
#include "fa_kernels.hpp"

namespace fa {
namespace {

// 8 consecutive elements <-> f32 (bf16: one 16-byte access, f32: two)
__device__ __forceinline__ void load8(const bf16 *p, float v[8]) {
    const bf16x8 a = as_bf16x8(ld_global_16(p));
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (float)a[j];
}
__device__ __forceinline__ void load8(const float *p, float v[8]) {
    const f32x4 a = __builtin_bit_cast(f32x4, ld_global_16(p));
    const f32x4 b = __builtin_bit_cast(f32x4, ld_global_16(p + 4));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = a[j];
        v[4 + j] = b[j];
    }
}
__device__ __forceinline__ void store8(bf16 *p, const float v[8]) {
    bf16x8 a;
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = f32_to_bf16(v[j]);
    *reinterpret_cast<bf16x8 *>(p) = a;
}
__device__ __forceinline__ void store8(float *p, const float v[8]) {
    *reinterpret_cast<f32x4 *>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4 *>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

// x rounded to the storage type T, back in f32
template <typename T>
__device__ __forceinline__ float round_to(float x) {
    return (float)(T)x;
}

// Sum over the wave, the same value in every lane: within each 16-lane row by
// DPP (partners lane^1, lane^2, then the mirrors within 8 and within 16 lanes;
// each step adds a disjoint group's partial, so every lane of a row ends with
// the same sum), then rows by lane^16 and lane^32 exchanges.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float s) {
    s += dpp_f32<0xB1>(s);   // quad_perm [1,0,3,2]
    s += dpp_f32<0x4E>(s);   // quad_perm [2,3,0,1]
    s += dpp_f32<0x141>(s);  // row_half_mirror
    s += dpp_f32<0x140>(s);  // row_mirror
    s += __shfl_xor(s, 16, 64);
    return sum_xor32(s);
}

// One wave per row; lane l holds elements k*512 + 8*l .. +8 for k < MAXCH.
// GATED: the row is first the gated residual x + g * b, rounded to T as the
// gated-residual op rounds it (the same fma), stored to sum (and sum2), and
// the statistics are those of the rounded sum: the bits of the gated
// residual followed by this kernel on its output.
template <typename T, int MAXCH, bool GATED>
__global__ __launch_bounds__(256) void ln_mod_fwd_kernel(LnModParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.N) return;
    const int C = p.C;
    const T *x = static_cast<const T *>(p.x) + row * p.ldx;
    float v[MAXCH][8];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < MAXCH; ++k) {
        const int e = k * 512 + lane * 8;
        if (e < C) {
            load8(x + e, v[k]);
            if constexpr (GATED) {
                float gv[8], bv[8];
                load8(static_cast<const T *>(p.g) + e, gv);
                load8(static_cast<const T *>(p.b) + row * p.ldb + e, bv);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[k][j] = round_to<T>(__builtin_fmaf(gv[j], bv[j], v[k][j]));
                store8(static_cast<T *>(p.sum) + row * p.ldsum + e, v[k]);
                if (p.sum2) store8(static_cast<T *>(p.sum2) + row * p.ldsum2 + e, v[k]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) s += v[k][j];
        }
    }
    const float mean = wave_sum(s) / (float)C;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < MAXCH; ++k) {
        const int e = k * 512 + lane * 8;
        if (e < C) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float d = v[k][j] - mean;
                q += d * d;
            }
        }
    }
    const float var = wave_sum(q) / (float)C;
    const float den = sqrtf(var + p.eps);
    const float inv = 1.f / den;
    const T *shift = static_cast<const T *>(p.shift), *scale = static_cast<const T *>(p.scale);
    T *y = static_cast<T *>(p.y) + row * p.ldy;
#pragma unroll
    for (int k = 0; k < MAXCH; ++k) {
        const int e = k * 512 + lane * 8;
        if (e < C) {
            float sh[8], sc[8], o[8];
            load8(shift + e, sh);
            load8(scale + e, sc);
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = (v[k][j] - mean) * inv * (sc[j] + 1.f) + sh[j];
            store8(y + e, o);
        }
    }
    if (lane == 0 && p.mean) {
        p.mean[row] = mean;
        p.rstd[row] = 1.f / den;
    }
}

// GATE_OUT: also gdx = g * dx, from dx as rounded to T (the same fma as the
// gated-residual op with no x), the gradient through a gated branch whose
// output fed this layer norm's input.
template <typename T, int MAXCH, bool GATE_OUT>
__global__ __launch_bounds__(256) void ln_mod_bwd_kernel(LnModParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.N) return;
    const int C = p.C;
    const T *x = static_cast<const T *>(p.x) + row * p.ldx;
    const T *dy = static_cast<const T *>(p.dy) + row * p.lddy;
    const T *scale = static_cast<const T *>(p.scale);
    const float mean = p.mean[row], rstd = p.rstd[row];
    float n[MAXCH][8], dn[MAXCH][8];
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int k = 0; k < MAXCH; ++k) {
        const int e = k * 512 + lane * 8;
        if (e < C) {
            float xv[8], gv[8], sc[8];
            load8(x + e, xv);
            load8(dy + e, gv);
            load8(scale + e, sc);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                n[k][j] = (xv[j] - mean) * rstd;
                dn[k][j] = gv[j] * (sc[j] + 1.f);
                a += dn[k][j];
                b += dn[k][j] * n[k][j];
            }
        }
    }
    const float ma = wave_sum(a) / (float)C, mb = wave_sum(b) / (float)C;
    const T *dres = static_cast<const T *>(p.dres);
    T *dx = static_cast<T *>(p.dx) + row * p.lddx;
#pragma unroll
    for (int k = 0; k < MAXCH; ++k) {
        const int e = k * 512 + lane * 8;
        if (e < C) {
            float o[8], r[8];
            if (dres) {
                load8(dres + row * p.ldres + e, r);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) r[j] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = r[j] + rstd * (dn[k][j] - ma - n[k][j] * mb);
            store8(dx + e, o);
            if constexpr (GATE_OUT) {
                float gv[8], go[8];
                load8(static_cast<const T *>(p.g) + e, gv);
#pragma unroll
                for (int j = 0; j < 8; ++j) go[j] = __builtin_fmaf(gv[j], round_to<T>(o[j]), 0.f);
                store8(static_cast<T *>(p.gdx) + row * p.ldgdx + e, go);
            }
        }
    }
}

// Elementwise over an [N, C] view, 8 elements per thread (C % 8 == 0).
// op 0: y = x + g * b (x may be null: y = g * b);  1: y = gelu(b);
// op 2: y = x * gelu'(b) (x = upstream gradient);  3: y = silu(b)
// gelu(u) = u/2 * (1 + tanh(z)), z = k0 * (u + k1 u^3), evaluated as
// u * sigmoid(2z) (the same function: (1 + tanh z) / 2 = sigmoid(2z)) with one
// exp2 and one reciprocal; gelu'(u) = sg + 2 u sg (1 - sg) k0 (1 + 3 k1 u^2),
// sg = sigmoid(2z).
constexpr float kGeluK0 = 0.7978845608028654f;  // sqrt(2/pi)
constexpr float kGeluK1 = 0.044715f;

// sigmoid(2 k0 (u + k1 u^3)) of the tanh-GELU
__device__ __forceinline__ float gelu_sigmoid(float u) {
    const float z2 = (2.f * kGeluK0) * (u + kGeluK1 * u * u * u);
    return __builtin_amdgcn_rcpf(1.f + exp2_fast(-kLog2e * z2));
}

// Grid: x over 128-lane groups of a row's 8-element chunks, y over rows
// (striding by gridDim.y), so no lane divides to find its row.
constexpr int kEltLanes = 128;
template <typename T, int OP>
__global__ __launch_bounds__(kEltLanes) void elementwise_kernel(EltParams p) {
    const int e = (blockIdx.x * kEltLanes + threadIdx.x) * 8;
    if (e >= p.C) return;
    const T *g = static_cast<const T *>(p.g);
    for (int64_t row = blockIdx.y; row < p.N; row += gridDim.y) {
        float bv[8], o[8];
        load8(static_cast<const T *>(p.b) + row * p.ldb + e, bv);
        if constexpr (OP == 0) {
            float gv[8], xv[8];
            load8(g + e, gv);
            if (p.x) {
                load8(static_cast<const T *>(p.x) + row * p.ldx + e, xv);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) xv[j] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = __builtin_fmaf(gv[j], bv[j], xv[j]);
        } else if constexpr (OP == 1) {
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = bv[j] * gelu_sigmoid(bv[j]);
        } else if constexpr (OP == 2) {
            float xv[8];
            load8(static_cast<const T *>(p.x) + row * p.ldx + e, xv);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float u = bv[j];
                const float sg = gelu_sigmoid(u);
                const float d = sg + (2.f * kGeluK0) * u * (sg - sg * sg) * (1.f + (3.f * kGeluK1) * u * u);
                o[j] = xv[j] * d;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = bv[j] / (1.f + exp2_fast(-kLog2e * bv[j]));
        }
        store8(static_cast<T *>(p.y) + row * p.ldy + e, o);
    }
}

// SwiGLU over [N, C] views, 8 elements per thread.  Forward: y = T(T(silu(g))
// * u).  Backward: du = T(dy * T(silu(g))), dg = T(T(dy * u) * silu'(g)) with
// silu'(g) = s (1 + g (1 - s)), s = 1 / (1 + e^-g); T() = round to storage.
template <typename T, bool BWD>
__global__ __launch_bounds__(256) void swiglu_kernel(SwigluParams p) {
    const int64_t per_row = p.C / 8;
    const int64_t total = (int64_t)p.N * per_row;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t row = i / per_row;
        const int e = (int)(i - row * per_row) * 8;
        float gv[8], uv[8], o[8];
        load8(static_cast<const T *>(p.gate) + row * p.ldg + e, gv);
        load8(static_cast<const T *>(p.up) + row * p.ldu + e, uv);
        if constexpr (!BWD) {
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = round_to<T>(gv[j] / (1.f + exp2_fast(-kLog2e * gv[j]))) * uv[j];
        } else {
            float dv[8], du[8];
            load8(static_cast<const T *>(p.dy) + row * p.lddy + e, dv);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float g = gv[j];
                const float sg = 1.f / (1.f + exp2_fast(-kLog2e * g));
                const float silu = round_to<T>(g / (1.f + exp2_fast(-kLog2e * g)));
                du[j] = dv[j] * silu;
                o[j] = round_to<T>(dv[j] * uv[j]) * (sg * (1.f + g * (1.f - sg)));
            }
            store8(static_cast<T *>(p.dup) + row * p.lddup + e, du);
        }
        store8(static_cast<T *>(p.y) + row * p.ldy + e, o);
    }
}

// AdamW, weight decay 0, in the reference's operation order:
//   m' = m*b1 + g*(1-b1);  v' = v*b2 + (g*g)*(1-b2)
//   p' = p - ((m' * ibc1) / (sqrt(v' * ibc2) + eps)) * lr
// each product / sum rounded separately (contraction off for the
// expressions written here), IEEE sqrt and division, p' rounded to T.
template <typename T, typename H>
__device__ __forceinline__ void adamw_elem(T *w, const float *grad, float *mm, float *vv, int64_t i, const H &h) {
#pragma clang fp contract(off)
    const float g = grad[i];
    const float m = mm[i] * h.b1 + g * h.one_m_b1;
    const float gg = g * g;
    const float v = vv[i] * h.b2 + gg * h.one_m_b2;
    const float mhat = m * h.ibc1;
    const float den = sqrtf(v * h.ibc2) + h.eps;
    const float delta = (mhat / den) * h.lr;
    w[i] = (T)((float)w[i] - delta);
    mm[i] = m;
    vv[i] = v;
}

template <typename T>
__global__ __launch_bounds__(256) void adamw_kernel(AdamwParams p) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < p.n; i += (int64_t)gridDim.x * 256)
        adamw_elem(static_cast<T *>(p.param), p.grad, p.m, p.v, i, p);
}

// Several tensors of one AdamW step in one launch: tensor k owns blocks
// [block0[k], block0[k + 1]) and strides over its elements with them.  Same
// per-element arithmetic as adamw_kernel, so the same bits.
template <typename T>
__global__ __launch_bounds__(256) void adamw_many_kernel(AdamwMany p) {
    const int b = blockIdx.x;
    int k = 0;
    while (k + 1 < p.count && p.block0[k + 1] <= b) ++k;
    const int nb = p.block0[k + 1] - p.block0[k];
    T *w = static_cast<T *>(p.param[k]);
    for (int64_t i = (int64_t)(b - p.block0[k]) * 256 + threadIdx.x; i < p.n[k]; i += (int64_t)nb * 256)
        adamw_elem(w, p.grad[k], p.m[k], p.v[k], i, p);
}

// Strided 2D copies of several small arrays in one launch: view k owns
// blocks [block0[k], block0[k + 1]) and strides over its rows * cols elements.
template <typename E>
__global__ __launch_bounds__(256) void copy2d_many_kernel(Copy2dMany p) {
    const int b = blockIdx.x;
    int k = 0;
    while (k + 1 < p.count && p.block0[k + 1] <= b) ++k;
    const int nb = p.block0[k + 1] - p.block0[k];
    const int cols = p.cols[k];
    const int64_t n = (int64_t)p.rows[k] * cols;
    const E *src = static_cast<const E *>(p.src[k]);
    E *dst = static_cast<E *>(p.dst[k]);
    for (int64_t i = (int64_t)(b - p.block0[k]) * 256 + threadIdx.x; i < n; i += (int64_t)nb * 256) {
        const int64_t r = i / cols, c = i - r * cols;
        dst[r * p.dst_rs[k] + c * p.dst_cs[k]] = src[r * p.src_rs[k] + c * p.src_cs[k]];
    }
}

inline int elt_grid(int64_t n8) {
    const int64_t blocks = (n8 + 255) / 256;
    return (int)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

}  // namespace

// MAXCH (512-element chunks per row): 2 up to C = 1024, 6 up to 3072 (the
// blocks' width: fewer registers, so a whole 4608-row grid is resident in one
// round), 8 up to 4096.
template <typename T, bool F>
static hipError_t ln_fwd_t(const LnModParams &p, hipStream_t s) {
    const dim3 grid((unsigned)((p.N + 3) / 4)), block(256);
    if (p.C <= 1024)
        hipLaunchKernelGGL((ln_mod_fwd_kernel<T, 2, F>), grid, block, 0, s, p);
    else if (p.C <= 3072)
        hipLaunchKernelGGL((ln_mod_fwd_kernel<T, 6, F>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((ln_mod_fwd_kernel<T, 8, F>), grid, block, 0, s, p);
    return hipGetLastError();
}
template <typename T, bool F>
static hipError_t ln_bwd_t(const LnModParams &p, hipStream_t s) {
    const dim3 grid((unsigned)((p.N + 3) / 4)), block(256);
    if (p.C <= 1024)
        hipLaunchKernelGGL((ln_mod_bwd_kernel<T, 2, F>), grid, block, 0, s, p);
    else if (p.C <= 3072)
        hipLaunchKernelGGL((ln_mod_bwd_kernel<T, 6, F>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((ln_mod_bwd_kernel<T, 8, F>), grid, block, 0, s, p);
    return hipGetLastError();
}
template <typename T>
static hipError_t ln_fwd_t(const LnModParams &p, hipStream_t s) {
    return p.b ? ln_fwd_t<T, true>(p, s) : ln_fwd_t<T, false>(p, s);
}
template <typename T>
static hipError_t ln_bwd_t(const LnModParams &p, hipStream_t s) {
    return p.gdx ? ln_bwd_t<T, true>(p, s) : ln_bwd_t<T, false>(p, s);
}

hipError_t launch_ln_mod_fwd(const LnModParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? ln_fwd_t<bf16>(p, s) : ln_fwd_t<float>(p, s);
}
hipError_t launch_ln_mod_bwd(const LnModParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? ln_bwd_t<bf16>(p, s) : ln_bwd_t<float>(p, s);
}

template <typename T>
static hipError_t elt_t(const EltParams &p, int op, hipStream_t s) {
    const unsigned gx = (unsigned)((p.C / 8 + kEltLanes - 1) / kEltLanes);
    // about 64K workgroups in all; at most 65535 row groups
    int64_t gy = ((int64_t)1 << 16) / gx;
    if (gy > p.N) gy = p.N;
    if (gy > 65535) gy = 65535;
    if (gy < 1) gy = 1;
    const dim3 grid(gx, (unsigned)gy), block(kEltLanes);
    switch (op) {
        case 0: hipLaunchKernelGGL((elementwise_kernel<T, 0>), grid, block, 0, s, p); break;
        case 1: hipLaunchKernelGGL((elementwise_kernel<T, 1>), grid, block, 0, s, p); break;
        case 2: hipLaunchKernelGGL((elementwise_kernel<T, 2>), grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL((elementwise_kernel<T, 3>), grid, block, 0, s, p); break;
    }
    return hipGetLastError();
}
hipError_t launch_elementwise(const EltParams &p, int op, int dtype, hipStream_t s) {
    return dtype == 0 ? elt_t<bf16>(p, op, s) : elt_t<float>(p, op, s);
}

template <typename T>
static hipError_t swiglu_t(const SwigluParams &p, bool bwd, hipStream_t s) {
    const dim3 grid(elt_grid((int64_t)p.N * (p.C / 8))), block(256);
    if (bwd)
        hipLaunchKernelGGL((swiglu_kernel<T, true>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((swiglu_kernel<T, false>), grid, block, 0, s, p);
    return hipGetLastError();
}
hipError_t launch_swiglu(const SwigluParams &p, bool bwd, int dtype, hipStream_t s) {
    return dtype == 0 ? swiglu_t<bf16>(p, bwd, s) : swiglu_t<float>(p, bwd, s);
}

hipError_t launch_adamw_many(AdamwMany p, int dtype, hipStream_t s) {
    int blocks = 0;
    for (int k = 0; k < p.count; ++k) {
        p.block0[k] = blocks;
        const int64_t nb = (p.n[k] + 255) / 256;
        blocks += (int)(nb < 1024 ? nb : 1024);
    }
    p.block0[p.count] = blocks;
    const dim3 grid(blocks), block(256);
    if (dtype == 0)
        hipLaunchKernelGGL((adamw_many_kernel<bf16>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((adamw_many_kernel<float>), grid, block, 0, s, p);
    return hipGetLastError();
}

hipError_t launch_copy2d_many(Copy2dMany p, int elt_bytes, hipStream_t s) {
    int blocks = 0;
    for (int k = 0; k < p.count; ++k) {
        p.block0[k] = blocks;
        const int64_t nb = ((int64_t)p.rows[k] * p.cols[k] + 255) / 256;
        blocks += (int)(nb < 256 ? nb : 256);
    }
    p.block0[p.count] = blocks;
    if (elt_bytes == 2)
        hipLaunchKernelGGL(copy2d_many_kernel<uint16_t>, dim3(blocks), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(copy2d_many_kernel<uint32_t>, dim3(blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_adamw(const AdamwParams &p, int dtype, hipStream_t s) {
    const dim3 grid(elt_grid(p.n)), block(256);
    if (dtype == 0)
        hipLaunchKernelGGL((adamw_kernel<bf16>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((adamw_kernel<float>), grid, block, 0, s, p);
    return hipGetLastError();
}

}  // namespace fa
