// Fused QK prologue for gfx950: RMSNorm -> axial rotate-half RoPE -> write
// into the joint [B,S,H,D] attention buffer at the stream's sequence offset.
//
// Forward semantics, with the reference's cast points:
//   rms_norm   crates/foundry-spike/src/lib.rs:45-58
//              n = x_f32 / sqrt(mean(x^2) + eps), cast to dtype, * weight in dtype
//   apply_rope lib.rs:107-129
//              out = n*cos + rot(n)*sin in f32, rot = [x1|x2] -> [-x2|x1] per
//              axis segment; cast back
//   concat     lib.rs:363-365 (txt rows first, then img rows)
// One row (b, token, head) is D elements; D*elt/16 lanes hold it with one
// 16-byte load each, the sum of squares reduces over those lanes, and the
// rotation partner (d +- half) is exchanged through LDS.  HBM-bound: one read
// of x, one write of y, tables and weight from L2.
//
// Backward (chain rule, f32, casts treated as identity):
//   g  = dy*cos + rot^T(dy*sin),  rot^T = [a1|a2] -> [a2|-a1]
//   dn = g * w;  n = x / sigma
//   dx = (dn - n * mean(dn * n)) / sigma
#include <math.h>

#include "fa_device.hpp"
#include "fa_kernels.hpp"

namespace fa {
namespace {

template <typename T>
__device__ __forceinline__ float ld_elt(const T *p, int i) {
    return (float)p[i];
}

template <typename T>
__device__ __forceinline__ T cast_out(float v) {
    return (T)v;
}

template <typename T>
__device__ __forceinline__ float round_dt(float v) {
    return (float)(T)v;  // identity for float, RNE to bf16 for bf16
}

// partner index and sign for the rotate-half of element d:
// first half of a segment takes -x[d+half], second half takes +x[d-half].
__device__ __forceinline__ void rope_partner(const QkPrologueParams &p, int d, int &partner,
                                             float &sign) {
    int off = 0;
    partner = d;
    sign = 0.f;
    for (int a = 0; a < p.n_axes; ++a) {
        const int w = p.axes[a], half = w >> 1;
        if (d >= off && d < off + w) {
            if (d - off < half) {
                partner = d + half;
                sign = -1.f;
            } else {
                partner = d - half;
                sign = 1.f;
            }
        }
        off += w;
    }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void qk_prologue_fwd_kernel(QkPrologueParams p) {
    // one rounding per reference op: no FMA contraction of x*cos + rot*sin
#pragma clang fp contract(off)
    constexpr int EPL = 16 / sizeof(T);   // elements per lane
    constexpr int LPR = D / EPL;          // lanes per row
    constexpr int RPB = 256 / LPR;        // rows per block
    __shared__ float buf[RPB][D];
    const int tid = threadIdx.x, lr = tid / LPR, part = tid % LPR;
    const int64_t rows = (int64_t)p.B * p.T * p.H;
    const int64_t row = (int64_t)blockIdx.x * RPB + lr;
    const bool live = row < rows;
    int b = 0, t = 0, h = 0;
    if (live) {
        h = row % p.H;
        t = (row / p.H) % p.T;
        b = row / ((int64_t)p.H * p.T);
    }
    const T *x = static_cast<const T *>(p.x) + b * p.x_sb + t * p.x_ss + h * p.x_sh;
    float xv[EPL];
    float ss = 0.f;
    if (live) {
        const u32x4 raw = ld_global_16(x + part * EPL);
        const T *e = reinterpret_cast<const T *>(&raw);
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            xv[i] = (float)e[i];
            ss += xv[i] * xv[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < EPL; ++i) xv[i] = 0.f;
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float sc = sqrtf(ss / (float)D + p.eps);
    const T *w = static_cast<const T *>(p.w);
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int d = part * EPL + i;
        const float nv = round_dt<T>(xv[i] / sc);
        buf[lr][d] = round_dt<T>(nv * ld_elt(w, d));
    }
    __syncthreads();
    if (!live) return;
    const T *cs = static_cast<const T *>(p.cos) + (int64_t)t * D;
    const T *sn = static_cast<const T *>(p.sin) + (int64_t)t * D;
    T out[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int d = part * EPL + i;
        int pd;
        float sg;
        rope_partner(p, d, pd, sg);
        const float a = buf[lr][d] * ld_elt(cs, d);
        const float r = sg * buf[lr][pd] * ld_elt(sn, d);
        out[i] = cast_out<T>(a + r);
    }
    T *y = static_cast<T *>(p.y) + b * p.y_sb + (int64_t)(p.y_off + t) * p.y_ss + h * p.y_sh;
    st_global_16(y + part * EPL, *reinterpret_cast<const u32x4 *>(out));
}

template <typename T, int D>
__global__ __launch_bounds__(256) void qk_prologue_bwd_kernel(QkPrologueParams p) {
    constexpr int EPL = 16 / sizeof(T);
    constexpr int LPR = D / EPL;
    constexpr int RPB = 256 / LPR;
    __shared__ float buf[RPB][D];
    const int tid = threadIdx.x, lr = tid / LPR, part = tid % LPR;
    const int64_t rows = (int64_t)p.B * p.T * p.H;
    const int64_t row = (int64_t)blockIdx.x * RPB + lr;
    const bool live = row < rows;
    int b = 0, t = 0, h = 0;
    if (live) {
        h = row % p.H;
        t = (row / p.H) % p.T;
        b = row / ((int64_t)p.H * p.T);
    }
    const T *cs = static_cast<const T *>(p.cos) + (int64_t)t * D;
    const T *sn = static_cast<const T *>(p.sin) + (int64_t)t * D;
    float xv[EPL], dyv[EPL];
    float ss = 0.f;
    if (live) {
        const T *x = static_cast<const T *>(p.x) + b * p.x_sb + t * p.x_ss + h * p.x_sh;
        const T *dy =
            static_cast<const T *>(p.dy) + b * p.y_sb + (int64_t)(p.y_off + t) * p.y_ss + h * p.y_sh;
        const u32x4 rx = ld_global_16(x + part * EPL), rd = ld_global_16(dy + part * EPL);
        const T *ex = reinterpret_cast<const T *>(&rx);
        const T *ed = reinterpret_cast<const T *>(&rd);
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            xv[i] = (float)ex[i];
            dyv[i] = (float)ed[i];
            ss += xv[i] * xv[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < EPL; ++i) xv[i] = dyv[i] = 0.f;
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float sigma = sqrtf(ss / (float)D + p.eps);
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int d = part * EPL + i;
        buf[lr][d] = live ? dyv[i] * ld_elt(sn, d) : 0.f;
    }
    __syncthreads();
    const T *w = static_cast<const T *>(p.w);
    float dn[EPL], nv[EPL];
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int d = part * EPL + i;
        int pd;
        float sg;
        rope_partner(p, d, pd, sg);
        // rot^T takes the partner with the opposite sign of rot
        const float gv = live ? dyv[i] * ld_elt(cs, d) - sg * buf[lr][pd] : 0.f;
        dn[i] = gv * ld_elt(w, d);
        nv[i] = xv[i] / sigma;
        dot += dn[i] * nv[i];
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
    if (!live) return;
    const float mdot = dot / (float)D;
    T out[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) out[i] = cast_out<T>((dn[i] - nv[i] * mdot) / sigma);
    T *dx = static_cast<T *>(p.dx) + b * p.dx_sb + t * p.dx_ss + h * p.dx_sh;
    st_global_16(dx + part * EPL, *reinterpret_cast<const u32x4 *>(out));
}

template <typename T, int D, bool BWD>
hipError_t launch_prologue(const QkPrologueParams &p, hipStream_t s) {
    constexpr int LPR = D * sizeof(T) / 16;
    constexpr int RPB = 256 / LPR;
    const int64_t rows = (int64_t)p.B * p.T * p.H;
    const dim3 grid((unsigned)((rows + RPB - 1) / RPB)), block(256);
    if (BWD)
        hipLaunchKernelGGL((qk_prologue_bwd_kernel<T, D>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((qk_prologue_fwd_kernel<T, D>), grid, block, 0, s, p);
    return hipGetLastError();
}

template <bool BWD>
hipError_t dispatch(const QkPrologueParams &p, int dtype, hipStream_t s) {
    if (dtype == 0)
        return p.D == 128 ? launch_prologue<bf16, 128, BWD>(p, s) : launch_prologue<bf16, 64, BWD>(p, s);
    return p.D == 128 ? launch_prologue<float, 128, BWD>(p, s) : launch_prologue<float, 64, BWD>(p, s);
}

}  // namespace

hipError_t launch_qk_prologue_fwd(const QkPrologueParams &p, int dtype, hipStream_t s) {
    return dispatch<false>(p, dtype, s);
}

hipError_t launch_qk_prologue_bwd(const QkPrologueParams &p, int dtype, hipStream_t s) {
    return dispatch<true>(p, dtype, s);
}

}  // namespace fa
