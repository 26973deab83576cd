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

#include <type_traits>

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

// The forward's x rows (read once) and y rows (written once) go through
// non-temporal loads and stores, which leave the L2 to the reused cos / sin
// rows and weights: c2 Q + K 2-3% faster.  The backward's loads measured
// slower that way and stay plain.
template <typename T>
__device__ __forceinline__ void load_row_once(const T *ptr, float (&v)[16 / sizeof(T)]) {
    constexpr int EPL = 16 / sizeof(T);
    const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(ptr));
    const T *e = reinterpret_cast<const T *>(&raw);
#pragma unroll
    for (int i = 0; i < EPL; ++i) v[i] = (float)e[i];
}
__device__ __forceinline__ void store_row_once(void *ptr, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(ptr));
}

// Round two f32 values to bf16 (RNE) and back with one v_cvt_pk_bf16_f32.
__device__ __forceinline__ void round2_bf16(float &a, float &b) {
    const uint32_t w = pack_bf16x2(a, b);
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
}

// bf16 rows take the fast row statistics: the sum of squares by FMA and one
// v_rsq_f32 (within 1 ulp) for 1/sigma, then x * (1/sigma) for the division.
// Their results are cast to bf16 right after (lib.rs:53-56), which an ulp of
// f32 error changes only for values within that ulp of a bf16 rounding
// boundary.  f32 rows keep the correctly rounded sqrt and division.
template <typename T>
constexpr bool kFastStats = sizeof(T) == 2;

// x / d for every x of a row with one reciprocal per row: q0 = x * r (r =
// v_rcp_f32(d), within 1 ulp), the exact remainder e = x - q0 * d by FMA, and
// q = q0 + e * r: the correctly rounded quotient except for rare operands
// within a fraction of an ulp of a rounding midpoint (Markstein's correction
// step).  Replaces the IEEE division sequence, about 10 instructions each.
__device__ __forceinline__ float div_by(float x, float d, float r) {
    const float q0 = x * r;
    const float e = __builtin_fmaf(-q0, d, x);
    return __builtin_fmaf(e, r, q0);
}

// 16 / sizeof(T) consecutive elements as f32: one 16-byte load when VEC (the
// pointer is 16-byte aligned), else element loads.
template <typename T, bool VEC>
__device__ __forceinline__ void load_row_part(const T *ptr, float (&v)[16 / sizeof(T)]) {
    constexpr int EPL = 16 / sizeof(T);
    if constexpr (VEC) {
        const u32x4 raw = ld_global_16(ptr);
        const T *e = reinterpret_cast<const T *>(&raw);
#pragma unroll
        for (int i = 0; i < EPL; ++i) v[i] = (float)e[i];
    } else {
#pragma unroll
        for (int i = 0; i < EPL; ++i) v[i] = (float)ptr[i];
    }
}

// Sum over the LPR consecutive lanes holding one row; every lane gets the
// sum.  LPR <= 16 stays in registers through DPP (quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror, row_mirror: each step adds a disjoint partner
// group, so after log2(LPR) steps every lane holds the full sum); wider rows
// (the f32 D = 128 layout) use cross-lane shuffles.
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
    if constexpr (LPR <= 16) {
        auto dpp = [](float x, auto ctrl) {
            return __builtin_bit_cast(
                float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value, 0xF, 0xF, false));
        };
        v += dpp(v, std::integral_constant<int, 0xB1>{});
        if constexpr (LPR >= 4) v += dpp(v, std::integral_constant<int, 0x4E>{});
        if constexpr (LPR >= 8) v += dpp(v, std::integral_constant<int, 0x141>{});
        if constexpr (LPR >= 16) v += dpp(v, std::integral_constant<int, 0x140>{});
    } else {
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    }
    return v;
}

// Rotate-half partner table: tab[d] = partner(d) - d, whose sign gives the
// sign of rot (first half of a segment takes -x[d + half]).  Threads d < D
// fill it; the kernel's barrier orders the fill before any read.
template <int D>
__device__ __forceinline__ void fill_partner_table(const QkPrologueParams &p, signed char *tab) {
    const int d = threadIdx.x;
    if (d < D) {
        int pd;
        float sg;
        rope_partner(p, d, pd, sg);
        tab[d] = (signed char)(pd - d);
    }
}

// Token and head of row r0 + off of batch item blockIdx.y, with (t0, h0) the
// workgroup's first row: off < 128 and h0 < H keep u = h0 + off small
// enough for an f32 quotient estimate within one of u / H, corrected by one
// step either way (exact for every H <= 1024 and off < 128, checked
// exhaustively against integer division).
__device__ __forceinline__ void row_token_head(const QkPrologueParams &p, int t0, int h0, int off, int &t, int &h) {
    const int u = h0 + off;
    int q = (int)((float)u * p.inv_h);
    int r = u - (int)__umul24((unsigned)q, (unsigned)p.H);  // q <= u / H + 1, H < 2^24
    if (r >= p.H) {
        ++q;
        r -= p.H;
    } else if (r < 0) {
        --q;
        r += p.H;
    }
    t = t0 + q;
    h = r;
}

// Element offset of row (t, h) within its batch item.  The ABI bounds the
// token and head strides below 2^24 elements and a batch item's rows below
// 2^31 elements, so two 24-bit products (full-rate VALU) give it in 32 bits.
__device__ __forceinline__ uint32_t row_offset(int t, int h, int64_t ss, int64_t sh) {
    return __umul24((unsigned)t, (unsigned)ss) + __umul24((unsigned)h, (unsigned)sh);
}

// Rows are (b, token, head) triples in row-major order; a workgroup covers
// R passes of RPP rows, every lane holding 16 bytes of one row per pass.  All
// global loads of the R rows (x, and the token's cos / sin rows) are issued
// before any arithmetic.  Rows past the end load the last row and store
// nothing.  VEC: cos, sin and weight are 16-byte aligned.
template <typename T, int D, int R, bool VEC, bool TOK, bool QUAD>
__device__ __forceinline__ void qk_prologue_fwd_body(const QkPrologueParams &p, int bx, int64_t b) {
    // one rounding per reference op: no FMA contraction of x*cos + rot*sin
#pragma clang fp contract(off)
    constexpr int EPL = 16 / sizeof(T);   // elements per lane
    constexpr int LPR = D / EPL;          // lanes per row
    constexpr int RPP = 256 / LPR;        // rows per pass
    // the staged values (n * w) are exact in T: stage them as T
    __shared__ __attribute__((aligned(16))) T buf[R][RPP][D];
    const int tid = threadIdx.x, lr = tid / LPR, part = tid % LPR;
    const int rows = p.T * p.H;  // per batch item (< 2^31, checked by the ABI)
    const int r0 = bx * (R * RPP);
    const int t0 = r0 / p.H, h0 = r0 - t0 * p.H;
    __shared__ __attribute__((aligned(16))) signed char ptab[D];
    fill_partner_table<D>(p, ptab);
    float wv[EPL];
    load_row_part<T, VEC>(static_cast<const T *>(p.w) + part * EPL, wv);
    // TOK: the lane's R rows are R adjacent heads of one token (H % R == 0),
    // so one cos / sin load serves them all; otherwise rows k*RPP + lr
    constexpr int NTAB = TOK ? 1 : R;
    float xv[R][EPL], cv[NTAB][EPL], sv[NTAB][EPL];
    // rows of batch item b: 32-bit element offsets from uniform bases
    const T *xb = static_cast<const T *>(p.x) + b * p.x_sb;
    T *yb = static_cast<T *>(p.y) + b * p.y_sb + (int64_t)p.y_off * p.y_ss;
    uint32_t yoff[R];
    bool live[R];
    int ti, hi;
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int off0 = TOK ? lr * R + k : k * RPP + lr;
        live[k] = r0 + off0 < rows;
        if (!TOK || k == 0) {
            const int off = live[k] ? off0 : rows - 1 - r0;
            row_token_head(p, t0, h0, off, ti, hi);
        } else if (live[k]) {
            ++hi;  // the next head of the same token
        }
        const uint32_t xo = row_offset(ti, hi, p.x_ss, p.x_sh) + part * EPL;
        load_row_once<T>(xb + xo, xv[k]);
        if (!TOK || k == 0) {
            const uint32_t to = (uint32_t)ti * D + part * EPL;
            load_row_part<T, VEC>(static_cast<const T *>(p.cos) + to, cv[TOK ? 0 : k]);
            load_row_part<T, VEC>(static_cast<const T *>(p.sin) + to, sv[TOK ? 0 : k]);
        }
        yoff[k] = row_offset(ti, hi, p.y_ss, p.y_sh) + part * EPL;
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
        if constexpr (kFastStats<T>) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < EPL; ++i) ss = __builtin_fmaf(xv[k][i], xv[k][i], ss);
            ss = row_sum<LPR>(ss);
            const float rs = __builtin_amdgcn_rsqf(ss * (1.f / (float)D) + p.eps);
#pragma unroll
            for (int i = 0; i < EPL; i += 2) {
                float n0 = xv[k][i] * rs, n1 = xv[k][i + 1] * rs;
                round2_bf16(n0, n1);  // n cast to bf16
                n0 *= wv[i];
                n1 *= wv[i + 1];
                round2_bf16(n0, n1);  // n * w in bf16
                xv[k][i] = n0;
                xv[k][i + 1] = n1;
            }
        } else {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < EPL; ++i) ss += xv[k][i] * xv[k][i];
            ss = row_sum<LPR>(ss);
            const float sc = sqrtf(ss / (float)D + p.eps);
            const float rc = __builtin_amdgcn_rcpf(sc);
#pragma unroll
            for (int i = 0; i < EPL; ++i) {
                const float nv = round_dt<T>(div_by(xv[k][i], sc, rc));
                xv[k][i] = round_dt<T>(nv * wv[i]);  // the normed, weighted row (n * w)
            }
        }
#pragma unroll
        for (int i = 0; i < EPL; ++i) buf[k][lr][part * EPL + i] = (T)xv[k][i];
    }
    __syncthreads();
    if constexpr (QUAD) {
        // Every axis half is a multiple of 4: the partners of an aligned
        // group of 4 elements are an aligned group of 4 with one sign, read
        // from LDS in one access (8 bytes of bf16, 16 of f32).
        using Group = std::conditional_t<sizeof(T) == 2, u32x2, u32x4>;
        constexpr int NG = EPL / 4;
        int pq[NG];
        float sq[NG];
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const int o = ptab[part * EPL + 4 * j];
            pq[j] = part * EPL + 4 * j + o;
            sq[j] = o > 0 ? -1.f : 1.f;
        }
#pragma unroll
        for (int k = 0; k < R; ++k) {
            if (!live[k]) continue;
            T out[EPL];
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                const Group raw = *reinterpret_cast<const Group *>(&buf[k][lr][pq[j]]);
                const T *pv = reinterpret_cast<const T *>(&raw);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * j + e;
                    const float a = xv[k][i] * cv[TOK ? 0 : k][i];
                    const float r = (float)pv[e] * sv[TOK ? 0 : k][i];
                    out[i] = cast_out<T>(__builtin_fmaf(sq[j], r, a));
                }
            }
            store_row_once(yb + yoff[k], *reinterpret_cast<const u32x4 *>(out));
        }
        return;
    }
    int pd[EPL];
    float sg[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int o = ptab[part * EPL + i];
        pd[i] = part * EPL + i + o;
        sg[i] = o > 0 ? -1.f : 1.f;
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
        if (!live[k]) continue;
        T out[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            // x*cos + rot(x)*sin with rot = sign * partner: the sign
            // product is exact, so one FMA gives the reference's rounding
            // of the sum of the two rounded products
            const float a = xv[k][i] * cv[TOK ? 0 : k][i];
            const float r = (float)buf[k][lr][pd[i]] * sv[TOK ? 0 : k][i];
            out[i] = cast_out<T>(__builtin_fmaf(sg[i], r, a));
        }
        store_row_once(yb + yoff[k], *reinterpret_cast<const u32x4 *>(out));
    }
}

template <typename T, int D, int R, bool VEC, bool TOK, bool QUAD>
__device__ __forceinline__ void qk_prologue_bwd_body(const QkPrologueParams &p, int bx, int64_t b) {
    constexpr int EPL = 16 / sizeof(T);
    constexpr int LPR = D / EPL;
    constexpr int RPP = 256 / LPR;
    __shared__ __attribute__((aligned(16))) float buf[R][RPP][D];
    const int tid = threadIdx.x, lr = tid / LPR, part = tid % LPR;
    const int rows = p.T * p.H;
    const int r0 = bx * (R * RPP);
    const int t0 = r0 / p.H, h0 = r0 - t0 * p.H;
    __shared__ __attribute__((aligned(16))) signed char ptab[D];
    fill_partner_table<D>(p, ptab);
    float wv[EPL];
    load_row_part<T, VEC>(static_cast<const T *>(p.w) + part * EPL, wv);
    // TOK: as in the forward, the lane's R rows share one token's cos / sin
    constexpr int NTAB = TOK ? 1 : R;
    float xv[R][EPL], dyv[R][EPL], cv[NTAB][EPL], sv[NTAB][EPL];
    // rows of batch item b: 32-bit element offsets from uniform bases
    const T *xb = static_cast<const T *>(p.x) + b * p.x_sb;
    const T *dyb = static_cast<const T *>(p.dy) + b * p.y_sb + (int64_t)p.y_off * p.y_ss;
    T *dxb = static_cast<T *>(p.dx) + b * p.dx_sb;
    uint32_t dxoff[R];
    bool live[R];
    int ti, hi;
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int off0 = TOK ? lr * R + k : k * RPP + lr;
        live[k] = r0 + off0 < rows;
        if (!TOK || k == 0) {
            const int off = live[k] ? off0 : rows - 1 - r0;
            row_token_head(p, t0, h0, off, ti, hi);
        } else if (live[k]) {
            ++hi;  // the next head of the same token
        }
        load_row_part<T, true>(xb + row_offset(ti, hi, p.x_ss, p.x_sh) + part * EPL, xv[k]);
        load_row_part<T, true>(dyb + row_offset(ti, hi, p.y_ss, p.y_sh) + part * EPL, dyv[k]);
        if (!TOK || k == 0) {
            const uint32_t to = (uint32_t)ti * D + part * EPL;
            load_row_part<T, VEC>(static_cast<const T *>(p.cos) + to, cv[TOK ? 0 : k]);
            load_row_part<T, VEC>(static_cast<const T *>(p.sin) + to, sv[TOK ? 0 : k]);
        }
        dxoff[k] = row_offset(ti, hi, p.dx_ss, p.dx_sh) + part * EPL;
    }
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
        for (int i = 0; i < EPL; ++i) buf[k][lr][part * EPL + i] = dyv[k][i] * sv[TOK ? 0 : k][i];
    __syncthreads();
    // QUAD: partners in aligned groups of 4 with one sign (as in the
    // forward), read as one 16-byte LDS access of the f32 staging rows
    constexpr int NG = EPL / 4;
    int pd[EPL], pq[NG > 0 ? NG : 1];
    float sg[EPL], sq[NG > 0 ? NG : 1];
    if constexpr (QUAD) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const int o = ptab[part * EPL + 4 * j];
            pq[j] = part * EPL + 4 * j + o;
            sq[j] = o > 0 ? -1.f : 1.f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int o = ptab[part * EPL + i];
            pd[i] = part * EPL + i + o;
            sg[i] = o > 0 ? -1.f : 1.f;
        }
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) ss += xv[k][i] * xv[k][i];
        ss = row_sum<LPR>(ss);
        float sigma = 0.f, rs;
        if constexpr (kFastStats<T>) {
            rs = __builtin_amdgcn_rsqf(ss * (1.f / (float)D) + p.eps);
        } else {
            sigma = sqrtf(ss / (float)D + p.eps);
            rs = __builtin_amdgcn_rcpf(sigma);
        }
        // x / sigma: one multiply for bf16 rows, the corrected quotient for f32
        auto over_sigma = [&](float v) { return kFastStats<T> ? v * rs : div_by(v, sigma, rs); };
        float dn[EPL], nv[EPL];
        float dot = 0.f;
        // the partner value of element i and the sign of rot for it
        float pv[EPL], ps[EPL];
        if constexpr (QUAD) {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                const f32x4 g4 = *reinterpret_cast<const f32x4 *>(&buf[k][lr][pq[j]]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pv[4 * j + e] = g4[e];
                    ps[4 * j + e] = sq[j];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < EPL; ++i) {
                pv[i] = buf[k][lr][pd[i]];
                ps[i] = sg[i];
            }
        }
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            // rot^T takes the partner with the opposite sign of rot
            const float gv = __builtin_fmaf(-ps[i], pv[i], dyv[k][i] * cv[TOK ? 0 : k][i]);
            dn[i] = gv * wv[i];
            nv[i] = over_sigma(xv[k][i]);
            dot += dn[i] * nv[i];
        }
        dot = row_sum<LPR>(dot);
        if (!live[k]) continue;
        const float mdot = dot * (1.f / (float)D);
        T out[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) out[i] = cast_out<T>(over_sigma(dn[i] - nv[i] * mdot));
        st_global_16(dxb + dxoff[k], *reinterpret_cast<const u32x4 *>(out));
    }
}

// Rows per lane (passes per workgroup).  Measured at c2's Q + K (HIP-graph
// replay): the forward with rows sharing a token runs 4% faster at 4 rows
// (80 VGPRs) than at 2; the backward, and rows of different tokens (105
// VGPRs at 4), stay at 2.
constexpr int kPrologueRows = 2;
constexpr int kPrologueRowsFwdTok = 4;

// Several prologue segments (Q and K of the txt and img streams) in one
// launch: the grid's x blocks are the segments' blocks end to end, and a
// workgroup finds its segment from the prefix table (wave-uniform), so the
// launch ramp and each workgroup's setup serve every segment at once.
struct QkPrologueMulti {
    QkPrologueParams seg[kMaxPrologueSegs];
    int wg0[kMaxPrologueSegs + 1];  // first grid x block of each segment; wg0[count] = grid x
    int count;
};

template <typename T, int D, int R, bool VEC, bool BWD, bool TOK, bool QUAD>
__global__ __launch_bounds__(256) void qk_prologue_multi_kernel(QkPrologueMulti m) {
    const int bx = blockIdx.x;
    int sgi = 0;
#pragma unroll
    for (int i = 1; i < kMaxPrologueSegs; ++i)
        if (i < m.count && bx >= m.wg0[i]) sgi = i;
    // one segment's parameters, selected by constant index (kernel-argument
    // loads, no copy to scratch)
    auto run = [&](const QkPrologueParams &p) {
        if ((int)blockIdx.y >= p.B) return;  // a segment with a smaller batch
        if constexpr (BWD)
            qk_prologue_bwd_body<T, D, R, VEC, TOK, QUAD>(p, bx - m.wg0[sgi], blockIdx.y);
        else
            qk_prologue_fwd_body<T, D, R, VEC, TOK, QUAD>(p, bx - m.wg0[sgi], blockIdx.y);
    };
    if (sgi == 0) run(m.seg[0]);
    else if (sgi == 1) run(m.seg[1]);
    else if (sgi == 2) run(m.seg[2]);
    else run(m.seg[3]);
}

template <typename T, int D, bool BWD, bool VEC, int R, bool TOK, bool QUAD = false>
hipError_t launch_prologue_r(const QkPrologueParams *ps, int n, hipStream_t s) {
    constexpr int LPR = D * sizeof(T) / 16;
    constexpr int RPB = 256 / LPR * R;
    QkPrologueMulti m{};
    m.count = n;
    int64_t wg = 0;
    unsigned by = 1;
    for (int i = 0; i < n; ++i) {
        m.seg[i] = ps[i];
        m.seg[i].inv_h = 1.f / (float)ps[i].H;
        m.wg0[i] = (int)wg;
        wg += ((int64_t)ps[i].T * ps[i].H + RPB - 1) / RPB;
        by = by > (unsigned)ps[i].B ? by : (unsigned)ps[i].B;
    }
    if (wg >= (int64_t(1) << 31)) return hipErrorInvalidConfiguration;
    for (int i = n; i <= kMaxPrologueSegs; ++i) m.wg0[i] = (int)wg;
    const dim3 grid((unsigned)wg, by), block(256);
    hipLaunchKernelGGL((qk_prologue_multi_kernel<T, D, R, VEC, BWD, TOK, QUAD>), grid, block, 0, s, m);
    return hipGetLastError();
}

// A lane's rows share a token when every segment's head count is a multiple
// of the rows per lane (the workgroup's first row is then one too).
template <typename T, int D, bool BWD, bool VEC>
hipError_t launch_prologue_v(const QkPrologueParams *ps, int n, hipStream_t s) {
    auto all_heads = [&](int r) {
        for (int i = 0; i < n; ++i)
            if (ps[i].H % r) return false;
        return true;
    };
    // rotate-half partners are read 4 at a time when every axis half of
    // every segment is a multiple of 4
    bool quad = true;
    for (int i = 0; i < n; ++i)
        for (int a = 0; a < ps[i].n_axes; ++a) quad = quad && (ps[i].axes[a] / 2) % 4 == 0;
    if constexpr (!BWD) {
        if (all_heads(kPrologueRowsFwdTok))
            return quad ? launch_prologue_r<T, D, BWD, VEC, kPrologueRowsFwdTok, true, true>(ps, n, s)
                        : launch_prologue_r<T, D, BWD, VEC, kPrologueRowsFwdTok, true, false>(ps, n, s);
    }
    if (quad)
        return all_heads(kPrologueRows) ? launch_prologue_r<T, D, BWD, VEC, kPrologueRows, true, true>(ps, n, s)
                                        : launch_prologue_r<T, D, BWD, VEC, kPrologueRows, false, true>(ps, n, s);
    if (all_heads(kPrologueRows)) return launch_prologue_r<T, D, BWD, VEC, kPrologueRows, true>(ps, n, s);
    return launch_prologue_r<T, D, BWD, VEC, kPrologueRows, false>(ps, n, s);
}

template <typename T, int D, bool BWD>
hipError_t launch_prologue(const QkPrologueParams *ps, int n, hipStream_t s) {
    bool vec = true;
    for (int i = 0; i < n; ++i)
        vec = vec && reinterpret_cast<uintptr_t>(ps[i].w) % 16 == 0 && reinterpret_cast<uintptr_t>(ps[i].cos) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(ps[i].sin) % 16 == 0;
    return vec ? launch_prologue_v<T, D, BWD, true>(ps, n, s) : launch_prologue_v<T, D, BWD, false>(ps, n, s);
}

template <bool BWD>
hipError_t dispatch(const QkPrologueParams *ps, int n, int dtype, hipStream_t s) {
    if (n < 1 || n > kMaxPrologueSegs) return hipErrorInvalidValue;
    const int D = ps[0].D;
    if (dtype == 0)
        return D == 128 ? launch_prologue<bf16, 128, BWD>(ps, n, s) : launch_prologue<bf16, 64, BWD>(ps, n, s);
    return D == 128 ? launch_prologue<float, 128, BWD>(ps, n, s) : launch_prologue<float, 64, BWD>(ps, n, s);
}

}  // namespace

hipError_t launch_qk_prologue_fwd(const QkPrologueParams *ps, int n, int dtype, hipStream_t s) {
    return dispatch<false>(ps, n, dtype, s);
}

hipError_t launch_qk_prologue_bwd(const QkPrologueParams *ps, int n, int dtype, hipStream_t s) {
    return dispatch<true>(ps, n, dtype, s);
}

}  // namespace fa
