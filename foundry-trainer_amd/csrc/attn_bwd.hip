// Flash-attention backward for gfx950 (CDNA4).
//
// Computes the gradients of foundry-spike's AttnBwd::bwd
// (crates/foundry-spike/src/lib.rs:216-263) without materialising any S x S
// tensor:
//   P    = exp(scale * Q K^T - LSE)        recomputed from the forward's LSE
//   dP   = dO V^T
//   D_i  = rowsum(dO * O)_i                (= rowsum(dP * P)_i in exact
//                                           arithmetic; the reference's
//                                           lib.rs:246-247 form)
//   dS   = P * (dP - D_i) * scale
//   dV   = P^T dO,  dK = dS^T Q,  dQ = dS K
// Three launches, no atomics, bit-identical on repeat:
//   1. delta:  D = rowsum(dO * O)                    (HBM-bound)
//   2. dk/dv:  one workgroup per 128 keys (4 waves x 32 keys), looping over
//              all queries in 64-query LDS stages.  S = Q K^T puts keys on the
//              accumulator's lanes, so P and dS feed the dV / dK MFMAs as A
//              operands straight from registers.
//   3. dq:     one workgroup per 128 queries (4 waves x 32), looping over
//              64-key LDS stages.  S^T = K Q^T puts queries on the lanes, so
//              dS^T feeds dQ^T = K^T dS^T as the B operand.
// All GEMMs run on v_mfma_f32_32x32x16_bf16 (bf16 storage) or
// v_mfma_f32_32x32x2_f32 (f32 storage) with f32 accumulation.
#include <math.h>

#include "fa_device.hpp"
#include "fa_kernels.hpp"
#include "fa_tiles.hpp"

namespace fa {
namespace {

// ---------------------------------------------------------------------------
// 1. delta = rowsum(dO * O) in f32, written [B,H,S]
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(AttnBwdParams p) {
    constexpr int EPL = 16 / sizeof(T);  // elements per 16-byte load
    constexpr int LPR = D / EPL;         // lanes per row
    const int64_t rows = (int64_t)p.B * p.S * p.H;
    const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR;
    const int part = threadIdx.x % LPR;
    float acc = 0.f;
    int b = 0, s = 0, h = 0;
    if (row < rows) {
        h = row % p.H;
        s = (row / p.H) % p.S;
        b = row / ((int64_t)p.H * p.S);
        const T *o = static_cast<const T *>(p.o) + b * p.o_sb + s * p.o_ss + h * p.o_sh + part * EPL;
        const T *d =
            static_cast<const T *>(p.dout) + b * p.do_sb + s * p.do_ss + h * p.do_sh + part * EPL;
        const u32x4 ov = ld_global_16(o), dv = ld_global_16(d);
        if constexpr (sizeof(T) == 2) {
            const bf16x8 a = as_bf16x8(ov), c = as_bf16x8(dv);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += (float)a[e] * (float)c[e];
        } else {
            // bit-cast the whole vector: a bit cast of a vector-element lvalue
            // (ov[e]) reads element 0 whatever e is
            const f32x4 a = __builtin_bit_cast(f32x4, ov), c = __builtin_bit_cast(f32x4, dv);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc += a[e] * c[e];
        }
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (row < rows && part == 0) p.delta[((int64_t)b * p.H + h) * p.S + s] = acc;
}

// ---------------------------------------------------------------------------
// 2. dK / dV (bf16)
// ---------------------------------------------------------------------------
constexpr int kKT = 128;  // keys per workgroup
constexpr int kQB = 64;   // queries per LDS stage

template <int D>
struct DkvSmem {
    static constexpr int Q_RM = 0;
    static constexpr int Q_TR = Q_RM + Tile64<D>::BYTES;
    static constexpr int DO_RM = Q_TR + Tile64<D>::BYTES;
    static constexpr int DO_TR = DO_RM + Tile64<D>::BYTES;
    static constexpr int LSE = DO_TR + Tile64<D>::BYTES;  // 64 f32: lse * log2(e)
    static constexpr int DELTA = LSE + kQB * 4;          // 64 f32
    static constexpr int BYTES = DELTA + kQB * 4;
};

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_bf16_kernel(AttnBwdParams p) {
    using L = DkvSmem<D>;
    extern __shared__ __align__(16) char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nk = (S + kKT - 1) / kKT;
    const int work = xcd_remap(blockIdx.x, gridDim.x);
    const int kt = work % nk, bh = work / nk;
    const int h = bh % H, b = bh / H;

    const bf16 *qbase = static_cast<const bf16 *>(p.q) + b * p.q_sb + h * p.q_sh;
    const bf16 *kbase = static_cast<const bf16 *>(p.k) + b * p.k_sb + h * p.k_sh;
    const bf16 *vbase = static_cast<const bf16 *>(p.v) + b * p.v_sb + h * p.v_sh;
    const bf16 *dobase = static_cast<const bf16 *>(p.dout) + b * p.do_sb + h * p.do_sh;
    const float *lse = p.lse + ((int64_t)b * H + h) * S;
    const float *delta = p.delta + ((int64_t)b * H + h) * S;
    const int kj = kt * kKT + wave * 32 + n;  // this lane's key
    const bool key_kept = kj < S && (!p.keep || p.keep[(int64_t)b * S + kj]);

    // K^T and V^T B-operand fragments: lane holds row kj, features kd*16+g*8..+8
    bf16x8 kf[D / 16], vf[D / 16];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) {
        const bool in = kj < S;
        kf[kd] = as_bf16x8(in ? ld_global_16(kbase + kj * p.k_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
        vf[kd] = as_bf16x8(in ? ld_global_16(vbase + kj * p.v_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
    }
    f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[dt][r] = dv[dt][r] = 0.f;
    const float c = p.scale_log2;

    const int nqb = (S + kQB - 1) / kQB;
    for (int qb = 0; qb < nqb; ++qb) {
        const int q0 = qb * kQB;
        {
            u32x4 rq[Tile64<D>::PAIR_LOADS], rd[Tile64<D>::PAIR_LOADS];
            tile_load_pairs<D>(rq, qbase, p.q_ss, q0, S, tid);
            tile_load_pairs<D>(rd, dobase, p.do_ss, q0, S, tid);
            float lv = INFINITY, dlt = 0.f;  // rows past S contribute P = 0
            if (tid < kQB && q0 + tid < S) {
                const float l = lse[q0 + tid];
                // a row with every key masked has LSE = -inf and P = 0
                lv = l == -INFINITY ? INFINITY : l * kLog2e;
                dlt = delta[q0 + tid];
            }
            __syncthreads();  // previous stage fully consumed
            tile_store_rm_pairs<D>(rq, smem + L::Q_RM, tid);
            tile_store_tr<D>(rq, smem + L::Q_TR, tid);
            tile_store_rm_pairs<D>(rd, smem + L::DO_RM, tid);
            tile_store_tr<D>(rd, smem + L::DO_TR, tid);
            if (tid < kQB) {
                reinterpret_cast<float *>(smem + L::LSE)[tid] = lv;
                reinterpret_cast<float *>(smem + L::DELTA)[tid] = dlt;
            }
            __syncthreads();
        }
        const float *lse_s = reinterpret_cast<const float *>(smem + L::LSE);
        const float *dlt_s = reinterpret_cast<const float *>(smem + L::DELTA);

#pragma unroll
        for (int sub = 0; sub < kQB / 32; ++sub) {
            // S = Q K^T and dP = dO V^T for 32 queries x this lane-column's key
            f32x16 s, dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
            for (int kd = 0; kd < D / 16; ++kd) {
                s = mfma_32x32x16(rm_frag<D>(smem + L::Q_RM, sub * 32 + n, kd, g), kf[kd], s);
                dp = mfma_32x32x16(rm_frag<D>(smem + L::DO_RM, sub * 32 + n, kd, g), vf[kd], dp);
            }
            bf16x8 pf[2], df[2];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int qi = sub * 32 + acc_row(r, lane);
                float pv = exp2_fast(s[r] * c - lse_s[qi]);
                pv = key_kept ? pv : 0.f;
                const float ds = pv * (dp[r] - dlt_s[qi]);
                pf[r >> 3][r & 7] = f32_to_bf16(pv);
                df[r >> 3][r & 7] = f32_to_bf16(ds);
            }
            // dV += P^T dO, dK += dS^T Q  (contraction over the 32 queries)
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const int f = dt * 32 + n;
                    dv[dt] = mfma_32x32x16(pf[ks], tr_frag(smem + L::DO_TR, f, sub * 2 + ks, g), dv[dt]);
                    dk[dt] = mfma_32x32x16(df[ks], tr_frag(smem + L::Q_TR, f, sub * 2 + ks, g), dk[dt]);
                }
        }
    }

    // dk/dv accumulators: element r of lane = (key kt*128 + wave*32 + acc_row(r), d = dt*32 + n)
    bf16 *dkb = static_cast<bf16 *>(p.dk) + b * p.dk_sb + h * p.dk_sh;
    bf16 *dvb = static_cast<bf16 *>(p.dv) + b * p.dv_sb + h * p.dv_sh;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int key = kt * kKT + wave * 32 + acc_row(r, lane);
        if (key < S) {
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                dkb[key * p.dk_ss + dt * 32 + n] = f32_to_bf16(dk[dt][r] * p.scale);
                dvb[key * p.dv_ss + dt * 32 + n] = f32_to_bf16(dv[dt][r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// 3. dQ (bf16)
// ---------------------------------------------------------------------------
constexpr int kQT = 128;  // queries per workgroup
constexpr int kKB = 64;   // keys per LDS stage

template <int D>
struct DqSmem {
    static constexpr int K_RM = 0;
    static constexpr int K_TR = K_RM + Tile64<D>::BYTES;
    static constexpr int V_RM = K_TR + Tile64<D>::BYTES;
    static constexpr int BYTES = V_RM + Tile64<D>::BYTES;
};

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_bf16_kernel(AttnBwdParams p) {
    using L = DqSmem<D>;
    extern __shared__ __align__(16) char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nq = (S + kQT - 1) / kQT;
    const int work = xcd_remap(blockIdx.x, gridDim.x);
    const int qt = work % nq, bh = work / nq;
    const int h = bh % H, b = bh / H;

    const bf16 *qbase = static_cast<const bf16 *>(p.q) + b * p.q_sb + h * p.q_sh;
    const bf16 *kbase = static_cast<const bf16 *>(p.k) + b * p.k_sb + h * p.k_sh;
    const bf16 *vbase = static_cast<const bf16 *>(p.v) + b * p.v_sb + h * p.v_sh;
    const bf16 *dobase = static_cast<const bf16 *>(p.dout) + b * p.do_sb + h * p.do_sh;
    const uint8_t *keep = p.keep ? p.keep + (int64_t)b * S : nullptr;
    const int qi = qt * kQT + wave * 32 + n;

    bf16x8 qf[D / 16], of[D / 16];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) {
        const bool in = qi < S;
        qf[kd] = as_bf16x8(in ? ld_global_16(qbase + qi * p.q_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
        of[kd] = as_bf16x8(in ? ld_global_16(dobase + qi * p.do_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
    }
    float lse2 = INFINITY, dlt = 0.f;
    if (qi < S) {
        const float l = p.lse[((int64_t)b * H + h) * S + qi];
        lse2 = l == -INFINITY ? INFINITY : l * kLog2e;
        dlt = p.delta[((int64_t)b * H + h) * S + qi];
    }
    f32x16 dq[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[dt][r] = 0.f;
    const float c = p.scale_log2;

    const int nkb = (S + kKB - 1) / kKB;
    for (int kb = 0; kb < nkb; ++kb) {
        const int k0 = kb * kKB;
        {
            u32x4 rk[Tile64<D>::PAIR_LOADS], rv[Tile64<D>::RM_LOADS];
            tile_load_pairs<D>(rk, kbase, p.k_ss, k0, S, tid);
            tile_load_rm<D>(rv, vbase, p.v_ss, k0, S, tid);
            __syncthreads();
            tile_store_rm_pairs<D>(rk, smem + L::K_RM, tid);
            tile_store_tr<D>(rk, smem + L::K_TR, tid);
            tile_store_rm<D>(rv, smem + L::V_RM, tid);
            __syncthreads();
        }
        uint64_t km = ~0ull;
        if (keep || k0 + kKB > S) {
            const int key = k0 + lane;
            km = __ballot(key < S && (!keep || keep[key]));
        }
        // S^T = K Q^T and dP^T = V dO^T: two 32-key tiles each
        f32x16 s[2], dp[2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[t][r] = dp[t][r] = 0.f;
#pragma unroll
        for (int kd = 0; kd < D / 16; ++kd)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                s[t] = mfma_32x32x16(rm_frag<D>(smem + L::K_RM, t * 32 + n, kd, g), qf[kd], s[t]);
                dp[t] = mfma_32x32x16(rm_frag<D>(smem + L::V_RM, t * 32 + n, kd, g), of[kd], dp[t]);
            }
        bf16x8 df[4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kk = t * 32 + acc_row(r, lane);
                float pv = exp2_fast(s[t][r] * c - lse2);
                pv = ((km >> kk) & 1) ? pv : 0.f;
                df[t * 2 + (r >> 3)][r & 7] = f32_to_bf16(pv * (dp[t][r] - dlt));
            }
        // dQ^T += K^T dS^T
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                dq[dt] = mfma_32x32x16(tr_frag(smem + L::K_TR, dt * 32 + n, ks, g), df[ks], dq[dt]);
    }

    if (qi < S) {
        bf16 *row = static_cast<bf16 *>(p.dq) + b * p.dq_sb + h * p.dq_sh + qi * p.dq_ss;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                const int d = dt * 32 + grp * 8 + g * 4;
                u32x2 w;
                w[0] = pack_bf16x2(dq[dt][grp * 4 + 0] * p.scale, dq[dt][grp * 4 + 1] * p.scale);
                w[1] = pack_bf16x2(dq[dt][grp * 4 + 2] * p.scale, dq[dt][grp * 4 + 3] * p.scale);
                *reinterpret_cast<u32x2 *>(row + d) = w;
            }
    }
}

// ---------------------------------------------------------------------------
// f32 backward (FA_DTYPE_F32): exact f32 MFMA, one wave per 32 keys (dK/dV)
// or 32 queries (dQ), 32-row blocks.  Parity path for the reference's f32 run.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64) void attn_bwd_dkdv_f32_kernel(AttnBwdParams p) {
    __shared__ float Qs[32][D + 1];
    __shared__ float Os[32][D + 1];  // dO block
    __shared__ float Ls[32], Ds[32];
    const int lane = threadIdx.x, n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nk = (S + 31) / 32;
    const int kt = blockIdx.x % nk, bh = blockIdx.x / nk;
    const int h = bh % H, b = bh / H;
    const float *qbase = static_cast<const float *>(p.q) + b * p.q_sb + h * p.q_sh;
    const float *kbase = static_cast<const float *>(p.k) + b * p.k_sb + h * p.k_sh;
    const float *vbase = static_cast<const float *>(p.v) + b * p.v_sb + h * p.v_sh;
    const float *dobase = static_cast<const float *>(p.dout) + b * p.do_sb + h * p.do_sh;
    const float *lse = p.lse + ((int64_t)b * H + h) * S;
    const float *delta = p.delta + ((int64_t)b * H + h) * S;
    const int kj = kt * 32 + n;
    const bool kept = kj < S && (!p.keep || p.keep[(int64_t)b * S + kj]);
    float kf[D / 2], vf[D / 2];
#pragma unroll
    for (int kd = 0; kd < D / 2; ++kd) {
        kf[kd] = kj < S ? kbase[kj * p.k_ss + 2 * kd + g] : 0.f;
        vf[kd] = kj < S ? vbase[kj * p.v_ss + 2 * kd + g] : 0.f;
    }
    f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[dt][r] = dv[dt][r] = 0.f;
    const float c = p.scale_log2;
    for (int q0 = 0; q0 < S; q0 += 32) {
        __syncthreads();
        for (int e = lane; e < 32 * D; e += 64) {
            const int row = e / D, d = e % D, qi = q0 + row;
            Qs[row][d] = qi < S ? qbase[qi * p.q_ss + d] : 0.f;
            Os[row][d] = qi < S ? dobase[qi * p.do_ss + d] : 0.f;
        }
        if (lane < 32) {
            const int qi = q0 + lane;
            const float l = qi < S ? lse[qi] : INFINITY;
            Ls[lane] = l == -INFINITY ? INFINITY : l * kLog2e;
            Ds[lane] = qi < S ? delta[qi] : 0.f;
        }
        __syncthreads();
        f32x16 s, dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
        for (int kd = 0; kd < D / 2; ++kd) {
            s = mfma_32x32x2_f32(Qs[n][2 * kd + g], kf[kd], s);
            dp = mfma_32x32x2_f32(Os[n][2 * kd + g], vf[kd], dp);
        }
        f32x16 pm, dsm;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int qi = acc_row(r, lane);
            const float pv = kept ? exp2f(s[r] * c - Ls[qi]) : 0.f;
            pm[r] = pv;
            dsm[r] = pv * (dp[r] - Ds[qi]);
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int qi = acc_row(t, lane);
                dv[dt] = mfma_32x32x2_f32(pm[t], Os[qi][dt * 32 + n], dv[dt]);
                dk[dt] = mfma_32x32x2_f32(dsm[t], Qs[qi][dt * 32 + n], dk[dt]);
            }
    }
    float *dkb = static_cast<float *>(p.dk) + b * p.dk_sb + h * p.dk_sh;
    float *dvb = static_cast<float *>(p.dv) + b * p.dv_sb + h * p.dv_sh;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int key = kt * 32 + acc_row(r, lane);
        if (key < S)
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                dkb[key * p.dk_ss + dt * 32 + n] = dk[dt][r] * p.scale;
                dvb[key * p.dv_ss + dt * 32 + n] = dv[dt][r];
            }
    }
}

template <int D>
__global__ __launch_bounds__(64) void attn_bwd_dq_f32_kernel(AttnBwdParams p) {
    __shared__ float Ks[32][D + 1];
    __shared__ float Vs[32][D + 1];
    const int lane = threadIdx.x, n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nq = (S + 31) / 32;
    const int qt = blockIdx.x % nq, bh = blockIdx.x / nq;
    const int h = bh % H, b = bh / H;
    const float *qbase = static_cast<const float *>(p.q) + b * p.q_sb + h * p.q_sh;
    const float *kbase = static_cast<const float *>(p.k) + b * p.k_sb + h * p.k_sh;
    const float *vbase = static_cast<const float *>(p.v) + b * p.v_sb + h * p.v_sh;
    const float *dobase = static_cast<const float *>(p.dout) + b * p.do_sb + h * p.do_sh;
    const uint8_t *keep = p.keep ? p.keep + (int64_t)b * S : nullptr;
    const int qi = qt * 32 + n;
    float qf[D / 2], of[D / 2];
#pragma unroll
    for (int kd = 0; kd < D / 2; ++kd) {
        qf[kd] = qi < S ? qbase[qi * p.q_ss + 2 * kd + g] : 0.f;
        of[kd] = qi < S ? dobase[qi * p.do_ss + 2 * kd + g] : 0.f;
    }
    float lse2 = INFINITY, dlt = 0.f;
    if (qi < S) {
        const float l = p.lse[((int64_t)b * H + h) * S + qi];
        lse2 = l == -INFINITY ? INFINITY : l * kLog2e;
        dlt = p.delta[((int64_t)b * H + h) * S + qi];
    }
    f32x16 dq[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[dt][r] = 0.f;
    const float c = p.scale_log2;
    for (int k0 = 0; k0 < S; k0 += 32) {
        __syncthreads();
        for (int e = lane; e < 32 * D; e += 64) {
            const int row = e / D, d = e % D, key = k0 + row;
            Ks[row][d] = key < S ? kbase[key * p.k_ss + d] : 0.f;
            Vs[row][d] = key < S ? vbase[key * p.v_ss + d] : 0.f;
        }
        __syncthreads();
        bool kept = false;
        if (lane < 32) kept = k0 + lane < S && (!keep || keep[k0 + lane]);
        const uint64_t km = __ballot(kept);
        f32x16 s, dp;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
        for (int kd = 0; kd < D / 2; ++kd) {
            s = mfma_32x32x2_f32(Ks[n][2 * kd + g], qf[kd], s);
            dp = mfma_32x32x2_f32(Vs[n][2 * kd + g], of[kd], dp);
        }
        f32x16 dsm;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int kk = acc_row(r, lane);
            const float pv = ((km >> kk) & 1) ? exp2f(s[r] * c - lse2) : 0.f;
            dsm[r] = pv * (dp[r] - dlt);
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int t = 0; t < 16; ++t)
                dq[dt] = mfma_32x32x2_f32(Ks[acc_row(t, lane)][dt * 32 + n], dsm[t], dq[dt]);
    }
    if (qi < S) {
        float *row = static_cast<float *>(p.dq) + b * p.dq_sb + h * p.dq_sh + qi * p.dq_ss;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) row[dt * 32 + acc_row(r, lane)] = dq[dt][r] * p.scale;
    }
}

template <typename T, int D>
hipError_t launch_delta(const AttnBwdParams &p, hipStream_t s) {
    constexpr int LPR = D * sizeof(T) / 16;
    const int64_t threads = (int64_t)p.B * p.S * p.H * LPR;
    const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    hipLaunchKernelGGL((attn_bwd_delta_kernel<T, D>), grid, block, 0, s, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_bwd_bf16(const AttnBwdParams &p, int D, hipStream_t s) {
    hipError_t e = D == 128 ? launch_delta<bf16, 128>(p, s) : launch_delta<bf16, 64>(p, s);
    if (e != hipSuccess) return e;
    const int nk = (p.S + kKT - 1) / kKT, nq = (p.S + kQT - 1) / kQT;
    const dim3 gk(p.B * p.H * nk), gq(p.B * p.H * nq), block(256);
    if (D == 128) {
        hipLaunchKernelGGL(attn_bwd_dkdv_bf16_kernel<128>, gk, block, DkvSmem<128>::BYTES, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(attn_bwd_dq_bf16_kernel<128>, gq, block, DqSmem<128>::BYTES, s, p);
    } else {
        hipLaunchKernelGGL(attn_bwd_dkdv_bf16_kernel<64>, gk, block, DkvSmem<64>::BYTES, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(attn_bwd_dq_bf16_kernel<64>, gq, block, DqSmem<64>::BYTES, s, p);
    }
    return hipGetLastError();
}

hipError_t launch_attn_bwd_f32(const AttnBwdParams &p, int D, hipStream_t s) {
    hipError_t e = D == 128 ? launch_delta<float, 128>(p, s) : launch_delta<float, 64>(p, s);
    if (e != hipSuccess) return e;
    const int n32 = (p.S + 31) / 32;
    const dim3 grid(p.B * p.H * n32), block(64);
    if (D == 128) {
        hipLaunchKernelGGL(attn_bwd_dkdv_f32_kernel<128>, grid, block, 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(attn_bwd_dq_f32_kernel<128>, grid, block, 0, s, p);
    } else {
        hipLaunchKernelGGL(attn_bwd_dkdv_f32_kernel<64>, grid, block, 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(attn_bwd_dq_f32_kernel<64>, grid, block, 0, s, p);
    }
    return hipGetLastError();
}

hipError_t prepare_bwd_kernels() {
    hipError_t e;
    if ((e = hipFuncSetAttribute((const void *)attn_bwd_dkdv_bf16_kernel<128>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                 DkvSmem<128>::BYTES)) != hipSuccess)
        return e;
    if ((e = hipFuncSetAttribute((const void *)attn_bwd_dkdv_bf16_kernel<64>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                 DkvSmem<64>::BYTES)) != hipSuccess)
        return e;
    if ((e = hipFuncSetAttribute((const void *)attn_bwd_dq_bf16_kernel<128>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                 DqSmem<128>::BYTES)) != hipSuccess)
        return e;
    return hipFuncSetAttribute((const void *)attn_bwd_dq_bf16_kernel<64>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, DqSmem<64>::BYTES);
}

}  // namespace fa
