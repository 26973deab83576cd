// Flash-attention forward for gfx950 (CDNA4), emitting O and the row LSE.
//
// Semantics follow foundry-spike's attn_fwd (crates/foundry-spike/src/lib.rs:
// 131-149): scores = (Q K^T) * scale in f32, softmax in f32, P cast to the
// storage dtype, O = P V with f32 accumulation.  The softmax is computed
// online (running max / sum per query row) so the (H,S,S) score tensor the
// reference materialises never exists; the natural-log row logsumexp is
// written for the backward.
//
// bf16 kernel layout (one workgroup = 4 waves = 128 queries of one (b, h)):
//   - Each wave owns 32 queries.  It computes S^T = K Q^T for a 64-key block
//     on v_mfma_f32_32x32x16_bf16: K (A operand) is read from LDS, Q (B
//     operand) stays in registers for the whole kernel.  In the S^T
//     accumulator every lane holds 16 keys of ONE query (lane % 32), so the
//     row max / row sum need a single cross-lane step (lane ^ 32).
//   - O^T = V^T P^T is the second MFMA: V^T (A operand) comes from a
//     transposed LDS tile, P^T (B operand) is the S^T accumulator converted to
//     bf16 in registers — no LDS round trip for P.
//   - K and V^T tiles are double-buffered in LDS; the next block's global
//     loads are in flight while the current block computes (one barrier per
//     block).
//   - Workgroups are remapped so the 8 XCDs each take contiguous runs of
//     (b, h) query tiles and share K/V in their own L2.
#include <math.h>

#include "fa_device.hpp"
#include "fa_kernels.hpp"
#include "fa_tiles.hpp"

namespace fa {
namespace {

constexpr int kBM = 128;  // queries per workgroup
constexpr int kBN = 64;   // keys per block
constexpr int kThreads = 256;

template <int D>
struct FwdTile {
    static constexpr int K_BYTES = Tile64<D>::BYTES;  // K tile, row-major swizzled
    static constexpr int V_BYTES = Tile64<D>::BYTES;  // V^T tile
    static constexpr int STAGE = K_BYTES + V_BYTES;
    static constexpr int SMEM = 2 * STAGE;
};

template <int D>
struct TileRegs {
    u32x4 k[Tile64<D>::RM_LOADS];
    u32x4 v[Tile64<D>::PAIR_LOADS];
};

// Global -> registers for key block kb (rows >= S read as zero).
template <int D>
__device__ __forceinline__ void load_tile(TileRegs<D> &t, const bf16 *kbase, const bf16 *vbase,
                                          int64_t k_ss, int64_t v_ss, int kb, int S, int tid) {
    tile_load_rm<D>(t.k, kbase, k_ss, kb * kBN, S, tid);
    tile_load_pairs<D>(t.v, vbase, v_ss, kb * kBN, S, tid);
}

// Registers -> LDS stage: K swizzled row-major, V transposed to V^T.
template <int D>
__device__ __forceinline__ void store_tile(const TileRegs<D> &t, char *stage, int tid) {
    tile_store_rm<D>(t.k, stage, tid);
    tile_store_tr<D>(t.v, stage + FwdTile<D>::K_BYTES, tid);
}

template <int D>
__global__ __launch_bounds__(kThreads) void attn_fwd_bf16_kernel(AttnFwdParams p) {
    using T = FwdTile<D>;
    extern __shared__ __align__(16) char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nq = (S + kBM - 1) / kBM;
    const int work = xcd_remap(blockIdx.x, gridDim.x);
    const int qt = work % nq, bh = work / nq;
    const int h = bh % H, b = bh / H;

    const bf16 *qbase = static_cast<const bf16 *>(p.q) + b * p.q_sb + h * p.q_sh;
    const bf16 *kbase = static_cast<const bf16 *>(p.k) + b * p.k_sb + h * p.k_sh;
    const bf16 *vbase = static_cast<const bf16 *>(p.v) + b * p.v_sb + h * p.v_sh;
    const uint8_t *keep = p.keep ? p.keep + (int64_t)b * S : nullptr;
    const int qi = qt * kBM + wave * 32 + n;  // this lane's query row

    // Q^T fragments (B operand): lane holds Q[qi][kd*16 + g*8 .. +8].
    bf16x8 qf[D / 16];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd)
        qf[kd] = qi < S ? as_bf16x8(ld_global_16(qbase + qi * p.q_ss + kd * 16 + g * 8))
                        : as_bf16x8(u32x4{0, 0, 0, 0});

    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const float c = p.scale_log2;

    const int nkb = (S + kBN - 1) / kBN;
    TileRegs<D> regs;
    load_tile<D>(regs, kbase, vbase, p.k_ss, p.v_ss, 0, S, tid);
    store_tile<D>(regs, smem, tid);
    __syncthreads();

    for (int kb = 0; kb < nkb; ++kb) {
        const char *stage = smem + (kb & 1) * T::STAGE;
        if (kb + 1 < nkb) load_tile<D>(regs, kbase, vbase, p.k_ss, p.v_ss, kb + 1, S, tid);

        // key-keep bits of this block (uniform over the workgroup)
        uint64_t km = ~0ull;
        const bool tail = (kb + 1) * kBN > S;
        if (keep || tail) {
            const int key = kb * kBN + lane;
            const bool kept = key < S && (!keep || keep[key]);
            km = __ballot(kept);
        }

        // S^T = K Q^T : two 32-key tiles
        f32x16 s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) s0[r] = s1[r] = 0.f;
#pragma unroll
        for (int kd = 0; kd < D / 16; ++kd) {
            const bf16x8 a0 = rm_frag<D>(stage, n, kd, g);
            const bf16x8 a1 = rm_frag<D>(stage, 32 + n, kd, g);
            s0 = mfma_32x32x16(a0, qf[kd], s0);
            s1 = mfma_32x32x16(a1, qf[kd], s1);
        }
        if (km != ~0ull) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kk = acc_row(r, lane);
                if (!((km >> kk) & 1)) s0[r] = -INFINITY;
                if (!((km >> (kk + 32)) & 1)) s1[r] = -INFINITY;
            }
        }

        // online softmax (exp2 domain; m_run in raw score units)
        float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
        mx = fmaxf(mx, xor32(mx));
        const float m_new = fmaxf(m_run, mx);
        const float m_sc = m_new == -INFINITY ? 0.f : m_new * c;
        const float alpha = exp2_fast(m_run * c - m_sc);
        m_run = m_new;
        float psum = 0.f;
        bf16x8 pf[4];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p0 = exp2_fast(s0[r] * c - m_sc);
            const float p1 = exp2_fast(s1[r] * c - m_sc);
            psum += p0 + p1;
            pf[r >> 3][r & 7] = f32_to_bf16(p0);
            pf[2 + (r >> 3)][r & 7] = f32_to_bf16(p1);
        }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;

        // O^T += V^T P^T
        const char *vt = stage + T::K_BYTES;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 a = tr_frag(vt, dt * 32 + n, ks, g);
                o[dt] = mfma_32x32x16(a, pf[ks], o[dt]);
            }

        if (kb + 1 < nkb) store_tile<D>(regs, smem + ((kb + 1) & 1) * T::STAGE, tid);
        __syncthreads();
    }

    // finalize: O = O / l, LSE = m*scale + ln(l)
    const float l_tot = l_run + xor32(l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qi < S) {
        bf16 *orow = static_cast<bf16 *>(p.o) + b * p.o_sb + h * p.o_sh + qi * p.o_ss;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                const int d = dt * 32 + grp * 8 + g * 4;
                u32x2 w;
                w[0] = pack_bf16x2(o[dt][grp * 4 + 0] * inv, o[dt][grp * 4 + 1] * inv);
                w[1] = pack_bf16x2(o[dt][grp * 4 + 2] * inv, o[dt][grp * 4 + 3] * inv);
                *reinterpret_cast<u32x2 *>(orow + d) = w;
            }
        if (g == 0)
            p.lse[((int64_t)b * H + h) * S + qi] =
                l_tot > 0.f ? m_run * p.scale + log2_fast(l_tot) * 0.6931471805599453f : -INFINITY;
    }
}

// ---------------------------------------------------------------------------
// f32 forward (FA_DTYPE_F32): exact f32 products on v_mfma_f32_32x32x2_f32,
// one wave per 32 queries, 32-key blocks.  This is the parity path for the
// reference's f32 CPU run; P stays f32 as in lib.rs:147 for f32 inputs.
// ---------------------------------------------------------------------------
constexpr int kF32BN = 32;

template <int D>
__global__ __launch_bounds__(64) void attn_fwd_f32_kernel(AttnFwdParams p) {
    __shared__ float Ks[kF32BN][D + 1];
    __shared__ float Vs[kF32BN][D];
    const int lane = threadIdx.x, n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nq = (S + 31) / 32;
    const int work = blockIdx.x;
    const int qt = work % nq, bh = work / nq;
    const int h = bh % H, b = bh / H;
    const float *qbase = static_cast<const float *>(p.q) + b * p.q_sb + h * p.q_sh;
    const float *kbase = static_cast<const float *>(p.k) + b * p.k_sb + h * p.k_sh;
    const float *vbase = static_cast<const float *>(p.v) + b * p.v_sb + h * p.v_sh;
    const uint8_t *keep = p.keep ? p.keep + (int64_t)b * S : nullptr;
    const int qi = qt * 32 + n;

    float qf[D / 2];
#pragma unroll
    for (int kd = 0; kd < D / 2; ++kd) qf[kd] = qi < S ? qbase[qi * p.q_ss + 2 * kd + g] : 0.f;
    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const float c = p.scale_log2;

    for (int kb = 0; kb * kF32BN < S; ++kb) {
        __syncthreads();
        for (int e = lane; e < kF32BN * D; e += 64) {
            const int row = e / D, d = e % D, key = kb * kF32BN + row;
            Ks[row][d] = key < S ? kbase[key * p.k_ss + d] : 0.f;
            Vs[row][d] = key < S ? vbase[key * p.v_ss + d] : 0.f;
        }
        __syncthreads();
        bool kept = false;
        if (lane < kF32BN) {
            const int key = kb * kF32BN + lane;
            kept = key < S && (!keep || keep[key]);
        }
        const uint64_t km = __ballot(kept);

        f32x16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
        for (int kd = 0; kd < D / 2; ++kd) s = mfma_32x32x2_f32(Ks[n][2 * kd + g], qf[kd], s);
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (!((km >> acc_row(r, lane)) & 1)) s[r] = -INFINITY;

        float mx = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        mx = fmaxf(mx, xor32(mx));
        const float m_new = fmaxf(m_run, mx);
        const float m_sc = m_new == -INFINITY ? 0.f : m_new * c;
        const float alpha = exp2f(m_run * c - m_sc);
        m_run = m_new;
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = exp2f(s[r] * c - m_sc);
            psum += s[r];
        }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int key = acc_row(j, lane);  // key of element j in this lane half
                o[dt] = mfma_32x32x2_f32(Vs[key][dt * 32 + n], s[j], o[dt]);
            }
        }
    }
    const float l_tot = l_run + xor32(l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qi < S) {
        float *orow = static_cast<float *>(p.o) + b * p.o_sb + h * p.o_sh + qi * p.o_ss;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) orow[dt * 32 + acc_row(r, lane)] = o[dt][r] * inv;
        if (g == 0)
            p.lse[((int64_t)b * H + h) * S + qi] =
                l_tot > 0.f ? m_run * p.scale + logf(l_tot) : -INFINITY;
    }
}

}  // namespace

hipError_t launch_attn_fwd_bf16(const AttnFwdParams &p, int D, hipStream_t s) {
    const int nq = (p.S + kBM - 1) / kBM;
    const dim3 grid(p.B * p.H * nq), block(kThreads);
    if (D == 128)
        hipLaunchKernelGGL(attn_fwd_bf16_kernel<128>, grid, block, FwdTile<128>::SMEM, s, p);
    else
        hipLaunchKernelGGL(attn_fwd_bf16_kernel<64>, grid, block, FwdTile<64>::SMEM, s, p);
    return hipGetLastError();
}

hipError_t launch_attn_fwd_f32(const AttnFwdParams &p, int D, hipStream_t s) {
    const int nq = (p.S + 31) / 32;
    const dim3 grid(p.B * p.H * nq), block(64);
    if (D == 128)
        hipLaunchKernelGGL(attn_fwd_f32_kernel<128>, grid, block, 0, s, p);
    else
        hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, grid, block, 0, s, p);
    return hipGetLastError();
}

hipError_t prepare_fwd_kernels() {
    hipError_t e = hipFuncSetAttribute((const void *)attn_fwd_bf16_kernel<128>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       FwdTile<128>::SMEM);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute((const void *)attn_fwd_bf16_kernel<64>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, FwdTile<64>::SMEM);
}

}  // namespace fa
