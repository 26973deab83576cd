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
//   - O^T = V^T P^T is the second MFMA: V^T is the A operand, P^T (B operand)
//     is the S^T accumulator converted to bf16 in registers — no LDS round
//     trip for P; the row sum comes from v_dot2 over the packed P.
//   - K and V tiles are loaded straight into LDS (buffer_load ... lds, no
//     register staging), double-buffered: the next block's loads are in
//     flight while the current block computes (one barrier per block).  V^T
//     operands come from the row-major V tile through ds_read_b64_tr_b16.
//   - The running max is rescaled lazily (only when it grows by > 2^8), so
//     the O rescale leaves the inner loop.
//   - Workgroups are remapped so the 8 XCDs each take contiguous runs of
//     (b, h) query tiles and share K/V in their own L2.
#include <math.h>

#include "fa_device.hpp"
#include "fa_kernels.hpp"
#include "fa_lds.hpp"

namespace fa {
namespace {

constexpr int kBM = 128;  // queries per workgroup (4 waves x 32)
constexpr int kBN = 64;   // keys per block
constexpr int kThreads = 256;
// Lazy rescaling: the running max used as the exp2 reference only moves when
// a row's max grows by more than 2^8 in the exp2 domain, so P <= 256 and the
// O / l rescale (64 + 1 multiplies per lane) runs in a handful of blocks.
constexpr float kRescaleLog2 = 8.f;

template <int D>
struct FwdTile {
    using T = LdsTile<D, kBN>;
    static constexpr int K_OFF = 0;                  // K tile, row-major
    static constexpr int V_OFF = T::BYTES;           // V tile, row-major
    static constexpr int STAGE = 2 * T::BYTES;
    static constexpr int SMEM = 2 * STAGE;           // double buffered
    static constexpr int WI = T::WAVE_INSTS / 4;     // wave-instructions per wave per tile
};

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_bf16_kernel(AttnFwdParams p) {
    using F = FwdTile<D>;
    using T = typename F::T;
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

    // K and V tiles go straight from HBM/L2 into LDS; rows >= S read as zero
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kbase, (uint32_t)(((S - 1) * p.k_ss + D) * 2));
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vbase, (uint32_t)(((S - 1) * p.v_ss + D) * 2));
    const uint32_t kvo = tile_src_off<D>(wave, lane, p.k_ss);
    const uint32_t vvo = tile_src_off<D>(wave, lane, p.v_ss);
    const uint32_t ki_step = tile_inst_row_step<D>(p.k_ss), vi_step = tile_inst_row_step<D>(p.v_ss);
    const uint32_t kstep = (uint32_t)(kBN * p.k_ss * 2), vstep = (uint32_t)(kBN * p.v_ss * 2);
    auto issue = [&](int kb, int buf) {
        char *st = smem + buf * F::STAGE;
#pragma unroll
        for (int i = 0; i < F::WI; ++i)
            buffer_to_lds_16(krs, st + F::K_OFF + (i * 4 + wave) * 1024, kvo, kb * kstep + i * ki_step);
#pragma unroll
        for (int i = 0; i < F::WI; ++i)
            buffer_to_lds_16(vrs, st + F::V_OFF + (i * 4 + wave) * 1024, vvo, kb * vstep + i * vi_step);
    };

    // loop-invariant LDS operand offsets
    uint32_t koff[D / 16];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) koff[kd] = row_frag_off<D>(n, kd, g);
    uint32_t voff[D / 32][2];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        voff[dt][0] = col_frag_off<D>(0, 0, dt, lane);
        voff[dt][1] = col_frag_off<D>(0, 1, dt, lane);
    }

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
    float m_run = -INFINITY, m_sc = 0.f, l_run = 0.f;
    const float c = p.scale_log2;
    const bf16x2 ones = {(bf16)1.f, (bf16)1.f};

    const int nkb = (S + kBN - 1) / kBN;
    issue(0, 0);
    for (int kb = 0; kb < nkb; ++kb) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // tile kb landed for every wave; tile kb-1 fully consumed
        if (kb + 1 < nkb) issue(kb + 1, (kb + 1) & 1);
        const char *ks_t = smem + (kb & 1) * F::STAGE + F::K_OFF;
        const char *vs_t = smem + (kb & 1) * F::STAGE + F::V_OFF;

        // key-keep bits of this block (uniform over the workgroup)
        uint64_t km = ~0ull;
        if (keep || (kb + 1) * kBN > S) {
            const int key = kb * kBN + lane;
            km = __ballot(key < S && (!keep || keep[key]));
        }

        // S^T = K Q^T : two 32-key tiles
        f32x16 s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) s0[r] = s1[r] = 0.f;
#pragma unroll
        for (int kd = 0; kd < D / 16; ++kd) {
            const bf16x8 a0 = lds_read_row_frag(ks_t, koff[kd]);
            const bf16x8 a1 = lds_read_row_frag(ks_t, koff[kd] + 32 * T::ROWB);
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

        // online softmax, exp2 domain, lazily rescaled
        float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
        mx = fmaxf(mx, xor32(mx));
        const float m_new = fmaxf(m_run, mx);
        if (__any((m_new - m_run) * c > kRescaleLog2)) {
            const float m_sc_new = m_new == -INFINITY ? 0.f : m_new * c;
            const float alpha = m_run == -INFINITY ? 0.f : exp2_fast(m_sc - m_sc_new);
            m_run = m_new;
            m_sc = m_sc_new;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
        }
        bf16x8 pf[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const f32x16 &sv = (ks >> 1) ? s1 : s0;
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = (ks & 1) * 8 + 2 * e;
                const uint32_t word =
                    pack_bf16x2(exp2_fast(sv[r] * c - m_sc), exp2_fast(sv[r + 1] * c - m_sc));
                w[e] = word;
                // row sum of the bf16 P actually multiplied into O
                l_run = __builtin_amdgcn_fdot2_f32_bf16(u32_as_bf16x2(word), ones, l_run, false);
            }
            pf[ks] = as_bf16x8(w);
        }

        // O^T += V^T P^T  (V^T fragments by transpose reads of the row-major V tile)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 a = lds_read_col_frag(vs_t, voff[dt][0] + ks * 16 * T::ROWB,
                                                   voff[dt][1] + ks * 16 * T::ROWB);
                o[dt] = mfma_32x32x16(a, pf[ks], o[dt]);
            }
    }

    // finalize: O = O / l, LSE = m*scale + ln(l)   (P and l share the reference m_run)
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
