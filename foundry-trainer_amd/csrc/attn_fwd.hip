// Flash-attention forward for gfx950 (CDNA4), emitting O and the row LSE.
//
// Semantics follow foundry-spike's attn_fwd (crates/foundry-spike/src/lib.rs:
// 131-149): scores = (Q K^T) * scale in f32, softmax in f32, P cast to the
// storage dtype, O = P V with f32 accumulation.  The softmax is computed
// online (running max / sum per query row) so the (H,S,S) score tensor the
// reference materialises never exists; the natural-log row logsumexp is
// written for the backward.
//
// bf16 kernel layout (one workgroup = NW = 8 waves = 256 queries of one
// (b, h), or 4 waves = 128 queries for short sequences; all waves share each
// K/V tile, so 8 waves halve the L2 -> LDS bytes per FLOP):
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
//   - The exp2 reference (a past row max) moves only when a block's P could
//     grow large (its row sum exceeds 2^12), so the common block runs no
//     max reduction and no O rescale.
//   - Each 64-key block interleaves three independent streams: the next
//     block's scores, this block's P, and O += P V of the previous block.
//   - Workgroups are remapped so the 8 XCDs each take contiguous runs of
//     (b, h) query tiles and share K/V in their own L2.
#include <math.h>

#include <type_traits>

#include "fa_device.hpp"
#include "fa_kernels.hpp"
#include "fa_lds.hpp"

namespace fa {
namespace {

// A workgroup is NW waves x 32 queries (NW = 4 or 8) sharing each K/V tile:
// 8 waves halve the K/V bytes streamed into LDS per FLOP.
constexpr int kBN = 64;   // keys per block
// Lazy rescaling: P = exp2(s*c - m_sc) against a reference m_sc that is a
// past row max.  A block whose per-lane P sum (32 values) stays <= 2^12 has
// every P <= 2^12, far from bf16/f32 overflow, and is used as is; otherwise
// (or while a row has seen no kept key) the wave moves the reference to the
// block's row max, rescales O and l, and recomputes that block's P.  The
// common block runs no max reduction at all.
constexpr float kRescaleSum = 4096.f;

// LDS: K0, K1, V0, V1, each a row-major 64-row tile.  Iteration j reads
// K_{j+1} (for the next scores) and V_{j-1} (for the previous block's P V).
template <int D, int NW>
struct FwdTile {
    using T = LdsTile<D, kBN>;
    static constexpr int BM = NW * 32;              // queries per workgroup
    static constexpr int WI = T::WAVE_INSTS / NW;  // wave-instructions per wave per tile
    static_assert(WI >= 1 && WI * NW == T::WAVE_INSTS, "tile split over waves");
};

// Per-lane state of one query tile after a range of key blocks: the O^T
// accumulators and this lane's half of the row sum, both relative to the exp2
// reference m_sc = m_run * scale_log2 (0 while m_run = -inf).
template <int D>
struct FwdState {
    f32x16 o[D / 32];
    float m_run, m_sc, l_run;
};

// Key blocks [kb0, kb1) of query tile t (t = (b*H + h)*nq + qt).  KEEP: a
// key mask is given (p.keep); blocks with no kept key are not streamed.
template <int D, int NW, bool KEEP>
__device__ __forceinline__ void fwd_tile(const AttnFwdParams &p, int t, int kb0, int kb1, FwdState<D> &st) {
    using F = FwdTile<D, NW>;
    constexpr int kBM = F::BM;
    using T = typename F::T;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nq = (S + kBM - 1) / kBM;
    const int qt = t % nq, bh = t / nq;
    const int h = bh % H, b = bh / H;

    const bf16 *qbase = static_cast<const bf16 *>(p.q) + b * p.q_sb + h * p.q_sh;
    const bf16 *kbase = static_cast<const bf16 *>(p.k) + b * p.k_sb + h * p.k_sh;
    const bf16 *vbase = static_cast<const bf16 *>(p.v) + b * p.v_sb + h * p.v_sh;
    const uint8_t *keep = KEEP ? p.keep + (int64_t)b * S : nullptr;
    const int qi = qt * kBM + wave * 32 + n;  // this lane's query row

    // KEEP: the live 64-key blocks of [kb0, kb1) (uniform over the
    // workgroup).  The pipeline walks live blocks only: cur is the block
    // being processed, nx1 and nx2 the next two live blocks (kb1 past the
    // last); they are set in the prologue.  Without a mask every block is
    // live.  The keep-byte loads go out first, beside the Q rows.
    __shared__ uint32_t live[KEEP ? kLiveWords : 1];
    const bool track = KEEP && kb1 <= kLiveWords * 32;
    constexpr int kLiveU = 128 / NW;  // blocks per wave whose keep bytes load up front
    uint32_t lv[kLiveU];
    const __amdgpu_buffer_rsrc_t keep_rs = make_rsrc(keep, (uint32_t)S);
    if (track) live_mask_issue<NW, kBN, kLiveU>(keep_rs, kb0, live, lv);
    auto next_live = [&](int from) -> int { return track ? next_live_block(live, from, kb1) : from; };
    int cur = kb0, nx1 = kb0 + 1, nx2 = kb0 + 2;

    // K and V tiles go straight from HBM/L2 into LDS; rows >= S read as zero
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kbase, (uint32_t)(((S - 1) * p.k_ss + D) * 2));
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vbase, (uint32_t)(((S - 1) * p.v_ss + D) * 2));
    const uint32_t kvo = tile_src_off<D>(wave, lane, p.k_ss);
    const uint32_t vvo = tile_src_off<D>(wave, lane, p.v_ss);
    const uint32_t ki_step = tile_inst_row_step<D, NW>(p.k_ss), vi_step = tile_inst_row_step<D, NW>(p.v_ss);
    const uint32_t kstep = (uint32_t)(kBN * p.k_ss * 2), vstep = (uint32_t)(kBN * p.v_ss * 2);
    // The four stage buffers are distinct LDS objects: the compiler can then
    // tell a read of one stage from the DMA still filling another and emits no
    // wait for the prefetch (one shared buffer makes it drain the prefetch
    // before every transpose read).
    __shared__ __align__(16) char ks0[T::BYTES], ks1[T::BYTES], vs0[T::BYTES], vs1[T::BYTES];
    auto issue_k = [&](int kb, char *dst) {
#pragma unroll
        for (int i = 0; i < F::WI; ++i)
            buffer_to_lds_16(krs, dst + (i * NW + wave) * 1024, kvo, kb * kstep + i * ki_step);
    };
    auto issue_v = [&](int kb, char *dst) {
#pragma unroll
        for (int i = 0; i < F::WI; ++i)
            buffer_to_lds_16(vrs, dst + (i * NW + wave) * 1024, vvo, kb * vstep + i * vi_step);
    };

    // loop-invariant LDS operand offsets
    uint32_t koff[D / 16];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) koff[kd] = row_frag_off<D>(n, kd, g);
    uint32_t voff[D / 32];  // rows +8 come from col_frag_hi8
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) voff[dt] = col_frag_off<D>(0, 0, dt, lane);

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

    // S^T = K Q^T for a 64-key tile: MFMAs kd_lo .. kd_hi-1 of the 2 x D/16.
    auto qk_part = [&](const char *kt, f32x16 &s0, f32x16 &s1, int kd_lo, int kd_hi) {
#pragma unroll
        for (int kd = kd_lo; kd < kd_hi; ++kd) {
            const bf16x8 a0 = lds_read_row_frag(kt, koff[kd]);
            const bf16x8 a1 = lds_read_row_frag(kt, koff[kd] + 32 * T::ROWB);
            s0 = mfma_32x32x16(a0, qf[kd], s0);
            s1 = mfma_32x32x16(a1, qf[kd], s1);
        }
    };

    // P of block kb against the current reference m_sc: 32 scores per lane
    // -> 16 packed bf16 words, and the lane's row sum of the bf16 P actually
    // multiplied into O.  Slice ks (16 keys) is pw[ks].
    auto make_p = [&](const f32x16 &c0, const f32x16 &c1, u32x4 (&pw)[4], float &lp, int ks) {
        const f32x16 &sv = (ks >> 1) ? c1 : c0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = (ks & 1) * 8 + 2 * e;
            const uint32_t word = pack_bf16x2(exp2_fast(sv[r] * c - m_sc), exp2_fast(sv[r + 1] * c - m_sc));
            pw[ks][e] = word;
            lp = __builtin_amdgcn_fdot2_f32_bf16(u32_as_bf16x2(word), ones, lp, false);
        }
    };
    // Move the reference to the row max of block kb's scores (rare path):
    // O and l, accumulated under the old reference, are rescaled to it.
    auto move_reference = [&](const f32x16 &c0, const f32x16 &c1) {
        float mx = fmaxf(c0[0], c1[0]);
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(c0[r], c1[r]));
        mx = max_xor32(mx);
        const float m_new = fmaxf(m_run, mx);
        const float m_sc_new = m_new == -INFINITY ? 0.f : m_new * c;
        const float alpha = m_run == -INFINITY ? 0.f : exp2_fast(m_sc - m_sc_new);
        m_run = m_new;
        m_sc = m_sc_new;
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
    };
    // O^T += V^T P^T for one 16-key slice of a block's P (V^T fragments by
    // transpose reads of the row-major V tile).
    auto pv_slice = [&](const char *vt, const u32x4 &w, int ks) {
        const bf16x8 pf = as_bf16x8(w);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
            const bf16x8 a = lds_read_col_frag(vt, voff[dt] + ks * 16 * T::ROWB,
                                               col_frag_hi8<D>(voff, dt) + ks * 16 * T::ROWB);
            o[dt] = mfma_32x32x16(a, pf, o[dt]);
        }
    };

    // Keep byte of this lane's key in block kb, loaded one block ahead so its
    // latency hides behind a block of work: with one 8-wave workgroup per CU,
    // a load right after the barrier would stall every wave of the CU at once.
    auto keep_byte = [&](int kb) -> uint32_t { return KEEP ? keep[min(kb * kBN + lane, S - 1)] : 1u; };
    uint32_t kbyte = 1u;

    // One key block (cur), a three-stage software pipeline with no dependency
    // inside the block: the scores of block nx1 (MFMA), P of block cur (VALU,
    // from scores computed one block earlier) and O += P V for the previous
    // block (MFMA, with P kept in registers from the previous block) are
    // interleaved slice by slice.  The reference check closes the block, so
    // its body is one straight-line region.  The j-th block streamed has K in
    // ks[j%2] and V in vs[j%2]; PAR = j % 2 makes every LDS stage offset an
    // immediate.  FIRST (j == 0) has no previous block.  The block ends by
    // advancing cur, nx1, nx2 to the next live blocks.
    auto block = [&](auto par, auto first, f32x16 &c0, f32x16 &c1, f32x16 &n0, f32x16 &n1, u32x4 (&pw)[4]) {
        constexpr int P = decltype(par)::value;
        constexpr bool FIRST = decltype(first)::value;
        const int kb = cur;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // K_{kb+1}, V_{kb-1} landed; K_kb and V_{kb-2} fully consumed
        const char *kn = P ? ks0 : ks1;  // K_{kb+1}
        const char *vp = P ? vs0 : vs1;  // V_{kb-1}

        // key-keep bits of block kb (uniform over the workgroup).  The byte
        // was loaded one block ago and has landed under the wait above; the
        // empty asm keeps its use here (hoisted into the previous block, its
        // wait would also drain the DMA issued after the load).
        uint64_t km = ~0ull;
        if (KEEP || (kb + 1) * kBN > S) {
            if (KEEP) asm volatile("" : "+v"(kbyte));
            const int key = kb * kBN + lane;
            km = __ballot(key < S && kbyte != 0);
        }
        if (KEEP && nx1 < kb1) kbyte = keep_byte(nx1);
#pragma unroll
        for (int r = 0; r < 16; ++r) n0[r] = n1[r] = 0.f;
        if (km != ~0ull) {
            // acc_row(r, lane) = (r/4)*8 + 4*g + r%4: one lane-dependent shift,
            // then constant bit positions
            const uint32_t k0 = (uint32_t)(km >> (4 * g)), k1 = (uint32_t)(km >> (32 + 4 * g));
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kk = (r >> 2) * 8 + (r & 3);
                if (!((k0 >> kk) & 1)) c0[r] = -INFINITY;
                if (!((k1 >> kk) & 1)) c1[r] = -INFINITY;
            }
        }
        if (FIRST) move_reference(c0, c1);
        u32x4 prev[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) prev[ks] = pw[ks];
        float lp = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            // The DMA for K_{kb+2} and V_kb goes out after the first and the
            // second slice rather than in one burst at the barrier, where it
            // met every wave's first LDS reads (1% off the forward); both
            // buffers are free from the barrier on, and are read next block.
            if (ks == 1 && nx2 < kb1) issue_k(nx2, P ? ks1 : ks0);
            if (ks == 2) issue_v(kb, P ? vs1 : vs0);
            make_p(c0, c1, pw, lp, ks);
            // The last block computes scores of a stale K tile that are never
            // used: keeping the MFMAs unconditional keeps them interleavable.
            qk_part(kn, n0, n1, ks * (D / 16) / 4, (ks + 1) * (D / 16) / 4);
            if (!FIRST) pv_slice(vp, prev[ks], ks);
        }
        // Every P <= 2^12 when the lane's block sum is (P >= 0); a row with
        // no kept key so far (m_run = -inf) has no reference yet.
        if (!FIRST && __any(m_run == -INFINITY || !(lp <= kRescaleSum))) {
            move_reference(c0, c1);
            lp = 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) make_p(c0, c1, pw, lp, ks);
        }
        l_run += lp;
        cur = nx1;
        nx1 = nx2;
        nx2 = next_live(nx2 + 1);
    };

    // prologue: K of the first live block -> its scores; the next live
    // block's K in flight.  With a tracked mask, K of block kb0 goes out
    // before the live blocks are known (kb0 is live in most ranges), so its
    // latency overlaps the keep bytes'.
    f32x16 sa0, sa1, sb0, sb1;
    u32x4 pw[4];
    if (track) {
        issue_k(kb0, ks0);
        barrier_keep_dma<F::WI>();  // zeroed words visible; keep bytes and Q rows landed
        live_mask_finish<NW, kBN, kLiveU>(keep_rs, kb0, kb1, live, lv);
        barrier_keep_dma<F::WI>();  // live bits visible
        cur = next_live(kb0);
        if (cur >= kb1) {  // no kept key in the range: O = 0, LSE = -inf
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the early DMA lands before the exit
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) st.o[dt][r] = 0.f;
            st.m_run = -INFINITY;
            st.m_sc = 0.f;
            st.l_run = 0.f;
            return;
        }
        nx1 = next_live(cur + 1);
        nx2 = next_live(nx1 + 1);
        if (cur != kb0) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // block kb0's tile landed, then is replaced
            issue_k(cur, ks0);
        }
    } else {
        issue_k(cur, ks0);
    }
    if (KEEP) kbyte = keep_byte(cur);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (nx1 < kb1) issue_k(nx1, ks1);
#pragma unroll
    for (int r = 0; r < 16; ++r) sa0[r] = sa1[r] = 0.f;
    qk_part(ks0, sa0, sa1, 0, D / 16);
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    int nblk = 1;  // blocks streamed (KEEP; otherwise kb1 - kb0)
    block(I0{}, std::true_type{}, sa0, sa1, sb0, sb1, pw);
    while (cur < kb1) {
        block(I1{}, std::false_type{}, sb0, sb1, sa0, sa1, pw);
        ++nblk;
        if (cur < kb1) {
            block(I0{}, std::false_type{}, sa0, sa1, sb0, sb1, pw);
            ++nblk;
        }
    }
    // epilogue: O += P V for the last block, whose V that block issued
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    {
        const int last = KEEP ? nblk - 1 : kb1 - 1 - kb0;
        const char *vl = (last & 1) ? vs1 : vs0;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) pv_slice(vl, pw[ks], ks);
    }
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) st.o[dt] = o[dt];
    st.m_run = m_run;
    st.m_sc = m_sc;
    st.l_run = l_run;

}

// O = O / l and LSE = (m_sc + log2 l) * ln 2 for query tile t.
template <int D, int NW>
__device__ __forceinline__ void fwd_store(const AttnFwdParams &p, int t, const FwdState<D> &st) {
    constexpr int kBM = FwdTile<D, NW>::BM;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nq = (S + kBM - 1) / kBM;
    const int qt = t % nq, bh = t / nq;
    const int h = bh % H, b = bh / H;
    const int qi = qt * kBM + wave * 32 + n;
    const float l_tot = sum_xor32(st.l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qi < S) {
        bf16 *orow = static_cast<bf16 *>(p.o) + b * p.o_sb + h * p.o_sh + qi * p.o_ss;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                const int d = dt * 32 + grp * 8 + g * 4;
                u32x2 w;
                w[0] = pack_bf16x2(st.o[dt][grp * 4 + 0] * inv, st.o[dt][grp * 4 + 1] * inv);
                w[1] = pack_bf16x2(st.o[dt][grp * 4 + 2] * inv, st.o[dt][grp * 4 + 3] * inv);
                *reinterpret_cast<u32x2 *>(orow + d) = w;
            }
        if (g == 0)
            p.lse[((int64_t)b * H + h) * S + qi] =
                l_tot > 0.f ? (st.m_sc + log2_fast(l_tot)) * 0.6931471805599453f : -INFINITY;
    }
}

// Split partial of query tile t over one key range: O / l in f32 and the
// range's natural-log LSE (-inf when none of its keys is kept).
template <int D, int NW>
__device__ __forceinline__ void fwd_store_part(const AttnFwdParams &p, int t, int part, const FwdState<D> &st) {
    constexpr int kBM = FwdTile<D, NW>::BM;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S;
    const int nq = (S + kBM - 1) / kBM;
    const int qt = t % nq, bh = t / nq;
    const int qi = qt * kBM + wave * 32 + n;
    const float l_tot = sum_xor32(st.l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qi < S) {
        const int64_t row = ((int64_t)part * p.B * p.H + bh) * S + qi;
        float *orow = p.part_o + row * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = st.o[dt][grp * 4 + e] * inv;
                *reinterpret_cast<f32x4 *>(orow + dt * 32 + grp * 8 + g * 4) = w;
            }
        if (g == 0)
            p.part_lse[row] = l_tot > 0.f ? (st.m_sc + log2_fast(l_tot)) * 0.6931471805599453f : -INFINITY;
    }
}

// One workgroup per NW*32-query tile; 2 waves per SIMD (<= 256 VGPRs).
// SPLIT: p.split workgroups per tile, each over one key range.  KEEP: a key
// mask is given.
template <int D, int NW, bool SPLIT, bool KEEP>
__global__ __launch_bounds__(NW * 64, 2) void attn_fwd_bf16_kernel(AttnFwdParams p) {
    const int nkb = (p.S + kBN - 1) / kBN;
    const int w = xcd_remap(blockIdx.x, gridDim.x);
    FwdState<D> st;
    if constexpr (SPLIT) {
        constexpr int kBM = FwdTile<D, NW>::BM;
        const int nq = (p.S + kBM - 1) / kBM;
        const int qt = w % nq, part = (w / nq) % p.split, bh = w / (nq * p.split);
        int c0, c1;
        split_chunks(p.S, p.split, part, c0, c1);
        constexpr int kBPC = kSplitChunk / kBN;  // key blocks per chunk
        const int t = bh * nq + qt;
        fwd_tile<D, NW, KEEP>(p, t, c0 * kBPC, min(c1 * kBPC, nkb), st);
        fwd_store_part<D, NW>(p, t, part, st);
    } else {
        fwd_tile<D, NW, KEEP>(p, w, 0, nkb, st);
        fwd_store<D, NW>(p, w, st);
    }
}

// Combines the split partials of each query row through their LSEs:
// LSE = log sum_p exp(LSE_p), O = sum_p exp(LSE_p - LSE) O_p, summed in
// partition order.  One thread per 8 features of a row.
template <int D>
__global__ __launch_bounds__(256) void attn_fwd_combine_kernel(AttnFwdParams p) {
    constexpr int kCPR = D / 8;  // threads per row
    const int64_t rows = (int64_t)p.B * p.H * p.S;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * kCPR) return;
    const int64_t row = idx / kCPR;
    const int c = (int)(idx % kCPR);
    const int S = p.S, H = p.H;
    const int s = (int)(row % S), h = (int)((row / S) % H), b = (int)(row / ((int64_t)S * H));
    float m = -INFINITY;
    for (int q = 0; q < p.split; ++q) m = fmaxf(m, p.part_lse[q * rows + row]);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float lse = -INFINITY;
    if (m != -INFINITY) {
        float den = 0.f;
        for (int q = 0; q < p.split; ++q) {
            const float wq = expf(p.part_lse[q * rows + row] - m);
            den += wq;
            const f32x4 *src = reinterpret_cast<const f32x4 *>(p.part_o + (q * rows + row) * D + c * 8);
            const f32x4 lo = src[0], hi = src[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[e] += wq * lo[e];
                acc[4 + e] += wq * hi[e];
            }
        }
        const float inv = 1.f / den;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= inv;
        lse = m + logf(den);
    }
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(acc[2 * e], acc[2 * e + 1]);
    bf16 *orow = static_cast<bf16 *>(p.o) + b * p.o_sb + h * p.o_sh + s * p.o_ss;
    *reinterpret_cast<u32x4 *>(orow + c * 8) = w;
    if (c == 0) p.lse[row] = lse;
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

// Workgroup shape, shared by the forward and backward bf16 kernels.  An
// 8-wave workgroup fills a CU's registers alone (2 waves per SIMD), so its
// grid runs in whole-CU rounds; 4-wave workgroups pair up per CU, and in a
// sparse last round run alone at higher speed.  8 waves halve the streamed
// L2 -> LDS bytes per FLOP but only pay when the 8-wave grid's last round is
// at least half full: measured on MI355X, c2 (B1 H24 S4608: last round 69%
// full) +3.6% and c5 (B2 S6656: 88%) +3% fwd+bwd, c3 (B4 S1536: 25%) -13%.
// CU count of the current device (cached per device; 256 if unknown).
int device_cu_count() {
    static int cus[64];
    int dev = 0;
    int n = 256;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
        int c = __atomic_load_n(&cus[dev], __ATOMIC_RELAXED);
        if (c == 0 && hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            c > 0)
            __atomic_store_n(&cus[dev], c, __ATOMIC_RELAXED);
        if (c > 0) n = c;
    }
    return n;
}

int attn_waves(int B, int H, int S) {
    if (S < 512) return 4;  // fewer than two 256-row tiles per (b, h)
    if (attn_split(B, H, S) > 1) return 8;
    const int n = device_cu_count();
    const int64_t wg = (int64_t)B * H * ((S + 255) / 256);
    const int64_t last = wg % n == 0 ? n : wg % n;
    return 2 * last >= n ? 8 : 4;
}

// Range split for grids that leave most CUs idle: with at most half the CUs
// busy even at 8 waves (B*H*ceil(S/256) <= CUs/2, e.g. 3 or 6 heads at
// S = 4608, one GPU's share of 24 heads over 8 or 4 GPUs), each tile's key
// range (forward, dQ) or query range (dK/dV) is cut into `split` parts of at
// least 512 rows, so the grid grows to about one workgroup per CU.  The
// partials cost an f32 write and read of split x O (or of each gradient).
int attn_split(int B, int H, int S) {
    if (S < 1024) return 1;
    const int n = device_cu_count();
    const int64_t wg = (int64_t)B * H * ((S + 255) / 256);
    if (2 * wg > n) return 1;
    const int nc = (S + kSplitChunk - 1) / kSplitChunk;
    int64_t split = n / wg;
    split = split < nc / 4 ? split : nc / 4;  // >= 4 chunks (512 rows) per part
    split = split < 16 ? split : 16;
    return split > 1 ? (int)split : 1;
}

size_t attn_split_elems(int B, int H, int S, int D, int split) {
    return split > 1 ? (size_t)split * B * H * S * D : 0;
}

// p.split > 1 (set by the caller from attn_split, with the partial buffers):
// 8-wave split grid, then the combine pass.
hipError_t launch_attn_fwd_bf16(const AttnFwdParams &p, int D, hipStream_t s) {
    if (p.split > 1) {
        const int nq = (p.S + 255) / 256;
        const dim3 grid(p.B * p.H * nq * p.split), block(512);
        if (D == 128 && p.keep)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<128, 8, true, true>), grid, block, 0, s, p);
        else if (D == 128)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<128, 8, true, false>), grid, block, 0, s, p);
        else if (p.keep)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<64, 8, true, true>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<64, 8, true, false>), grid, block, 0, s, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t threads = (int64_t)p.B * p.H * p.S * (D / 8);
        const dim3 cgrid((unsigned)((threads + 255) / 256)), cblock(256);
        if (D == 128)
            hipLaunchKernelGGL(attn_fwd_combine_kernel<128>, cgrid, cblock, 0, s, p);
        else
            hipLaunchKernelGGL(attn_fwd_combine_kernel<64>, cgrid, cblock, 0, s, p);
        return hipGetLastError();
    }
    const int nw = attn_waves(p.B, p.H, p.S);
    const int bm = nw * 32;
    const int nq = (p.S + bm - 1) / bm;
    const dim3 grid(p.B * p.H * nq), block(nw * 64);
    if (p.keep) {
        if (D == 128 && nw == 8)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<128, 8, false, true>), grid, block, 0, s, p);
        else if (D == 128)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<128, 4, false, true>), grid, block, 0, s, p);
        else if (nw == 8)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<64, 8, false, true>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<64, 4, false, true>), grid, block, 0, s, p);
    } else {
        if (D == 128 && nw == 8)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<128, 8, false, false>), grid, block, 0, s, p);
        else if (D == 128)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<128, 4, false, false>), grid, block, 0, s, p);
        else if (nw == 8)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<64, 8, false, false>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<64, 4, false, false>), grid, block, 0, s, p);
    }
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

hipError_t prepare_fwd_kernels() { return hipSuccess; }  // static LDS only

}  // namespace fa
