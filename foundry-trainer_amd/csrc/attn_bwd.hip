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
// Three launches (two when dQ does the pre-pass, see dq_block), no atomics,
// bit-identical on repeat:
//   1. delta:  D = rowsum(dO * O)                    (HBM-bound)
//   2. dk/dv:  one workgroup per NW*32 keys (NW = 4 or 8 waves x 32 keys),
//              looping over all queries in 64-query LDS stages.  S = Q K^T puts keys on the
//              accumulator's lanes, so P and dS feed the dV / dK MFMAs as A
//              operands straight from registers.
//   3. dq:     one workgroup per NW*32 queries (NW waves x 32), looping over
//              32-key LDS units.  S^T = K Q^T puts queries on the lanes, so
//              dS^T feeds dQ^T = K^T dS^T as the B operand.
// With a workspace for it (8-wave bf16 grids, p.ds), dK/dV also stores every
// bf16 dS value and dQ becomes 3': an HBM-bound dQ^T = K^T dS^T over the
// stored dS, the same products in the same key order as 3, so the same bits
// without 3's recompute of S and dP (2 of its 3G of matrix work).
// Tiles move HBM -> LDS with buffer_load ... lds (double-buffered, zero fill
// past S); every transposed operand (dO^T, Q^T, K^T) is read from the same
// row-major tile with ds_read_b64_tr_b16.  Eight-wave workgroups share each
// streamed tile between twice as many rows, halving the L2 -> LDS bytes per
// FLOP; attn_waves (attn_fwd.hip) picks the shape.
// All GEMMs run on v_mfma_f32_32x32x16_bf16 (bf16 storage) or
// v_mfma_f32_32x32x2_f32 (f32 storage) with f32 accumulation.
#include <math.h>

#include "fa_device.hpp"
#include "fa_kernels.hpp"
#include "fa_lds.hpp"

namespace fa {
namespace {

// Cache policy of the dS stores and loads: non-temporal (each byte is
// written once and read once; measured 2-4% off the backward at c2 and c5
// against the default policy).
constexpr int kDsCachePolicy = 2;

// ---------------------------------------------------------------------------
// 1. delta = rowsum(dO * O) in f32, written [B,H,S]; also lse2 = LSE*log2(e)
//    (+inf for a fully masked row, so P = exp2(s*c - lse2) = 0 there)
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
    if (row < rows && part == 0) {
        const int64_t i = ((int64_t)b * p.H + h) * p.S + s;
        p.delta[i] = acc;
        const float l = p.lse[i];
        p.lse2[i] = l == -INFINITY ? INFINITY : l * kLog2e;
    }
}

// ---------------------------------------------------------------------------
// 2. dK / dV (bf16): a workgroup owns NW*32 keys (NW waves x 32); it streams the
//    queries in 64-row stages (Q, dO, lse2, delta) straight into LDS,
//    double-buffered.  S = Q K^T and dP = dO V^T put the wave's keys on the
//    accumulator lanes, so P^T and dS^T are A operands from registers; dO^T
//    and Q^T come from the row-major tiles by transpose reads.
// ---------------------------------------------------------------------------
constexpr int kQB = 64;   // queries per LDS stage

template <int D, int NW>
struct DkvTile {
    using T = LdsTile<D, kQB>;
    static constexpr int KT = NW * 32;  // keys per workgroup
    static constexpr int Q_OFF = 0;
    static constexpr int DO_OFF = T::BYTES;
    static constexpr int LSE_OFF = 2 * T::BYTES;        // 64 f32
    static constexpr int DELTA_OFF = LSE_OFF + kQB * 4;  // 64 f32
    static constexpr int STAGE = DELTA_OFF + kQB * 4;
    static constexpr int WI = T::WAVE_INSTS / NW;
    static_assert(WI >= 1 && WI * NW == T::WAVE_INSTS, "tile split over waves");
};

// SPLIT: the workgroup streams only its partition's query blocks and leaves
// unscaled f32 partial dK, dV (the reduce pass applies the mask and scale).
// DS: also store every (key, query) element of dS for the dQ product (p.ds,
// unsplit only; zero for an excluded key or a key past S), in 1 KiB blocks
// of 32 keys (a wave's) x 16 queries: element (key, q) of block (key / 32,
// q / 16) at ((key % 32) + 32 * (q % 16 / 8)) * 16 + (q % 8) * 2, blocks
// [key / 32][q / 16] with ds_ld / 16 blocks per row.  One permlane32 swap per
// word puts 8 consecutive queries of the lane's key in each lane, so a wave
// stores a whole block with one 16-byte store per lane.
template <int D, int NW, bool SPLIT, bool DS = false>
__device__ __forceinline__ void dkdv_block(const AttnBwdParams &p, int work) {
    static_assert(!(SPLIT && DS), "dS is stored by the unsplit kernel only");
    using F = DkvTile<D, NW>;
    constexpr int kKT = F::KT;
    using T = typename F::T;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nk = (S + kKT - 1) / kKT;
    const int nqb = (S + kQB - 1) / kQB;
    const int kt = work % nk;
    int bh, qpart = 0, qb0 = 0, qb1 = nqb;  // qpart: this workgroup's query range
    if constexpr (SPLIT) {
        qpart = (work / nk) % p.split;
        bh = work / (nk * p.split);
        int c0, c1;
        split_chunks(S, p.split, qpart, c0, c1);
        constexpr int kBPC = kSplitChunk / kQB;
        qb0 = c0 * kBPC;
        qb1 = min(c1 * kBPC, nqb);
    } else {
        bh = work / nk;
    }
    const int h = bh % H, b = bh / H;

    const bf16 *qbase = static_cast<const bf16 *>(p.q) + b * p.q_sb + h * p.q_sh;
    const bf16 *kbase = static_cast<const bf16 *>(p.k) + b * p.k_sb + h * p.k_sh;
    const bf16 *vbase = static_cast<const bf16 *>(p.v) + b * p.v_sb + h * p.v_sh;
    const bf16 *dobase = static_cast<const bf16 *>(p.dout) + b * p.do_sb + h * p.do_sh;
    const int64_t row0 = ((int64_t)b * H + h) * S;
    const int kj = kt * kKT + wave * 32 + n;  // this lane's key
    // keep byte of the workgroup's key tid (loaded first; unsplit with a mask)
    const bool test_keys = !SPLIT && p.keep != nullptr;
    const int tkey = kt * kKT + tid;
    const uint32_t tkeep =
        test_keys && tid < kKT ? (uint32_t)p.keep[(int64_t)b * S + min(tkey, S - 1)] & (tkey < S ? 0xffu : 0u) : 0u;
    // dS^T rows of this head; rows past S (keys of the last tile) lie past
    // the descriptor's range and are dropped
    const int64_t ds_head = (int64_t)((S + 31) / 32) * 32 * p.ds_ld;  // elements per head
    const __amdgpu_buffer_rsrc_t dsrs = make_rsrc(DS ? static_cast<bf16 *>(p.ds) + bh * ds_head : nullptr,
                                                  DS ? (uint32_t)(ds_head * 2) : 0u);
    const uint32_t ds_row = (uint32_t)(kt * (kKT / 32) + wave) * (uint32_t)(p.ds_ld / 16);  // this wave's first block
    const bool dkeep = !DS || (kj < S && (!p.keep || p.keep[(int64_t)b * S + kj]));
    // wave-uniform: some lane of this wave has a key to zero (excluded, or past S)
    const bool ds_zero = DS && (p.keep != nullptr || kt * kKT + wave * 32 + 32 > S);

    // K and V rows of this lane's key (B operands): features kd*16 + g*8 .. +8
    bf16x8 kf[D / 16], vf[D / 16];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) {
        const bool in = kj < S;
        kf[kd] = as_bf16x8(in ? ld_global_16(kbase + kj * p.k_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
        vf[kd] = as_bf16x8(in ? ld_global_16(vbase + kj * p.v_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
    }

    // stage loads: Q and dO tiles (rows >= S read as zero), lse2 and delta
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qbase, (uint32_t)(((S - 1) * p.q_ss + D) * 2));
    const __amdgpu_buffer_rsrc_t ors = make_rsrc(dobase, (uint32_t)(((S - 1) * p.do_ss + D) * 2));
    const __amdgpu_buffer_rsrc_t lrs = make_rsrc(p.lse2 + row0, (uint32_t)(S * 4));
    const __amdgpu_buffer_rsrc_t drs = make_rsrc(p.delta + row0, (uint32_t)(S * 4));
    const uint32_t qvo = tile_src_off<D>(wave, lane, p.q_ss);
    const uint32_t ovo = tile_src_off<D>(wave, lane, p.do_ss);
    const uint32_t qi_step = tile_inst_row_step<D, NW>(p.q_ss), oi_step = tile_inst_row_step<D, NW>(p.do_ss);
    const uint32_t qstep = (uint32_t)(kQB * p.q_ss * 2), ostep = (uint32_t)(kQB * p.do_ss * 2);
    // one LDS object per stage: the compiler then keeps the prefetch DMA in
    // flight across the transpose reads of the other stage
    __shared__ __align__(16) char stage0[F::STAGE], stage1[F::STAGE];
    auto issue = [&](int qb, int buf) {
        char *st = buf ? stage1 : stage0;
#pragma unroll
        for (int i = 0; i < F::WI; ++i)
            buffer_to_lds_16(qrs, st + F::Q_OFF + (i * NW + wave) * 1024, qvo, qb * qstep + i * qi_step);
#pragma unroll
        for (int i = 0; i < F::WI; ++i)
            buffer_to_lds_16(ors, st + F::DO_OFF + (i * NW + wave) * 1024, ovo, qb * ostep + i * oi_step);
        if (wave == 0)
            buffer_to_lds_4(lrs, st + F::LSE_OFF, lane * 4, qb * kQB * 4);
        else if (wave == 1)
            buffer_to_lds_4(drs, st + F::DELTA_OFF, lane * 4, qb * kQB * 4);
    };

    // loop-invariant LDS operand offsets
    const RowFragAddr ra = row_frag_addr<D>(n, g);
    const ColFragAddr ca0 = col_frag_addr<D>(0, lane);

    f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[dt][r] = dv[dt][r] = 0.f;
    const float c = p.scale_log2;

    // A workgroup whose keys are all excluded by the mask streams no queries:
    // its dK and dV rows are stored as zero below (the unsplit kernel; a
    // split range's partials are needed by the reduce).  The first stage is
    // issued before the test, which rarely fails.
    issue(qb0, 0);
    bool live = true;
    if (test_keys) {
        live = __syncthreads_or(tkeep != 0u) != 0;
        if (!live) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the stage lands before the exit
    }
    const int qend = live ? qb1 : qb0;
    if constexpr (DS) {
        // a workgroup streaming no queries still leaves its keys' dS blocks
        // (zero) for the dQ product
        if (!live) {
            const u32x4 z = {0u, 0u, 0u, 0u};
            for (int blk = 0; blk < p.ds_ld / 16; ++blk) {
                __builtin_amdgcn_raw_buffer_store_b128(z, dsrs, (uint32_t)lane * 16, (ds_row + (uint32_t)blk) * 1024,
                                                       kDsCachePolicy);
                asm volatile("s_nop 1" ::"v"(z));  // see the stores below
            }
        }
    }
    auto stage = [&](auto par, int qb) {
        constexpr int P = decltype(par)::value;  // (qb - qb0) % 2
        // Vector memory operations complete in issue order, so with DS the
        // stage's DMA (issued before the previous stage's 4 dS stores) has
        // landed once at most 4 operations are outstanding.
        if (DS && qb != qb0)
            asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (qb + 1 < qb1) issue(qb + 1, P ^ 1);
        const char *st = P ? stage1 : stage0;
        const char *qs_t = st + F::Q_OFF, *os_t = st + F::DO_OFF;
        const float *lse_s = reinterpret_cast<const float *>(st + F::LSE_OFF);
        const float *dlt_s = reinterpret_cast<const float *>(st + F::DELTA_OFF);

#pragma unroll 1
        for (int sub = 0; sub < kQB / 32; ++sub) {
            // S = Q K^T, dP = dO V^T : 32 queries x this lane's key
            f32x16 sa, dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) sa[r] = dp[r] = 0.f;
#pragma unroll
            for (int kd = 0; kd < D / 16; ++kd) {
                const uint32_t o = row_frag_at(ra, kd) + sub * 32 * T::ROWB;
                sa = mfma_32x32x16(lds_read_row_frag(qs_t, o), kf[kd], sa);
                dp = mfma_32x32x16(lds_read_row_frag(os_t, o), vf[kd], dp);
            }
            bf16x8 pf[2], df[2];
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                // queries sub*32 + grp*8 + g*4 + 0..3 of elements r = grp*4 + 0..3
                const f32x4 l4 = *reinterpret_cast<const f32x4 *>(lse_s + sub * 32 + grp * 8 + g * 4);
                const f32x4 d4 = *reinterpret_cast<const f32x4 *>(dlt_s + sub * 32 + grp * 8 + g * 4);
                float pv[4], dsv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = grp * 4 + e;
                    pv[e] = exp2_fast(sa[r] * c - l4[e]);
                    dsv[e] = pv[e] * (dp[r] - d4[e]);
                }
                u32x2 pw, dw;
                pw[0] = pack_bf16x2(pv[0], pv[1]);
                pw[1] = pack_bf16x2(pv[2], pv[3]);
                dw[0] = pack_bf16x2(dsv[0], dsv[1]);
                dw[1] = pack_bf16x2(dsv[2], dsv[3]);
                set_half(pf[grp >> 1], grp & 1, pw);
                set_half(df[grp >> 1], grp & 1, dw);
            }
            // dV += P^T dO, dK += dS^T Q  (contraction over the 32 queries)
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const uint32_t o0 = col_frag_at(ca0, dt) + (sub * 2 + ks) * 16 * T::ROWB;
                    const uint32_t o1 = col_frag_at_hi8<D>(ca0, dt) + (sub * 2 + ks) * 16 * T::ROWB;
                    dv[dt] = mfma_32x32x16(pf[ks], lds_read_col_frag(os_t, o0, o1), dv[dt]);
                    dk[dt] = mfma_32x32x16(df[ks], lds_read_col_frag(qs_t, o0, o1), dk[dt]);
                }
            if constexpr (DS) {
                // after the last MFMA that reads df, so the swaps work in its
                // registers; df[j]: queries 16j + {4g .. 4g+3} (words 0, 1) and 16j + 8 + {4g ..} (words 2, 3);
                // after the swap lane (n, g) holds queries 16j + 8g .. +8 of key n
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const u32x4 u = as_u32x4(df[j]);
                    const auto r0 = __builtin_amdgcn_permlane32_swap(u[0], u[2], false, false);
                    const auto r1 = __builtin_amdgcn_permlane32_swap(u[1], u[3], false, false);
                    u32x4 w = u32x4{r0[0], r1[0], r0[1], r1[1]};
                    if (ds_zero && !dkeep) w = u32x4{0u, 0u, 0u, 0u};
                    __builtin_amdgcn_raw_buffer_store_b128(w, dsrs, (uint32_t)lane * 16,
                                                           (ds_row + (uint32_t)(qb * 4 + sub * 2 + j)) * 1024,
                                                           kDsCachePolicy);
                    // A VALU write to a data VGPR of a 16-byte store in the
                    // next cycle corrupted the stored first dword (measured:
                    // every dword 0 of the blocks, nondeterministically; the
                    // compiler emitted the write right after the store).
                    // Holding the data live across wait states keeps the
                    // write back.
                    asm volatile("s_nop 1" ::"v"(w));
                }
            }
        }
    };
    for (int qb = qb0; qb < qend; qb += 2) {
        stage(std::integral_constant<int, 0>{}, qb);
        if (qb + 1 < qb1) stage(std::integral_constant<int, 1>{}, qb + 1);
    }

    if constexpr (SPLIT) {
        // element r of lane: key kt*KT + wave*32 + acc_row(r), d = dt*32 + n
        const int64_t rows = (int64_t)p.B * H * S;
        float *pk = p.part_dk + (qpart * rows + (int64_t)bh * S) * D;
        float *pv = p.part_dv + (qpart * rows + (int64_t)bh * S) * D;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kt * kKT + wave * 32 + acc_row(r, lane);
            if (key < S) {
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt) {
                    pk[(int64_t)key * D + dt * 32 + n] = dk[dt][r];
                    pv[(int64_t)key * D + dt * 32 + n] = dv[dt][r];
                }
            }
        }
        return;
    }

    // accumulators: element r of lane = (key kt*KT + wave*32 + acc_row(r), d = dt*32 + n).
    // A lane's P / dS values feed only its own key's rows of dV / dK (the A
    // operand row), so an excluded key is handled here: its rows are zero
    // (selected, not multiplied: its unmasked P may have overflowed).
    bf16 *dkb = static_cast<bf16 *>(p.dk) + b * p.dk_sb + h * p.dk_sh;
    bf16 *dvb = static_cast<bf16 *>(p.dv) + b * p.dv_sb + h * p.dv_sh;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int key = kt * kKT + wave * 32 + acc_row(r, lane);
        if (key < S) {
            const bool kept = !p.keep || p.keep[(int64_t)b * S + key];
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                dkb[key * p.dk_ss + dt * 32 + n] = f32_to_bf16(kept ? dk[dt][r] * p.scale : 0.f);
                dvb[key * p.dv_ss + dt * 32 + n] = f32_to_bf16(kept ? dv[dt][r] : 0.f);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// 3. dQ (bf16): a workgroup owns NW*32 queries (NW waves x 32) and streams K/V in
//    32-key units straight into LDS, four buffers deep.  S^T = K Q^T and
//    dP^T = V dO^T put the wave's queries on the lanes; dQ^T = K^T dS^T takes
//    K^T from the row-major K tile by transpose reads.  Software pipeline per
//    unit u: the MFMAs of unit u+1's S^T / dP^T are interleaved with unit u's
//    dS^T VALU work and dQ^T MFMAs, unit u+2 is in flight and unit u+3 is
//    issued into the buffer unit u-1 just released.
// ---------------------------------------------------------------------------
constexpr int kKU = 32;   // keys per unit

template <int D, int NW>
struct DqTile {
    using T = LdsTile<D, kKU>;
    static constexpr int QT = NW * 32;              // queries per workgroup
    static constexpr int WI = T::WAVE_INSTS / NW;  // wave-instructions per wave per tile
    static_assert(WI >= 1 && WI * NW == T::WAVE_INSTS, "tile split over waves");
};

// KEEP: a key mask is given (p.keep != nullptr).  The unmasked instance has
// no per-unit loads besides the tile DMA.
// DELTA: the kernel also does the pre-pass for its own queries (delta =
// rowsum(dO * O) and lse2 from LSE, written to the workspace for dK/dV, which
// then runs after it), so the whole backward is two launches.  The row sum
// follows the pre-pass's order exactly -- sequential sums over 8-element
// parts, then an xor butterfly over the parts -- so both give the same bits.
// SPLIT: the workgroup streams only its partition's key units and leaves an
// unscaled f32 partial dQ; with DELTA, key range 0 stores the pre-pass rows.
template <int D, bool KEEP, int NW, bool DELTA, bool SPLIT>
__device__ __forceinline__ void dq_block(const AttnBwdParams &p, int work) {
    using F = DqTile<D, NW>;
    constexpr int kQT = F::QT;
    using T = typename F::T;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nq = (S + kQT - 1) / kQT;
    const int qt = work % nq;
    const int nku4 = (((S + kKU - 1) / kKU) + 3) & ~3;
    int bh, kpart = 0, u0 = 0, u1 = nku4;  // kpart: this workgroup's key range
    if constexpr (SPLIT) {
        kpart = (work / nq) % p.split;
        bh = work / (nq * p.split);
        int c0, c1;
        split_chunks(S, p.split, kpart, c0, c1);
        constexpr int kUPC = kSplitChunk / kKU;  // 4 units per chunk
        u0 = c0 * kUPC;
        u1 = c1 * kUPC;  // the last part ends at nku4
    } else {
        bh = work / nq;
    }
    const int h = bh % H, b = bh / H;

    const bf16 *qbase = static_cast<const bf16 *>(p.q) + b * p.q_sb + h * p.q_sh;
    const bf16 *kbase = static_cast<const bf16 *>(p.k) + b * p.k_sb + h * p.k_sh;
    const bf16 *vbase = static_cast<const bf16 *>(p.v) + b * p.v_sb + h * p.v_sh;
    const bf16 *dobase = static_cast<const bf16 *>(p.dout) + b * p.do_sb + h * p.do_sh;
    const uint8_t *keep = KEEP ? p.keep + (int64_t)b * S : nullptr;
    const int qi = qt * kQT + wave * 32 + n;

    // KEEP: groups of four units (128 keys) with no kept key are not
    // streamed.  Their keep bytes load first, beside the Q and dO rows.
    __shared__ uint32_t live[KEEP ? kLiveWords : 1];
    const int g1 = u1 >> 2;
    const bool track = KEEP && g1 <= kLiveWords * 32;
    constexpr int kLiveU = 64 / NW;  // groups per wave whose keep bytes load up front
    uint32_t lv[kLiveU];
    const __amdgpu_buffer_rsrc_t keep_rs = make_rsrc(keep, (uint32_t)S);
    if (track) live_mask_issue<NW, 4 * kKU, kLiveU>(keep_rs, u0 >> 2, live, lv);

    // distinct LDS objects per buffer (see attn_fwd.hip: lets the compiler
    // keep the prefetch DMA in flight across reads of the other buffers)
    __shared__ __align__(16) char k0[T::BYTES], k1[T::BYTES], k2[T::BYTES], k3[T::BYTES];
    __shared__ __align__(16) char v0[T::BYTES], v1[T::BYTES], v2[T::BYTES], v3[T::BYTES];
    auto kb_ = [&](int i) -> char * { return i == 0 ? k0 : i == 1 ? k1 : i == 2 ? k2 : k3; };
    auto vb_ = [&](int i) -> char * { return i == 0 ? v0 : i == 1 ? v1 : i == 2 ? v2 : v3; };

    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kbase, (uint32_t)(((S - 1) * p.k_ss + D) * 2));
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vbase, (uint32_t)(((S - 1) * p.v_ss + D) * 2));
    const uint32_t kvo = tile_src_off<D>(wave, lane, p.k_ss);
    const uint32_t vvo = tile_src_off<D>(wave, lane, p.v_ss);
    const uint32_t ki_step = tile_inst_row_step<D, NW>(p.k_ss), vi_step = tile_inst_row_step<D, NW>(p.v_ss);
    const uint32_t kstep = (uint32_t)(kKU * p.k_ss * 2), vstep = (uint32_t)(kKU * p.v_ss * 2);
    auto issue = [&](int u, char *kd, char *vd) {
#pragma unroll
        for (int i = 0; i < F::WI; ++i)
            buffer_to_lds_16(krs, kd + (i * NW + wave) * 1024, kvo, u * kstep + i * ki_step);
#pragma unroll
        for (int i = 0; i < F::WI; ++i)
            buffer_to_lds_16(vrs, vd + (i * NW + wave) * 1024, vvo, u * vstep + i * vi_step);
    };

    // loop-invariant LDS operand offsets
    uint32_t roff[D / 16];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) roff[kd] = row_frag_off<D>(n, kd, g);
    uint32_t coff[D / 32];  // rows +8 come from col_frag_hi8
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) coff[dt] = col_frag_off<D>(0, 0, dt, lane);

    bf16x8 qf[D / 16], of[D / 16];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) {
        const bool in = qi < S;
        qf[kd] = as_bf16x8(in ? ld_global_16(qbase + qi * p.q_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
        of[kd] = as_bf16x8(in ? ld_global_16(dobase + qi * p.do_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
    }
    float lse2 = INFINITY, dlt = 0.f;
    const int64_t qrow = ((int64_t)b * H + h) * S + qi;
    if constexpr (DELTA) {
        // part 2*kd + g = features [16 kd + 8 g, +8): this lane holds the
        // parts of one parity, its lane ^ 32 partner the others
        const bf16 *obase = static_cast<const bf16 *>(p.o) + b * p.o_sb + h * p.o_sh;
        float part[D / 16];
#pragma unroll
        for (int kd = 0; kd < D / 16; ++kd) {
            const bf16x8 ov =
                as_bf16x8(qi < S ? ld_global_16(obase + qi * p.o_ss + kd * 16 + g * 8) : u32x4{0, 0, 0, 0});
            float acc = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += (float)ov[e] * (float)of[kd][e];
            part[kd] = acc;
        }
        // butterfly: part offsets D/16 .. 2 pair parts of one lane (kd ^ m),
        // offset 1 pairs the lane with its partner
#pragma unroll
        for (int m = D / 32; m >= 1; m >>= 1) {
            float nxt[D / 16];
#pragma unroll
            for (int kd = 0; kd < D / 16; ++kd) nxt[kd] = part[kd] + part[kd ^ m];
#pragma unroll
            for (int kd = 0; kd < D / 16; ++kd) part[kd] = nxt[kd];
        }
        dlt = sum_xor32(part[0]);
        if (qi < S) {
            const float l = p.lse[qrow];
            lse2 = l == -INFINITY ? INFINITY : l * kLog2e;
            if (g == 0 && kpart == 0) {
                p.delta[qrow] = dlt;
                p.lse2[qrow] = lse2;
            }
        }
    } else if (qi < S) {
        lse2 = p.lse2[qrow];
        dlt = p.delta[qrow];
    }
    f32x16 dq[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[dt][r] = 0.f;
    const float c = p.scale_log2;

    // S^T = K Q^T and dP^T = V dO^T of one unit, MFMAs kd_lo .. kd_hi-1
    auto sdp = [&](const char *kt, const char *vt, f32x16 &sa, f32x16 &dp, int kd_lo, int kd_hi) {
#pragma unroll
        for (int kd = kd_lo; kd < kd_hi; ++kd) {
            sa = mfma_32x32x16(lds_read_row_frag(kt, roff[kd]), qf[kd], sa);
            dp = mfma_32x32x16(lds_read_row_frag(vt, roff[kd]), of[kd], dp);
        }
    };

    // Units run in groups of four (padding units lie past S: they read zeros
    // and are fully masked).  Every unit issues its prefetch and its next
    // keep-byte load unconditionally, so each unit sees the same loads in
    // flight and the only waits are the explicit ones at the barriers.
    // KEEP: ucur is the first unit of the group being processed, unext that
    // of the next live group (u1 past the last), both set in the prologue;
    // the j-th unit streamed sits in buffer j % 4.
    auto next_group = [&](int ufrom) -> int {  // first unit of the first live group at or after ufrom
        return track ? 4 * next_live_block(live, ufrom >> 2, g1) : ufrom;
    };
    int ucur = u0, unext = u0 + 4;
    // keep byte of this lane's key in unit u (clamped address; KEEP only)
    auto keep_byte = [&](int u) -> uint32_t { return KEEP ? keep[min(u * kKU + n, S - 1)] : 1u; };
    uint32_t kbyte = 1u;
    auto unit = [&](auto par, f32x16 &sc, f32x16 &dc, f32x16 &sn, f32x16 &dn) {
        constexpr int P = decltype(par)::value;  // position in the group
        const int u = ucur + P;
        const int u_after = P < 3 ? u + 1 : unext;             // the unit streamed next
        const int u_issue = P == 0 ? ucur + 3 : unext + P - 1;  // three units ahead
        // unit u+1 landed (unit u+2, 2*WI loads per wave, may still be in
        // flight, as may the keep byte issued after it); unit u-1 consumed
        barrier_keep_dma<2 * F::WI>();
        // key-keep bits of unit u, lanes 0..31 (uniform over the workgroup).
        // The byte was loaded one unit ago and has landed under the barrier's
        // wait; the empty asm keeps its use here (hoisted into the previous
        // unit, its wait would also drain the prefetch issued after it).
        if constexpr (KEEP) asm volatile("" : "+v"(kbyte));
        const int key = u * kKU + n;
        const uint64_t km = __ballot(key < S && kbyte != 0);
        kbyte = keep_byte(u_after);
        issue(u_issue, kb_((P + 3) & 3), vb_((P + 3) & 3));
        const char *kc = kb_(P), *kn = kb_((P + 1) & 3), *vn = vb_((P + 1) & 3);

#pragma unroll
        for (int r = 0; r < 16; ++r) sn[r] = dn[r] = 0.f;
        // next unit's scores (a zero or stale tile after the last unit, never
        // used) interleave with this unit's work
        sdp(kn, vn, sn, dn, 0, 2);
        if (km != ~0ull) {
            // acc_row(r, lane) = (r/4)*8 + 4*g + r%4: one lane shift, then
            // constant bit positions
            const uint32_t kb32 = (uint32_t)(km >> (4 * g));
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (!((kb32 >> ((r >> 2) * 8 + (r & 3))) & 1)) sc[r] = -INFINITY;
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bf16x8 df;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                u32x2 w;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    float d2[2];
#pragma unroll
                    for (int v = 0; v < 2; ++v) {
                        const int r = (ks * 2 + hh) * 4 + 2 * e + v;
                        const float pv = exp2_fast(sc[r] * c - lse2);
                        d2[v] = pv * (dc[r] - dlt);
                    }
                    w[e] = pack_bf16x2(d2[0], d2[1]);
                }
                set_half(df, hh, w);
            }
            sdp(kn, vn, sn, dn, 2 + ks * (D / 16 - 2) / 2, 2 + (ks + 1) * (D / 16 - 2) / 2);
            // dQ^T += K^T dS^T over this 16-key step
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
                dq[dt] = mfma_32x32x16(lds_read_col_frag(kc, coff[dt] + ks * 16 * T::ROWB,
                                                         col_frag_hi8<D>(coff, dt) + ks * 16 * T::ROWB),
                                       df, dq[dt]);
        }
    };

    // prologue: the first live group's units 0..2 issued, unit 0's scores
    // computed (a range with no live group skips everything: dQ = 0).  With
    // a tracked mask, group u0 / 4 goes out before the live groups are known
    // (it is live in most ranges), so its latency overlaps the keep bytes'.
    issue(u0, k0, v0);
    issue(u0 + 1, k1, v1);
    issue(u0 + 2, k2, v2);
    if (track) {
        barrier_keep_dma<6 * F::WI>();  // zeroed words visible; keep bytes landed
        live_mask_finish<NW, 4 * kKU, kLiveU>(keep_rs, u0 >> 2, g1, live, lv);
        barrier_keep_dma<6 * F::WI>();  // live bits visible
        ucur = next_group(u0);
        if (ucur < u1) {
            unext = next_group(ucur + 4);
            if (ucur != u0) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // group u0's units landed, then are replaced
                issue(ucur, k0, v0);
                issue(ucur + 1, k1, v1);
                issue(ucur + 2, k2, v2);
            }
        }
    }
    if (ucur >= u1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the early DMA lands before the exit
    if (ucur < u1) {
        if (KEEP) kbyte = keep_byte(ucur);
        barrier_keep_dma<0>();
        f32x16 sa0, da0, sa1, da1;
#pragma unroll
        for (int r = 0; r < 16; ++r) sa0[r] = da0[r] = 0.f;
        sdp(k0, v0, sa0, da0, 0, D / 16);
        while (ucur < u1) {
            unit(std::integral_constant<int, 0>{}, sa0, da0, sa1, da1);
            unit(std::integral_constant<int, 1>{}, sa1, da1, sa0, da0);
            unit(std::integral_constant<int, 2>{}, sa0, da0, sa1, da1);
            unit(std::integral_constant<int, 3>{}, sa1, da1, sa0, da0);
            ucur = unext;
            unext = next_group(unext + 4);
        }
        // the last prefetches are still writing LDS: they must land before
        // the workgroup can end
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    if constexpr (SPLIT) {
        if (qi < S) {
            float *row = p.part_dq + ((int64_t)kpart * p.B * H * S + (int64_t)bh * S + qi) * D;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                for (int grp = 0; grp < 4; ++grp) {
                    f32x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = dq[dt][grp * 4 + e];
                    *reinterpret_cast<f32x4 *>(row + dt * 32 + grp * 8 + g * 4) = w;
                }
        }
        return;
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
// 3'. dQ from the stored dS (p.ds): dQ^T = K^T dS^T.  A workgroup of 8 waves
//     owns 256 queries of one (b, h) and streams 64-key blocks: the K tile
//     and the dS blocks of the 64 keys x 256 queries (two runs of 16
//     contiguous 1 KiB blocks) go HBM -> LDS by DMA, three blocks deep.  Both
//     MFMA operands are transpose reads: K^T column fragments of the
//     row-major K tile, and dS^T fragments gathered from the blocks (the
//     transpose read takes any 8-byte address per lane: lane j of a 16-lane
//     group reads key +j/4, queries 4(j%4) .. +3, and receives query j's four
//     keys).  Keys past S read as zero in both.  The same products in the
//     same key order as the recomputing dQ kernel's dQ^T MFMAs.
// ---------------------------------------------------------------------------
constexpr int kDsKB = 64;  // keys per block

template <int D>
struct DqDsTile {
    using KT = LdsTile<D, kDsKB>;  // K: 64 keys x D features
    static constexpr int NW = 8;
    static constexpr int QT = 256;                     // queries per workgroup
    static constexpr int SBYTES = kDsKB * QT * 2;      // dS of a block: 32 KiB
    static constexpr int KWI = KT::WAVE_INSTS / NW;    // K wave-instructions per wave
    static constexpr int SWI = SBYTES / 1024 / NW;     // dS wave-instructions per wave
    static constexpr int LOADS = KWI + SWI;            // per wave per block
    static_assert(KWI >= 1 && KWI * NW == KT::WAVE_INSTS, "K tile split over waves");
};

template <int D>
__global__ __launch_bounds__(512) void attn_bwd_dq_ds_kernel(AttnBwdParams p) {
    using F = DqDsTile<D>;
    using KT = typename F::KT;
    constexpr int NW = F::NW;
    const int work = xcd_remap(blockIdx.x, gridDim.x);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, g = lane >> 5;
    const int S = p.S, H = p.H;
    const int nq = (S + F::QT - 1) / F::QT;
    const int qt = work % nq, bh = work / nq;
    const int h = bh % H, b = bh / H;
    const int nkb = (S + kDsKB - 1) / kDsKB;

    const bf16 *kbase = static_cast<const bf16 *>(p.k) + b * p.k_sb + h * p.k_sh;
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kbase, (uint32_t)(((S - 1) * p.k_ss + D) * 2));
    const uint32_t kvo = tile_src_off<D>(wave, lane, p.k_ss);
    const uint32_t ki_step = tile_inst_row_step<D, NW>(p.k_ss);
    const uint32_t kstep = (uint32_t)(kDsKB * p.k_ss * 2);
    // dS blocks of this head: [S / 32 key tiles][ds_ld / 16 query blocks] x 1 KiB
    const int64_t ds_head = (int64_t)((S + 31) / 32) * 32 * p.ds_ld;
    const __amdgpu_buffer_rsrc_t srs =
        make_rsrc(static_cast<const bf16 *>(p.ds) + bh * ds_head, (uint32_t)(ds_head * 2));
    const uint32_t row_blocks = (uint32_t)(p.ds_ld / 16);

    // distinct LDS objects per buffer: the compiler tells the DMA into one
    // from the reads of another
    __shared__ __align__(16) char k0[KT::BYTES], k1[KT::BYTES], k2[KT::BYTES];
    __shared__ __align__(16) char s0[F::SBYTES], s1[F::SBYTES], s2[F::SBYTES];
    auto issue = [&](int kb, char *kd, char *sd) {
#pragma unroll
        for (int i = 0; i < F::KWI; ++i)
            buffer_to_lds_16(krs, kd + (i * NW + wave) * 1024, kvo, kb * kstep + i * ki_step);
        // LDS block c = key tile c / 16 of the two, query block c % 16 of the 16
#pragma unroll
        for (int i = 0; i < F::SWI; ++i) {
            const int c = i * NW + wave;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                srs, (__attribute__((address_space(3))) void *)(sd + c * 1024), 16, (uint32_t)lane * 16,
                ((uint32_t)(2 * kb + c / 16) * row_blocks + (uint32_t)(qt * 16 + c % 16)) * 1024, 0, kDsCachePolicy);
        }
    };

    // A operand K^T: column tile dt of the K tile.  B operand dS^T for this
    // wave's 32 queries: lane j of 16-lane group G (g = G / 2, query half
    // G % 2) reads key 4g + j/4 (+8 for the second half, +16 per k-step
    // within a key tile), queries wave*32 + 16(G % 2) + 4(j % 4) .. +3.
    uint32_t ko0[D / 32], ko1[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        ko0[dt] = col_frag_off<D>(0, 0, dt, lane);
        ko1[dt] = col_frag_off<D>(0, 1, dt, lane);
    }
    const int jj = lane & 15, gg = lane >> 5, dh = (lane >> 4) & 1;
    const uint32_t so = (uint32_t)((wave * 2 + dh) * 1024 + (4 * gg + (jj >> 2) + 32 * ((jj & 3) >> 1)) * 16 +
                                   8 * (jj & 1));

    f32x16 dq[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[dt][r] = 0.f;

    // block kb in (kt, st): wait for it (block kb+1 may stay in flight), then
    // refill the buffers block kb-1 used with block kb+2 (unconditionally:
    // past the last block the tiles read as zero)
    auto stage = [&](int kb, const char *kt, const char *st, char *kn, char *sn) {
        barrier_keep_dma<F::LOADS>();
        issue(kb + 2, kn, sn);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < kDsKB / 16; ++ks) {
            // key tile ks / 2 (16 KiB apart), keys 16 (ks % 2) + 8 half
            const uint32_t o = so + (ks >> 1) * 16384 + (ks & 1) * 256;
            const bf16x8 bfr = lds_read_col_frag(st, o, o + 128);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
                dq[dt] = mfma_32x32x16(
                    lds_read_col_frag(kt, ko0[dt] + ks * 16 * KT::ROWB, ko1[dt] + ks * 16 * KT::ROWB), bfr, dq[dt]);
        }
    };
    issue(0, k0, s0);
    issue(1, k1, s1);
    // whole groups of three blocks (the padding blocks read zeros), so every
    // buffer is a compile-time LDS object
    for (int kb = 0; kb < nkb; kb += 3) {
        stage(kb, k0, s0, k2, s2);
        stage(kb + 1, k1, s1, k0, s0);
        stage(kb + 2, k2, s2, k1, s1);
    }
    // the prefetches past the last block are still writing LDS
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const int qi = qt * F::QT + wave * 32 + n;
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

// 2 waves per SIMD (<= 256 VGPRs) for either workgroup size.
template <int D, int NW, bool SPLIT, bool DS = false>
__global__ __launch_bounds__(NW * 64, 2) void attn_bwd_dkdv_bf16_kernel(AttnBwdParams p) {
    dkdv_block<D, NW, SPLIT, DS>(p, xcd_remap(blockIdx.x, gridDim.x));
}

template <int D, bool KEEP, int NW, bool DELTA, bool SPLIT>
__global__ __launch_bounds__(NW * 64, 2) void attn_bwd_dq_bf16_kernel(AttnBwdParams p) {
    dq_block<D, KEEP, NW, DELTA, SPLIT>(p, xcd_remap(blockIdx.x, gridDim.x));
}

template <int D, int NW, bool DELTA, bool SPLIT>
void launch_dq(const AttnBwdParams &p, dim3 grid, dim3 block, hipStream_t s) {
    if (p.keep)
        hipLaunchKernelGGL((attn_bwd_dq_bf16_kernel<D, true, NW, DELTA, SPLIT>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((attn_bwd_dq_bf16_kernel<D, false, NW, DELTA, SPLIT>), grid, block, 0, s, p);
}

// Sums the split partials of gradients [z0, z0 + nz) (0 dQ, 1 dK, 2 dV) in
// partition order and stores them as the unsplit kernels do: dQ and dK times
// the scale, dK and dV rows of an excluded key zero (selected: a masked key's
// partials may hold overflowed values).  One thread per 8 features of a row.
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_reduce_kernel(AttnBwdParams p, int z0) {
    constexpr int kCPR = D / 8;
    const int64_t rows = (int64_t)p.B * p.H * p.S;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * kCPR) return;
    const int z = z0 + (int)blockIdx.y;
    const int64_t row = idx / kCPR;
    const int c = (int)(idx % kCPR);
    const int S = p.S, H = p.H;
    const int s = (int)(row % S), h = (int)((row / S) % H), b = (int)(row / ((int64_t)S * H));
    const float *src = z == 0 ? p.part_dq : z == 1 ? p.part_dk : p.part_dv;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int q = 0; q < p.split; ++q) {
        const f32x4 *v = reinterpret_cast<const f32x4 *>(src + (q * rows + row) * D + c * 8);
        const f32x4 lo = v[0], hi = v[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc[e] += lo[e];
            acc[4 + e] += hi[e];
        }
    }
    const bool kept = z == 0 || !p.keep || p.keep[(int64_t)b * S + s];
    const float f = z == 2 ? 1.f : p.scale;
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        w[e] = pack_bf16x2(kept ? acc[2 * e] * f : 0.f, kept ? acc[2 * e + 1] * f : 0.f);
    bf16 *dst;
    if (z == 0)
        dst = static_cast<bf16 *>(p.dq) + b * p.dq_sb + h * p.dq_sh + s * p.dq_ss;
    else if (z == 1)
        dst = static_cast<bf16 *>(p.dk) + b * p.dk_sb + h * p.dk_sh + s * p.dk_ss;
    else
        dst = static_cast<bf16 *>(p.dv) + b * p.dv_sb + h * p.dv_sh + s * p.dv_ss;
    *reinterpret_cast<u32x4 *>(dst + c * 8) = w;
}

hipError_t launch_reduce(const AttnBwdParams &p, int D, int z0, int nz, hipStream_t s) {
    const int64_t threads = (int64_t)p.B * p.H * p.S * (D / 8);
    const dim3 grid((unsigned)((threads + 255) / 256), nz), block(256);
    if (D == 128)
        hipLaunchKernelGGL(attn_bwd_reduce_kernel<128>, grid, block, 0, s, p, z0);
    else
        hipLaunchKernelGGL(attn_bwd_reduce_kernel<64>, grid, block, 0, s, p, z0);
    return hipGetLastError();
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

// Split backward (p.split > 1, 8-wave dK/dV; dQ with 8 waves at D = 128, 4
// at D = 64), in order on one stream.  All phases: dQ partials (partition 0
// also writing the pre-pass rows), dK/dV partials, one reduce of all three.
// Phase 2 / 3 alone: the partials, then their own reduce (dK/dV and dQ use
// separate partial buffers, so they may run concurrently after the pre-pass).
hipError_t launch_attn_bwd_split(const AttnBwdParams &p, int D, int phase, hipStream_t s) {
    hipError_t e = hipSuccess;
    if (phase == 1) return D == 128 ? launch_delta<bf16, 128>(p, s) : launch_delta<bf16, 64>(p, s);
    if (phase == 0 || phase == 3) {
        const int nw_q = D == 128 ? 8 : 4;
        const dim3 grid(p.B * p.H * ((p.S + nw_q * 32 - 1) / (nw_q * 32)) * p.split), block(nw_q * 64);
        const bool delta = phase == 0;
        if (D == 128)
            delta ? launch_dq<128, 8, true, true>(p, grid, block, s) : launch_dq<128, 8, false, true>(p, grid, block, s);
        else
            delta ? launch_dq<64, 4, true, true>(p, grid, block, s) : launch_dq<64, 4, false, true>(p, grid, block, s);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (phase == 3) return launch_reduce(p, D, 0, 1, s);
    }
    const dim3 grid(p.B * p.H * ((p.S + 255) / 256) * p.split), block(512);
    if (D == 128)
        hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<128, 8, true>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<64, 8, true>), grid, block, 0, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return phase == 0 ? launch_reduce(p, D, 0, 3, s) : launch_reduce(p, D, 1, 2, s);
}

// Unsplit backward through the stored dS^T (p.ds): pre-pass, dK/dV storing
// dS^T, then dQ from it -- in this order (dQ reads what dK/dV stored).
hipError_t launch_attn_bwd_ds(const AttnBwdParams &p, int D, int phase, hipStream_t s) {
    hipError_t e = hipSuccess;
    if (phase == 0 || phase == 1) {
        e = D == 128 ? launch_delta<bf16, 128>(p, s) : launch_delta<bf16, 64>(p, s);
        if (e != hipSuccess) return e;
    }
    if (phase == 0 || phase == 2) {
        const int nw = attn_waves(p.B, p.H, p.S);
        const dim3 grid(p.B * p.H * ((p.S + nw * 32 - 1) / (nw * 32))), block(nw * 64);
        if (D == 128 && nw == 8)
            hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<128, 8, false, true>), grid, block, 0, s, p);
        else if (D == 128)
            hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<128, 4, false, true>), grid, block, 0, s, p);
        else if (nw == 8)
            hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<64, 8, false, true>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<64, 4, false, true>), grid, block, 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (phase == 0 || phase == 3) {
        const dim3 grid(p.B * p.H * ((p.S + DqDsTile<128>::QT - 1) / DqDsTile<128>::QT)), block(512);
        if (D == 128)
            hipLaunchKernelGGL(attn_bwd_dq_ds_kernel<128>, grid, block, 0, s, p);
        else
            hipLaunchKernelGGL(attn_bwd_dq_ds_kernel<64>, grid, block, 0, s, p);
        e = hipGetLastError();
    }
    return e;
}

hipError_t launch_attn_bwd_bf16(const AttnBwdParams &p, int D, int phase, hipStream_t s) {
    if (p.split > 1) return launch_attn_bwd_split(p, D, phase, s);
    if (p.ds) return launch_attn_bwd_ds(p, D, phase, s);
    // workgroup shape as for the forward (attn_waves); dQ at D = 64 streams
    // 4 KiB units, too small to split over 8 waves.
    const int nw = attn_waves(p.B, p.H, p.S);
    const int nw_q = D == 128 ? nw : 4;
    // The whole backward with 8-wave kernels runs in order on one stream:
    // dQ first, doing the pre-pass for its own queries, then dK/dV.
    const bool fused = phase == 0 && nw == 8;
    hipError_t e = hipSuccess;
    if (!fused && (phase == 0 || phase == 1)) {
        e = D == 128 ? launch_delta<bf16, 128>(p, s) : launch_delta<bf16, 64>(p, s);
        if (e != hipSuccess) return e;
    }
    auto dq = [&](bool delta) {
        const dim3 grid(p.B * p.H * ((p.S + nw_q * 32 - 1) / (nw_q * 32))), block(nw_q * 64);
        if (D == 128 && nw_q == 8)
            delta ? launch_dq<128, 8, true, false>(p, grid, block, s)
                  : launch_dq<128, 8, false, false>(p, grid, block, s);
        else if (D == 128)
            delta ? launch_dq<128, 4, true, false>(p, grid, block, s)
                  : launch_dq<128, 4, false, false>(p, grid, block, s);
        else
            delta ? launch_dq<64, 4, true, false>(p, grid, block, s) : launch_dq<64, 4, false, false>(p, grid, block, s);
        return hipGetLastError();
    };
    if (fused && (e = dq(true)) != hipSuccess) return e;
    if (phase == 0 || phase == 2) {
        const dim3 grid(p.B * p.H * ((p.S + nw * 32 - 1) / (nw * 32))), block(nw * 64);
        if (D == 128 && nw == 8)
            hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<128, 8, false>), grid, block, 0, s, p);
        else if (D == 128)
            hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<128, 4, false>), grid, block, 0, s, p);
        else if (nw == 8)
            hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<64, 8, false>), grid, block, 0, s, p);
        else
            hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<64, 4, false>), grid, block, 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (!fused && (phase == 0 || phase == 3)) e = dq(false);
    return e;
}

hipError_t launch_attn_bwd_f32(const AttnBwdParams &p, int D, int phase, hipStream_t s) {
    hipError_t e = hipSuccess;
    if (phase == 0 || phase == 1) {
        e = D == 128 ? launch_delta<float, 128>(p, s) : launch_delta<float, 64>(p, s);
        if (e != hipSuccess) return e;
    }
    const dim3 grid(p.B * p.H * ((p.S + 31) / 32)), block(64);
    if (phase == 0 || phase == 2) {
        if (D == 128)
            hipLaunchKernelGGL(attn_bwd_dkdv_f32_kernel<128>, grid, block, 0, s, p);
        else
            hipLaunchKernelGGL(attn_bwd_dkdv_f32_kernel<64>, grid, block, 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (phase == 0 || phase == 3) {
        if (D == 128)
            hipLaunchKernelGGL(attn_bwd_dq_f32_kernel<128>, grid, block, 0, s, p);
        else
            hipLaunchKernelGGL(attn_bwd_dq_f32_kernel<64>, grid, block, 0, s, p);
        e = hipGetLastError();
    }
    return e;
}

hipError_t prepare_bwd_kernels() { return hipSuccess; }  // static LDS only

}  // namespace fa
