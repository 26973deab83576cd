// bf16 GEMM for gfx950 with fused epilogues: the frozen linears of the c4
// block's MLP (foundry-spike's linear_scaled base product, lib.rs:270-287,
// applied at throughput.rs:254-256) and the elementwise op that follows them.
//
//   C[M, N] = A[M, K] B[N, K]^T     (x W^T: both operands K-contiguous)
//
// Epilogues (the accumulator is rounded to the storage type first, the
// reference's cast point for a bf16 matmul):
//   NONE   c = T(acc)
//   GELU   c = pre = T(acc), c2 = T(gelu(pre))           (W1 forward + GELU)
//   DGELU  c = T(T(acc) * gelu'(aux))                    (dX of W2, times the
//                                                         GELU derivative at
//                                                         the saved pre)
// gelu is the tanh form, evaluated as the elementwise kernels do.
//
// Layout: a workgroup of 8 waves computes a 256 x 256 tile, each wave a
// 128 x 64 part as 4 x 2 accumulators of v_mfma_f32_32x32x16_bf16 (128 f32
// per lane, in VGPRs: two waves per SIMD, so that one wave's MFMAs cover the
// other's LDS reads).  K runs in 64-wide
// stages: the 256 x 64 A and B tiles go HBM/L2 -> LDS by buffer_load ... lds
// (double-buffered, distinct LDS objects per stage, chunk-swizzled rows), and
// every MFMA operand is a row fragment (ds_read_b128).  The MFMA computes
// C^T tiles (W rows as the A operand), so each lane ends up holding 4
// consecutive outputs of one row per accumulator group: 8-byte stores.
// Workgroups are ordered so that each XCD owns a band of N tiles: the W tiles
// of a band are read by all M tiles on one XCD's L2.
#include <math.h>

#include "fa_device.hpp"
#include "fa_kernels.hpp"
#include "fa_lds.hpp"

namespace fa {
namespace {

constexpr int kGM = 256, kGN = 256;
constexpr int kGW = 8;  // waves per workgroup (2 along M x 4 along N)

constexpr float kGeluK0 = 0.7978845608028654f;  // sqrt(2/pi)
constexpr float kGeluK1 = 0.044715f;
// sigmoid(2 k0 (u + k1 u^3)): gelu(u) = u * s, gelu'(u) = s + 2 u s (1 - s) k0 (1 + 3 k1 u^2)
__device__ __forceinline__ float gelu_sig(float u) {
    const float z2 = (2.f * kGeluK0) * (u + kGeluK1 * u * u * u);
    return __builtin_amdgcn_rcpf(1.f + exp2_fast(-kLog2e * z2));
}
__device__ __forceinline__ float gelu_grad(float u) {
    const float sg = gelu_sig(u);
    return sg + (2.f * kGeluK0) * u * (sg - sg * sg) * (1.f + (3.f * kGeluK1) * u * u);
}

constexpr int kGK = 64;                        // K columns per LDS stage
using GTile = LdsTile<kGK, 256>;               // 256 rows x 64 k, 32 KiB
constexpr int kGWI = GTile::WAVE_INSTS / kGW;  // DMA wave-instructions per wave per operand

template <int EPI>
__global__ __launch_bounds__(kGW * 64, 2) void gemm_tn_bf16_kernel(GemmParams p) {
    // one LDS object per stage and operand: the compiler then tells a DMA
    // destination from the reads of the other stage
    __shared__ __align__(16) char a0[GTile::BYTES], a1[GTile::BYTES];
    __shared__ __align__(16) char b0[GTile::BYTES], b1[GTile::BYTES];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, g = lane >> 5;
    const int MT = p.M / kGM, NT = p.N / kGN;
    const int w = xcd_remap(blockIdx.x, gridDim.x);
    // bands of group_m M tiles; within a band the M tile runs fastest
    const int band = w / (p.group_m * NT), m0 = band * p.group_m;
    const int gsz = min(p.group_m, MT - m0), wb = w - band * p.group_m * NT;
    const int mt = m0 + wb % gsz, nt = wb / gsz;
    const int wm = wave & 1, wn = wave >> 1;  // the wave's part: rows wm*128 .. +128, cols wn*64 .. +64

    const bf16 *abase = static_cast<const bf16 *>(p.a) + (int64_t)mt * kGM * p.lda;
    const bf16 *bbase = static_cast<const bf16 *>(p.b) + (int64_t)nt * kGN * p.ldb;
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(abase, (uint32_t)((kGM - 1) * p.lda * 2 + p.K * 2));
    const __amdgpu_buffer_rsrc_t brs = make_rsrc(bbase, (uint32_t)((kGN - 1) * p.ldb * 2 + p.K * 2));
    const uint32_t avo = tile_src_off<kGK>(wave, lane, p.lda), bvo = tile_src_off<kGK>(wave, lane, p.ldb);
    const uint32_t a_step = tile_inst_row_step<kGK, kGW>(p.lda), b_step = tile_inst_row_step<kGK, kGW>(p.ldb);
    auto issue = [&](int kt, char *ad, char *bd) {
#pragma unroll
        for (int i = 0; i < kGWI; ++i)
            buffer_to_lds_16(ars, ad + (i * kGW + wave) * 1024, avo, kt * kGK * 2 + i * a_step);
#pragma unroll
        for (int i = 0; i < kGWI; ++i)
            buffer_to_lds_16(brs, bd + (i * kGW + wave) * 1024, bvo, kt * kGK * 2 + i * b_step);
    };

    // Row fragments: A rows wm*128 + i*32 + n, B rows wn*64 + j*32 + n.  The
    // chunk swizzle repeats every 16 rows, so every i (j) shares one key.
    const RowFragAddr fa_ = row_frag_addr<kGK>(wm * 128 + n, g);
    const RowFragAddr fb_ = row_frag_addr<kGK>(wn * 64 + n, g);

    f32x16 acc[2][4];  // acc[j][i]: C^T tile (B rows j, A rows i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

    // One K stage kt, held in (as, bs).  Stage kt+1 goes into the other
    // buffers right after the barrier (every wave is then done with stage
    // kt-1) and unconditionally: past the last stage it reads in-range
    // columns or zeros that are never used.  The scheduling barrier keeps
    // the issue there: left to the scheduler it sinks below the MFMAs, and a
    // conditional issue made the compiler wait for it before the first LDS
    // read.
    auto stage = [&](int kt, const char *as, const char *bs, char *an, char *bn) {
        barrier_keep_dma<0>();  // stage kt landed; stage kt-1 fully read
        issue(kt + 1, an, bn);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < kGK / 16; ++ks) {
            bf16x8 af[4], bfr[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = lds_read_row_frag(as, row_frag_at(fa_, ks) + i * 32 * GTile::ROWB);
#pragma unroll
            for (int j = 0; j < 2; ++j) bfr[j] = lds_read_row_frag(bs, row_frag_at(fb_, ks) + j * 32 * GTile::ROWB);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][i] = mfma_32x32x16(bfr[j], af[i], acc[j][i]);
        }
    };
    // K / 64 stages: whole pairs in the loop, with no condition inside it
    // (the compiler's wait-count analysis merges the paths around a skipped
    // stage and then waits for a prefetch that may stay in flight), and an
    // odd last stage after it.
    const int nk = p.K / kGK;
    issue(0, a0, b0);
    for (int kt = 0; kt + 1 < nk; kt += 2) {
        stage(kt, a0, b0, a1, b1);
        stage(kt + 1, a1, b1, a0, b0);
    }
    if (nk & 1) stage(nk - 1, a0, b0, a1, b1);
    // the prefetch past the last stage is still writing LDS: it must land
    // before the workgroup can end
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // acc[j][i] element r of lane: C[m][c], m = mt*256 + wm*128 + i*32 + n,
    // c = nt*256 + wn*64 + j*32 + (r/4)*8 + 4g + r%4: 4 consecutive columns
    // per group r/4.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = (int64_t)mt * kGM + wm * 128 + i * 32 + n;
        bf16 *crow = static_cast<bf16 *>(p.c) + m * p.ldc;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = nt * kGN + wn * 64 + j * 32 + q * 8 + 4 * g;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = (float)(bf16)acc[j][i][q * 4 + e];  // T(acc)
                if constexpr (EPI == kGemmDgelu) {
                    const u32x2 pu = *reinterpret_cast<const u32x2 *>(static_cast<const bf16 *>(p.aux) +
                                                                      m * p.ldaux + c);
                    const bf16x4 pre = __builtin_bit_cast(bf16x4, pu);
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] *= gelu_grad((float)pre[e]);
                }
                u32x2 out;
                out[0] = pack_bf16x2(v[0], v[1]);
                out[1] = pack_bf16x2(v[2], v[3]);
                *reinterpret_cast<u32x2 *>(crow + c) = out;
                if constexpr (EPI == kGemmGelu) {
                    u32x2 act;
                    act[0] = pack_bf16x2(v[0] * gelu_sig(v[0]), v[1] * gelu_sig(v[1]));
                    act[1] = pack_bf16x2(v[2] * gelu_sig(v[2]), v[3] * gelu_sig(v[3]));
                    *reinterpret_cast<u32x2 *>(static_cast<bf16 *>(p.c2) + m * p.ldc2 + c) = act;
                }
            }
    }
}

}  // namespace

// Tile order: bands of 8 M tiles, so that the 32 workgroups an XCD runs at
// once cover 8 M x 4 N tiles (12 distinct 256-row panels) rather than a
// whole M column of tiles; at 8192^3 this took the kernel from 1.37 to
// 0.94 ms, at the c4 shapes it is neutral.
constexpr int kGroupM = 8;

hipError_t launch_gemm_tn_bf16(const GemmParams &p0, hipStream_t s) {
    GemmParams p = p0;
    p.group_m = min(kGroupM, p.M / kGM);
    const dim3 grid((p.M / kGM) * (p.N / kGN)), block(kGW * 64);
    if (p.epi == kGemmGelu)
        hipLaunchKernelGGL(gemm_tn_bf16_kernel<kGemmGelu>, grid, block, 0, s, p);
    else if (p.epi == kGemmDgelu)
        hipLaunchKernelGGL(gemm_tn_bf16_kernel<kGemmDgelu>, grid, block, 0, s, p);
    else
        hipLaunchKernelGGL(gemm_tn_bf16_kernel<kGemmNone>, grid, block, 0, s, p);
    return hipGetLastError();
}

}  // namespace fa
