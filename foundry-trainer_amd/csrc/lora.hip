// LoRA down/up kernels for gfx950 — the adapter term of foundry-spike's
// linear_scaled (crates/foundry-spike/src/lib.rs:270-287):
//     y = x W^T (+ b) + scale * (x A^T) B^T,   A [r, K], B [M, r]
// The base GEMM x W^T is the caller's; these kernels add the rank-r term and
// produce its gradients.
//
//   rowdot  out[n][j] = s * sum_k X[n][k] W[j][k]      (x A^T, and dy B as
//           dy (B^T)^T): a skinny GEMM.  bf16 (lora_rowdot16_kernel): 1, 2
//           or 4 16-row slabs per 8-wave workgroup (chosen per call from the
//           grid's fit to the CUs) on v_mfma_f32_16x16x32_bf16, each wave's
//           k-steps of X and W staged in its own LDS region by DMA in
//           row-segment lane order and read back in operand order.  f32 (the
//           parity path): one wave per 32 rows, operands from global memory.
//           HBM-bound: one read of X.
//   expand  Y[n][c] += s * sum_j U[n][j] Wt[c][j]       (y += s u B^T, and
//           dx += du A).  bf16 (lora_expand_mfma_kernel): one wave per 32
//           rows x 64 columns on v_mfma_f32_32x32x16_bf16, the result
//           transposed through LDS so Y is updated with 16-byte accesses.  f32
//           (the parity path): one thread per output column and row phase,
//           Wt rows staged in LDS.  HBM-bound: one read and one write of Y.
//   colsum  out[j][c] = s * sum_n U[n][j] X[n][c]      (dB^T = s u^T dy and
//           dA = du^T x).  bf16: a skinny MFMA GEMM, X^T (by transpose reads
//           of 32-token x 128-column tiles streamed into LDS) times U^T (read
//           the same way from a 32- or 64-column tile of U's rows streamed
//           beside them, or from a staged fragment-major copy when U is not
//           16-byte aligned), split over tokens; the splits are summed in a
//           fixed order by a second kernel — deterministic, no atomics.  One
//           set of launches serves up to 16 products of any token counts.
//           f32 (the parity path): each workgroup owns 64 columns and sweeps
//           all rows in a fixed order.
#include <type_traits>

#include "fa_device.hpp"
#include "fa_kernels.hpp"
#include "fa_lds.hpp"

namespace fa {
namespace {

// ---- rowdot -------------------------------------------------------------
// X: [N, K] (ldx), W: [R, K] contiguous, out: f32 [N, R] (ldo), R <= 32.
template <typename T>
__global__ __launch_bounds__(256) void lora_rowdot_kernel(const T *__restrict__ X, int64_t ldx,
                                                          const T *__restrict__ W, float *out,
                                                          int64_t ldo, int N, int K, int R,
                                                          float s) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 31, g = lane >> 5;
    const int row0 = (blockIdx.x * 4 + wave) * 32;
    if (row0 >= N) return;
    const int xr = row0 + n;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    if constexpr (sizeof(T) == 2) {
        const bool xin = xr < N, win = n < R;
        const bf16 *xp = reinterpret_cast<const bf16 *>(X) + (int64_t)xr * ldx + g * 8;
        const bf16 *wp = reinterpret_cast<const bf16 *>(W) + (int64_t)n * K + g * 8;
        for (int k0 = 0; k0 < K; k0 += 16) {
            const bf16x8 a = as_bf16x8(xin ? ld_global_16(xp + k0) : u32x4{0, 0, 0, 0});
            const bf16x8 b = as_bf16x8(win ? ld_global_16(wp + k0) : u32x4{0, 0, 0, 0});
            acc = mfma_32x32x16(a, b, acc);
        }
    } else {
        const float *xp = reinterpret_cast<const float *>(X) + (int64_t)xr * ldx;
        const float *wp = reinterpret_cast<const float *>(W) + (int64_t)n * K;
        for (int k0 = 0; k0 < K; k0 += 2) {
            const float a = xr < N ? xp[k0 + g] : 0.f;
            const float b = n < R ? wp[k0 + g] : 0.f;
            acc = mfma_32x32x2_f32(a, b, acc);
        }
    }
    // acc element r: row row0 + acc_row(r), column j = n
    if (n < R)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = row0 + acc_row(r, lane);
            if (row < N) out[(int64_t)row * ldo + n] = acc[r] * s;
        }
}

// ---- expand -------------------------------------------------------------
// Y[n][c] += s * sum_j U[n][j] * Wt[c][j];  U f32 [N, R] (ldu), Wt [C, R]
// contiguous, Y [N, C] (ldy).  Block = 64 columns x 4 row phases; the 64 Wt
// rows are staged in LDS, U rows are broadcast reads.
template <typename T>
__global__ __launch_bounds__(256) void lora_expand_kernel(const float *__restrict__ U, int64_t ldu,
                                                          const T *__restrict__ Wt, T *Y,
                                                          int64_t ldy, int N, int C, int R,
                                                          float s, int rows_per_block) {
    __shared__ float wsh[64][33];
    const int cl = threadIdx.x & 63, ph = threadIdx.x >> 6;
    const int c0 = blockIdx.x * 64;
    for (int e = threadIdx.x; e < 64 * R; e += 256) {
        const int cc = e / R, j = e % R;
        wsh[cc][j] = c0 + cc < C ? (float)Wt[(int64_t)(c0 + cc) * R + j] : 0.f;
    }
    __syncthreads();
    const int col = c0 + cl;
    if (col >= C) return;
    const int n0 = blockIdx.y * rows_per_block;
    const int n1 = min(N, n0 + rows_per_block);
    for (int row = n0 + ph; row < n1; row += 4) {
        const float *u = U + (int64_t)row * ldu;
        float acc = 0.f;
        for (int j = 0; j < R; ++j) acc += u[j] * wsh[cl][j];
        T *y = Y + (int64_t)row * ldy + col;
        *y = (T)((float)*y + s * acc);
    }
}

// ---- rowdot / expand, bf16 (MFMA) ---------------------------------------
// rowdot: out[n][j] = s * sum_k X[n][k] W[j][k], R <= 16 * NT.  A workgroup
// of 8 waves owns 16 rows; wave w takes k-steps (32 wide) w, w + 8, ..., and
// the 8 partial tiles are summed in LDS in a fixed order (deterministic, no
// workspace).
//
// Loads: the MFMA operand order (lane = row + 16 * chunk) spreads each quad of
// lanes over 4 rows, and loads in that order ran at half the rate of the same
// bytes read with each quad in one 64-byte row segment (X and A of 4096 x
// 3072, r 16: 6.6 against 3.4 us).  So each wave stages its own k-steps in a
// private LDS region by buffer_load ... lds in the row-segment order (lane =
// 4 * row + chunk, X rows then W rows, 1 KiB per 16 rows) and reads them back
// in operand order.  Within a 64-byte row the chunk is XORed with (row / 4) %
// 4, so that both the DMA (a quad still covers one segment) and the operand
// reads (16 rows at one chunk hit 16 distinct bank groups) are conflict-free.
// G k-steps per stage, two stages per wave in flight; no barrier inside the
// loop (the regions are private).  Rows >= N and j >= R load from a clamped (valid) row:
// output element (n, j) depends on row n of X and row j of W only, and those
// outputs are not stored.  K % 32 == 16 leaves a half k-step whose upper 16
// columns are zeroed in the operand.
// One k-step per stage: two k-steps per stage (twice the LDS) was no faster
// alone and slower in the c4 step, where a workgroup's LDS decides whether it
// can share a CU with the other stream's kernels.
template <int NT, int MT = 1>
struct RowdotStage {
    static constexpr int G = 1;                        // k-steps per stage
    static constexpr int STEP = 1024 * (MT + NT);      // LDS bytes per k-step: MT X slabs, then NT W tiles
    static constexpr int WAVE = G * STEP;              // one wave's stage
    static constexpr int BYTES = 8 * WAVE;             // the workgroup's stage
};

// MT: 16-row slabs per workgroup.  Each k-step's W tiles are then read once
// for MT slabs of X; at rank 48 the W bytes (from L2) outweigh X's three to
// one for a single slab.
template <int NT, typename TO, int MT = 1>
__global__ __launch_bounds__(512) void lora_rowdot16_kernel(const bf16 *__restrict__ X, int64_t ldx,
                                                            const bf16 *__restrict__ W, TO *out, int64_t ldo,
                                                            int N, int K, int R, float s) {
    using RS = RowdotStage<NT, MT>;
    constexpr int G = RS::G;
    // two distinct LDS objects: the compiler then tells the DMA into one
    // stage from the reads of the other
    __shared__ __align__(16) char sa[RS::BYTES], sb[RS::BYTES];
    // the 8 partial tiles of one slab reuse sa once the k-steps are done
    static_assert(sizeof(float) * 8 * NT * 4 * 64 <= RS::BYTES, "partials fit in a stage");
    float (*part)[NT][4][64] = reinterpret_cast<float (*)[NT][4][64]>(sa);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m = lane & 15, q = lane >> 4;
    const int row0 = blockIdx.x * 16 * MT;

    // DMA source offsets: lane 4 r + p fetches chunk p ^ ((r / 4) % 4) of row
    // r of a 16-row, 32-column k-step (the k-step itself goes in soffset)
    const int r = lane >> 2, c = (lane & 3) ^ ((r >> 2) & 3);
    const int xrows = min(16 * MT, N - row0);
    const __amdgpu_buffer_rsrc_t xrs =
        make_rsrc(X + (int64_t)row0 * ldx, (uint32_t)(((int64_t)(xrows - 1) * ldx + K) * 2));
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W, (uint32_t)((int64_t)R * K * 2));
    uint32_t xvo[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xvo[mt] = (uint32_t)((min(mt * 16 + r, xrows - 1) * ldx + c * 8) * 2);
    uint32_t wvo[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) wvo[t] = (uint32_t)((min(t * 16 + r, R - 1) * (int64_t)K + c * 8) * 2);
    // operand reads: lane (m, q) takes chunk q of row m
    const int rd = m * 64 + ((q ^ ((m >> 2) & 3)) << 4);

    const int nks = (K + 31) / 32;                               // k-steps, the last maybe half
    const int J = nks > wave ? (nks - wave + 7) / 8 : 0;         // this wave's k-steps
    const bool half = K % 32 != 0;
    // stage of k-steps j0 .. j0+G-1 of this wave into dst; past J it loads a
    // clamped (valid) k-step that is never read, so every stage issues the
    // same G (1 + NT) loads and the waits can count them
    auto issue = [&](int j0, char *dst) {
        char *d = dst + wave * RS::WAVE;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int ks = wave + 8 * min(j0 + g, J - 1);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                buffer_to_lds_16(xrs, d + g * RS::STEP + 1024 * mt, xvo[mt], (uint32_t)ks * 64);
#pragma unroll
            for (int t = 0; t < NT; ++t)
                buffer_to_lds_16(wrs, d + g * RS::STEP + 1024 * (MT + t), wvo[t], (uint32_t)ks * 64);
        }
    };
    const u32x4 zero = {0, 0, 0, 0};
    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int j0, const char *src) {
        const char *d = src + wave * RS::WAVE;
#pragma unroll
        for (int g = 0; g < G; ++g)
            if (j0 + g < J) {
                u32x4 wf[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) wf[t] = ld_lds_16(d + g * RS::STEP + 1024 * (MT + t), rd);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    u32x4 a = ld_lds_16(d + g * RS::STEP + 1024 * mt, rd);
                    if (half && wave + 8 * (j0 + g) == nks - 1 && q >= 2) a = zero;  // columns past K
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[mt][t] = mfma_16x16x32(as_bf16x8(a), as_bf16x8(wf[t]), acc[mt][t]);
                }
            }
    };
    if (J > 0) {
        constexpr int VM = G * (MT + NT);  // loads per stage
        issue(0, sa);
        issue(G, sb);
        // No exit between the halves: with one, the compiler's wait-count
        // analysis sees a path from a refill of sa straight to the reads of
        // sa and drains every load there.  A half past J reads nothing.
        for (int j0 = 0; j0 < J; j0 += 2 * G) {
            wait_vmcnt<VM>();  // stage j0 landed, the next one may stay in flight
            consume(j0, sa);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the DMA refills sa
            issue(j0 + 2 * G, sa);
            wait_vmcnt<VM>();
            consume(j0 + G, sb);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(j0 + 3 * G, sb);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the stages issued past J land before LDS is reused
    }
    // one slab at a time through sa: the 8 waves' partial tiles, summed in a
    // fixed order
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        __syncthreads();  // every wave is done with sa (its stage, or the previous slab's partials)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) part[wave][t][e][lane] = acc[mt][t][e];
        __syncthreads();
        if (wave < NT) {
            const int t = wave, col = t * 16 + m;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = part[0][t][e][lane];
#pragma unroll
                for (int w = 1; w < 8; ++w) v += part[w][t][e][lane];
                const int row = row0 + mt * 16 + 4 * q + e;
                if (row < N && col < R) out[(int64_t)row * ldo + col] = (TO)(v * s);
            }
        }
    }
}

// expand: Y[n][c] += s * sum_j U[n][j] Wt[c][j], U f32 [N, R] rounded to bf16
// for the MFMA, Wt [C, R] bf16 contiguous, R <= 64.  One wave per 32 rows x
// 64 columns (two 32x32 output tiles, k = j).  VEC (16-byte loads of U and
// Wt rows) needs R % 8 == 0 and 16-byte aligned U and Wt.
template <bool VEC>
__device__ __forceinline__ bf16x8 load8_u_as_bf16(const bf16 *p, int j0, int R) {
    if (VEC && j0 + 8 <= R) return as_bf16x8(ld_global_16(p));
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = j0 + e < R ? p[e] : (bf16)0.f;
    return o;
}
template <bool VEC>
__device__ __forceinline__ bf16x8 load8_u_as_bf16(const float *p, int j0, int R) {
    float v[8];
    if (VEC && j0 + 8 <= R) {
        const f32x4 a = __builtin_bit_cast(f32x4, ld_global_16(p));
        const f32x4 b = __builtin_bit_cast(f32x4, ld_global_16(p + 4));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = a[e];
            v[4 + e] = b[e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = j0 + e < R ? p[e] : 0.f;
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = f32_to_bf16(v[e]);
    return o;
}
template <bool VEC>
__device__ __forceinline__ bf16x8 load8_guarded_bf16(const bf16 *p, int j0, int R) {
    if (VEC && j0 + 8 <= R) return as_bf16x8(ld_global_16(p));
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = j0 + e < R ? p[e] : (bf16)0.f;
    return o;
}

template <bool VEC, bool Y16, typename TU, int KS>
__global__ __launch_bounds__(256) void lora_expand_mfma_kernel(const TU *__restrict__ U, int64_t ldu,
                                                               const bf16 *__restrict__ Wt, bf16 *Y, int64_t ldy,
                                                               int N, int C, int R, float s) {
    // per-wave half (16 rows x 64 columns) of the f32 result tile, used twice;
    // rows padded to 68 floats (16-byte aligned).  17 KiB per workgroup lets
    // six workgroups share a CU, so the c4 grids run in one round.
    __shared__ __attribute__((aligned(16))) float tile[4][16][68];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31, g = lane >> 5;
    const int row0 = blockIdx.y * 32;
    const int col0 = (blockIdx.x * 4 + wave) * 64;
    const bool active = col0 < C;  // wave-uniform
    const int urow = min(row0 + n, N - 1);
    // Every load goes out before the first is used: the Y chunks this lane
    // updates at the end (they do not depend on the product), then the U and
    // Wt operands of all KS = ceil(R / 16) rank steps, so the kernel waits on
    // memory once rather than once per rank step and again for Y.
    bf16x8 yv[4];
    if constexpr (Y16) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int row = row0 + (lane >> 3) + 8 * k, col = col0 + 8 * (lane & 7);
            yv[k] = active && row < N && col < C ? as_bf16x8(ld_global_16(Y + (int64_t)row * ldy + col))
                                                 : as_bf16x8(u32x4{0, 0, 0, 0});
        }
    }
    bf16x8 a[KS], b[KS][2];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int ja = ks * 16 + g * 8;
        const bool in = active && ja < R;
        a[ks] = in ? load8_u_as_bf16<VEC>(U + (int64_t)urow * ldu + ja, ja, R) : as_bf16x8(u32x4{0, 0, 0, 0});
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int col = min(col0 + t * 32 + n, C - 1);
            b[ks][t] = in ? load8_guarded_bf16<VEC>(Wt + (int64_t)col * R + ja, ja, R) : as_bf16x8(u32x4{0, 0, 0, 0});
        }
    }
    if (!active) return;  // wave-uniform; the LDS buffer below is the wave's own
    f32x16 acc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[t] = mfma_32x32x16(a[ks], b[ks][t], acc[t]);
    // acc[t] element r: row acc_row(r, lane), column t*32 + n of the wave's
    // tile.  Elements r < 8 hold rows 0..15, r >= 8 rows 16..31: half h goes
    // through the buffer in pass h.  Each lane updates four 8-column chunks:
    // chunk c = lane + 64k covers tile row c / 8, columns 8 * (c % 8) .. + 7
    // (C % 16 == 0 keeps a chunk whole); chunks k = 2h, 2h + 1 lie in half h.
    // Lanes exchange values through the wave's own buffer: a wait for the
    // LDS operations with a compiler memory barrier separates each pass's
    // writes from its reads, and pass 0's reads from pass 1's writes.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 8 * h; r < 8 * h + 8; ++r) tile[wave][acc_row(r, lane) - 16 * h][t * 32 + n] = acc[t][r];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int k = 2 * h; k < 2 * h + 2; ++k) {
            const int tr = (lane >> 3) + 8 * k, tc = 8 * (lane & 7);
            const int row = row0 + tr, col = col0 + tc;
            if (row >= N || col >= C) continue;
            const f32x4 lo = *reinterpret_cast<const f32x4 *>(&tile[wave][tr - 16 * h][tc]);
            const f32x4 hi = *reinterpret_cast<const f32x4 *>(&tile[wave][tr - 16 * h][tc + 4]);
            bf16 *y = Y + (int64_t)row * ldy + col;
            if constexpr (Y16) {
                bf16x8 v = yv[k];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = f32_to_bf16((float)v[e] + s * lo[e]);
                    v[4 + e] = f32_to_bf16((float)v[4 + e] + s * hi[e]);
                }
                st_global_16(y, as_u32x4(v));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[e] = f32_to_bf16((float)y[e] + s * lo[e]);
                    y[4 + e] = f32_to_bf16((float)y[4 + e] + s * hi[e]);
                }
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
}

// ---- colsum -------------------------------------------------------------
// out[j][c] = s * sum_n U[n][j] * X[n][c]  (U f32 [N, R], X [N, C] ldx).
// Written to out at (j * os_j + c * os_c) so the same kernel yields dA [R, K]
// (os_j = K, os_c = 1) and dB [M, R] (os_j = 1, os_c = R).
// Block: 64 columns x 4 row-phases; each thread accumulates R partial sums
// for one column over rows phase, phase+4, ..., then the 4 phases are summed
// in a fixed order.
template <typename T>
__global__ __launch_bounds__(256) void lora_colsum_kernel(const float *__restrict__ U, int64_t ldu,
                                                          const T *__restrict__ X, int64_t ldx,
                                                          float *out, int64_t os_j, int64_t os_c,
                                                          int N, int C, int R, float s) {
    __shared__ float part[4][64][33];
    const int cl = threadIdx.x & 63, ph = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + cl;
    float acc[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) acc[j] = 0.f;
    if (col < C) {
        for (int row = ph; row < N; row += 4) {
            const float xv = (float)X[(int64_t)row * ldx + col];
            const float *u = U + (int64_t)row * ldu;
#pragma unroll
            for (int j = 0; j < 32; ++j)
                if (j < R) acc[j] += u[j] * xv;
        }
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) part[ph][cl][j] = acc[j];
    __syncthreads();
    if (ph == 0 && col < C)
        for (int j = 0; j < R; ++j)
            out[j * os_j + (int64_t)col * os_c] =
                s * (((part[0][cl][j] + part[1][cl][j]) + part[2][cl][j]) + part[3][cl][j]);
}

// ---- colsum, bf16 (MFMA) ------------------------------------------------
// U^T as MFMA B operands, fragment-major: for 32-row block h (j / 32),
// 16-token step k and lane L = j % 32 + 32 g, the lane's 8 values are the 16
// bytes at ((h * npad / 16 + k) * 64 + L) * 8, so a wave's operand load for
// one step is 1 KiB in lane order (loads whose quads of lanes span 4 rows
// ran at about half the rate).  Lane half g holds positions 16 k + 8 g ..
// +7, and within each 16-token group the tokens are stored as {0..3, 8..11,
// 4..7, 12..15}: lane half g then holds tokens {4g..4g+3, 8+4g..8+4g+3} —
// the k order of the transpose-read A operand.  Rows j >= R and tokens >= N
// are zero.  One thread per element, in storage order.
__device__ __forceinline__ void ut_frag_coords(int64_t e, int npad, int &j, int &n) {
    const int e8 = (int)(e & 7), L = (int)((e >> 3) & 63);
    const int64_t rest = e >> 9;
    const int nk = npad >> 4, h = (int)(rest / nk), k = (int)(rest % nk);
    j = h * 32 + (L & 31);
    const int p = k * 16 + (L >> 5) * 8 + e8;  // position within the padded token axis
    const int q = p & 15;
    n = (p >> 4) * 16 + ((q & 4) ? 8 : 0) + ((q & 8) ? 4 : 0) + (q & 3);
}
template <typename TU>
__global__ void lora_ut_kernel(const TU *__restrict__ U, int64_t ldu, bf16 *ut, int N, int R, int npad) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)32 * npad) return;
    int j, n;
    ut_frag_coords(e, npad, j, n);
    ut[e] = j < R && n < N ? (bf16)U[(int64_t)n * ldu + j] : (bf16)0.f;
}

constexpr int kCsCols = 128;  // columns per workgroup (4 waves x 32)
// Tokens per LDS stage.  32 rather than 64: 24 KiB of LDS per workgroup
// (two stages of X and U) lets six workgroups share a CU instead of three;
// the c4 step's 12 gradient products 41.0 -> 38.4 us, the single block's
// four 110.3 -> 103.8 us, same bits (a 4-product q/k/v set 23.7 -> 24.9 us).
constexpr int kCsRows = 32;

// Workgroup (column tile ct, token split sp): part[sp][c][j] = sum over the
// split's tokens of X[n][c] U[n][j], for the tile's 128 columns and j < 32.
__global__ __launch_bounds__(256) void lora_colsum_mfma_kernel(const bf16 *__restrict__ X, int64_t ldx,
                                                               const bf16 *__restrict__ ut, int npad,
                                                               float *part, int N, int C, int chunk) {
    using T = LdsTile<128, kCsRows>;
    constexpr int WI = T::WAVE_INSTS / 4;
    __shared__ __align__(16) char st0[T::BYTES], st1[T::BYTES];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31;
    const int c0 = blockIdx.x * kCsCols;
    const int t_begin = blockIdx.y * chunk, t_end = min(t_begin + chunk, npad);
    // rows >= N (and, in the last row, columns >= C) read as zero
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(X + c0, (uint32_t)(((int64_t)(N - 1) * ldx + (C - c0)) * 2));
    const uint32_t xvo = tile_src_off<128>(wave, lane, ldx);
    const uint32_t row_step = tile_inst_row_step<128>(ldx);
    const uint32_t stage_step = (uint32_t)(kCsRows * ldx * 2);
    auto issue = [&](int t0, char *dst) {
#pragma unroll
        for (int i = 0; i < WI; ++i)
            buffer_to_lds_16(xrs, dst + (i * 4 + wave) * 1024, xvo, (uint32_t)(t0 / kCsRows) * stage_step + i * row_step);
    };
    uint32_t coff[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) coff[dt] = col_frag_off<128>(0, 0, dt, lane);
    const bf16 *ub = ut + lane * 8;  // fragment-major: 512 values per 16-token step
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    // a stage's U^T fragments are loaded before the next stage's DMA, so that
    // waiting for them leaves that DMA in flight (in-order completion)
    constexpr int KS = kCsRows / 16;
    auto loadu = [&](int t0, bf16x8 (&b)[KS]) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) b[ks] = as_bf16x8(ld_global_16(ub + ((t0 >> 4) + ks) * 512));
    };
    auto stage = [&](const char *tile, const bf16x8 (&b)[KS]) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const bf16x8 a = lds_read_col_frag(tile, coff[wave] + ks * 16 * T::ROWB,
                                               col_frag_hi8<128>(coff, wave) + ks * 16 * T::ROWB);
            acc = mfma_32x32x16(a, b[ks], acc);
        }
    };
    bf16x8 bu[KS];
    issue(t_begin, st0);
    for (int t0 = t_begin; t0 < t_end; t0 += 2 * kCsRows) {
        barrier_keep_dma<0>();
        loadu(t0, bu);
        if (t0 + kCsRows < t_end) issue(t0 + kCsRows, st1);
        stage(st0, bu);
        if (t0 + kCsRows < t_end) {
            barrier_keep_dma<0>();
            loadu(t0 + kCsRows, bu);
            if (t0 + 2 * kCsRows < t_end) issue(t0 + 2 * kCsRows, st0);
            stage(st1, bu);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // acc element r: column c0 + wave*32 + acc_row(r, lane), j = n
    float *pp = part + (int64_t)blockIdx.y * C * 32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int c = c0 + wave * 32 + acc_row(r, lane);
        if (c < C) pp[(int64_t)c * 32 + n] = acc[r];
    }
}

// sum_sp p[sp * stride] for sp = 0, 1, ..., n - 1, added in that order; the
// loads go out eight at a time, so a thread waits for memory once per eight
// splits rather than once per split.
__device__ __forceinline__ float sum_splits(const float *p, int64_t stride, int n) {
    float acc = 0.f;
    int sp = 0;
    for (; sp + 8 <= n; sp += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = p[(int64_t)(sp + i) * stride];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc += v[i];
    }
    for (; sp < n; ++sp) acc += p[(int64_t)sp * stride];
    return acc;
}

// out[j * os_j + c * os_c] = s * sum_sp part[sp][c][j] (fixed order), j < R.
__global__ void lora_colsum_reduce_kernel(const float *__restrict__ part, float *out, int64_t os_j,
                                          int64_t os_c, int C, int R, int splits, float s) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)C * 32) return;
    const int c = (int)(e >> 5), j = (int)(e & 31);
    if (j >= R) return;
    out[j * os_j + (int64_t)c * os_c] = s * sum_splits(part + e, (int64_t)C * 32, splits);
}

// ---- colsum over several products in one set of launches -----------------
// Products k = 0..count-1, each of its own token count N_k: out_k = s_k *
// U_k^T X_k (or its transpose), U_k bf16 [N_k, R_k <= 64].  The same three steps as above,
// each one launch for all products: U^T in operand order (rw = 32 or 64 rows),
// split partials over [splits_k][C_k][rw] (R_k > 32: a second accumulator
// over U^T rows 32..63 shares each X tile), fixed-order sum.  Per output the
// arithmetic is that of the single-product kernels, so the same bits.
constexpr int kGradMany = 16;
struct GradProblem {
    const bf16 *u;
    int64_t ldu;
    const bf16 *x;
    int64_t ldx;
    float *out;
    int64_t os_j, os_c;
    bf16 *ut;     // [rw][npad]
    float *part;  // [splits][C][rw]
    float s;
    int C, R, rw, splits, chunk, wg0;  // wg0: the product's first colsum workgroup
    int N, npad;  // tokens, and tokens rounded up to whole stages (kCsRows)
};
struct GradMany {
    GradProblem p[kGradMany];
    int count;
};

__global__ void lora_ut_many_kernel(GradMany g) {
    const GradProblem &q = g.p[blockIdx.y];
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= q.rw * q.npad) return;
    int j, n;
    ut_frag_coords(e, q.npad, j, n);
    q.ut[e] = j < q.R && n < q.N ? q.u[(int64_t)n * q.ldu + j] : (bf16)0.f;
}

// One workgroup: column tile, token split of product q.  DIRECT (every
// product's U 16-byte aligned with 16-byte rows): U's rows for a stage
// (kCsRows tokens x 32 or 64 columns) come into LDS by DMA beside the X tile,
// and the B operand is a column fragment of that tile -- the same transpose
// read, hence the same token
// order, as X's A operand; columns j >= R hold whatever follows U's rows and
// only reach outputs j >= R, which are not stored.  Otherwise the B operand
// is read from the staged fragment-major U^T.  The values multiplied are the
// same either way, so are the bits.
// The LDS arrays are the kernel's own (not pointer arguments of a helper):
// the compiler then tells the DMA into one stage from the reads of the other.
template <bool DIRECT>
__global__ __launch_bounds__(256) void lora_colsum_many_kernel(GradMany g) {
    // one workgroup per (product, split, column tile): product k's
    // workgroups start at wg0, split-major
    int k = 0;
    while (k + 1 < g.count && g.p[k + 1].wg0 <= (int)blockIdx.x) ++k;
    const GradProblem &q = g.p[k];
    const int ntiles = (q.C + kCsCols - 1) / kCsCols;
    const int wi = (int)blockIdx.x - q.wg0, split = wi / ntiles, tile = wi - split * ntiles;
    using T = LdsTile<128, kCsRows>;
    using UT = LdsTile<64, kCsRows>;  // the widest U tile (R > 32)
    constexpr int WI = T::WAVE_INSTS / 4;
    __shared__ __align__(16) char st0[T::BYTES], st1[T::BYTES];
    __shared__ __align__(16) char uu0[DIRECT ? UT::BYTES : 16], uu1[DIRECT ? UT::BYTES : 16];
    const int N = q.N, npad = q.npad;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 31;
    const int C = q.C;
    const int64_t ldx = q.ldx;
    const int c0 = tile * kCsCols;
    const int t_begin = split * q.chunk, t_end = min(t_begin + q.chunk, npad);
    const bool two = q.rw == 64;
    // rows >= N (and, in the last row, columns >= C) read as zero
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(q.x + c0, (uint32_t)(((int64_t)(N - 1) * ldx + (C - c0)) * 2));
    const uint32_t xvo = tile_src_off<128>(wave, lane, ldx);
    const uint32_t row_step = tile_inst_row_step<128>(ldx);
    const uint32_t stage_step = (uint32_t)(kCsRows * ldx * 2);
    // U rows >= N read as zero.  The range ends at a whole dword: the
    // buffer range check zeroes a dword that crosses it, which for odd R
    // would drop the last row's column R - 1 (column R, the dword's other
    // half, lies in the row's 16-byte stride).
    const __amdgpu_buffer_rsrc_t urs =
        make_rsrc(q.u, (uint32_t)((int64_t)(N - 1) * q.ldu * 2 + ((q.R * 2 + 3) & ~3)));
    const uint32_t ustage_step = (uint32_t)(kCsRows * q.ldu * 2);
    auto issue_x = [&](int t0, char *dst) {
#pragma unroll
        for (int i = 0; i < WI; ++i)
            buffer_to_lds_16(xrs, dst + (i * 4 + wave) * 1024, xvo, (uint32_t)(t0 / kCsRows) * stage_step + i * row_step);
    };
    uint32_t coff[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) coff[dt] = col_frag_off<128>(0, 0, dt, lane);
    const bf16 *ub = q.ut + lane * 8;            // fragment-major: 512 values per 16-token step
    const bf16 *ub2 = ub + (int64_t)32 * npad;   // rows 32..63
    f32x16 acc, acc2;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        acc[r] = 0.f;
        acc2[r] = 0.f;
    }
    // Staged: a stage's U^T fragments are loaded before the next stage's DMA
    // is issued: memory operations complete in issue order, so waiting for
    // them then leaves that DMA in flight during this stage's MFMAs.
    constexpr int KS = kCsRows / 16;
    auto loadu = [&](int t0, bf16x8 (&b)[2 * KS]) {
        if constexpr (!DIRECT) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                b[ks] = as_bf16x8(ld_global_16(ub + ((t0 >> 4) + ks) * 512));
                if (two) b[KS + ks] = as_bf16x8(ld_global_16(ub2 + ((t0 >> 4) + ks) * 512));
            }
        }
    };
    if constexpr (DIRECT) {
        // The U tile is as wide as the product needs: 32 columns (R <= 32,
        // 4 KiB a stage) or 64 (8 KiB); body<UW> is the whole pipeline for
        // one width, so each keeps its loop free of conditions.
        auto body = [&](auto uwc) {
            constexpr int UW = decltype(uwc)::value;
            using U = LdsTile<UW, kCsRows>;
            constexpr int UWI = U::WAVE_INSTS / 4;
            const uint32_t uvo = tile_src_off<UW>(wave, lane, q.ldu);
            const uint32_t urow_step = tile_inst_row_step<UW>(q.ldu);
            uint32_t cu[UW / 32];
#pragma unroll
            for (int f = 0; f < UW / 32; ++f) cu[f] = col_frag_off<UW>(0, 0, f, lane);
            auto issue = [&](int t0, char *dst, char *udst) {
                issue_x(t0, dst);
                if constexpr (UWI == 0) {
                    if (wave < U::WAVE_INSTS)
                        buffer_to_lds_16(urs, udst + wave * 1024, uvo, (uint32_t)(t0 / kCsRows) * ustage_step);
                } else {
#pragma unroll
                    for (int i = 0; i < UWI; ++i)
                        buffer_to_lds_16(urs, udst + (i * 4 + wave) * 1024, uvo,
                                         (uint32_t)(t0 / kCsRows) * ustage_step + i * urow_step);
                }
            };
            auto stage = [&](const char *tile, const char *utile) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const bf16x8 a = lds_read_col_frag(tile, coff[wave] + ks * 16 * T::ROWB,
                                                       col_frag_hi8<128>(coff, wave) + ks * 16 * T::ROWB);
                    const bf16x8 b0 = lds_read_col_frag(utile, cu[0] + ks * 16 * U::ROWB,
                                                        col_frag_hi8<UW>(cu, 0) + ks * 16 * U::ROWB);
                    acc = mfma_32x32x16(a, b0, acc);
                    if constexpr (UW == 64) {
                        const bf16x8 b1 = lds_read_col_frag(utile, cu[1] + ks * 16 * U::ROWB,
                                                            col_frag_hi8<UW>(cu, 1) + ks * 16 * U::ROWB);
                        acc2 = mfma_32x32x16(a, b1, acc2);
                    }
                }
            };
            // Each stage's refill goes out unconditionally (past the split's
            // range it reads rows of the next split or zeros, never used): a
            // conditional issue made the compiler wait for the refill of one
            // stage before reading the other.  Only the second stage's reads
            // are conditional.  (A ring of three stages, two in flight, ran
            // slower: 72 KiB of LDS leaves two workgroups per CU, not three.)
            issue(t_begin, st0, uu0);
            for (int t0 = t_begin; t0 < t_end; t0 += 2 * kCsRows) {
                barrier_keep_dma<0>();
                issue(t0 + kCsRows, st1, uu1);
                stage(st0, uu0);
                barrier_keep_dma<0>();
                issue(t0 + 2 * kCsRows, st0, uu0);
                if (t0 + kCsRows < t_end) stage(st1, uu1);
            }
        };
        if (two)
            body(std::integral_constant<int, 64>{});
        else
            body(std::integral_constant<int, 32>{});
    } else {
        auto issue = [&](int t0, char *dst, char *) { issue_x(t0, dst); };
        auto stage = [&](const char *tile, const char *, const bf16x8 (&b)[2 * KS]) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const bf16x8 a = lds_read_col_frag(tile, coff[wave] + ks * 16 * T::ROWB,
                                                   col_frag_hi8<128>(coff, wave) + ks * 16 * T::ROWB);
                acc = mfma_32x32x16(a, b[ks], acc);
                if (two) acc2 = mfma_32x32x16(a, b[KS + ks], acc2);
            }
        };
        bf16x8 bu[2 * KS];
        issue(t_begin, st0, uu0);
        for (int t0 = t_begin; t0 < t_end; t0 += 2 * kCsRows) {
            barrier_keep_dma<0>();
            loadu(t0, bu);
            if (t0 + kCsRows < t_end) issue(t0 + kCsRows, st1, uu1);
            stage(st0, uu0, bu);
            if (t0 + kCsRows < t_end) {
                barrier_keep_dma<0>();
                loadu(t0 + kCsRows, bu);
                if (t0 + 2 * kCsRows < t_end) issue(t0 + 2 * kCsRows, st0, uu0);
                stage(st1, uu1, bu);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // acc element r: column c0 + wave*32 + acc_row(r, lane), j = n (acc2: j = 32 + n)
    const int rw = q.rw;
    float *pp = q.part + (int64_t)split * C * rw;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int c = c0 + wave * 32 + acc_row(r, lane);
        if (c < C) {
            pp[(int64_t)c * rw + n] = acc[r];
            if (two) pp[(int64_t)c * rw + 32 + n] = acc2[r];
        }
    }
}

// out[j * os_j + c * os_c] = s * sum_sp part[sp][c][j] (fixed order), j < R.
__global__ void lora_colsum_reduce_many_kernel(GradMany g) {
    const GradProblem &q = g.p[blockIdx.y];
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)q.C * q.rw) return;
    const int c = (int)(e / q.rw), j = (int)(e - (int64_t)c * q.rw);
    if (j >= q.R) return;
    q.out[j * q.os_j + (int64_t)c * q.os_c] = q.s * sum_splits(q.part + e, (int64_t)q.C * q.rw, q.splits);
}

// Small transpose [R][C] -> [C][R] (dtype).
template <typename T>
__global__ void lora_transpose_kernel(const T *__restrict__ src, T *dst, int R, int C) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)R * C) return;
    const int r = e / C, c = e % C;
    dst[(int64_t)c * R + r] = src[e];
}

// 16-row slabs per rowdot workgroup, 1, 2 or 4.  A CU's LDS-DMA rate bounds
// these kernels, so the time goes as the most bytes any one CU stages:
// (workgroups on the busiest CU) x (MT X slabs + NT W tiles) per k-step.  More
// slabs per workgroup share each W tile among more rows but leave CUs idle
// once the grid is smaller than the chip (4096 rows: 256 workgroups of one
// slab fill 256 CUs once; 4608 rows: 288 of one slab put two on 32 CUs, 144
// of two slabs put at most one on any).  Which slab count runs changes no
// bits: each 16-row tile's k-steps are the same, in the same order.
int rowdot_slabs(int N, int NT) {
    const int cus = device_cu_count();
    int best = 1;
    int64_t best_cost = -1;
    for (int mt : {1, 2, 4}) {
        const int64_t wgs = (N + 16 * mt - 1) / (16 * mt);
        const int64_t cost = (wgs + cus - 1) / cus * (mt + NT);
        if (best_cost < 0 || cost < best_cost) best = mt, best_cost = cost;
    }
    return best;
}

template <typename T>
hipError_t rowdot(const T *X, int64_t ldx, const T *W, float *out, int64_t ldo, int N, int K,
                  int R, float s, hipStream_t st) {
    if constexpr (sizeof(T) == 2) {
        auto go = [&](auto mtc) {
            constexpr int MT = decltype(mtc)::value;
            const dim3 grid((unsigned)((N + 16 * MT - 1) / (16 * MT))), block(512);
            if (R <= 16)
                hipLaunchKernelGGL((lora_rowdot16_kernel<1, float, MT>), grid, block, 0, st, X, ldx, W, out, ldo, N, K,
                                   R, s);
            else
                hipLaunchKernelGGL((lora_rowdot16_kernel<2, float, MT>), grid, block, 0, st, X, ldx, W, out, ldo, N, K,
                                   R, s);
        };
        switch (rowdot_slabs(N, (R + 15) / 16)) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        default: go(std::integral_constant<int, 4>{}); break;
        }
    } else {
        const dim3 grid((N + 127) / 128), block(256);
        hipLaunchKernelGGL(lora_rowdot_kernel<T>, grid, block, 0, st, X, ldx, W, out, ldo, N, K, R, s);
    }
    return hipGetLastError();
}

// bf16 Y += s * U Wt^T, U f32 or bf16 rows of stride ldu (16-byte U loads
// when each U row of R elements starts 16-byte aligned).
template <typename TU>
hipError_t expand_mfma(const TU *U, int64_t ldu, const bf16 *Wt, bf16 *Y, int64_t ldy, int N, int C, int R, float s,
                       hipStream_t st) {
    if (R < 1 || R > 64) return hipErrorInvalidValue;  // one to four 16-wide rank steps
    const dim3 grid((unsigned)((C + 255) / 256), (unsigned)((N + 31) / 32)), block(256);
    const bool vec = R % 8 == 0 && (ldu * (int64_t)sizeof(TU)) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(U) % 16 == 0 && reinterpret_cast<uintptr_t>(Wt) % 16 == 0;
    const bool y16 = ldy % 8 == 0 && reinterpret_cast<uintptr_t>(Y) % 16 == 0;
    // the rank steps are a template argument, so a rank-16 launch holds the
    // registers of one step's operands (more waves per SIMD), not four
    auto pick = [&](auto ksc) {
        constexpr int KS = decltype(ksc)::value;
        return vec ? (y16 ? lora_expand_mfma_kernel<true, true, TU, KS> : lora_expand_mfma_kernel<true, false, TU, KS>)
                   : (y16 ? lora_expand_mfma_kernel<false, true, TU, KS>
                          : lora_expand_mfma_kernel<false, false, TU, KS>);
    };
    const int ks = (R + 15) / 16;
    auto kern = ks == 1   ? pick(std::integral_constant<int, 1>{})
                : ks == 2 ? pick(std::integral_constant<int, 2>{})
                : ks == 3 ? pick(std::integral_constant<int, 3>{})
                          : pick(std::integral_constant<int, 4>{});
    hipLaunchKernelGGL(kern, grid, block, 0, st, U, ldu, Wt, Y, ldy, N, C, R, s);
    return hipGetLastError();
}

template <typename T>
hipError_t expand(const float *U, int64_t ldu, const T *Wt, T *Y, int64_t ldy, int N, int C,
                  int R, float s, hipStream_t st) {
    if constexpr (sizeof(T) == 2) return expand_mfma<float>(U, ldu, Wt, Y, ldy, N, C, R, s, st);
    const int rpb = 64;
    const dim3 grid((C + 63) / 64, (N + rpb - 1) / rpb), block(256);
    hipLaunchKernelGGL(lora_expand_kernel<T>, grid, block, 0, st, U, ldu, Wt, Y, ldy, N, C, R, s,
                       rpb);
    return hipGetLastError();
}

// Token splits of the bf16 colsum: up to about 256 workgroups per product,
// each split a whole number of stages and at least 1024 tokens long.  A workgroup's fixed part (first stage's wait, partial store) and the
// partial bytes the reduce reads favour long splits: the c4 double block's 12
// products (4096 and 512 tokens, C = 3072) in one call took 48.0 us with
// splits of at least 4 stages (11 splits of 384 tokens at 4096), 45.2 with 8,
// 40.8 with 16 and 40.8-43 with 32 (but its q/k/v group alone 23.8 us at 16
// against 28.1 at 32); a ring of three stages lost to the occupancy it cost.
inline int colsum_splits(int N, int C) {
    const int tiles = (C + kCsCols - 1) / kCsCols;
    const int stages = (N + kCsRows - 1) / kCsRows;
    int sp = (256 + tiles - 1) / tiles;
    if (sp > stages / (1024 / kCsRows)) sp = stages / (1024 / kCsRows);  // splits of >= 1024 tokens
    return sp < 1 ? 1 : sp;
}
inline int colsum_npad(int N) { return (N + kCsRows - 1) / kCsRows * kCsRows; }

// bf16: U (f32 [N, R]) -> ut (bf16, operand order) -> split partials -> out.
template <typename TU>
hipError_t colsum_bf16(const TU *U, int64_t ldu, const bf16 *X, int64_t ldx, float *out, int64_t os_j,
                       int64_t os_c, int N, int C, int R, float s, bf16 *ut, float *part, hipStream_t st) {
    const int npad = colsum_npad(N), splits = colsum_splits(N, C);
    const int stages = npad / kCsRows;
    const int chunk = (stages + splits - 1) / splits * kCsRows;
    hipLaunchKernelGGL(lora_ut_kernel<TU>, dim3((unsigned)((32 * (int64_t)npad + 255) / 256)), dim3(256), 0, st, U,
                       ldu, ut, N, R, npad);
    hipLaunchKernelGGL(lora_colsum_mfma_kernel, dim3((unsigned)((C + kCsCols - 1) / kCsCols), (unsigned)splits),
                       dim3(256), 0, st, X, ldx, ut, npad, part, N, C, chunk);
    hipLaunchKernelGGL(lora_colsum_reduce_kernel, dim3((unsigned)((C * 32 + 255) / 256)), dim3(256), 0, st, part,
                       out, os_j, os_c, C, R, splits, s);
    return hipGetLastError();
}

template <typename T>
hipError_t colsum(const float *U, int64_t ldu, const T *X, int64_t ldx, float *out, int64_t os_j,
                  int64_t os_c, int N, int C, int R, float s, hipStream_t st) {
    const dim3 grid((C + 63) / 64), block(256);
    hipLaunchKernelGGL(lora_colsum_kernel<T>, grid, block, 0, st, U, ldu, X, ldx, out, os_j, os_c,
                       N, C, R, s);
    return hipGetLastError();
}

template <typename T>
hipError_t transpose(const T *src, T *dst, int R, int C, hipStream_t st) {
    const int64_t n = (int64_t)R * C;
    hipLaunchKernelGGL(lora_transpose_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       src, dst, R, C);
    return hipGetLastError();
}

template <typename T>
hipError_t lora_fwd_t(const LoraParams &p, hipStream_t st) {
    hipError_t e = rowdot<T>(static_cast<const T *>(p.x), p.ldx, static_cast<const T *>(p.a), p.u,
                             p.r, p.N, p.K, p.r, 1.f, st);
    if (e != hipSuccess) return e;
    // y += s * u B^T : B is [M, r] = Wt for expand
    return expand<T>(p.u, p.r, static_cast<const T *>(p.b), static_cast<T *>(p.y), p.ldy, p.N, p.M,
                     p.r, p.scale, st);
}

inline size_t al256(size_t x) { return (x + 255) & ~size_t(255); }

// Workspace layout (bytes, each 256-aligned): du f32 [N, r] | B^T [r, M] |
// A^T [K, r] | bf16 colsum only: ut bf16 [32, npad] | partials f32
// [splits(N, C) * C * 32], the larger of C = K and C = M
template <typename T>
hipError_t lora_bwd_t(const LoraParams &p, hipStream_t st) {
    char *ws = reinterpret_cast<char *>(p.work);
    float *du = reinterpret_cast<float *>(ws);
    const size_t du_b = al256((size_t)p.N * p.r * 4);
    T *bt = reinterpret_cast<T *>(ws + du_b);
    const size_t bt_b = al256((size_t)p.r * p.M * sizeof(T));
    T *at = reinterpret_cast<T *>(ws + du_b + bt_b);
    const size_t at_b = al256((size_t)p.K * p.r * sizeof(T));
    bf16 *ut = reinterpret_cast<bf16 *>(ws + du_b + bt_b + at_b);
    float *part = reinterpret_cast<float *>(ws + du_b + bt_b + at_b + al256((size_t)32 * colsum_npad(p.N) * 2));
    hipError_t e;
    // dB[o][j] = s * sum_n dy[n][o] u[n][j]
    if constexpr (sizeof(T) == 2)
        e = colsum_bf16<float>(p.u, p.r, static_cast<const bf16 *>(p.dy), p.lddy, p.db, 1, p.r, p.N, p.M, p.r,
                               p.scale, ut, part, st);
    else
        e = colsum<T>(p.u, p.r, static_cast<const T *>(p.dy), p.lddy, p.db, 1, p.r, p.N, p.M, p.r, p.scale, st);
    if (e != hipSuccess) return e;
    // du = s * dy B  (B^T as the [r, M] row operand)
    if ((e = transpose<T>(static_cast<const T *>(p.b), bt, p.M, p.r, st)) != hipSuccess) return e;
    if ((e = rowdot<T>(static_cast<const T *>(p.dy), p.lddy, bt, du, p.r, p.N, p.M, p.r, p.scale,
                       st)) != hipSuccess)
        return e;
    // dA[j][k] = sum_n du[n][j] x[n][k]
    if constexpr (sizeof(T) == 2)
        e = colsum_bf16<float>(du, p.r, static_cast<const bf16 *>(p.x), p.ldx, p.da, p.K, 1, p.N, p.K, p.r, 1.f,
                               ut, part, st);
    else
        e = colsum<T>(du, p.r, static_cast<const T *>(p.x), p.ldx, p.da, p.K, 1, p.N, p.K, p.r, 1.f, st);
    if (e != hipSuccess) return e;
    if (p.dx) {
        // dx += du A  (A^T [K, r] as Wt)
        if ((e = transpose<T>(static_cast<const T *>(p.a), at, p.r, p.K, st)) != hipSuccess) return e;
        if ((e = expand<T>(du, p.r, at, static_cast<T *>(p.dx), p.lddx, p.N, p.K, p.r, 1.f, st)) !=
            hipSuccess)
            return e;
    }
    return hipSuccess;
}

}  // namespace

size_t lora_bwd_workspace_bytes(int N, int K, int M, int r, int elt) {
    const size_t base = al256((size_t)N * r * 4) + al256((size_t)r * M * elt) + al256((size_t)K * r * elt);
    if (elt != 2) return base;
    // the two colsum calls (C = M for dB, C = K for dA) share the partials
    const size_t pk = (size_t)colsum_splits(N, K) * K, pm = (size_t)colsum_splits(N, M) * M;
    return base + al256((size_t)32 * colsum_npad(N) * 2) + al256((pk > pm ? pk : pm) * 32 * 4);
}

hipError_t launch_lora_fwd(const LoraParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? lora_fwd_t<bf16>(p, s) : lora_fwd_t<float>(p, s);
}

hipError_t launch_lora_bwd(const LoraParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? lora_bwd_t<bf16>(p, s) : lora_bwd_t<float>(p, s);
}

// ---- bf16 pieces for adapters folded into the base GEMMs -----------------
hipError_t launch_lora_down_bf16(const void *x, int64_t ldx, const void *a, int N, int K, int R, float scale,
                                 void *u, int64_t ldu, hipStream_t st) {
    const bf16 *X = static_cast<const bf16 *>(x), *A = static_cast<const bf16 *>(a);
    bf16 *U = static_cast<bf16 *>(u);
    auto go = [&](auto mtc) {
        constexpr int MT = decltype(mtc)::value;
        const dim3 grid((unsigned)((N + 16 * MT - 1) / (16 * MT))), block(512);
        // R <= 64: up to four 16-column tiles per workgroup (a stack of adapters
        // that share x, e.g. q/k/v, runs as one product)
        if (R <= 16)
            hipLaunchKernelGGL((lora_rowdot16_kernel<1, bf16, MT>), grid, block, 0, st, X, ldx, A, U, ldu, N, K, R, scale);
        else if (R <= 32)
            hipLaunchKernelGGL((lora_rowdot16_kernel<2, bf16, MT>), grid, block, 0, st, X, ldx, A, U, ldu, N, K, R, scale);
        else if (R <= 48)
            hipLaunchKernelGGL((lora_rowdot16_kernel<3, bf16, MT>), grid, block, 0, st, X, ldx, A, U, ldu, N, K, R, scale);
        else
            hipLaunchKernelGGL((lora_rowdot16_kernel<4, bf16, MT>), grid, block, 0, st, X, ldx, A, U, ldu, N, K, R, scale);
    };
    switch (rowdot_slabs(N, (R + 15) / 16)) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    default: go(std::integral_constant<int, 4>{}); break;
    }
    return hipGetLastError();
}

hipError_t launch_lora_up_bf16(const void *u, int64_t ldu, const void *b, int N, int M, int R, float scale, void *y,
                               int64_t ldy, hipStream_t st) {
    return expand_mfma<bf16>(static_cast<const bf16 *>(u), ldu, static_cast<const bf16 *>(b), static_cast<bf16 *>(y),
                             ldy, N, M, R, scale, st);
}

namespace {
inline int grad_rows(int R) { return R > 32 ? 64 : 32; }
inline size_t grad_item_bytes(int N, int C, int R) {
    return al256((size_t)grad_rows(R) * colsum_npad(N) * 2) +
           al256((size_t)colsum_splits(N, C) * C * grad_rows(R) * 4);
}
}  // namespace

size_t lora_grad_many_workspace_bytes(const LoraGradItem *items, int count) {
    // sets of kGradMany products run one after another over the same bytes
    size_t most = 0;
    for (int k0 = 0; k0 < count; k0 += kGradMany) {
        size_t b = 0;
        for (int k = k0; k < count && k < k0 + kGradMany; ++k)
            b += grad_item_bytes(items[k].N, items[k].C, items[k].R);
        most = b > most ? b : most;
    }
    return most;
}

hipError_t launch_lora_grad_many_bf16(const LoraGradItem *items, int count, void *work, hipStream_t st) {
    for (int k0 = 0; k0 < count; k0 += kGradMany) {
        GradMany g{};
        g.count = count - k0 < kGradMany ? count - k0 : kGradMany;
        char *ws = static_cast<char *>(work);
        int wgs = 0, max_out = 1, max_npad = kCsRows;
        bool staged = false;
        for (int k = 0; k < g.count; ++k) {
            const LoraGradItem &it = items[k0 + k];
            GradProblem &q = g.p[k];
            q.u = static_cast<const bf16 *>(it.u);
            q.ldu = it.ldu;
            staged = staged || reinterpret_cast<uintptr_t>(it.u) % 16 != 0 || (it.ldu * 2) % 16 != 0;
            q.x = static_cast<const bf16 *>(it.x);
            q.ldx = it.ldx;
            q.out = it.grad;
            // grad [R, C] (lora_a layout): (j, c) at j * C + c; transposed [C, R]: c * R + j
            q.os_j = it.transpose ? 1 : it.C;
            q.os_c = it.transpose ? it.R : 1;
            q.s = it.scale;
            q.C = it.C;
            q.R = it.R;
            q.rw = grad_rows(it.R);
            q.N = it.N;
            q.npad = colsum_npad(it.N);
            q.splits = colsum_splits(it.N, it.C);
            q.chunk = (q.npad / kCsRows + q.splits - 1) / q.splits * kCsRows;
            q.wg0 = wgs;
            q.ut = reinterpret_cast<bf16 *>(ws);
            ws += al256((size_t)q.rw * q.npad * 2);
            q.part = reinterpret_cast<float *>(ws);
            ws += al256((size_t)q.splits * it.C * q.rw * 4);
            wgs += (it.C + kCsCols - 1) / kCsCols * q.splits;
            max_out = it.C * q.rw > max_out ? it.C * q.rw : max_out;
            max_npad = q.npad > max_npad ? q.npad : max_npad;
        }
        if (staged)
            hipLaunchKernelGGL(lora_ut_many_kernel, dim3((unsigned)((64 * max_npad + 255) / 256), (unsigned)g.count),
                               dim3(256), 0, st, g);
        if (staged)
            hipLaunchKernelGGL(lora_colsum_many_kernel<false>, dim3((unsigned)wgs), dim3(256), 0, st, g);
        else
            hipLaunchKernelGGL(lora_colsum_many_kernel<true>, dim3((unsigned)wgs), dim3(256), 0, st, g);
        hipLaunchKernelGGL(lora_colsum_reduce_many_kernel, dim3((unsigned)((max_out + 255) / 256), (unsigned)g.count),
                           dim3(256), 0, st, g);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace fa
