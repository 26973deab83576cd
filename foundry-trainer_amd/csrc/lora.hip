// LoRA down/up kernels for gfx950 — the adapter term of foundry-spike's
// linear_scaled (crates/foundry-spike/src/lib.rs:270-287):
//     y = x W^T (+ b) + scale * (x A^T) B^T,   A [r, K], B [M, r]
// The base GEMM x W^T is the caller's; these kernels add the rank-r term and
// produce its gradients.
//
//   rowdot  out[n][j] = s * sum_k X[n][k] W[j][k]      (x A^T, and dy B as
//           dy (B^T)^T): skinny GEMM on v_mfma_f32_32x32x16_bf16, one wave
//           per 32 rows, operands straight from global memory (16-byte loads,
//           both run along k).  HBM-bound: one read of X.
//   expand  Y[n][c] += s * sum_j U[n][j] Wt[c][j]       (y += s u B^T, and
//           dx += du A): one thread per output column and row phase, Wt rows
//           staged in LDS.  HBM-bound: one read and one write of Y.
//   colsum  out[j][c] = s * sum_n U[n][j] X[n][c]      (dB^T = s u^T dy and
//           dA = du^T x): each workgroup owns 64 columns and sweeps all rows
//           in a fixed order — deterministic, no atomics.
#include "fa_device.hpp"
#include "fa_kernels.hpp"

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

// Small transpose [R][C] -> [C][R] (dtype).
template <typename T>
__global__ void lora_transpose_kernel(const T *__restrict__ src, T *dst, int R, int C) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)R * C) return;
    const int r = e / C, c = e % C;
    dst[(int64_t)c * R + r] = src[e];
}

template <typename T>
hipError_t rowdot(const T *X, int64_t ldx, const T *W, float *out, int64_t ldo, int N, int K,
                  int R, float s, hipStream_t st) {
    const dim3 grid((N + 127) / 128), block(256);
    hipLaunchKernelGGL(lora_rowdot_kernel<T>, grid, block, 0, st, X, ldx, W, out, ldo, N, K, R, s);
    return hipGetLastError();
}

template <typename T>
hipError_t expand(const float *U, int64_t ldu, const T *Wt, T *Y, int64_t ldy, int N, int C,
                  int R, float s, hipStream_t st) {
    const int rpb = 64;
    const dim3 grid((C + 63) / 64, (N + rpb - 1) / rpb), block(256);
    hipLaunchKernelGGL(lora_expand_kernel<T>, grid, block, 0, st, U, ldu, Wt, Y, ldy, N, C, R, s,
                       rpb);
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

// Workspace layout (bytes, each 256-aligned): du f32 [N, r] | B^T [r, M] | A^T [K, r]
template <typename T>
hipError_t lora_bwd_t(const LoraParams &p, hipStream_t st) {
    char *ws = reinterpret_cast<char *>(p.work);
    float *du = reinterpret_cast<float *>(ws);
    const size_t du_b = ((size_t)p.N * p.r * 4 + 255) & ~size_t(255);
    T *bt = reinterpret_cast<T *>(ws + du_b);
    const size_t bt_b = ((size_t)p.r * p.M * sizeof(T) + 255) & ~size_t(255);
    T *at = reinterpret_cast<T *>(ws + du_b + bt_b);
    hipError_t e;
    // dB[o][j] = s * sum_n dy[n][o] u[n][j]
    if ((e = colsum<T>(p.u, p.r, static_cast<const T *>(p.dy), p.lddy, p.db, 1, p.r, p.N, p.M, p.r,
                       p.scale, st)) != hipSuccess)
        return e;
    // du = s * dy B  (B^T as the [r, M] row operand)
    if ((e = transpose<T>(static_cast<const T *>(p.b), bt, p.M, p.r, st)) != hipSuccess) return e;
    if ((e = rowdot<T>(static_cast<const T *>(p.dy), p.lddy, bt, du, p.r, p.N, p.M, p.r, p.scale,
                       st)) != hipSuccess)
        return e;
    // dA[j][k] = sum_n du[n][j] x[n][k]
    if ((e = colsum<T>(du, p.r, static_cast<const T *>(p.x), p.ldx, p.da, p.K, 1, p.N, p.K, p.r,
                       1.f, st)) != hipSuccess)
        return e;
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
    const size_t du_b = ((size_t)N * r * 4 + 255) & ~size_t(255);
    const size_t bt_b = ((size_t)r * M * elt + 255) & ~size_t(255);
    const size_t at_b = ((size_t)K * r * elt + 255) & ~size_t(255);
    return du_b + bt_b + at_b;
}

hipError_t launch_lora_fwd(const LoraParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? lora_fwd_t<bf16>(p, s) : lora_fwd_t<float>(p, s);
}

hipError_t launch_lora_bwd(const LoraParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? lora_bwd_t<bf16>(p, s) : lora_bwd_t<float>(p, s);
}

}  // namespace fa
