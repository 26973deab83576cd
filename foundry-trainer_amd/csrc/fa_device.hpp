// Device-side helpers shared by the gfx950 kernels: vector types, the
// bf16 MFMA wrappers, conversions, LDS swizzles and the XCD-aware block map.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// v_mfma_f32_32x32x16_bf16.  Operand lane layout (wave64):
//   A[m][k]: lane = m + 32*(k/8), element k%8     (m, k < 32, 16)
//   B[k][n]: lane = n + 32*(k/8), element k%8
//   C[m][n]: lane = n + 32*((m/4)%2), element (m/8)*4 + m%4
// Only the m/n placement matters to the kernels: any k permutation applied
// identically to A and B leaves the product unchanged.
__device__ __forceinline__ f32x16 mfma_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16: A[m][k] lane = m + 16*(k/8) (8 consecutive k per
// lane), B[k][n] lane = n + 16*(k/8); D element i of lane l is
// D[4*(l/16) + i][l%16].
__device__ __forceinline__ f32x4 mfma_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x2_f32: A[m][k] lane = m + 32*k, B[k][n] lane = n + 32*k.
__device__ __forceinline__ f32x16 mfma_32x32x2_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row index (within a 32-row tile) of accumulator element r of `lane`.
__device__ __forceinline__ int acc_row(int r, int lane) {
    return (r >> 2) * 8 + ((lane >> 5) << 2) + (r & 3);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_fast(float x) { return __builtin_amdgcn_logf(x); }

__device__ __forceinline__ float bf16_to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ bf16 f32_to_bf16(float x) { return (bf16)x; }  // RNE

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v = {(bf16)lo, (bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ u32x4 ld_global_16(const void *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}
__device__ __forceinline__ void st_global_16(void *p, u32x4 v) {
    *reinterpret_cast<u32x4 *>(p) = v;
}
__device__ __forceinline__ u32x4 ld_lds_16(const char *smem, int byte_off) {
    return *reinterpret_cast<const u32x4 *>(smem + byte_off);
}
__device__ __forceinline__ void st_lds_16(char *smem, int byte_off, u32x4 v) {
    *reinterpret_cast<u32x4 *>(smem + byte_off) = v;
}
__device__ __forceinline__ void st_lds_4(char *smem, int byte_off, uint32_t v) {
    *reinterpret_cast<uint32_t *>(smem + byte_off) = v;
}

// Bit casts take their operand BY VALUE: clang's __builtin_bit_cast applied
// directly to a vector-element lvalue (v[i]) reads element 0 whatever i is.
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ bf16x2 u32_as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2, v); }
__device__ __forceinline__ u32x4 as_u32x4(bf16x8 v) { return __builtin_bit_cast(u32x4, v); }

// Swap values between lane l and lane l^32.
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// max / sum of a lane's value and its lane ^ 32 partner in one VALU exchange
// (v_permlane32_swap: the returned pair is (x[l], x[l+32]) on lanes < 32 and
// (x[l-32], x[l]) on lanes >= 32, so both halves combine the same operands in
// the same order and get bit-identical results).
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Map a linear block id to a logical work id so that consecutive logical ids
// land on the same XCD.  Workgroups are dispatched round-robin over the 8
// XCDs (bid % 8); tiles of one (b, h) then share that XCD's L2 for K and V.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    const int q = nblocks >> 3, r = nblocks & 7;
    const int x = bid & 7, i = bid >> 3;
    return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
}

// Range split: a sequence of S rows (queries or keys) is cut into 128-row
// chunks, and partition `part` of `split` covers chunks [c0, c1).  Work ids
// of a split grid run (b*H + h, part, tile), so the tiles that stream the
// same range are neighbours and share an XCD's L2.
constexpr int kSplitChunk = 128;
__host__ __device__ __forceinline__ void split_chunks(int S, int split, int part, int &c0, int &c1) {
    const int nc = (S + kSplitChunk - 1) / kSplitChunk;
    c0 = part * nc / split;
    c1 = (part + 1) * nc / split;
}

}  // namespace fa
