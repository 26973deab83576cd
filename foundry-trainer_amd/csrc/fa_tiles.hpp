// Global -> register -> LDS movers for 64-row bf16 tiles, used by every
// attention kernel (256 threads per workgroup).
//
// Two LDS layouts of a 64 x D tile (rows = keys or queries, D features):
//   row-major ("rm"): 64 rows of D/8 16-byte chunks, chunk XOR-swizzled with
//     the row (swz_off).  Serves MFMA operands whose lanes index rows and
//     whose 8 elements run along D.
//   transposed ("tr"): D feature rows of 64 row-entries (128 bytes), in MFMA
//     operand order within 16-row groups and chunk-swizzled (tr64_*).  Serves
//     operands whose elements run along the 64 rows (P V, P^T dO, dS^T Q,
//     dS K products).
// A "pair" load gives each thread rows (2*pp, 2*pp+1) for the same chunks, so
// one register copy can be written to both layouts.
#pragma once
#include "fa_device.hpp"

namespace fa {

template <int D>
struct Tile64 {
    static constexpr int DCH = D / 8;          // 16-byte chunks per row
    static constexpr int BYTES = 64 * D * 2;   // either layout
    static constexpr int RM_LOADS = 64 * DCH / 256;
    static constexpr int PAIR_CH = DCH / 8;    // chunks per thread and row (pair loads)
    static constexpr int PAIR_LOADS = 2 * PAIR_CH;
};

// Row-major assignment: thread covers chunk c = j*256 + tid (row c/DCH).
template <int D>
__device__ __forceinline__ void tile_load_rm(u32x4 (&r)[Tile64<D>::RM_LOADS], const bf16 *base,
                                             int64_t row_stride, int row0, int nrows, int tid) {
    using T = Tile64<D>;
#pragma unroll
    for (int j = 0; j < T::RM_LOADS; ++j) {
        const int c = j * 256 + tid, row = c / T::DCH, ch = c % T::DCH;
        r[j] = row0 + row < nrows ? ld_global_16(base + (int64_t)(row0 + row) * row_stride + ch * 8)
                                  : u32x4{0, 0, 0, 0};
    }
}

template <int D>
__device__ __forceinline__ void tile_store_rm(const u32x4 (&r)[Tile64<D>::RM_LOADS], char *dst,
                                              int tid) {
    using T = Tile64<D>;
#pragma unroll
    for (int j = 0; j < T::RM_LOADS; ++j) {
        const int c = j * 256 + tid;
        st_lds_16(dst, swz_off<T::DCH>(c / T::DCH, c % T::DCH), r[j]);
    }
}

// Pair assignment: thread holds rows 2*pp and 2*pp+1 (pp = tid % 32) for
// chunks cb + 8*j (cb = tid / 32).  r[2j] is row 2pp, r[2j+1] row 2pp+1.
template <int D>
__device__ __forceinline__ void tile_load_pairs(u32x4 (&r)[Tile64<D>::PAIR_LOADS],
                                                const bf16 *base, int64_t row_stride, int row0,
                                                int nrows, int tid) {
    using T = Tile64<D>;
    const int pp = tid & 31, cb = tid >> 5;
    const int r0 = row0 + 2 * pp;
#pragma unroll
    for (int j = 0; j < T::PAIR_CH; ++j) {
        const int ch = cb + 8 * j;
        r[2 * j] = r0 < nrows ? ld_global_16(base + (int64_t)r0 * row_stride + ch * 8)
                              : u32x4{0, 0, 0, 0};
        r[2 * j + 1] = r0 + 1 < nrows ? ld_global_16(base + (int64_t)(r0 + 1) * row_stride + ch * 8)
                                      : u32x4{0, 0, 0, 0};
    }
}

template <int D>
__device__ __forceinline__ void tile_store_tr(const u32x4 (&r)[Tile64<D>::PAIR_LOADS], char *dst,
                                              int tid) {
    using T = Tile64<D>;
    const int pp = tid & 31, cb = tid >> 5;
#pragma unroll
    for (int j = 0; j < T::PAIR_CH; ++j) {
        const int ch = cb + 8 * j;
        const u32x4 a = r[2 * j], b = r[2 * j + 1];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t lo = (a[w] & 0xffffu) | (b[w] << 16);
            const uint32_t hi = (a[w] >> 16) | (b[w] & 0xffff0000u);
            st_lds_4(dst, tr64_pair_off(ch * 8 + 2 * w, 2 * pp), lo);
            st_lds_4(dst, tr64_pair_off(ch * 8 + 2 * w + 1, 2 * pp), hi);
        }
    }
}

template <int D>
__device__ __forceinline__ void tile_store_rm_pairs(const u32x4 (&r)[Tile64<D>::PAIR_LOADS],
                                                    char *dst, int tid) {
    using T = Tile64<D>;
    const int pp = tid & 31, cb = tid >> 5;
#pragma unroll
    for (int j = 0; j < T::PAIR_CH; ++j) {
        const int ch = cb + 8 * j;
        st_lds_16(dst, swz_off<T::DCH>(2 * pp, ch), r[2 * j]);
        st_lds_16(dst, swz_off<T::DCH>(2 * pp + 1, ch), r[2 * j + 1]);
    }
}

// MFMA operand reads ------------------------------------------------------
// Row-major tile, row `row`, 16-d step kd, lane half g: 8 features
// kd*16 + g*8 .. +8 of that row.
template <int D>
__device__ __forceinline__ bf16x8 rm_frag(const char *tile, int row, int kd, int g) {
    return as_bf16x8(ld_lds_16(tile, swz_off<Tile64<D>::DCH>(row, kd * 2 + g)));
}
// Transposed tile, feature row f, 16-row step ks, lane half g.
__device__ __forceinline__ bf16x8 tr_frag(const char *tile, int f, int ks, int g) {
    return as_bf16x8(ld_lds_16(tile, tr64_read_off(f, ks, g)));
}

}  // namespace fa
