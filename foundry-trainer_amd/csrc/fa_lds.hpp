// LDS movement for gfx950 attention kernels: direct buffer->LDS tile loads
// and the operand reads that consume them.
//
// Tile layout: R rows x D bf16 features, row-major, 2*D bytes per row, the
// 16-byte chunk c of row r stored at chunk position c ^ chunk_swz<D>(r).
//
// Loads: `buffer_load_dwordx4 ... lds` writes lane l's 16 bytes to
// LDS[M0 + 16*l], so a wave-instruction fills 1 KiB of the tile; each lane
// picks the global chunk that belongs at its LDS slot (this is where the
// swizzle is applied).  The buffer resource's num_records bounds the tensor:
// rows past the end read as zero, with 32-bit offsets only.
//
// Operand reads:
//   row fragment  (ds_read_b128): 8 consecutive features of one row — the
//                 MFMA operand whose lanes index rows (Q/K/V/dO as stored).
//   col fragment  (2 x ds_read_b64_tr_b16): 8 rows of one feature — the
//                 operand whose lanes index features and whose elements run
//                 along rows (V^T, dO^T, Q^T, K^T).  Within each 16-lane
//                 group the instruction hands lane i element (i % 4) of the
//                 8 bytes addressed by lane 4e + i/4 (e = 0..3); pointing lane
//                 j at row base + j/4, features f0 + 4*(j % 4) gives lane i the
//                 four values X[base + e][f0 + i].
#pragma once
#include "fa_device.hpp"

namespace fa {

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    // raw buffer, stride 0, 32-bit data format (GFX9 word 3)
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// Live key blocks under a key-padding mask.  Bit kb of `words` is set when
// block kb (keys [kb*BLK, kb*BLK + BLK) of one batch item) holds a kept key;
// the kernels then stream only live blocks.  kLiveWords words track
// kLiveWords*32 blocks; a range with more blocks is not tracked (every block
// treated as live).  Built once per workgroup in two steps, so that the
// keep-byte loads share their latency with the kernel's first loads:
//   live_mask_issue: zero `words` and issue the keep-byte loads of the first
//     batch: wave w takes the U consecutive blocks kb0 + w*U .. + U - 1, one
//     byte per lane per load (BLK/64 loads per block) through a buffer
//     resource over the row's S bytes, so keys past S read as zero;
//   (the caller issues its own first loads, then a barrier that waits for
//    LDS writes and for the keep bytes)
//   live_mask_finish: one ballot per block, the wave's live bits gathered
//     in a scalar register (blocks >= kb1 dropped) and ORed into at most two
//     words; further batches of U*NW blocks when the range has more; the
//     caller's next barrier publishes the words.
constexpr int kLiveWords = 128;
template <int BLK, int U>
__device__ __forceinline__ void live_mask_load(__amdgpu_buffer_rsrc_t keep_rs, int first, uint32_t (&v)[U]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        v[u] = 0u;
#pragma unroll
        for (int j = 0; j < BLK; j += 64)
            v[u] |= __builtin_amdgcn_raw_buffer_load_b8(keep_rs, (first + u) * BLK + j + lane, 0, 0);
    }
}

template <int NW, int BLK, int U>
__device__ __forceinline__ void live_mask_issue(__amdgpu_buffer_rsrc_t keep_rs, int kb0, uint32_t *words,
                                                uint32_t (&v)[U]) {
    static_assert(U <= 32, "a wave's blocks span at most two words");
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int i = tid; i < kLiveWords; i += NW * 64) words[i] = 0u;
    live_mask_load<BLK, U>(keep_rs, kb0 + wave * U, v);
}

template <int NW, int BLK, int U>
__device__ __forceinline__ void live_mask_finish(__amdgpu_buffer_rsrc_t keep_rs, int kb0, int kb1, uint32_t *words,
                                                 uint32_t (&v)[U]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    for (int base = kb0;; base += U * NW) {
        const int first = base + wave * U;
        uint32_t m = 0u;  // bit u: block first + u is live (wave-uniform)
#pragma unroll
        for (int u = 0; u < U; ++u) m |= (__ballot(v[u] != 0u) != 0ull ? 1u : 0u) << u;
        const int n = kb1 - first;  // blocks of this wave inside the range
        m = n <= 0 ? 0u : n >= 32 ? m : m & ((1u << n) - 1u);
        if (m != 0u && lane == 0) {
            const uint64_t mm = (uint64_t)m << (first & 31);
            atomicOr(&words[first >> 5], (uint32_t)mm);
            if ((uint32_t)(mm >> 32)) atomicOr(&words[(first >> 5) + 1], (uint32_t)(mm >> 32));
        }
        if (base + U * NW >= kb1) break;
        live_mask_load<BLK, U>(keep_rs, base + U * NW + wave * U, v);
    }
}

// First live block >= from (wave-uniform), or `end` when blocks [from, end)
// hold no kept key.  `words` as built by build_live_mask over [kb0, end).
__device__ __forceinline__ int next_live_block(const uint32_t *words, int from, int end) {
    if (from >= end) return end;
    int w = from >> 5;
    uint32_t bits = __builtin_amdgcn_readfirstlane(words[w]) & (~0u << (from & 31));
    const int wend = (end + 31) >> 5;
    while (bits == 0u) {
        if (++w >= wend) return end;
        bits = __builtin_amdgcn_readfirstlane(words[w]);
    }
    const int r = (w << 5) + __builtin_ctz(bits);
    return r < end ? r : end;
}

// One wave-instruction: 16 bytes per lane from rsrc at (voff + soff) to
// LDS[dst + 16*lane].  dst must be wave-uniform.
__device__ __forceinline__ void buffer_to_lds_16(__amdgpu_buffer_rsrc_t rsrc, char *dst, uint32_t voff,
                                                 uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)dst, 16,
                                             voff, soff, 0, 0);
}

// 4 bytes per lane to LDS[dst + 4*lane] (a 64-entry f32 vector per wave).
__device__ __forceinline__ void buffer_to_lds_4(__amdgpu_buffer_rsrc_t rsrc, char *dst, uint32_t voff,
                                                uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)dst, 4,
                                             voff, soff, 0, 0);
}

// Workgroup barrier that keeps buffer->LDS loads in flight.  __syncthreads()
// drains every outstanding one (its workgroup release fence counts them as
// pending LDS writes), which would cap a prefetch at one stage.  Here each
// wave first waits until at most VM of its vector-memory loads are
// outstanding (the DMA the next reads need has landed) and for its own LDS
// reads, then meets the others; the "memory" clobbers keep the compiler from
// moving LDS accesses across the barrier.
#define FA_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(" #n ") lgkmcnt(0)" ::: "memory")
template <int VM>
__device__ __forceinline__ void barrier_keep_dma() {
    static_assert(VM >= 0 && VM <= 12, "vmcnt literal");
    if constexpr (VM == 0) FA_WAIT_VM(0);
    else if constexpr (VM == 1) FA_WAIT_VM(1);
    else if constexpr (VM == 2) FA_WAIT_VM(2);
    else if constexpr (VM == 3) FA_WAIT_VM(3);
    else if constexpr (VM == 4) FA_WAIT_VM(4);
    else if constexpr (VM == 5) FA_WAIT_VM(5);
    else if constexpr (VM == 6) FA_WAIT_VM(6);
    else if constexpr (VM == 7) FA_WAIT_VM(7);
    else if constexpr (VM == 8) FA_WAIT_VM(8);
    else if constexpr (VM == 9) FA_WAIT_VM(9);
    else if constexpr (VM == 10) FA_WAIT_VM(10);
    else if constexpr (VM == 11) FA_WAIT_VM(11);
    else FA_WAIT_VM(12);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
#undef FA_WAIT_VM

// Wait until at most VM of this wave's vector-memory loads are outstanding
// (no barrier: for LDS a wave fills and reads itself).
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(VM >= 0 && VM <= 8, "vmcnt literal");
    if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if constexpr (VM == 1) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
    else if constexpr (VM == 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else if constexpr (VM == 3) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
    else if constexpr (VM == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if constexpr (VM == 5) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
    else if constexpr (VM == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    else if constexpr (VM == 7) asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
}

// Replace elements 4*half .. 4*half+3 of an MFMA operand with two packed words.
__device__ __forceinline__ void set_half(bf16x8 &v, int half, u32x2 w) {
    u32x4 u = as_u32x4(v);
    u[2 * half] = w[0];
    u[2 * half + 1] = w[1];
    v = as_bf16x8(u);
}

// XOR key of row r's chunks.  Two read shapes must both hit distinct banks:
//   row fragments: 16 consecutive rows at one logical chunk -> the key must
//     be a bijection of r % 16 (of r % 8 within any 8 aligned rows);
//   transpose reads: 4 aligned rows x 2 (or 4) adjacent chunks -> the keys of
//     the 4 rows must differ in chunk bits 1..2 (and 2..3).
// The plain key r % 16 fails the second (rows 4i..4i+3 only permute chunks
// inside one aligned group).  With r = (r3 r2 r1 r0):
//   key = (r1^r3) << 3 | r0 << 2 | r1 << 1 | (r2^r1)
// is linear and invertible over GF(2) (r0 = k2, r1 = k1, r2 = k0^k1,
// r3 = k3^k1), and over the 4 rows of a transpose read (r2, r3 fixed) bits
// 1..2 take (r1, r0) and bits 2..3 take (r0, r1^r3): all distinct.  It depends
// on r % 16 only.  D = 64 tiles have 8 chunks per row and use bits 0..2,
// D = 32 tiles (4 chunks) bits 0..1.
template <int D>
__device__ __forceinline__ int chunk_swz(int row) {
    static_assert(D == 32 || D == 64 || D == 128, "tile widths of 32, 64 or 128 features");
    const int r0 = row & 1, r1 = (row >> 1) & 1, r2 = (row >> 2) & 1, r3 = (row >> 3) & 1;
    const int k = (r2 ^ r1) | (r1 << 1) | (r0 << 2);
    return D >= 128 ? (k | ((r1 ^ r3) << 3)) : D == 64 ? k : (k & 3);
}

// Tile geometry for a D-feature bf16 tile of `ROWS` rows.
template <int D, int ROWS>
struct LdsTile {
    static constexpr int ROWB = 2 * D;               // bytes per row
    static constexpr int DCH = D / 8;                // chunks per row
    static constexpr int BYTES = ROWS * ROWB;
    static constexpr int WAVE_INSTS = BYTES / 1024;  // wave-instructions per tile
};

// Byte offset (relative to the tensor row base of the tile's first row) of
// the global chunk that lane `lane` of wave-instruction `inst` must fetch.
template <int D>
__device__ __forceinline__ uint32_t tile_src_off(int inst, int lane, int64_t row_stride_elems) {
    constexpr int DCH = D / 8;
    const int c = inst * 64 + lane;              // physical chunk index in the tile
    const int row = c / DCH, phys = c % DCH;
    const int logical = phys ^ chunk_swz<D>(row);
    return (uint32_t)((row * row_stride_elems + logical * 8) * 2);
}

// Wave-instruction `inst` of a tile covers rows inst*(1024/ROWB) ..; with
// NW waves sharing a tile, wave w issues instructions w, w+NW, ...  For a
// D=128 tile those are 4*NW rows apart (16 or 32), a multiple of the chunk
// swizzle's 16-row period, so they share one per-lane offset and differ only
// by the uniform row step (added to the scalar offset).
template <int D, int NW = 4>
__device__ __forceinline__ uint32_t tile_inst_row_step(int64_t row_stride_elems) {
    return (uint32_t)(NW * (1024 / (2 * D)) * row_stride_elems * 2);
}

// Row-fragment addressing split into a per-lane base and an XOR key:
//   offset(kd) = base + (((kd*2) ^ key) << 4)
// for row `row` (lane's row), lane half g.
struct RowFragAddr {
    uint32_t base, key;
};
template <int D>
__device__ __forceinline__ RowFragAddr row_frag_addr(int row, int g) {
    return {(uint32_t)(row * 2 * D), (uint32_t)(g ^ chunk_swz<D>(row))};
}
__device__ __forceinline__ uint32_t row_frag_at(RowFragAddr a, int kd) {
    return a.base + (((uint32_t)(kd * 2) ^ a.key) << 4);
}

// Column-fragment addressing for half `half`: offset(ft) = base + (((ft*4) ^ key) << 4)
// (valid for D = 128, where chunk = ft*4 + x with x < 4; for D = 64 the same
// form holds with ft*4 < 8).
struct ColFragAddr {
    uint32_t base, key;
};
template <int D>
__device__ __forceinline__ ColFragAddr col_frag_addr(int half, int lane) {
    const int j = lane & 15, G = lane >> 4;
    const int g = G >> 1, dhalf = G & 1;
    const int row = half * 8 + g * 4 + (j >> 2);
    const int f = dhalf * 16 + 4 * (j & 3);  // feature within the 32-feature tile
    const int x = f >> 3;                    // chunk within the tile, < 4
    return {(uint32_t)(row * 2 * D + (f & 7) * 2), (uint32_t)(x ^ chunk_swz<D>(row))};
}
__device__ __forceinline__ uint32_t col_frag_at(ColFragAddr a, int ft) {
    return a.base + (((uint32_t)(ft * 4) ^ a.key) << 4);
}
// The rows +8 half (col_frag_addr(1, lane)) from the rows +0 half: for D = 128
// chunk_swz(r + 8) = chunk_swz(r) ^ 8 swaps feature tiles dt and dt ^ 2; for
// D = 64 the key does not depend on row bit 3.
template <int D>
__device__ __forceinline__ uint32_t col_frag_at_hi8(ColFragAddr a0, int ft) {
    return col_frag_at(a0, D >= 128 ? ft ^ 2 : ft) + 8 * 2 * D;
}

// Row fragment: row `row`, features kd*16 + g*8 .. +8.
template <int D>
__device__ __forceinline__ uint32_t row_frag_off(int row, int kd, int g) {
    return (uint32_t)(row * 2 * D + (((kd * 2 + g) ^ chunk_swz<D>(row)) << 4));
}

__device__ __forceinline__ bf16x8 lds_read_row_frag(const char *smem, uint32_t off) {
    return as_bf16x8(*reinterpret_cast<const u32x4 *>(smem + off));
}

// Column-fragment lane address for the 4-row half `half` (0: rows +0..3 of
// the lane half's group, 1: rows +8..11) of a 16-row k-step, feature tile
// `ft` (32 features).  lane -> group G = lane/16, j = lane%16, g = lane/32.
template <int D>
__device__ __forceinline__ uint32_t col_frag_off(int ks, int half, int ft, int lane) {
    const int j = lane & 15, G = lane >> 4;
    const int g = G >> 1, dhalf = G & 1;
    const int row = ks * 16 + half * 8 + g * 4 + (j >> 2);
    const int f = ft * 32 + dhalf * 16 + 4 * (j & 3);
    return (uint32_t)(row * 2 * D + (((f >> 3) ^ chunk_swz<D>(row)) << 4) + (f & 7) * 2);
}

// Column-fragment offset of the rows +8 half from the rows +0 offsets of all
// feature tiles: chunk_swz(r + 8) = chunk_swz(r) ^ 8 flips chunk bit 3, which
// is feature tile bit 1 (D = 128) — so it is tile dt ^ 2 of the +0 half moved
// down 8 rows, an immediate.  For D = 64 (8 chunks) bit 3 is not used and the
// +8 half is the same tile.
template <int D>
__device__ __forceinline__ uint32_t col_frag_hi8(const uint32_t *off0, int dt) {
    return (D >= 128 ? off0[dt ^ 2] : off0[dt]) + 8 * 2 * D;
}

__device__ __forceinline__ i16x4 lds_read_tr16(const char *smem, uint32_t off) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4 *)(smem + off));
}

// Column fragment from two transpose reads: elements 0..3 from `off0`
// (rows +g*4+0..3), 4..7 from `off1` (rows +8+g*4+0..3).  This is the k order
// of an S^T / dS^T accumulator used as the other MFMA operand.
__device__ __forceinline__ bf16x8 lds_read_col_frag(const char *smem, uint32_t off0, uint32_t off1) {
    const i16x4 a = lds_read_tr16(smem, off0), b = lds_read_tr16(smem, off1);
    typedef short i16x8 __attribute__((ext_vector_type(8)));
    const i16x8 v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(bf16x8, v);
}

}  // namespace fa
