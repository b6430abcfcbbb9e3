// Device-side building blocks shared by the gfx950 kernels: bf16 packing, the 16x16x32 bf16 MFMA,
// wave reductions with a fixed order, and the tile layouts weights and caches are kept in.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tgx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

// A 16x16 block of C += A (16 x 32) * B (32 x 16), bf16 in, f32 accumulate. Lane l holds row
// l % 16 of A and column l % 16 of B, each with 8 of the 32 k in the same slots, and column
// l % 16, rows 4 (l / 16) .. 4 (l / 16) + 3 of C.
__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// f32 -> bf16 bits, rounding to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return bf16_bits(lo) | (bf16_bits(hi) << 16);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// The sum over the wave's 64 lanes, the same in every lane: a butterfly, then lane 0's value
// broadcast, so that every lane uses one rounding of it.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
    return __shfl(v, 0, WAVE);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, WAVE));
    return v;
}

// ---- layouts ----
//
// Weights, [N][K] row-major in the checkpoint, are kept in MFMA A-operand tiles: tile (n, kb) of
// 16 rows and 32 columns is 64 lanes x 8 bf16 (1 KiB), lane l holding row 16 n + l % 16, columns
// 32 kb + 8 (l / 16) .. + 7. Tiles of one strip of 16 rows follow each other along K, so that a
// wave reads its rows as whole 1 KiB runs.
__host__ __device__ constexpr size_t weight_tile_index(int n_strip, int kb, int kblocks) {
    return ((size_t)n_strip * kblocks + kb) * 512;  // in bf16 elements
}

// The q/k/v projection's rows are permuted so that each strip of 16 holds 8 of a head's RoPE
// pairs: strip rows 0..7 are the head's rows 8 q .. 8 q + 7 and rows 8..15 those 32 further
// (head_dim 64, four strips to a head). Row r of strip (head h, quarter q) is original row:
__host__ __device__ constexpr int qkv_row_of(int strip, int r, int head_dim) {
    return (strip / (head_dim / 16)) * head_dim + (strip % (head_dim / 16)) * 8 + (r < 8 ? r : head_dim / 2 + r - 8);
}

// The paged KV cache: per layer, block and KV head, a key tile and a value tile of 64 positions
// x 64 dimensions (4096 bf16 each), both in MFMA operand order.
//  keys: A operand of S^T = K Q^T: (p, d) at [p / 16][d / 32][lane = 16 ((d % 32) / 8) + p % 16][d % 8]
//  values: A operand of O^T = V^T P: (p, d) at [d / 16][p / 32][lane = 16 g + d % 16][s] where
//   within the 32 positions pp = p % 32 the slot is g = (pp % 16) / 4, s = pp % 4 + 4 (pp / 16),
//   the order in which a lane holds P after S^T, so P feeds the second product from registers.
constexpr int BLOCK_TOKENS = 64;
constexpr int HEAD_DIM = 64;
constexpr int KV_TILE = BLOCK_TOKENS * HEAD_DIM;  // bf16 per key or value tile

__host__ __device__ constexpr int key_index(int p, int d) {
    return (((p / 16) * 2 + d / 32) * 64 + ((d % 32) / 8) * 16 + p % 16) * 8 + d % 8;
}
__host__ __device__ constexpr int value_index(int p, int d) {
    return (((d / 16) * 2 + p / 32) * 64 + (((p % 32) % 16) / 4) * 16 + d % 16) * 8 + (p % 4) + 4 * ((p % 32) / 16);
}

}  // namespace tgx
