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

// x sigmoid(x) = x / (1 + e^-x), e^-x as 2^(-x log2 e) and the reciprocal by v_rcp_f32 (1 ulp),
// where a division takes ten instructions (an epilogue costs what its VALU instructions take).
__device__ __forceinline__ float silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> bf16, rounding to nearest even, packed lo | hi << 16 (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// f32 -> bf16 bits, rounding to nearest even.
__device__ __forceinline__ uint32_t bf16_bits(float f) { return pack_bf16x2(f, 0.f) & 0xffffu; }

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// The sum over the wave's 64 lanes, the same in every lane, in a fixed order: DPP moves within
// each row of 16 lanes (adjacent pairs, then quads, then the mirrored half row, then the
// mirrored row; each step adds two partial sums taken in the same order, so every lane of a row
// ends with the same value), then the four rows' sums read out and added in row order. No LDS
// round trip.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_move<0x141>(v);  // row_half_mirror
    v += dpp_move<0x140>(v);  // row_mirror
    return ((lane_value(v, 0) + lane_value(v, 16)) + lane_value(v, 32)) + lane_value(v, 48);
}

// ---- LDS staged by direct global-to-LDS loads, several stages in flight ----
//
// A stage of fragments lands in LDS by global_load_lds (lane l writes bytes 16 l .. of the
// fragment's 1 KiB). The compiler, seeing LDS written by such loads, waits for every load in
// flight before any ordinary LDS read; reading fragments through ds_read_b128 in asm instead
// leaves the waits to the kernel: wait_vm<N>() until at most N of this wave's loads are in flight
// (the later stages'), a barrier so that every wave's have landed, then lds_read16 and
// lds_landed() before the values are used.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ uint4 lds_read16(const uint4* p) {
    uint4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(lds_offset(p)) : "memory");
    return v;
}
// Eight fragments STRIDE bytes apart from byte `base` + OFF, the offsets in the instructions' own
// field (no address adds), in one asm statement.
template <int OFF, int STRIDE>
__device__ __forceinline__ void lds_read16_x8(uint32_t base, uint4 (&f)[8]) {
    static_assert(OFF >= 0 && OFF + 7 * STRIDE < 65536, "ds offsets hold 16 bits");
    asm volatile(
        "ds_read_b128 %0, %8 offset:%9\n\tds_read_b128 %1, %8 offset:%10\n\t"
        "ds_read_b128 %2, %8 offset:%11\n\tds_read_b128 %3, %8 offset:%12\n\t"
        "ds_read_b128 %4, %8 offset:%13\n\tds_read_b128 %5, %8 offset:%14\n\t"
        "ds_read_b128 %6, %8 offset:%15\n\tds_read_b128 %7, %8 offset:%16"
        : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]), "=&v"(f[7])
        : "v"(base), "n"(OFF), "n"(OFF + STRIDE), "n"(OFF + 2 * STRIDE), "n"(OFF + 3 * STRIDE), "n"(OFF + 4 * STRIDE),
          "n"(OFF + 5 * STRIDE), "n"(OFF + 6 * STRIDE), "n"(OFF + 7 * STRIDE)
        : "memory");
}
__device__ __forceinline__ void wait_lgkm() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// The values lds_read16 gave, usable: the wait, then each value passed through an asm the
// compiler must run after it, so that nothing reads a register before its load has returned.
template <int N>
__device__ __forceinline__ void lds_landed(uint4 (&v)[N]) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    wait_lgkm();
#pragma unroll
    for (int i = 0; i < N; ++i) {
        u32x4 t = __builtin_bit_cast(u32x4, v[i]);
        asm volatile("" : "+v"(t));
        v[i] = __builtin_bit_cast(uint4, t);
    }
}
// The values lds_read16 gave, usable once a wait for every LDS read before it has passed (an
// asm s_waitcnt lgkmcnt(0) of the caller's): each passed through an asm the compiler must run
// after that point, and no wait of its own.
template <int N>
__device__ __forceinline__ void lds_arrived(uint4 (&v)[N]) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int i = 0; i < N; ++i) {
        u32x4 t = __builtin_bit_cast(u32x4, v[i]);
        asm volatile("" : "+v"(t));
        v[i] = __builtin_bit_cast(uint4, t);
    }
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// wait_vm<N> as the compiler's own s_waitcnt, which its count of loads in flight takes in: after it
// the compiler knows the direct-to-LDS loads issued before the last N loads have landed, and
// waits for the later ones no more than their uses need (behind an asm wait it would wait for
// every load in flight before the first use of any).
template <int N>
__device__ __forceinline__ void wait_vm_seen() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    // gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in 15:14; expcnt (6:4) and lgkmcnt (11:8) at
    // their maxima, waiting for nothing.
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ void load_to_lds(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds((global_void*)src, (lds_void*)lds, 16, 0, 0);
}

// Lane l's value at lane l ^ 16 and l ^ 32, from the VALU's lane swaps (v_permlane16_swap: the
// odd rows of 16 of the first operand trade places with the even rows of the second;
// v_permlane32_swap: the upper half of the first with the lower half of the second), with no
// LDS round trip.
__device__ __forceinline__ float lane_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// A lane's two packed words of a RoPE pair's halves (lo: dimensions e, e + 1; hi: e + D / 2,
// e + 1 + D / 2) as 8 bytes of four consecutive dimensions, from a trade with lane l ^ 16, which
// holds e + 2 and e + 3 (v_permlane16_swap: the odd rows of 16 lanes of lo trade with the even
// rows of hi): an even row's lanes get lo and the partner's lo, an odd row's the partner's hi and
// hi. Every lane and its partner run it together (the same row: both spare or neither).
__device__ __forceinline__ uint2 quad_halves(uint32_t lo, uint32_t hi) {
    const auto r = __builtin_amdgcn_permlane16_swap(lo, hi, false, false);
    return make_uint2(r[0], r[1]);
}

// Two blocks' 8-byte pieces as one 16-byte piece a lane: lane l of an even row of 16 lanes holds
// columns c .. c + 3 of blocks a and b (two packed words each) and lane l ^ 16 columns c + 4 ..
// c + 7; after two v_permlane16_swap trades the even row's lane holds block a's c .. c + 7 and the
// odd row's block b's. Every lane and its partner run it together.
__device__ __forceinline__ uint4 pair_blocks(const uint32_t (&a)[2], const uint32_t (&b)[2]) {
    const auto r0 = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto r1 = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    return make_uint4(r0[0], r1[0], r0[1], r1[1]);
}

// Attention's online softmax over a turn of 16 PT keys (PT 4: a 64-key block at head_dim 64; PT 2:
// half a block at head_dim 128) for the 16 columns (query heads or (position, head) pairs) of a
// wave, from S^T = K Q^T in s[pt] (key 16 pt + 4 (lane / 16) + i, column lane % 16) and the turn's
// value fragments vin[dt KS + ks] (dimensions 16 dt .., positions 32 ks .. of the turn; KS = PT / 2):
// the running max m, kept in log2 units (scores times scale log2(e)), the running sum l of P and
// O^T in o (lane 16 g + c: column c, dimensions 16 dt + 4 g .. + 3, DT = head_dim / 16 tiles). P is
// rounded to bf16 for the product P V and summed as rounded, by an MFMA against ones. MASK: keys
// past the column's position `pos` count for nothing, and the values past `vlast` (the last
// position any column of the wave may see) read as zero: P is zero there, but a cache block past
// the position may hold anything, NaN included (a block handed on from a request that ended not
// finite), and 0 NaN is NaN. Turns wholly at or below every column's position need no mask. The
// first turn a column sees holds key 0 <= pos, so m is finite after it.
template <int PT, int DT>
struct OnlineSoftmax {
    static constexpr int KS = PT / 2;
    float m = -INFINITY, l = 0.f;
    f32x4 o[DT] = {};

    template <bool MASK>
    __device__ __forceinline__ void block(f32x4 (&s)[PT], const uint4 (&vin)[DT * KS], uint32_t p0, uint32_t pos, uint32_t vlast,
                                          float scale_log2) {
        const int lane = threadIdx.x % WAVE;
        uint4 vf[DT * KS];
#pragma unroll
        for (int i = 0; i < DT * KS; ++i) vf[i] = vin[i];
        if (MASK) {
            // Lane 16 g + d % 16 of value fragment dt KS + ks holds in its slot j the position
            // 32 ks + 16 (j / 4) + 4 g + j % 4 of the turn (value_index); word w holds slots 2 w and
            // 2 w + 1.
            const uint32_t g = (uint32_t)lane / 16;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                uint32_t keep[4];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t p = p0 + 32 * ks + 16 * (w / 2) + 4 * g + 2 * (w % 2);
                    keep[w] = (p <= vlast ? 0x0000ffffu : 0u) | (p + 1 <= vlast ? 0xffff0000u : 0u);
                }
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    uint4& f = vf[dt * KS + ks];
                    f.x &= keep[0];
                    f.y &= keep[1];
                    f.z &= keep[2];
                    f.w &= keep[3];
                }
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int pt = 0; pt < PT; ++pt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (MASK && p0 + pt * 16 + (lane / 16) * 4 + i > pos) s[pt][i] = -INFINITY;
                mx = fmaxf(mx, s[pt][i]);
            }
        mx = fmaxf(mx, lane_xor16(mx));
        mx = fmaxf(mx, lane_xor32(mx));
        const float m_new = fmaxf(m, mx * scale_log2);
        const float rescale = __builtin_amdgcn_exp2f(m - m_new);
        uint4 pf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint32_t words[4];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const f32x4 v = s[2 * ks + half];
                words[half * 2] = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(v[0], scale_log2, -m_new)),
                                              __builtin_amdgcn_exp2f(fmaf(v[1], scale_log2, -m_new)));
                words[half * 2 + 1] = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(v[2], scale_log2, -m_new)),
                                                  __builtin_amdgcn_exp2f(fmaf(v[3], scale_log2, -m_new)));
            }
            pf[ks] = make_uint4(words[0], words[1], words[2], words[3]);
        }
        // Column sums of P: every row of ones^T P is the sum (bf16 1.0 is 0x3f80).
        const uint4 ones = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) sum = mfma16(ones, pf[ks], sum);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            o[dt] *= rescale;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) o[dt] = mfma16(vf[dt * KS + ks], pf[ks], o[dt]);
        }
        l = l * rescale + sum[0];
        m = m_new;
    }
};

// scale log2(e): scores times this are in the units v_exp_f32 (2^x) takes.
__host__ __device__ constexpr float log2_scale(float scale) { return scale * 1.4426950408889634f; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, WAVE));
    return v;
}

// ---- layouts ----
//
// Weights, [N][K] row-major in the checkpoint, are kept in MFMA A-operand tiles of R rows (R of
// 4, 8 or 16, the strip height of the decoder's projections): tile (strip, kb) holds rows
// R strip .. R strip + R - 1, columns 32 kb .. 32 kb + 31, as [g][r][8] — lane 16 g + r (r < R)
// of a wave loads row r, columns 32 kb + 8 g .. + 7, 16 contiguous bytes; lanes with r >= R load
// nothing and hold zero rows. Tiles of one strip follow each other along K, so that a wave reads
// its rows as whole runs of R 64 bytes.
__host__ __device__ constexpr size_t weight_tile_index(int strip, int kb, int kblocks, int R) {
    return ((size_t)strip * kblocks + kb) * R * 32;  // in bf16 elements
}
__host__ __device__ constexpr int weight_lane_offset(int lane, int R) {
    return ((lane / 16) * R + lane % 16) * 8;
}

// The prefill's activations that feed a GEMM (the normed rows, the attention's output, the MLP's
// product), [M][K] bf16 kept as MFMA B-operand fragments of 16 rows by 32 columns, 1 KiB each,
// along K: (m, k) at fragment (m / 16, k / 32), lane 16 ((k % 32) / 8) + m % 16, slot k % 8. A
// GEMM reads each fragment as 1 KiB in a row; 8 columns k .. k + 7 (k a multiple of 8) sit
// together, as do 4.
__host__ __device__ constexpr size_t act_index(int m, int k, int K) {
    return ((size_t)(m / 16) * (K / 32) + k / 32) * 512 + (size_t)((((k % 32) / 8) * 16 + m % 16) * 8 + k % 8);
}

// The strip height of q/k/v and gate/up (the MFMA's rows); o_proj and down_proj take 4 or 16 by
// the batch (decode_residual_rows).
constexpr int QKV_ROWS = 16;

// Lane `lane`'s 16 bytes of the full 16-row fragment (strip S of 16 rows, k-block kb) of W kept
// in R-row strips: its rows r come from strip 16 S / R + r / R. For R = 16 this is lane 8.
template <int R>
__host__ __device__ constexpr size_t fragment_index(int S, int kb, int kblocks, int lane) {
    return weight_tile_index(S * (16 / R) + (lane % 16) / R, kb, kblocks, R) +
           weight_lane_offset((lane / 16) * 16 + (lane % 16) % R, R);
}

// The q/k/v projection's rows are permuted so that each strip of R holds R/2 of a head's RoPE
// pairs side by side: strip rows 2 k and 2 k + 1 are the head's rows p0 + k and p0 + k + head_dim/2
// (p0 = (s % (head_dim / R)) R/2; head_dim / R strips to a head), so that the four rows an MFMA
// lane holds of a strip are two whole pairs. Row r of strip s is original row:
__host__ __device__ constexpr int qkv_row_of(int strip, int r, int head_dim, int R) {
    return (strip / (head_dim / R)) * head_dim + (strip % (head_dim / R)) * (R / 2) + r / 2 + (r % 2) * (head_dim / 2);
}

// The paged KV cache: per layer, block and KV head, a key tile and a value tile of 64 positions
// x D dimensions (D = head_dim, 64 or 128; 64 D bf16 each), both in MFMA operand order.
//  keys: A operand of S^T = K Q^T: (p, d) at [p / 16][d / 32][lane = 16 ((d % 32) / 8) + p % 16][d % 8]
//   (a 16-position tile's D / 32 fragments together, so that 32 positions' keys are one run)
//  values: A operand of O^T = V^T P: (p, d) at [d / 16][p / 32][lane = 16 g + d % 16][s] where
//   within the 32 positions pp = p % 32 the slot is g = (pp % 16) / 4, s = pp % 4 + 4 (pp / 16),
//   the order in which a lane holds P after S^T, so P feeds the second product from registers.
constexpr int BLOCK_TOKENS = 64;
// The local stacks' head width (the encoder's and the DiT's), and the narrower of the LMs' two.
constexpr int HEAD_DIM = 64;
constexpr int KV_TILE = BLOCK_TOKENS * HEAD_DIM;  // bf16 per key or value tile at head_dim 64
__host__ __device__ constexpr int kv_tile(int head_dim) { return BLOCK_TOKENS * head_dim; }

__host__ __device__ constexpr int key_index(int p, int d, int head_dim = HEAD_DIM) {
    return (((p / 16) * (head_dim / 32) + d / 32) * 64 + ((d % 32) / 8) * 16 + p % 16) * 8 + d % 8;
}
__host__ __device__ constexpr int value_index(int p, int d) {
    return (((d / 16) * 2 + p / 32) * 64 + (((p % 32) % 16) / 4) * 16 + d % 16) * 8 + (p % 4) + 4 * ((p % 32) / 16);
}

}  // namespace tgx
