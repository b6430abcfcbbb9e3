// The local stack and the patch sampler on gfx950 (crates/graph/src/local/mod.rs:354-656 with
// local_{norm,qkv_rope,attention,partial,add_norm,gate_up}.comp; crates/graph/src/local/dit.rs
// with local_embed.comp, dit_euler.comp and cfm_noise.comp):
//
//   local_gemm      C = X W^T over up to a few hundred tokens, bf16 in, f32 accumulate: up to 64
//                   tokens straight from memory into each wave's registers beside its strips of
//                   W (local_gemm_direct); more in 64-token tiles streamed through a ring of LDS
//                   slots, read by the waves of a workgroup that each stream their own strips of
//                   W (local_gemm_ring). The epilogue fused: the row's RMSNorm scale with RoPE at
//                   each token's place in its sequence (local_qkv_rope.comp), the same scale with
//                   SiLU(gate) up (local_gate_up.comp), the f32 sums of one part of the columns
//                   (local_partial.comp), or over more than 64 tokens the parts added, the
//                   residual added and the next norm's input with its sums of squares
//                   (local_add_norm.comp)
//   local_attention every token of a sequence attends to every token of it, a wave to a
//                   sequence and query head, both products on MFMA (local_attention.comp)
//   local_add_norm  residual + the parts' sums in their order, then the next norm's input
//                   (local_add_norm.comp, local_norm.comp): up to 64 tokens, and the first and
//                   final norms
//   local_embed     a linear layer over a patch's frames into tokens, and tokens copied beside
//                   them (local_embed.comp)
//   dit_euler       out_proj's velocities, CFG-Zero* guidance and the Euler step (dit_euler.comp)
//   cfm_noise       x = temperature noise (cfm_noise.comp)
//
// The projections read each weight once for every token of a workgroup's tile, and a token's
// sums run in the same order whatever else is in its tile, so a row samples the same patch beside
// other rows as it does alone.
#include "local_kernels.hpp"

#include <math.h>

#include "dispatch.hpp"

namespace tgx {

namespace {


// The sums of squares of a row: one to each LOCAL_SQ_COLS columns (16 at hidden 1024), in
// column order. Each is four sums of 16 columns added as (a + b) + (c + d), each of those four of
// 4 columns, added as (a + b) + (c + d) again, each of those 4 squared and added in order from
// zero by fused multiply-adds: the order local_add_norm's lanes and local_gemm_ring's epilogue
// both keep, so that a row's scale is the same bits whichever wrote it.
constexpr int SQ_PARTS = 1024 / LOCAL_SQ_COLS;
__device__ __forceinline__ float squares4(float a, float b, float c, float d) {
    float s = 0.f;
    s = fmaf(a, a, s);
    s = fmaf(b, b, s);
    s = fmaf(c, c, s);
    return fmaf(d, d, s);
}
// The sum of squares of a token's LOCAL_SQ_COLS columns held a column to a lane (lane l: column l
// of the span), in the order above, by the VALU's lane moves: squares4 over lanes 4 i .. 4 i + 3
// (each quad's values broadcast, quad_perm), (a + b) + (c + d) over those of each 16 lanes (the
// 16 rotated right 12, 8 and 4 lanes, row_ror: the first lane of a 16 then holds lanes +4, +8,
// +12), then over the four 16s (lanes l ^ 16, l ^ 32). Every lane of the wave takes part; lane 0
// has the sum.
__device__ __forceinline__ float span_squares(float v) {
    const float s = squares4(dpp_move<0x00>(v), dpp_move<0x55>(v), dpp_move<0xAA>(v), dpp_move<0xFF>(v));
    const float t = (s + dpp_move<0x12C>(s)) + (dpp_move<0x128>(s) + dpp_move<0x124>(s));
    const float u = t + lane_xor16(t);
    return u + lane_xor32(u);
}
// 1 / rms of a row from its SQ_PARTS sums of squares, added in order.
__device__ __forceinline__ float row_scale_of(const float4 (&p)[SQ_PARTS / 4], int K, float eps) {
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < SQ_PARTS / 4; ++i) {
        total += p[i].x;
        total += p[i].y;
        total += p[i].z;
        total += p[i].w;
    }
    return 1.0f / sqrtf(total / (float)K + eps);
}
// A row's sums of squares, loaded ahead of the GEMM's own loads and pinned there (nothing
// computed from them moves above the point where they are settled).
struct RowSq {
    float4 p[SQ_PARTS / 4];
    __device__ void load(const float* row_sq, int m) {
#pragma unroll
        for (int i = 0; i < SQ_PARTS / 4; ++i) p[i] = *reinterpret_cast<const float4*>(row_sq + (size_t)m * SQ_PARTS + 4 * i);
    }
    __device__ void settle() {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int i = 0; i < SQ_PARTS / 4; ++i) {
            u32x4 t = __builtin_bit_cast(u32x4, p[i]);
            asm volatile("" : "+v"(t));
            p[i] = __builtin_bit_cast(float4, t);
        }
    }
};

// A wave's strips of W for work unit u: SW strips in a row, or for the gate/up projection (SW 2)
// gate strip u and the same rows of up, N / 32 strips on.
template <int EPI, int SW>
__device__ __forceinline__ void local_strips(int u, int N, int (&strip)[SW]) {
    static_assert(EPI != LEPI_SILU || SW == 2, "gate/up takes a gate strip and its up strip");
    if (EPI == LEPI_SILU) {
        strip[0] = u;
        strip[SW - 1] = u + N / 32;
    } else {
#pragma unroll
        for (int s = 0; s < SW; ++s) strip[s] = u * SW + s;
    }
}

// The epilogue of one 16 x 16 block: W rows 16 strip + 4 (lane / 16) + i against token
// mt + lane % 16, whose row scale is rs (QKV, SILU). SILU takes the gate's block in `acc` and the
// up's in `up`.
template <int EPI>
__device__ __forceinline__ void local_store(const LocalArgs& a, const LocalGemm& g, int strip, int mt, const f32x4& acc,
                                            const f32x4& up, float rs) {
    const int lane = threadIdx.x % WAVE, quad = lane / 16;
    const int m = mt + lane % 16;
    if (EPI == LEPI_PARTIAL) {
        const int n = strip * 16 + quad * 4;
        *reinterpret_cast<float4*>(g.partial + ((size_t)blockIdx.z * a.M_pad + m) * g.N + n) =
            make_float4(acc[0], acc[1], acc[2], acc[3]);
    } else if (EPI == LEPI_SILU) {
        if (m >= a.M) return;
        const int inner = g.N / 2, n = strip * 16 + quad * 4;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float gate = acc[i] * rs, u = up[i] * rs;
            v[i] = silu(gate) * u;
        }
        *reinterpret_cast<uint2*>(g.mlp + act_index(m, n, inner)) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    } else if (EPI == LEPI_QKV) {  // a lane's four rows of a strip are two RoPE pairs (qkv_row_of)
        const int H = a.heads, KV = a.kv_heads;
        const int head = strip / 4, qtr = strip % 4;
        // Rows 4 quad .. 4 quad + 3 of the strip: the pairs of dimensions (e, e + 32) and
        // (e + 1, e + 33), each first half then second; lanes l and l ^ 16 (the same token) trade
        // halves for the stores: the even quad stores dimensions e .. e + 3, the odd one
        // e + 30 .. e + 33.
        const int e = qtr * 8 + quad * 2;
        const int d0 = (quad & 1) ? e - 2 + HEAD_DIM / 2 : e;
        float lo[2], hi[2];  // dimensions e + k and e + k + 32
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            lo[k] = acc[2 * k] * rs;
            hi[k] = acc[2 * k + 1] * rs;
        }
        if (head < H + KV && a.rope) {
            const int place = m % a.T;
            const float2 co = *reinterpret_cast<const float2*>(a.cos + place * (HEAD_DIM / 2) + e);
            const float2 si = *reinterpret_cast<const float2*>(a.sin + place * (HEAD_DIM / 2) + e);
            // As upstream: x cos + rotate_half(x) sin (local_qkv_rope.comp:71-76), a pair
            // (x1, x2) to (x1 cos - x2 sin, x2 cos + x1 sin).
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const float cs = k ? co.y : co.x, sn = k ? si.y : si.x;
                const float x1 = lo[k], x2 = hi[k];
                lo[k] = __builtin_fmaf(x1, cs, -(x2 * sn));
                hi[k] = __builtin_fmaf(x2, cs, x1 * sn);
            }
        }
        const uint2 packed = quad_halves(pack_bf16x2(lo[0], lo[1]), pack_bf16x2(hi[0], hi[1]));
        if (m >= a.M) return;
        if (head < H)
            *reinterpret_cast<uint2*>(g.q + ((size_t)m * H + head) * HEAD_DIM + d0) = packed;
        else if (head < H + KV)
            *reinterpret_cast<uint2*>(g.k + ((size_t)m * KV + head - H) * HEAD_DIM + d0) = packed;
        else
            *reinterpret_cast<uint2*>(g.v + ((size_t)m * KV + head - H - KV) * HEAD_DIM + d0) = packed;
    }
}

template <int EPI, int SW, int TT>
__device__ __forceinline__ void local_epilogue(const LocalArgs& a, const LocalGemm& g, const int (&strip)[SW], int m0,
                                               const f32x4 (&acc)[SW][TT], const float (&rs)[TT]) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        if (EPI == LEPI_SILU) {
            local_store<EPI>(a, g, strip[0], m0 + 16 * t, acc[0][t], acc[SW - 1][t], rs[t]);
        } else {
#pragma unroll
            for (int s = 0; s < SW; ++s) local_store<EPI>(a, g, strip[s], m0 + 16 * t, acc[s][t], acc[s][t], rs[t]);
        }
    }
}

// A 16-byte load from global memory, as such: a pointer passed through an asm (WeightRing's)
// is no longer known to be global, and a flat load might read LDS, so the compiler would wait for
// every direct-to-LDS load in flight before issuing it.
__device__ __forceinline__ uint4 load16(const uint16_t* p) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(uint4, *(const __attribute__((address_space(1))) u32x4*)p);
}
// The scheduler may move nothing across this: every load above it is in flight before any value
// is used (left to itself it sinks loads towards their use to save registers).
__device__ __forceinline__ void all_issued() { __builtin_amdgcn_sched_barrier(0); }

// In both GEMMs below each output is one MFMA chain over its part's KBP k-blocks in k-block order,
// whatever tile it sits in, so that a token's sums are the same beside any other tokens. A wave
// keeps at most LG_INFLIGHT loads in flight, within its 6-bit count of them.
constexpr int LG_INFLIGHT = 48;

// A wave's ring of W fragments: its SW strips, DEPTH k-blocks ahead of the one it multiplies. The
// fragments are fetched in k-block order through one pointer a strip, moved on 1 KiB a fetch
// behind an asm the compiler cannot see through, so that it keeps one address a strip instead of
// one for every k-block of the unrolled loop.
template <int SW, int KBP, int DEPTH>
struct WeightRing {
    uint4 wf[DEPTH][SW];
    const uint16_t* next[SW];

    __device__ void start(const LocalGemm& g, const int (&strip)[SW], int kb0, int lane) {
#pragma unroll
        for (int s = 0; s < SW; ++s) next[s] = g.w + weight_tile_index(strip[s], kb0, g.K / 32, 16) + lane * 8;
    }
    // k-blocks [from, to) into their slots; calls follow each other in k-block order from 0
    __device__ void fetch(int from, int to) {
#pragma unroll
        for (int kb = from; kb < to; ++kb)
#pragma unroll
            for (int s = 0; s < SW; ++s) {
                wf[kb % DEPTH][s] = load16(next[s]);
                next[s] += 512;
                asm volatile("" : "+v"(next[s]));
            }
    }
};

// local_gemm_direct, for at most 64 tokens (M_pad = 16 TT): a workgroup of TT waves to a work unit
// (SW strips of W), wave t against token tile t, both operands straight from memory into
// registers, DEPTH k-blocks ahead (the waves read the same W; all but the first find it in cache).
// Grid (units, 1, parts).
template <int EPI, int SW, int TT, int KBP>
__global__ void __launch_bounds__(TT * WAVE) local_gemm_direct(LocalArgs a, LocalGemm g) {
    constexpr int DEPTH = LG_INFLIGHT / (SW + 1) < KBP ? LG_INFLIGHT / (SW + 1) : KBP;
    const int t = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int kb0 = blockIdx.z * KBP;
    int strip[SW];
    local_strips<EPI, SW>(blockIdx.x, g.N, strip);
    // The lane's token's sums of squares go first, the GEMM's loads behind them.
    constexpr bool SCALED = EPI == LEPI_QKV || EPI == LEPI_SILU;
    RowSq sq;
    if (SCALED) sq.load(g.row_sq, 16 * t + lane % 16);
    WeightRing<SW, KBP, DEPTH> w;
    w.start(g, strip, kb0, lane);
    const uint16_t* xp = g.x + act_index(16 * t, kb0 * 32, g.K) + lane * 8;  // the tile's fragments, 1 KiB each
    uint4 xf[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {  // k-block by k-block, so that the first MFMA waits for the first loads only
        w.fetch(d, d + 1);
        xf[d] = load16(xp + d * 512);
    }
    all_issued();
    if (SCALED) sq.settle();
    f32x4 acc[SW][1];
#pragma unroll
    for (int s = 0; s < SW; ++s) acc[s][0] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KBP; ++kb) {
        const int r = kb % DEPTH;
#pragma unroll
        for (int s = 0; s < SW; ++s) acc[s][0] = mfma16(w.wf[r][s], xf[r], acc[s][0]);
        if (kb + DEPTH < KBP) {
            w.fetch(kb + DEPTH, kb + DEPTH + 1);
            xf[r] = load16(xp + (kb + DEPTH) * 512);
        }
        all_issued();  // each k-block's refill stays where it is, DEPTH k-blocks ahead of its use
    }
    const float rs[1] = {SCALED ? row_scale_of(sq.p, g.K, a.eps) : 1.f};
    local_epilogue<EPI, SW, 1>(a, g, strip, 16 * t, acc, rs);
}

// local_gemm_ring, for more tokens (M_pad a multiple of 16 TT): a workgroup of 4 waves to 16 TT
// tokens (TT token tiles, 4 or 8) and 4 work units, wave w taking unit 4 blockIdx.x + w against
// every tile. A k-block's loads are a group: each wave's SW fragments of W, into registers
// (WeightRing), and its TT / 4 token tiles' fragments, straight from memory into a ring of RING
// LDS slots (TT KiB: the tiles' fragments of one k-block). The groups go out in k-block order RING ahead of their
// products, so a wave's count of loads in flight says which of its groups have landed, and the
// barrier after the wait says the same of every wave's; a wave reads a k-block's tiles from LDS
// while it multiplies the k-block before. No wave ever waits for more than the group it needs
// next. Each output is P chains of KBP k-blocks, the parts of local_gemm_direct in its order,
// added in part order as local_add_norm adds them.
// Grid (units / 4, M_pad / (16 TT)). Eight tiles halve the reads of W a token makes, at the cost of
// half the workgroups.
constexpr int ring_depth(int sw, int tt) { return tt == 8 ? 6 : sw == 1 ? 16 : 12; }
constexpr size_t ring_lds(int sw, int tt) {
    return (size_t)ring_depth(sw, tt) * tt * 64 * sizeof(uint4) + (16 * tt + 4 * 64) * sizeof(float);
}

// Waits until at most `n` of the wave's loads are in flight, `n` known when the loop is unrolled:
// the compiler's own wait (wait_vm_seen), so that it knows the loads before those n have landed
// and puts no wait of its own before their uses.
template <int N>
__device__ __forceinline__ void wait_vm_at_most(int n) {
    if constexpr (N == 0) {
        wait_vm_seen<0>();
    } else {
        if (n >= N)
            wait_vm_seen<N>();
        else
            wait_vm_at_most<N - 1>(n);
    }
}

template <int EPI, int SW, int KBP, int P, int TT>
__global__ void __launch_bounds__(4 * WAVE) __attribute__((amdgpu_waves_per_eu(2))) local_gemm_ring(LocalArgs a, LocalGemm g) {
    constexpr int KB = KBP * P;
    constexpr int RING = ring_depth(SW, TT);
    constexpr int XL = TT / 4;      // token tiles a wave loads
    constexpr int GROUP = SW + XL;  // a wave's loads of a k-block
    constexpr bool SCALED = EPI == LEPI_QKV || EPI == LEPI_SILU;
    static_assert(TT == 4 || TT == 8, "4 or 8 token tiles");
    static_assert(EPI != LEPI_ADD || TT == 4, "the sums of squares' reduction takes 64 tokens");
    static_assert(KB >= RING, "the ring fills before the first product");
    static_assert(RING * GROUP + SQ_PARTS / 4 < 64, "the loads in flight fit the wave's count");
    static_assert(EPI != LEPI_ADD || SW == 1, "a workgroup's columns are one span of a sum of squares");
    extern __shared__ uint4 xs[];  // [RING][TT tiles][64 lanes]
    float* scales = reinterpret_cast<float*>(xs + RING * TT * 64);  // [16 TT]: the tokens' row scales
    float* sq_part = scales + 16 * TT;                               // [4 waves][64 tokens]
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    const int m0 = blockIdx.y * 16 * TT;
    int strip[SW];
    local_strips<EPI, SW>(blockIdx.x * 4 + wv, g.N, strip);
    // The tokens' sums of squares (a lane to a token, 64 tokens to a wave, in every wave so that
    // each wave's count of loads is the same) go out before the groups: the wait for the first
    // group covers them.
    RowSq sq;
    if (SCALED) sq.load(g.row_sq, m0 + 64 * (wv % XL) + lane);
    WeightRing<SW, KB, RING> w;
    w.start(g, strip, 0, lane);
    // Tiles wv, wv + 4 ..'s fragments, 1 KiB each.
    const uint16_t* xp = g.x + act_index(m0 + 16 * wv, 0, g.K) + lane * 8;
    const size_t tile4 = (size_t)4 * (g.K / 32) * 512;  // four tiles on
    auto fetch = [&](int kb) __attribute__((always_inline)) {
        w.fetch(kb, kb + 1);
#pragma unroll
        for (int j = 0; j < XL; ++j) load_to_lds(xp + j * tile4 + kb * 512, &xs[((kb % RING) * TT + wv + 4 * j) * 64]);
    };
    // Each group stays behind the loads before it (the waits below count loads in issue order):
    // without a scheduling barrier between groups the compiler moves a later group's W loads
    // ahead of an earlier group's loads into LDS, and a wait that counts whole groups then lets a
    // wave read a slot whose load is still in flight.
    all_issued();
#pragma unroll
    for (int kb = 0; kb < RING; ++kb) {
        fetch(kb);
        all_issued();
    }
    f32x4 acc[P][SW][TT];
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
        for (int s = 0; s < SW; ++s)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[p][s][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Group 0 landed, every wave's; the scales into LDS, read after the barriers below. The store
    // is an asm the compiler cannot see: a store it knew of might share bytes with the loads into
    // the ring, for all it knows, and it would wait for every one of them before the first read.
    wait_vm_seen<(RING - 1) * GROUP>();
    if (SCALED) {
        const float rs = row_scale_of(sq.p, g.K, a.eps);
        if (wv < XL) asm volatile("ds_write_b32 %0, %1" ::"v"(lds_offset(&scales[64 * wv + lane])), "v"(rs) : "memory");
    }
    stage_barrier();
    uint4 xf[2][TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) xf[0][t] = lds_read16(&xs[t * 64 + lane]);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const int b = kb % 2;
        lds_landed(xf[b]);
        if (kb + 1 < KB) {
            // Group kb + 1 landed: the groups after it, up to kb + RING - 1, may be in flight. The
            // barrier also says every wave has its fragments of k-block kb, whose slot the fetch
            // below refills.
            wait_vm_at_most<(RING - 2) * GROUP>(GROUP * (RING - 2 < KB - 2 - kb ? RING - 2 : KB - 2 - kb));
            stage_barrier();
#pragma unroll
            for (int t = 0; t < TT; ++t) xf[1 - b][t] = lds_read16(&xs[(((kb + 1) % RING) * TT + t) * 64 + lane]);
        }
        const int r = kb % RING, p = kb / KBP;
#pragma unroll
        for (int s = 0; s < SW; ++s)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[p][s][t] = mfma16(w.wf[r][s], xf[b][t], acc[p][s][t]);
        if (kb + RING < KB) fetch(kb + RING);  // into the W registers just multiplied
        all_issued();
    }
    // The parts in part order.
    f32x4 sum[SW][TT];
#pragma unroll
    for (int s = 0; s < SW; ++s)
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            sum[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < P; ++p) sum[s][t] += acc[p][s][t];
        }
    if constexpr (EPI != LEPI_ADD) {
        float rs[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) rs[t] = SCALED ? scales[16 * t + lane % 16] : 1.f;
        local_epilogue<EPI, SW, TT>(a, g, strip, m0, sum, rs);
        return;
    }
    // LEPI_ADD: the residual added; with next_gain, the next norm's input and each token's sum of
    // squares over the wave's 16 columns (4 to a lane, then lanes l ^ 16, l ^ 32), the four
    // waves' added through LDS into the span of the workgroup's 64 columns.
    const int quad = lane / 16, n = strip[0] * 16 + quad * 4;
    float4 gn = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g.next_gain) gn = *reinterpret_cast<const float4*>(g.next_gain + n);
    float4 r[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) r[t] = *reinterpret_cast<const float4*>(g.residual + (size_t)(m0 + 16 * t + lane % 16) * g.N + n);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int m = m0 + 16 * t + lane % 16;
        float4 v;
        v.x = r[t].x + sum[0][t][0];
        v.y = r[t].y + sum[0][t][1];
        v.z = r[t].z + sum[0][t][2];
        v.w = r[t].w + sum[0][t][3];
        if (m < a.M) {
            *reinterpret_cast<float4*>(g.sum + (size_t)m * g.N + n) = v;
            if (g.next_gain)
                *reinterpret_cast<uint2*>(g.normed + act_index(m, n, g.N)) =
                    make_uint2(pack_bf16x2(v.x * gn.x, v.y * gn.y), pack_bf16x2(v.z * gn.z, v.w * gn.w));
        }
        if (g.next_gain) {
            float s4 = squares4(v.x, v.y, v.z, v.w);
            s4 += lane_xor16(s4);
            s4 += lane_xor32(s4);
            if (quad == 0) sq_part[wv * 64 + 16 * t + lane] = s4;
        }
    }
    if (!g.next_gain) return;
    __syncthreads();
    if (threadIdx.x < 64) {
        const int m = m0 + threadIdx.x;
        const float s = (sq_part[threadIdx.x] + sq_part[64 + threadIdx.x]) + (sq_part[128 + threadIdx.x] + sq_part[192 + threadIdx.x]);
        if (m < a.M) g.sum_sq[(size_t)m * SQ_PARTS + blockIdx.x] = s;
    }
}

// The GEMM of a projection whose epilogue is one of QKV, SILU or PARTIAL: `units` work units of
// SW strips (gate/up: pairs of strips), each output summed over the KBP k-blocks of its part. At
// most 64 tokens take the direct GEMM, more the ring (QKV and SILU only: its parts are added in
// the kernel, LEPI_ADD).
template <int EPI, int SW, int KBP>
void local_gemm(const char* label, const LocalArgs& a, const LocalGemm& g, int units, int parts, hipStream_t stream,
                DispatchTimer* timer) {
    if (a.M_pad <= 64) {
        const dim3 grid(units, 1, parts);
        switch (a.M_pad / 16) {
            case 1: dispatch(label, local_gemm_direct<EPI, SW, 1, KBP>, grid, dim3(WAVE), 0, stream, timer, a, g); break;
            case 2: dispatch(label, local_gemm_direct<EPI, SW, 2, KBP>, grid, dim3(2 * WAVE), 0, stream, timer, a, g); break;
            case 3: dispatch(label, local_gemm_direct<EPI, SW, 3, KBP>, grid, dim3(3 * WAVE), 0, stream, timer, a, g); break;
            default: dispatch(label, local_gemm_direct<EPI, SW, 4, KBP>, grid, dim3(4 * WAVE), 0, stream, timer, a, g); break;
        }
        return;
    }
    // Eight token tiles a workgroup for gate/up where the tokens come in 128s (its W, 16 MiB at
    // the sampler's shape, is the most read); four otherwise.
    if constexpr (EPI == LEPI_SILU) {
        if (a.M_pad % 128 == 0) {
            dispatch(label, local_gemm_ring<EPI, SW, KBP, 1, 8>, dim3(units / 4, a.M_pad / 128), dim3(4 * WAVE), ring_lds(SW, 8),
                     stream, timer, a, g);
            return;
        }
    }
    if constexpr (EPI != LEPI_PARTIAL)
        dispatch(label, local_gemm_ring<EPI, SW, KBP, 1, 4>, dim3(units / 4, a.M_pad / 64), dim3(4 * WAVE), ring_lds(SW, 4), stream,
                 timer, a, g);
}

// o_proj and down_proj over more than 64 tokens: the ring with the parts added and the residual
// added in its epilogue (LEPI_ADD), 16 or 32 k-blocks to each of 2 or 4 parts.
void local_gemm_add(const char* label, const LocalArgs& a, const LocalGemm& g, int kbp, int parts, hipStream_t stream,
                    DispatchTimer* timer) {
    const dim3 grid(g.N / 64, a.M_pad / 64), block(4 * WAVE);
    const size_t lds = ring_lds(1, 4);
    if (kbp == 16 && parts == 2)
        dispatch(label, local_gemm_ring<LEPI_ADD, 1, 16, 2, 4>, grid, block, lds, stream, timer, a, g);
    else if (kbp == 32 && parts == 2)
        dispatch(label, local_gemm_ring<LEPI_ADD, 1, 32, 2, 4>, grid, block, lds, stream, timer, a, g);
    else if (kbp == 16 && parts == 4)
        dispatch(label, local_gemm_ring<LEPI_ADD, 1, 16, 4, 4>, grid, block, lds, stream, timer, a, g);
    else
        dispatch(label, local_gemm_ring<LEPI_ADD, 1, 32, 4, 4>, grid, block, lds, stream, timer, a, g);
}

template <int EPI, int SW, int KBP, int P, int TT = 4>
hipError_t local_ring_lds() {
    return hipFuncSetAttribute((const void*)local_gemm_ring<EPI, SW, KBP, P, TT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)ring_lds(SW, TT));
}

// ---------------------------------------------------------------------------------------------
// local_attention: a wave to a (sequence, query head), 4 heads of one sequence to a workgroup.
// S^T = K Q^T by two MFMAs (keys as rows, the sequence's T <= 16 queries as columns, d in two
// halves of 32): lane l then holds query l % 16 against keys 4 (l / 16) .. + 3. The softmax over
// a query's keys is in-lane and across lanes l ^ 16, l ^ 32; P is rounded to bf16 and summed as
// rounded, and O^T = V^T P takes P straight from those registers as its B operand (k slots 0..3 =
// keys 4 (l / 16) + i, slots 4..7 zero), V^T gathered per lane as 4 keys of one dimension.
// Rows past T are read at the sequence's first token (in bounds) and masked or never written.
__global__ void __launch_bounds__(256) local_attention(LocalArgs a, const uint16_t* __restrict__ q,
                                                       const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                       uint16_t* __restrict__ attended) {
    const int seq = blockIdx.x, T = a.T, H = a.heads, KV = a.kv_heads;
    const int lane = threadIdx.x % WAVE, head = blockIdx.y * 4 + threadIdx.x / WAVE;
    const int kv = head / (H / KV), first = seq * T;
    const int r = lane % 16, g = lane / 16;
    const int row = first + (r < T ? r : 0);  // key row r, query column r
    const uint4* krow = reinterpret_cast<const uint4*>(k + ((size_t)row * KV + kv) * HEAD_DIM);
    const uint4* qrow = reinterpret_cast<const uint4*>(q + ((size_t)row * H + head) * HEAD_DIM);
    const uint4 ka = krow[g], kb = krow[4 + g], qa = qrow[g], qb = qrow[4 + g];
    // V^T rows: dimension 16 dt + r of keys 4 g + i.
    uint32_t vw[4][2];
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
        const int k0 = 4 * g + i < T ? first + 4 * g + i : first, k1 = 4 * g + i + 1 < T ? first + 4 * g + i + 1 : first;
        const uint16_t* v0 = v + ((size_t)k0 * KV + kv) * HEAD_DIM + r;
        const uint16_t* v1 = v + ((size_t)k1 * KV + kv) * HEAD_DIM + r;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) vw[dt][i / 2] = (uint32_t)v0[16 * dt] | ((uint32_t)v1[16 * dt] << 16);
    }
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    s = mfma16(ka, qa, s);
    s = mfma16(kb, qb, s);
    const float scale_log2 = log2_scale(a.scale);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (4 * g + i >= T) s[i] = -INFINITY;
        mx = fmaxf(mx, s[i]);
    }
    mx = fmaxf(mx, lane_xor16(mx));
    mx = fmaxf(mx, lane_xor32(mx));
    const float top = mx * scale_log2;
    uint32_t pw[2];
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
        pw[i / 2] = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(s[i], scale_log2, -top)),
                                __builtin_amdgcn_exp2f(fmaf(s[i + 1], scale_log2, -top)));
        total += bf16_lo(pw[i / 2]) + bf16_hi(pw[i / 2]);
    }
    total += lane_xor16(total);
    total += lane_xor32(total);
    const float inv = 1.0f / total;
    const uint4 pf = make_uint4(pw[0], pw[1], 0u, 0u);
    f32x4 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = mfma16(make_uint4(vw[dt][0], vw[dt][1], 0u, 0u), pf, f32x4{0.f, 0.f, 0.f, 0.f});
    if (r >= T) return;
    // Into attended in fragment order: dimensions 16 dt + 4 g .. + 3 of the head, 8 bytes.
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
        *reinterpret_cast<uint2*>(attended + act_index(first + r, head * HEAD_DIM + 16 * dt + 4 * g, H * HEAD_DIM)) =
            make_uint2(pack_bf16x2(o[dt][0] * inv, o[dt][1] * inv), pack_bf16x2(o[dt][2] * inv, o[dt][3] * inv));
}

// ---------------------------------------------------------------------------------------------
// local_add_norm: a wave to a token, lane l to its columns 16 l .. 16 l + 15 (hidden 1024).
// v = residual + the parts' sums in part order (written to `sum` when given). FINAL: RMSNorm with
// gain g in f32 into `out` (lane l squares its values in order, the lanes added by a butterfly).
// Else the next norm's input for the GEMM that applies the row's scale: normed = v g in bf16, and
// v's sums of squares over each 64 columns into row_sq, in the order local_gemm_ring's epilogue
// adds them (squares4 over 4 columns, (a + b) + (c + d) over a lane's 16, then over 4 lanes).
// PARTS (= parts, 0 to LOCAL_MAX_PARTS) is a template argument so that a lane's loads of every part
// are issued together, not one round trip a part.
template <bool FINAL, int PARTS>
__global__ void __launch_bounds__(256) local_add_norm(LocalArgs a, const float* __restrict__ partial, int parts,
                                                      const float* __restrict__ residual, float* __restrict__ sum,
                                                      const float* __restrict__ gain, uint16_t* __restrict__ normed,
                                                      float* __restrict__ row_sq, float* __restrict__ out) {
    const int m = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (m >= a.M) return;
    constexpr int K = 1024, PER = K / WAVE;
    const int base = lane * PER;
    float v[PER];
#pragma unroll
    for (int e = 0; e < PER; e += 4) {
        float4 r = *reinterpret_cast<const float4*>(residual + (size_t)m * K + base + e);
        if (PARTS > 0) {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int p = 0; p < PARTS; ++p) {
                const float4 s = *reinterpret_cast<const float4*>(partial + ((size_t)p * a.M_pad + m) * K + base + e);
                acc.x += s.x;
                acc.y += s.y;
                acc.z += s.z;
                acc.w += s.w;
            }
            r.x += acc.x;
            r.y += acc.y;
            r.z += acc.z;
            r.w += acc.w;
        }
        v[e] = r.x;
        v[e + 1] = r.y;
        v[e + 2] = r.z;
        v[e + 3] = r.w;
        if (sum) *reinterpret_cast<float4*>(sum + (size_t)m * K + base + e) = r;
    }
    if (FINAL) {
        float squares = 0.f;
#pragma unroll
        for (int e = 0; e < PER; ++e) squares += v[e] * v[e];
        const float scale = 1.0f / sqrtf(wave_sum(squares) / (float)K + a.eps);
#pragma unroll
        for (int e = 0; e < PER; e += 4) {
            float n[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) n[i] = v[e + i] * scale * gain[base + e + i];
            *reinterpret_cast<float4*>(out + (size_t)m * K + base + e) = make_float4(n[0], n[1], n[2], n[3]);
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < PER; e += 8) {
        float n[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) n[i] = v[e + i] * gain[base + e + i];
        *reinterpret_cast<uint4*>(normed + act_index(m, base + e, K)) =
            make_uint4(pack_bf16x2(n[0], n[1]), pack_bf16x2(n[2], n[3]), pack_bf16x2(n[4], n[5]), pack_bf16x2(n[6], n[7]));
    }
    float q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = squares4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    float s = (q[0] + q[1]) + (q[2] + q[3]);
    s += __shfl_xor(s, 1, WAVE);
    s += __shfl_xor(s, 2, WAVE);
    if (lane % 4 == 0) row_sq[(size_t)m * SQ_PARTS + lane / 4] = s;
}

// ---------------------------------------------------------------------------------------------
// local_embed: grid (hidden / 256, rows); thread n of the row: acc_f = bias[n] + sum_c W[n][c]
// frame_f[c] in channel order, for each of the row's frames, written as tokens first + f of both
// of the row's sequences; and the copied tokens.
constexpr int EMBED_MAX = 1024;     // channels x frames a row's patch may hold
constexpr int EMBED_CHANNELS = 64;  // channels at most (a row of W in 16 float4 loads)
constexpr int EMBED_COPIES = 2;     // copied tokens at most

// F frames to a patch, a template parameter so that every loop over them unrolls without a
// branch (a branch around a load makes the compiler wait for it where the paths join).
template <int F>
__global__ void __launch_bounds__(256) local_embed(LocalArgs a, EmbedArgs e) {
    __shared__ float frames[EMBED_MAX];  // [frames][channels]
    const int row = blockIdx.y, n = min(blockIdx.x * 256 + threadIdx.x, a.hidden - 1);
    const int C = e.channels;
    // The thread's row of W, every load in flight at once (indices clamped, not branched).
    float4 wq[EMBED_CHANNELS / 4];
#pragma unroll
    for (int v = 0; v < EMBED_CHANNELS / 4; ++v)
        wq[v] = *reinterpret_cast<const float4*>(e.w + (size_t)n * C + 4 * min(v, C / 4 - 1));
    // The copied tokens' values and the gain, loaded beside W.
    const int K = a.hidden;
    float cp[EMBED_COPIES];
#pragma unroll
    for (int t = 0; t < EMBED_COPIES; ++t)
        cp[t] = e.copy_src[((size_t)(e.shared ? 0 : row * e.copies) + min(t, e.copies - 1)) * K + n];
    const float g = e.gain ? e.gain[n] : 0.f;
    for (int i = threadIdx.x; i < C * F; i += 256) {
        const int f = i / C, c = i % C;
        frames[i] = e.src[((size_t)row * C + c) * F + f];
    }
    __syncthreads();  // hidden is a multiple of 256 (the launch checks): every lane has a column
    float acc[F];
    const float b = e.bias[n];
#pragma unroll
    for (int f = 0; f < F; ++f) acc[f] = b;
#pragma unroll
    for (int v = 0; v < EMBED_CHANNELS / 4; ++v) {
        if (4 * v >= C) break;
        const float w4[4] = {wq[v].x, wq[v].y, wq[v].z, wq[v].w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int f = 0; f < F; ++f) acc[f] += w4[i] * frames[f * C + 4 * v + i];
    }
    // Token m's value v of column n, and with a gain the first norm's input: v g in bf16 and the
    // sum of squares of the wave's 64 columns (uniform over the wave).
    auto put = [&](size_t m, float v) {
        e.x0[m * K + n] = v;
        if (!e.gain) return;
        // Columns n, n + 1 (lanes 2 i, 2 i + 1) side by side in fragment order: the even lane
        // stores both.
        const float vg = v * g, next = dpp_move<0xB1>(vg);  // quad_perm [1, 0, 3, 2]
        if (n % 2 == 0) *reinterpret_cast<uint32_t*>(e.normed + act_index((int)m, n, K)) = pack_bf16x2(vg, next);
        const float sq = span_squares(v);
        if (threadIdx.x % WAVE == 0) e.row_sq[m * SQ_PARTS + n / LOCAL_SQ_COLS] = sq;
    };
    for (int s = 0; s < e.seqs; ++s) {
        const size_t seq0 = (size_t)(row * e.seqs + s) * a.T;
#pragma unroll
        for (int f = 0; f < F; ++f) put(seq0 + e.first + f, acc[f]);
#pragma unroll
        for (int t = 0; t < EMBED_COPIES; ++t)
            if (t < e.copies) put(seq0 + e.copy_at + t, (e.guided && s > 0) ? 0.f : cp[t]);
    }
}

// ---------------------------------------------------------------------------------------------
// dit_euler: a workgroup of 8 waves to a row. out_proj's velocities are a 16-token product on
// the MFMA unit: W in 16-row bf16 tiles (the channels), the row's 2 frames tokens (the
// conditional sequence's, then the unconditional's; bf16, the other columns of the tile zero);
// wave w sums k-blocks 4 w .. 4 w + 3 with every load in flight at once, and the waves' tiles are
// added in wave order. Then CFG-Zero* (dit_euler.comp:81-110): alpha = <v_c, v_u> /
// (|v_u|^2 + 1e-8), guided = alpha v_u + cfg (v_c - alpha v_u), state -= dt guided.
constexpr int EULER_MAX_LEN = 512;  // channels x frames
constexpr int EULER_WAVES = 8;
constexpr int EULER_THREADS = EULER_WAVES * WAVE;
constexpr int EULER_STRIPS = 4;  // channels / 16 at most
constexpr int EULER_K = 1024;    // the DiT's width
constexpr int EULER_KB = EULER_K / 32 / EULER_WAVES;  // k-blocks to a wave

template <int F>
__global__ void __launch_bounds__(EULER_THREADS) dit_euler(LocalArgs a, EulerArgs e) {
    constexpr int TOKENS = 2 * F, K = EULER_K, KB = K / 32;
    __shared__ f32x4 red[EULER_WAVES][EULER_STRIPS][WAVE];
    __shared__ float vel[2 * EULER_MAX_LEN];
    __shared__ float sums[2][EULER_WAVES];
    const int row = blockIdx.x, C = e.channels, strips = C / 16;
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    // B operand: lane l holds token l % 16 (zero past the 2 F), columns 32 kb + 8 (l / 16) .. + 7.
    const int tm = lane % 16;
    const bool real = tm < TOKENS;
    const int tmc = real ? tm : 0;
    const size_t token = (size_t)(row * 2 + tmc / F) * a.T + e.first + tmc % F;
    const float* src = e.x + token * K + (lane / 16) * 8;
    const float* gain = e.gain + (lane / 16) * 8;
    RowSq sq;
    sq.load(e.row_sq, (int)token);
    float4 lo[EULER_KB], hi[EULER_KB], glo[EULER_KB], ghi[EULER_KB];
    uint4 wf[EULER_KB][EULER_STRIPS];
#pragma unroll
    for (int j = 0; j < EULER_KB; ++j) {
        const int kb = w * EULER_KB + j;
        lo[j] = *reinterpret_cast<const float4*>(src + kb * 32);
        hi[j] = *reinterpret_cast<const float4*>(src + kb * 32 + 4);
        glo[j] = *reinterpret_cast<const float4*>(gain + kb * 32);
        ghi[j] = *reinterpret_cast<const float4*>(gain + kb * 32 + 4);
#pragma unroll
        for (int s = 0; s < EULER_STRIPS; ++s)
            wf[j][s] = *reinterpret_cast<const uint4*>(e.w + weight_tile_index(min(s, strips - 1), kb, KB, 16) + lane * 8);
    }
    // The final norm: x / rms(x) g, its scale from the row's sums of squares.
    const float scale = row_scale_of(sq.p, K, a.eps);
    auto normed = [&](float4 v, float4 g4) { return make_float4(v.x * scale * g4.x, v.y * scale * g4.y, v.z * scale * g4.z, v.w * scale * g4.w); };
#pragma unroll
    for (int j = 0; j < EULER_KB; ++j) {
        lo[j] = normed(lo[j], glo[j]);
        hi[j] = normed(hi[j], ghi[j]);
    }
    f32x4 acc[EULER_STRIPS];
#pragma unroll
    for (int s = 0; s < EULER_STRIPS; ++s) acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < EULER_KB; ++j) {
        const uint4 b = real ? make_uint4(pack_bf16x2(lo[j].x, lo[j].y), pack_bf16x2(lo[j].z, lo[j].w),
                                          pack_bf16x2(hi[j].x, hi[j].y), pack_bf16x2(hi[j].z, hi[j].w))
                             : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int s = 0; s < EULER_STRIPS; ++s) acc[s] = mfma16(wf[j][s], b, acc[s]);
    }
#pragma unroll
    for (int s = 0; s < EULER_STRIPS; ++s) red[w][s][lane] = acc[s];
    __syncthreads();
    // Wave s < strips adds strip s over the waves in order: lane l holds token l % 16, channels
    // 16 s + 4 (l / 16) + i.
    if (w < strips && real) {
        f32x4 total = red[0][w][lane];
#pragma unroll
        for (int v = 1; v < EULER_WAVES; ++v) total += red[v][w][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = w * 16 + (lane / 16) * 4 + i;
            vel[(tm / F) * C * F + c * F + tm % F] = total[i] + e.bias[c];
        }
    }
    __syncthreads();
    const int len = C * F;
    float dot = 0.f, norm = 0.f;
    for (int i = threadIdx.x; i < len; i += EULER_THREADS) {
        dot += vel[i] * vel[len + i];
        norm += vel[len + i] * vel[len + i];
    }
    dot = wave_sum(dot);
    norm = wave_sum(norm);
    if (lane == 0) {
        sums[0][w] = dot;
        sums[1][w] = norm;
    }
    __syncthreads();
    dot = 0.f;
    norm = 0.f;
#pragma unroll
    for (int v = 0; v < EULER_WAVES; ++v) {
        dot += sums[0][v];
        norm += sums[1][v];
    }
    const float alpha = dot / (norm + 1e-8f);
    const float cfg = e.sampling[row * 2 + 1];
    for (int i = threadIdx.x; i < len; i += EULER_THREADS) {
        const float scaled = vel[len + i] * alpha;
        const float guided = scaled + cfg * (vel[i] - scaled);
        e.state[(size_t)row * len + i] -= guided * e.dt;
    }
}

__global__ void __launch_bounds__(256) cfm_noise(const float* __restrict__ noise, const float* __restrict__ sampling,
                                                 float* __restrict__ state, int rows, int len) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < rows * len) state[i] = sampling[(i / len) * 2] * noise[i];
}

}  // namespace

hipError_t launch_local_qkv(const LocalArgs& a, const LocalGemm& g, hipStream_t stream, DispatchTimer* timer) {
    if (g.K != a.hidden || g.N % 64 || a.M_pad != local_rows_padded(a.M)) return hipErrorInvalidValue;
    local_gemm<LEPI_QKV, 1, 32>("local_qkv_rope", a, g, g.N / 16, 1, stream, timer);
    return hipGetLastError();
}

hipError_t launch_local_attention(const LocalArgs& a, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* attended,
                                  hipStream_t stream, DispatchTimer* timer) {
    if (a.T < 1 || a.T > LOCAL_MAX_T || a.M % a.T || a.heads % 4 || a.kv_heads < 1 || a.heads % a.kv_heads) return hipErrorInvalidValue;
    dispatch("local_attention", local_attention, dim3(a.M / a.T, a.heads / 4), dim3(256), 0, stream, timer, a, q, k, v, attended);
    return hipGetLastError();
}

hipError_t launch_local_partial(const LocalArgs& a, const LocalGemm& g, int parts, hipStream_t stream, DispatchTimer* timer) {
    const int kbp = parts > 0 ? g.K / 32 / parts : 0;
    if (a.M_pad > 64 || a.M_pad != local_rows_padded(a.M) || parts < 1 || parts > LOCAL_MAX_PARTS || kbp * 32 * parts != g.K ||
        g.N % 64)
        return hipErrorInvalidValue;
    if (kbp == 16)
        local_gemm<LEPI_PARTIAL, 1, 16>("local_partial", a, g, g.N / 16, parts, stream, timer);
    else if (kbp == 32)
        local_gemm<LEPI_PARTIAL, 1, 32>("local_partial", a, g, g.N / 16, parts, stream, timer);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_local_add_norm(const LocalArgs& a, bool final, const float* partial, int parts, const float* residual, float* sum,
                                 const float* gain, uint16_t* normed, float* row_sq, float* out, hipStream_t stream,
                                 DispatchTimer* timer) {
    static_assert(LOCAL_MAX_PARTS == 4, "an instance for each count of parts");
    if (parts < 0 || parts > LOCAL_MAX_PARTS) return hipErrorInvalidValue;
    const dim3 rows4((a.M + 3) / 4);
    using Kernel = decltype(&local_add_norm<true, 0>);
    static constexpr Kernel finals[] = {local_add_norm<true, 0>, local_add_norm<true, 1>, local_add_norm<true, 2>,
                                        local_add_norm<true, 3>, local_add_norm<true, 4>};
    static constexpr Kernel adds[] = {local_add_norm<false, 0>, local_add_norm<false, 1>, local_add_norm<false, 2>,
                                      local_add_norm<false, 3>, local_add_norm<false, 4>};
    if (final)
        dispatch("local_final_norm", finals[parts], rows4, dim3(256), 0, stream, timer, a, partial, parts, residual, sum, gain, normed,
                 row_sq, out);
    else
        dispatch("local_add_norm", adds[parts], rows4, dim3(256), 0, stream, timer, a, partial, parts, residual, sum, gain, normed,
                 row_sq, out);
    return hipGetLastError();
}

hipError_t launch_local_add(const LocalArgs& a, const LocalGemm& g, int parts, hipStream_t stream, DispatchTimer* timer) {
    const int kbp = parts > 0 ? g.K / 32 / parts : 0;
    if (a.M_pad <= 64 || a.M_pad != local_rows_padded(a.M) || (parts != 2 && parts != 4) || (kbp != 16 && kbp != 32) ||
        kbp * 32 * parts != g.K || g.N != a.hidden)
        return hipErrorInvalidValue;
    local_gemm_add("local_add", a, g, kbp, parts, stream, timer);
    return hipGetLastError();
}

hipError_t launch_local_gate_up(const LocalArgs& a, const LocalGemm& g, hipStream_t stream, DispatchTimer* timer) {
    if (g.K != a.hidden || g.N != 2 * a.inner || a.M_pad != local_rows_padded(a.M)) return hipErrorInvalidValue;
    local_gemm<LEPI_SILU, 2, 32>("local_gate_up", a, g, a.inner / 16, 1, stream, timer);
    return hipGetLastError();
}

hipError_t launch_local_stack(const LocalArgs& a, const LocalLayer* layers, int nlayers, const float* final_norm,
                              const LocalBuffers& b, hipStream_t stream, DispatchTimer* timer) {
    if (!local_supported(a.hidden, a.inner, a.heads, a.kv_heads, b.o_parts, b.down_parts) || a.M_pad != local_rows_padded(a.M))
        return hipErrorInvalidValue;
    const int H = a.heads, KV = a.kv_heads;
    const int qkv_rows = (H + 2 * KV) * HEAD_DIM;
    // Over more than 64 tokens o_proj and down_proj add their parts and the residual themselves
    // (the ring GEMM); up to 64, their parts go out to `partial` for local_add_norm to add.
    const bool ring = a.M_pad > 64;
    hipError_t e = hipSuccess;
    // The first layer's input norm, unless the embedding wrote it.
    if (!b.normed0) e = launch_local_add_norm(a, false, nullptr, 0, b.x0, nullptr, layers[0].input_norm, b.normed, b.row_sq, nullptr, stream, timer);
    for (int l = 0; l < nlayers && e == hipSuccess; ++l) {
        const LocalLayer& L = layers[l];
        const bool last = l + 1 == nlayers;
        const float* input = l == 0 ? b.x0 : b.x;
        LocalGemm qkv{};
        qkv.w = L.qkv;
        qkv.x = l == 0 && b.normed0 ? b.normed0 : b.normed;
        qkv.K = a.hidden;
        qkv.N = qkv_rows;
        qkv.q = b.q;
        qkv.k = b.k;
        qkv.v = b.v;
        qkv.row_sq = l == 0 && b.normed0 ? b.row_sq0 : b.row_sq;
        e = launch_local_qkv(a, qkv, stream, timer);
        if (e == hipSuccess) e = launch_local_attention(a, b.q, b.k, b.v, b.attended, stream, timer);
        LocalGemm o{};
        o.w = L.o;
        o.x = b.attended;
        o.K = H * HEAD_DIM;
        o.N = a.hidden;
        if (ring) {
            o.residual = input;
            o.sum = b.h;
            o.next_gain = L.post_norm;
            o.normed = b.normed;
            o.sum_sq = b.row_sq;
            if (e == hipSuccess) e = launch_local_add(a, o, b.o_parts, stream, timer);
        } else {
            o.partial = b.partial;
            if (e == hipSuccess) e = launch_local_partial(a, o, b.o_parts, stream, timer);
            if (e == hipSuccess)
                e = launch_local_add_norm(a, false, b.partial, b.o_parts, input, b.h, L.post_norm, b.normed, b.row_sq, nullptr, stream, timer);
        }
        LocalGemm gu{};
        gu.w = L.gate_up;
        gu.x = b.normed;
        gu.K = a.hidden;
        gu.N = 2 * a.inner;
        gu.mlp = b.mlp;
        gu.row_sq = b.row_sq;
        if (e == hipSuccess) e = launch_local_gate_up(a, gu, stream, timer);
        LocalGemm down{};
        down.w = L.down;
        down.x = b.mlp;
        down.K = a.inner;
        down.N = a.hidden;
        // After the last layer, with no `out`, x and its sums of squares for the reader to norm.
        const float* next_gain = !last ? layers[l + 1].input_norm : b.out ? nullptr : final_norm;
        if (ring) {
            down.residual = b.h;
            down.sum = b.x;
            down.next_gain = next_gain;
            down.normed = b.normed;
            down.sum_sq = b.row_sq;
            if (e == hipSuccess) e = launch_local_add(a, down, b.down_parts, stream, timer);
            if (e == hipSuccess && last && b.out)
                e = launch_local_add_norm(a, true, nullptr, 0, b.x, nullptr, final_norm, nullptr, nullptr, b.out, stream, timer);
            continue;
        }
        down.partial = b.partial;
        if (e == hipSuccess) e = launch_local_partial(a, down, b.down_parts, stream, timer);
        if (e != hipSuccess) break;
        if (next_gain)
            e = launch_local_add_norm(a, false, b.partial, b.down_parts, b.h, b.x, next_gain, b.normed, b.row_sq, nullptr, stream, timer);
        else
            e = launch_local_add_norm(a, true, b.partial, b.down_parts, b.h, b.x, final_norm, nullptr, nullptr, b.out, stream, timer);
    }
    return e;
}

int local_stack_dispatches(const LocalArgs& a, const LocalBuffers& b, int nlayers) {
    const int norms = b.normed0 ? 0 : 1;
    if (a.M_pad > 64) return norms + 5 * nlayers + (b.out ? 1 : 0);
    return norms + 7 * nlayers;
}

bool local_supported(int hidden, int inner, int heads, int kv_heads, int o_parts, int down_parts) {
    // 2 or 4 parts of 16 or 32 k-blocks of 32 columns (the ring GEMM's instances).
    auto kbp_ok = [](int K, int parts) {
        return (parts == 2 || parts == 4) && K % (32 * parts) == 0 && (K / 32 / parts == 16 || K / 32 / parts == 32);
    };
    return hidden == 1024 && heads % 4 == 0 && kv_heads >= 1 && inner % 64 == 0 && kbp_ok(heads * HEAD_DIM, o_parts) &&
           kbp_ok(inner, down_parts);
}

int local_rows_padded(int M) { return M <= 64 ? (M + 15) / 16 * 16 : (M + 63) / 64 * 64; }

hipError_t local_prepare() {
    hipError_t e = local_ring_lds<LEPI_QKV, 1, 32, 1>();
    if (e == hipSuccess) e = local_ring_lds<LEPI_SILU, 2, 32, 1>();
    if (e == hipSuccess) e = local_ring_lds<LEPI_SILU, 2, 32, 1, 8>();
    if (e == hipSuccess) e = local_ring_lds<LEPI_ADD, 1, 16, 2>();
    if (e == hipSuccess) e = local_ring_lds<LEPI_ADD, 1, 32, 2>();
    if (e == hipSuccess) e = local_ring_lds<LEPI_ADD, 1, 16, 4>();
    if (e == hipSuccess) e = local_ring_lds<LEPI_ADD, 1, 32, 4>();
    return e;
}

hipError_t launch_local_embed(const LocalArgs& a, const EmbedArgs& e, int rows, hipStream_t stream, DispatchTimer* timer) {
    if (e.copies < 1 || e.copies > EMBED_COPIES || a.hidden % 256) return hipErrorInvalidValue;
    const dim3 grid((a.hidden + 255) / 256, rows), block(256);
    switch (e.frames) {
        case 1: dispatch("local_embed", local_embed<1>, grid, block, 0, stream, timer, a, e); break;
        case 2: dispatch("local_embed", local_embed<2>, grid, block, 0, stream, timer, a, e); break;
        case 3: dispatch("local_embed", local_embed<3>, grid, block, 0, stream, timer, a, e); break;
        case 4: dispatch("local_embed", local_embed<4>, grid, block, 0, stream, timer, a, e); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dit_euler(const LocalArgs& a, const EulerArgs& e, int rows, hipStream_t stream, DispatchTimer* timer) {
    if (a.hidden != EULER_K) return hipErrorInvalidValue;
    const dim3 grid(rows), block(EULER_THREADS);
    switch (e.frames) {
        case 1: dispatch("dit_euler", dit_euler<1>, grid, block, 0, stream, timer, a, e); break;
        case 2: dispatch("dit_euler", dit_euler<2>, grid, block, 0, stream, timer, a, e); break;
        case 3: dispatch("dit_euler", dit_euler<3>, grid, block, 0, stream, timer, a, e); break;
        case 4: dispatch("dit_euler", dit_euler<4>, grid, block, 0, stream, timer, a, e); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_cfm_noise(const float* noise, const float* sampling, float* state, int rows, int len, hipStream_t stream,
                            DispatchTimer* timer) {
    dispatch("cfm_noise", cfm_noise, dim3((rows * len + 255) / 256), dim3(256), 0, stream, timer, noise, sampling, state, rows, len);
    return hipGetLastError();
}

}  // namespace tgx
