// The prefill's kernels for gfx950 (crates/graph/src/prefill.rs:218-413 with norm_rows.comp,
// add_norm_rows.comp, rope_rows.comp, attention_rows.comp, silu_mul_rows.comp and the MLIR GEMM
// kernels/gpu/gemm.mlir), rewritten for the MFMA unit:
//
//   prefill_norm       RMSNorm of each row of the f32 stream into bf16 (norm_rows.comp, and the
//                      norm half of add_norm_rows.comp; the residual add is the GEMM's epilogue)
//   prefill_gemm       C = X W^T, bf16 in, f32 accumulate, a 256 x 128 tile to a workgroup of
//                      four waves staged through a ring of LDS stages, with the epilogue fused:
//                      RoPE and the cache write (rope_rows.comp), the residual add
//                      (add_norm_rows.comp), or SiLU(gate) up (silu_mul_rows.comp)
//   prefill_attention  causal attention over the paged cache, 32 positions of a run to a
//                      workgroup, keys and values staged through LDS a 64-position block at a time
//                      with an online softmax (attention_rows.comp)
#include "prefill_kernels.hpp"
#include "dispatch.hpp"

#include <math.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace tgx {

namespace {

// The GEMM's tile: 256 rows of W (16 strips) by TM rows of X, K 32 at a time (a k-block to a
// stage, in a ring of NBUF stages in LDS, all but one in flight while one is multiplied); wave
// (wn, wm) takes W rows 128 wn .. + 127 (8 strips) by X rows 64 wm .. + 63 (4 tiles of 16):
// 32 accumulators of 16 x 16. Two waves to a SIMD, so that one wave's products run while the
// other waits for LDS or the barrier:
//   TM 256: eight waves, a ring of four 32 KiB stages, a workgroup to a CU;
//   TM 128: four waves, a ring of three 24 KiB stages, two workgroups to a CU, so that one's
//           epilogue (its memory traffic) runs beside the other's products.
constexpr int TN = 256;
constexpr int W_STRIPS = TN / 16;   // 16
constexpr int WS = 8;               // a wave's W strips
constexpr int WT = 4;               // a wave's X tiles
constexpr int W_STAGE = W_STRIPS * 64;  // uint4 per stage: 16 KiB
constexpr int ROW_TILE_MAX = 256;   // M_pad is a multiple of this

template <int TM_>
struct GemmTile {
    static constexpr int TM = TM_;
    static constexpr int WAVES = TM / 32;  // 2 wave rows of W by TM / 64 of X
    static constexpr int THREADS = WAVES * WAVE;
    static constexpr int X_TILES = TM / 16;
    static constexpr int X_STAGE = X_TILES * 64;
    static constexpr int NBUF = TM == 256 ? 4 : 3;
    // The 1 KiB loads a wave issues a stage: the stage's W and X fragments over the waves.
    static constexpr int FB = (W_STRIPS + X_TILES) / WAVES;
    static_assert(FB * WAVES == W_STRIPS + X_TILES, "the fragments split evenly over the waves");
    static constexpr size_t LDS = (size_t)NBUF * (W_STAGE + X_STAGE) * 16 + TM * sizeof(float);
    static_assert(THREADS >= TM, "the q/k/v epilogue stages a row to a thread");
    static_assert(ROW_TILE_MAX % TM == 0, "M_pad is a multiple of TM");
    static_assert(NBUF * FB < 64, "the loads in flight fit the wave's counter");
};

__host__ __device__ constexpr bool residual_epilogue(int epi) { return epi == EPI_RESIDUAL || epi == EPI_RESIDUAL_IN; }

constexpr uint32_t TGX_SPARE_POS = 0xffffffffu;

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }


// The columns a sum of squares spans: a wave's 128 columns of W.
constexpr int SQ_SPAN = WS * 16;

// The scales 1 / rms of the tile's TM rows from their sums of squares (K / SQ_SPAN parts of
// SQ_SPAN columns, at most MAX_PARTS, added in order), a thread to a row; each 1 without
// row_sq. The parts are loaded at once, before the GEMM's own loads.
constexpr int MAX_PARTS = 4096 / SQ_SPAN;
template <int TM>
struct RowScale {
    float4 p[MAX_PARTS / 4];
    __device__ void load(const GemmArgs& g, int m0) {
        const int quads = g.K / SQ_SPAN / 4;
        const float* row = g.row_sq ? g.row_sq + (size_t)(m0 + threadIdx.x % TM) * (g.K / SQ_SPAN) : nullptr;
        if (!row) return;  // uniform
#pragma unroll
        for (int i = 0; i < MAX_PARTS / 4; ++i) p[i] = *reinterpret_cast<const float4*>(row + 4 * min(i, quads - 1));
    }
    // The loaded values pinned here: nothing computed from them moves above this point (the
    // compiler would otherwise wait for them before the GEMM's own loads are issued).
    __device__ void settle() {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int i = 0; i < MAX_PARTS / 4; ++i) {
            u32x4 t = __builtin_bit_cast(u32x4, p[i]);
            asm volatile("" : "+v"(t));
            p[i] = __builtin_bit_cast(float4, t);
        }
    }
    __device__ float scale(const PrefillArgs& a, const GemmArgs& g) const {
        if (!g.row_sq) return 1.f;
        const int quads = g.K / SQ_SPAN / 4;
        float total = 0.f;
#pragma unroll
        for (int i = 0; i < MAX_PARTS / 4; ++i) {
            if (i >= quads) break;
            total += p[i].x;
            total += p[i].y;
            total += p[i].z;
            total += p[i].w;
        }
        return 1.0f / sqrtf(total / (float)g.K + a.eps);
    }
};

// The global strip of W that strip `s` (0..7) of wave row `wn` of n-block `nb` takes.
template <int EPI>
__device__ __forceinline__ int strip_of(int nb, int wn, int s, int N) {
    if (EPI == EPI_SILU) {
        // 128 gate rows and the same 128 rows of up to a workgroup; a wave's first four strips are
        // gate, its last four the matching up.
        const int gate = nb * 8 + wn * 4 + (s % 4);
        return s < 4 ? gate : gate + N / 32;
    }
    return nb * W_STRIPS + wn * 8 + s;
}

// The workgroup's strip `sl` (0..15) in LDS order: wave row sl / 8, strip sl % 8.
template <int EPI>
__device__ __forceinline__ int stage_strip(int nb, int sl, int N) {
    return strip_of<EPI>(nb, sl / 8, sl % 8, N);
}

// The workgroup's tile (nb, mb). Workgroups go to the 8 XCDs in turn (id % 8), each XCD with its
// own L2; the ids are renumbered so that XCD x takes a contiguous eighth of the tiles, and the
// tiles in groups of GROUP_M M-tiles by every N-tile: an X tile (a band of positions) is then
// read only on its own XCD, by the N-tiles that share it there. A grid of fewer than a multiple
// of 8 workgroups keeps the plain order.
constexpr int GROUP_M = 4;
__device__ __forceinline__ void tile_of(int& nb, int& mb) {
    const int NB = gridDim.x, G = gridDim.x * gridDim.y;
    const int id = blockIdx.x + blockIdx.y * gridDim.x;
    const int v = G % 8 == 0 ? (id % 8) * (G / 8) + id / 8 : id;
    const int per_group = GROUP_M * NB;
    const int group = v / per_group, in = v % per_group;
    const int rows = min(GROUP_M, (int)gridDim.y - group * GROUP_M);  // the last group may be short
    mb = group * GROUP_M + in % rows;
    nb = in / rows;
}

// W in strips of WR rows (o_proj and down_proj: 4 or 16, the rest 16), gathered into 16-row
// fragments as it lands in LDS. D: the head width the q/k/v epilogue rotates and caches by.
template <int EPI, int WR, int TM, int D = HEAD_DIM>
__global__ void __launch_bounds__(GemmTile<TM>::THREADS) __attribute__((amdgpu_waves_per_eu(2)))
prefill_gemm(PrefillArgs a, GemmArgs g) {
    using T = GemmTile<TM>;
    constexpr int NBUF = T::NBUF, X_STAGE = T::X_STAGE;
    extern __shared__ uint4 lds[];
    uint4* ws = lds;                     // [NBUF][W_STAGE]
    uint4* xs = lds + NBUF * W_STAGE;    // [NBUF][X_STAGE]
    float* row_scale = reinterpret_cast<float*>(lds + NBUF * (W_STAGE + X_STAGE));  // [TM]
    int nb, mb;
    tile_of(nb, mb);
    // The wave's index, uniform: the branches on it below are the whole wave's.
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    const int lane = threadIdx.x % WAVE;
    const int wn = w / (T::WAVES / 2), wm = w % (T::WAVES / 2);
    const int kblocks = g.K / 32;
    const int stages = kblocks;
    const int m0 = mb * TM;

    // A stage is 16 weight fragments and TM / 16 vector fragments of 1 KiB, loaded straight from
    // memory into LDS: lane l of a load writes bytes 16 l .. 16 l + 15 of the fragment, the MFMA
    // operand order. Every wave loads FB of them (slot j of wave w is fragment FB w + j: the W
    // strips, then the X tiles), the same number every stage, so that its count in flight says
    // which stages have landed and no wave's loads hold the others at the barrier. Fragment j of
    // stage st is the lane's base + off[j] + st * fstep[j] (a k-block further along K), the
    // offsets 32-bit (a tensor holds fewer than 2^32 elements).
    constexpr int FB = T::FB;
    const uint16_t* fbase[FB];
    uint32_t off[FB], fstep[FB];
    uint4* fdst[FB];
    int fstride[FB];
#pragma unroll
    for (int j = 0; j < FB; ++j) {
        const int f = w * FB + j;
        if (f < W_STRIPS) {
            fbase[j] = g.w;
            off[j] = (uint32_t)fragment_index<WR>(stage_strip<EPI>(nb, f, g.N), 0, kblocks, lane);
            fstep[j] = WR * 32;
            fdst[j] = ws + f * 64;
            fstride[j] = W_STAGE;
        } else {
            const int x = f - W_STRIPS;
            fbase[j] = g.x;
            off[j] = (uint32_t)(m0 / 16 + x) * (uint32_t)kblocks * 512u + (uint32_t)lane * 8u;
            fstep[j] = 512;
            fdst[j] = xs + x * 64;
            fstride[j] = X_STAGE;
        }
    }
    // Stage st into buffer buf.
    auto fetch = [&](int st, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < FB; ++j) load_to_lds(fbase[j] + (off[j] + (uint32_t)st * fstep[j]), fdst[j] + buf * fstride[j]);
    };
    // Waits until a stage has landed for every wave: no more than the `after` stages fetched after
    // it in flight for this wave, then the barrier, which also says that every wave is done with
    // the step before (and with the buffers it read into registers).
    auto landed = [&](int after) __attribute__((always_inline)) {
        static_assert(NBUF <= 3, "up to two stages in flight past the one waited for");
        if (after >= 2)
            wait_vm<2 * FB>();
        else if (after == 1)
            wait_vm<FB>();
        else
            wait_vm<0>();
        stage_barrier();
    };

    // The accumulators start at zero, or with EPI_RESIDUAL_IN at the residual rows themselves
    // (rows past M read row M - 1, never stored): their loads go out first, ahead of the ring's,
    // so that the epilogue waits for no read.
    f32x4 acc[WS][WT];
    const int quad = lane / 16;
#pragma unroll
    for (int s = 0; s < WS; ++s)
#pragma unroll
        for (int t = 0; t < WT; ++t) {
            if constexpr (EPI == EPI_RESIDUAL_IN) {
                const int n = strip_of<EPI>(nb, wn, s, g.N) * 16 + quad * 4;
                const int m = min(m0 + (wm * WT + t) * 16 + lane % 16, a.M - 1);
                const float4 r = *reinterpret_cast<const float4*>(g.residual + (size_t)m * g.N + n);
                acc[s][t] = f32x4{r.x, r.y, r.z, r.w};
            } else {
                acc[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
    __builtin_amdgcn_sched_barrier(0);  // the residual's loads stay ahead of the ring's

    // The wave's fragments of stage st from LDS: fr[t] X tile t, fr[WT + s] W strip s.
    auto read = [&](int st, uint4 (&fr)[WT + WS]) __attribute__((always_inline)) {
        const int buf = st % NBUF;
#pragma unroll
        for (int t = 0; t < WT; ++t) fr[t] = lds_read16(&xs[buf * X_STAGE + (wm * WT + t) * 64 + lane]);
#pragma unroll
        for (int s = 0; s < WS; ++s) fr[WT + s] = lds_read16(&ws[buf * W_STAGE + (wn * WS + s) * 64 + lane]);
    };
    // Step st: the products of stage st from `cur` (read in the step before) while stage st + 1's
    // fragments are read into `next`, so that the LDS reads overlap the products. Two ways to keep
    // the ring fed (what suits q/k/v and gate/up slows o_proj and down_proj, whose X operands are
    // the larger and whose L2 more stages in flight crowd):
    //  AHEAD: past the barrier, stage st + NBUF into the buffer of stage st (read into registers
    //    in the step before, by every wave before this barrier), its loads spread between the
    //    products: NBUF stages in flight. Past the last stage the last is loaded again into a
    //    buffer no step reads after, and the last step reads the buffer of stage st + 1, which
    //    holds the last stage loaded again two steps before, landed, and which no load of that
    //    step writes (never used): every step the same, with no branch.
    //  otherwise: before the barrier, stage st + NBUF - 1 into the buffer of stage st - 1, which
    //    every wave had read by the end of step st - 2 (the prologue, for stage 0).
    constexpr bool AHEAD = !residual_epilogue(EPI);
    auto step = [&](int st, uint4 (&cur)[WT + WS], uint4 (&next)[WT + WS]) __attribute__((always_inline)) {
        if constexpr (AHEAD) {
            landed(NBUF - 2);  // stage st + 1
            read(st + 1, next);  // its buffer: (st + 1) % NBUF
#pragma unroll
            for (int s = 0; s < WS; ++s)
#pragma unroll
                for (int t = 0; t < WT; ++t) acc[s][t] = mfma16(cur[WT + s], cur[t], acc[s][t]);
            fetch(min(st + NBUF, stages - 1), st % NBUF);
            // A load after each WS WT / FB products (the few left over after the last load).
#pragma unroll
            for (int j = 0; j < FB; ++j) {
                __builtin_amdgcn_sched_group_barrier(0x008, WS * WT / FB, 0);  // MFMAs
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);             // a load
            }
            __builtin_amdgcn_sched_barrier(0);
            lds_landed(next);
        } else {
            if (st + NBUF - 1 < stages) fetch(st + NBUF - 1, (st + NBUF - 1) % NBUF);
            const bool more = st + 1 < stages;
            if (more) {
                landed(min(NBUF - 2, stages - 2 - st));  // stage st + 1
                read(st + 1, next);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < WS; ++s)
#pragma unroll
                for (int t = 0; t < WT; ++t) acc[s][t] = mfma16(cur[WT + s], cur[t], acc[s][t]);
            __builtin_amdgcn_sched_barrier(0);
            if (more) lds_landed(next);
        }
    };

    uint4 fa[WT + WS], fb[WT + WS];
    // The rows' scales (q/k/v, gate/up): their loads go first, the GEMM's behind them, and the
    // scales are taken once the first stage has landed (so have they), reaching LDS long before
    // the epilogue, past every barrier of the main loop.
    RowScale<TM> rs;
    const bool scales = !residual_epilogue(EPI) && threadIdx.x < TM;  // whole waves
    if (scales) rs.load(g, m0);
    // K >= 1024: 32 stages at least.
    constexpr int PRIMED = AHEAD ? NBUF : NBUF - 1;
    // The stages go out in stage order, the row scales' loads ahead of them: landed() counts
    // loads in issue order.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PRIMED; ++p) {
        fetch(p, p);
        __builtin_amdgcn_sched_barrier(0);
    }
    landed(PRIMED - 1);  // stage 0
    if (scales) {
        rs.settle();
        row_scale[threadIdx.x] = rs.scale(a, g);
    }
    read(0, fa);
    lds_landed(fa);
    // K is a multiple of 1024: the stages come in pairs, and the accumulators flow through no
    // branch (a branch around a step makes the compiler copy them out of their registers).
    for (int st = 0; st < stages; st += 2) {
        step(st, fa, fb);
        step(st + 1, fb, fa);
    }
    // No load to the LDS in flight (AHEAD's last ones), every wave done with the ring: the
    // epilogue below may reuse the LDS.
    wait_vm<0>();
    stage_barrier();

    // Epilogue: tile (s, t) holds W rows 16 strip + 4 (lane / 16) + i against X row
    // m0 + 16 (WT wm + t) + lane % 16.
    if (residual_epilogue(EPI)) {
        // The residual plus the products (EPI_RESIDUAL_IN: the accumulators hold both). With
        // next_gain: each lane's squares of its row's 32 values of the wave's 128 columns, in
        // strip order, then the 4 lanes of a row added (lanes l ^ 16, l ^ 32). EPI_RESIDUAL loads
        // the residual rows of four strips at once (rows past M read row M - 1, never stored).
        float sq[WT] = {};
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float4 r[4][WT], gn[4];
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int n = strip_of<EPI>(nb, wn, 4 * half + s4, g.N) * 16 + quad * 4;
                gn[s4] = *reinterpret_cast<const float4*>((g.next_gain ? g.next_gain : g.residual) + n);
#pragma unroll
                for (int t = 0; t < WT; ++t) {
                    const int m = min(m0 + (wm * WT + t) * 16 + lane % 16, a.M - 1);
                    r[s4][t] = EPI == EPI_RESIDUAL ? *reinterpret_cast<const float4*>(g.residual + (size_t)m * g.N + n)
                                                   : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
            // The next norm's bf16 operand two strips at a time: lanes l and l ^ 16 (the same row)
            // trade so that each stores 8 columns of one strip, 16 bytes (pair_blocks).
#pragma unroll
            for (int t = 0; t < WT; ++t) {
                const int m = m0 + (wm * WT + t) * 16 + lane % 16;
                if (m >= a.M) continue;
#pragma unroll
                for (int s2 = 0; s2 < 4; s2 += 2) {
                    uint32_t normed[2][2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int s4 = s2 + h, s = 4 * half + s4;
                        const int n = strip_of<EPI>(nb, wn, s, g.N) * 16 + quad * 4;
                        float4 o = make_float4(acc[s][t][0], acc[s][t][1], acc[s][t][2], acc[s][t][3]);
                        if (EPI == EPI_RESIDUAL) {
                            o.x = r[s4][t].x + acc[s][t][0];
                            o.y = r[s4][t].y + acc[s][t][1];
                            o.z = r[s4][t].z + acc[s][t][2];
                            o.w = r[s4][t].w + acc[s][t][3];
                        }
                        *reinterpret_cast<float4*>(g.out + (size_t)m * g.N + n) = o;
                        normed[h][0] = pack_bf16x2(o.x * gn[s4].x, o.y * gn[s4].y);
                        normed[h][1] = pack_bf16x2(o.z * gn[s4].z, o.w * gn[s4].w);
                        if (g.next_gain) {
                            sq[t] += o.x * o.x;
                            sq[t] += o.y * o.y;
                            sq[t] += o.z * o.z;
                            sq[t] += o.w * o.w;
                        }
                    }
                    if (g.next_gain) {
                        const int n = strip_of<EPI>(nb, wn, 4 * half + s2 + (quad & 1), g.N) * 16 + (quad & 2) * 4;
                        *reinterpret_cast<uint4*>(g.out_n + act_index(m, n, g.N)) = pair_blocks(normed[0], normed[1]);
                    }
                }
            }
        }
        if (g.next_gain) {
            const int parts = g.N / SQ_SPAN;
#pragma unroll
            for (int t = 0; t < WT; ++t) {
                float v = sq[t];
                v += lane_xor16(v);
                v += lane_xor32(v);
                const int m = m0 + (wm * WT + t) * 16 + lane % 16;
                if (quad == 0 && m < a.M) g.out_sq[(size_t)m * parts + nb * (TN / SQ_SPAN) + wn] = v;
            }
        }
    } else if (EPI == EPI_SILU) {
        const int inner = g.N / 2;
        const float* scale = row_scale;
        // silu(r g) (r u) for the row's scale r and the products g, u, as g u / ((1 + e) k) with
        // e = 2^(-r log2(e) g) and k = 1 / r^2: the row's two constants once, then four VALU
        // instructions and two transcendentals an output.
#pragma unroll
        for (int t = 0; t < WT; ++t) {
            const int j = (wm * WT + t) * 16 + lane % 16;
            const int m = m0 + j;
            if (m >= a.M) continue;
            const float rs = scale[j];
            const float c = -rs * 1.4426950408889634f, k = __builtin_amdgcn_rcpf(rs * rs);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int n = strip_of<EPI>(nb, wn, s, g.N) * 16 + quad * 4;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float gp = acc[s][t][i], up = acc[s + 4][t][i];
                    const float e = __builtin_amdgcn_exp2f(gp * c);
                    v[i] = (gp * up) * __builtin_amdgcn_rcpf(__builtin_fmaf(e, k, k));
                }
                uint2 packed = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                *reinterpret_cast<uint2*>(g.mlp + act_index(m, n, inner)) = packed;
            }
        }
    } else {  // EPI_QKV: a lane's four rows of a strip are two RoPE pairs (qkv_row_of)
        // Each of the tile's 256 rows' position, cache block and RoPE row, staged once in the LDS
        // the main loop is done with: a thread to a row, two round trips to memory in all.
        // A row's 32 values of cos and sin 36 floats apart, so that the 16 rows a wave's lanes read
        // at once (and the threads' rows as they store them) do not all fall on the same banks, as
        // 32 apart would put them.
        constexpr int RS = D / 2 + 4;
        static_assert((size_t)TM * (2 * RS + 2) * 4 <= T::LDS, "the rows' RoPE tables fit the ring's LDS");
        float* t_cos = reinterpret_cast<float*>(lds);          // [TM][RS]
        float* t_sin = t_cos + TM * RS;                        // [TM][RS]
        uint32_t* t_pos = reinterpret_cast<uint32_t*>(t_sin + TM * RS);  // [TM]
        uint32_t* t_blk = t_pos + TM;                           // [TM]
        const float* t_scale = row_scale;
        if (threadIdx.x < TM) {
            const int j = threadIdx.x;
            const int m = m0 + j;
            uint32_t pos = TGX_SPARE_POS, blk = TGX_SPARE_POS;
            if (m < a.M) {
                const uint32_t p = a.tok_pos[m], sl = a.tok_slot[m];
                if (p < (uint32_t)a.capacity && sl < (uint32_t)a.nslots) {
                    pos = p;
                    blk = a.table[(size_t)sl * a.max_blocks + p / BLOCK_TOKENS];
                    if (a.rope) {
#pragma unroll
                        for (int e = 0; e < D / 2; e += 4) {
                            *reinterpret_cast<float4*>(t_cos + j * RS + e) =
                                *reinterpret_cast<const float4*>(a.cos + (size_t)p * (D / 2) + e);
                            *reinterpret_cast<float4*>(t_sin + j * RS + e) =
                                *reinterpret_cast<const float4*>(a.sin + (size_t)p * (D / 2) + e);
                        }
                    }
                }
            }
            t_pos[j] = pos;
            t_blk[j] = blk;
        }
        __syncthreads();
        const int H = a.heads, KV = a.kv_heads;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int strip = strip_of<EPI>(nb, wn, s, g.N);
            const int head = strip / (D / 16), qtr = strip % (D / 16);
            // Rows 4 quad .. 4 quad + 3 of the strip: the pairs of dimensions (e, e + D / 2) and
            // (e + 1, e + 1 + D / 2), each first half then second. For the stores the lanes l and
            // l ^ 16 (quads 2 h and 2 h + 1, the same row) trade halves: the even quad stores
            // dimensions e .. e + 3 and the odd one e - 2 + D / 2 .. e + 1 + D / 2, 8 bytes each.
            const int e = qtr * 8 + quad * 2;
            const int d0 = (quad & 1) ? e - 2 + D / 2 : e;
            const bool rotate = head < H + KV && a.rope;
#pragma unroll
            for (int t = 0; t < WT; ++t) {
                const int j = (wm * WT + t) * 16 + lane % 16;  // the row within the tile
                const uint32_t pos = t_pos[j];
                if (pos == TGX_SPARE_POS) continue;
                const float rs = t_scale[j];
                float lo[2], hi[2];  // dimensions e + k and e + k + D / 2
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    lo[k] = acc[s][t][2 * k] * rs;
                    hi[k] = acc[s][t][2 * k + 1] * rs;
                }
                if (rotate) {
                    const float2 co = *reinterpret_cast<const float2*>(t_cos + j * RS + e);
                    const float2 si = *reinterpret_cast<const float2*>(t_sin + j * RS + e);
                    // As upstream: x cos + rotate_half(x) sin (rope_rows.comp:52-59), a pair
                    // (x1, x2) to (x1 cos - x2 sin, x2 cos + x1 sin).
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const float cs = k ? co.y : co.x, sn = k ? si.y : si.x;
                        const float x1 = lo[k], x2 = hi[k];
                        lo[k] = __builtin_fmaf(x1, cs, -(x2 * sn));
                        hi[k] = __builtin_fmaf(x2, cs, x1 * sn);
                    }
                }
                const int m = m0 + j;
                if (head < H) {
                    // q scaled by scale log2(e), the units the attention's softmax takes.
                    const float qs = log2_scale(a.scale);
                    const auto w4 = quad_halves(pack_bf16x2(lo[0] * qs, lo[1] * qs), pack_bf16x2(hi[0] * qs, hi[1] * qs));
                    *reinterpret_cast<uint2*>(g.q + ((size_t)m * H + head) * D + d0) = w4;
                    continue;
                }
                const uint32_t blk = t_blk[j];
                if (blk >= (uint32_t)a.nblocks) continue;
                const int kv = head < H + KV ? head - H : head - H - KV;
                constexpr int TILE = kv_tile(D);
                uint16_t* tl = g.kv + ((size_t)blk * KV + kv) * 2 * TILE;
                const int pp = (int)(pos % BLOCK_TOKENS);
                if (head < H + KV) {
                    // Four consecutive dimensions of a key sit side by side in its tile (d0 % 4 == 0).
                    *reinterpret_cast<uint2*>(tl + key_index(pp, d0, D)) = quad_halves(pack_bf16x2(lo[0], lo[1]), pack_bf16x2(hi[0], hi[1]));
                } else {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        tl[TILE + value_index(pp, e + k)] = (uint16_t)bf16_bits(lo[k]);
                        tl[TILE + value_index(pp, e + k + D / 2)] = (uint16_t)bf16_bits(hi[k]);
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// prefill_norm: a wave to a row: lane l sums the squares of its PL = K/64 elements in order, the
// lanes added by a butterfly (norm.glsl:12-29); rows past M are written zero. A lane issues all of
// its row's and gain's loads before it uses any.
template <bool FINAL, int PL>
__global__ void __launch_bounds__(256) prefill_norm(PrefillArgs a, const float* __restrict__ x, const float* __restrict__ gain,
                                                    uint16_t* __restrict__ out_bf16, float* __restrict__ out_f32) {
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (row >= a.M_pad) return;
    constexpr int K = PL * WAVE, per_lane = PL;
    if (row >= a.M) {
        if (!FINAL)
#pragma unroll
            for (int e = 0; e < per_lane; e += 8)
                *reinterpret_cast<uint4*>(out_bf16 + act_index(row, lane * per_lane + e, K)) = make_uint4(0, 0, 0, 0);
        return;
    }
    const float* r = x + (size_t)row * K + lane * per_lane;
    float4 xv[PL / 4], gv[PL / 4];
#pragma unroll
    for (int i = 0; i < PL / 4; ++i) xv[i] = *reinterpret_cast<const float4*>(r + 4 * i);
#pragma unroll
    for (int i = 0; i < PL / 4; ++i) gv[i] = *reinterpret_cast<const float4*>(gain + lane * per_lane + 4 * i);
    // The sum starts at a zero the compiler cannot see (it would fold 0 + x0 x0 to a product and
    // fuse the next term the other way round): every term is an FMA onto the sum, in order.
    float squares = 0.f;
    asm volatile("" : "+v"(squares));
#pragma unroll
    for (int i = 0; i < PL / 4; ++i) {
        const float4 v = xv[i];
        squares += v.x * v.x;
        squares += v.y * v.y;
        squares += v.z * v.z;
        squares += v.w * v.w;
    }
    const float scale = 1.0f / sqrtf(wave_sum(squares) / (float)K + a.eps);
#pragma unroll
    for (int e = 0; e < per_lane; e += 8) {
        const float4 v0 = xv[e / 4], v1 = xv[e / 4 + 1];
        const float4 g0 = gv[e / 4], g1 = gv[e / 4 + 1];
        const float n[8] = {v0.x * scale * g0.x, v0.y * scale * g0.y, v0.z * scale * g0.z, v0.w * scale * g0.w,
                            v1.x * scale * g1.x, v1.y * scale * g1.y, v1.z * scale * g1.z, v1.w * scale * g1.w};
        if (FINAL) {
            *reinterpret_cast<float4*>(out_f32 + (size_t)row * K + lane * per_lane + e) = make_float4(n[0], n[1], n[2], n[3]);
            *reinterpret_cast<float4*>(out_f32 + (size_t)row * K + lane * per_lane + e + 4) = make_float4(n[4], n[5], n[6], n[7]);
        } else {
            *reinterpret_cast<uint4*>(out_bf16 + act_index(row, lane * per_lane + e, K)) =
                make_uint4(pack_bf16x2(n[0], n[1]), pack_bf16x2(n[2], n[3]), pack_bf16x2(n[4], n[5]), pack_bf16x2(n[6], n[7]));
        }
    }
}

// ---------------------------------------------------------------------------------------------
// The prefill attention's online softmax, with a reference moved lazily. q comes scaled by
// scale log2(e) (the q/k/v epilogue), and the score MFMA's accumulator starts at -r, so that a
// block's scores arrive as s - r for the column's reference r, in the units v_exp_f32 (2^x) takes:
// P = 2^(s - r), in bf16. r moves only when a column's block maximum passes r + LAZY_SHIFT (and
// on block 0, which every column sees first), the column's o and l then rescaled; otherwise the
// block costs no subtract and no rescale. P <= 2^LAZY_SHIFT, and o and l stay in f32. A column
// whose reference stays computes the same bits whether or not others of its wave move theirs
// (it subtracts 0 and scales by 1), so that a position's result never depends on its neighbours.
// The values past `vlast` read as zero (as OnlineSoftmax's).
constexpr float LAZY_SHIFT = 8.0f;

// The largest of a column's scores over PT tiles (16 PT floats), in plain code: the compiler makes it a
// v_max3_f32 chain (quieting only the first two operands) and gives each read of an MFMA's result
// the wait states it needs, which it could not do for inline asm.
template <int PT>
__device__ __forceinline__ float peak_of(const f32x4 (&s)[PT]) {
    float m = fmaxf(s[0][0], s[0][1]);
#pragma unroll
    for (int k = 2; k < 4 * PT; k += 2) m = fmaxf(fmaxf(m, s[k / 4][k % 4]), s[(k + 1) / 4][(k + 1) % 4]);
    return m;
}

// A chunk's value fragments (the A operand of O^T = V^T P, value_index) past `vlast` zeroed:
// lane 16 g + d % 16 of fragment dt KS + ks holds in its slot j the position
// p0 + 32 ks + 16 (j / 4) + 4 g + j % 4; word w holds slots 2 w and 2 w + 1.
template <int KS, int DT>
__device__ __forceinline__ void zero_values_past(uint4 (&vf)[DT * KS], uint32_t p0, uint32_t vlast) {
    const uint32_t g = (uint32_t)(threadIdx.x % WAVE) / 16;
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

// A column's lazy softmax over chunks of 16 PT keys (PT tiles of 16 positions) into DT tiles of
// 16 output dimensions.
template <int PT, int DT>
struct LazySoftmax {
    static constexpr int KS = PT / 2;    // the chunk's k-blocks of 32 positions
    f32x4 neg_r = {0.f, 0.f, 0.f, 0.f};  // -r in each slot: the score MFMA's accumulator input
    f32x4 lsum = {0.f, 0.f, 0.f, 0.f};   // l, the column's sum of P (every slot alike)
    f32x4 o[DT] = {};

    // The chunk's scores less r, s, with the keys past the column's position `pos` at -inf when
    // MASK; returns the lane's largest.
    template <bool MASK>
    __device__ __forceinline__ float peak(f32x4 (&s)[PT], uint32_t p0, uint32_t pos) {
        const int lane = threadIdx.x % WAVE;
        if (MASK) {
#pragma unroll
            for (int pt = 0; pt < PT; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (p0 + pt * 16 + (lane / 16) * 4 + i > pos) s[pt][i] = -INFINITY;
        }
        return peak_of<PT>(s);
    }
    // The chunk's columns past the shift (or all on the first chunk) move r to their maximum (each
    // column's over its four lanes; mx the lane's largest, from peak), s and o, l rescaled. A
    // column that stays subtracts 0 and scales by 1: the same bits as no call.
    template <bool FIRST>
    __device__ __forceinline__ void rescale(f32x4 (&s)[PT], float mx) {
        float cm = fmaxf(mx, lane_xor16(mx));
        cm = fmaxf(cm, lane_xor32(cm));
        const float d = (FIRST || cm > LAZY_SHIFT) ? cm : 0.f;
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) s[pt] -= d;
        neg_r -= d;
        if (!FIRST) {
            const float f = __builtin_amdgcn_exp2f(-d);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] *= f;
            lsum *= f;
        }
    }
    // P = 2^s in bf16 (pf): s, the chunk's scores less r, after any rescale.
    __device__ __forceinline__ static void probs(const f32x4 (&s)[PT], uint4 (&pf)[KS]) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const f32x4 a = s[2 * ks], b = s[2 * ks + 1];
            pf[ks] = make_uint4(pack_bf16x2(__builtin_amdgcn_exp2f(a[0]), __builtin_amdgcn_exp2f(a[1])),
                                pack_bf16x2(__builtin_amdgcn_exp2f(a[2]), __builtin_amdgcn_exp2f(a[3])),
                                pack_bf16x2(__builtin_amdgcn_exp2f(b[0]), __builtin_amdgcn_exp2f(b[1])),
                                pack_bf16x2(__builtin_amdgcn_exp2f(b[2]), __builtin_amdgcn_exp2f(b[3])));
        }
    }
    // The MFMA half: column sums of P (every row of ones^T P is the sum; bf16 1.0 is 0x3f80) and
    // O^T += V^T P, each accumulator's products apart, the others between them. vf: the chunk's
    // values (fragment dt KS + ks), zeroed past the last position any column sees.
    __device__ __forceinline__ void accumulate(const uint4 (&pf)[KS], const uint4 (&vf)[DT * KS]) {
        const uint4 ones = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            lsum = mfma16(ones, pf[ks], lsum);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] = mfma16(vf[dt * KS + ks], pf[ks], o[dt]);
        }
    }
};

// ---------------------------------------------------------------------------------------------
// prefill_attention: workgroup (tile, kv): the tile's positions (up to 32, 32 / WAVES to a wave)
// for the `group` query heads KV head kv serves, heads of D dimensions. Columns of the MFMA are
// (position, head) pairs, 16 / group positions to a column group, CG column groups to a wave. The
// slot's positions from 0 to the tile's last are staged through LDS a chunk at a time (CHUNK
// positions: a 64-position block at D 64, half a block at D 128, so that a chunk's keys and values
// are 16 KiB either way); each column keeps its running maximum, sum and output
// (attention_rows.comp:71-116).
// A workgroup's tile, by the positions a column group holds (per_col = 16 / group, any group of 1
// to 16): ATTN_TILE positions at groups 1, 2 and 4 (a column group of 16, 8, 4 positions; one a
// wave); at group 3 (5 positions) ATTN_TILE_3 and at 5 (3 positions) ATTN_TILE_5, four waves of two
// column groups at D 64 and eight of one at D 128; at groups 6 to 8 (2 positions) 16 positions with
// four waves of two (eight of one at D 128), so that two workgroups share a CU: their barriers are
// their own, and one's softmax runs beside the other's products; at groups 9 to 16 a column group is
// one position's heads: eight waves of two column groups take 16 positions at D 64, and eight of one
// take 8 at D 128 (four column groups a wave, 32 positions, would hold more than a wave's registers
// and spill beside the ring's waits, which count loads in issue order).
constexpr int ATTN_TILE = 32;
constexpr int ATTN_TILE_3 = 40, ATTN_TILE_5 = 24;
constexpr int ATTN_TILE_8 = 16;
constexpr int ATTN_TILE_16 = 16, ATTN_TILE_16_D128 = 8;
// The positions a workgroup takes for `group` query heads to a KV head and heads of `head_dim`.
__host__ __device__ constexpr int attention_tile(int group, int head_dim) {
    return group > 8   ? (head_dim == 128 ? ATTN_TILE_16_D128 : ATTN_TILE_16)
           : group > 5 ? ATTN_TILE_8
           : group == 5 ? ATTN_TILE_5
           : group == 3 ? ATTN_TILE_3
                        : ATTN_TILE;
}
// The attention's ring of key-and-value stages: a stage is one chunk (16 KiB), ATTN_STAGES of them,
// up to ATTN_STAGES - 2 in flight beyond the two being taken.
constexpr int ATTN_STAGE = 2 * KV_TILE / 8;  // uint4: 16 fragments of 1 KiB
constexpr int ATTN_STAGES = 4;
constexpr int attention_chunk(int head_dim) { return head_dim == 64 ? BLOCK_TOKENS : BLOCK_TOKENS / 2; }

template <int TILE, int WAVES, int CG, int D>
__global__ void __launch_bounds__(WAVES * WAVE) __attribute__((amdgpu_waves_per_eu(2))) prefill_attention(PrefillArgs a, const uint16_t* __restrict__ q,
                                                                 const uint16_t* __restrict__ kvpool,
                                                                 uint16_t* __restrict__ attended,
                                                                 const PrefillTile* __restrict__ tiles) {
    constexpr int THREADS = WAVES * WAVE;
    constexpr int TOK = TILE / WAVES;          // positions to a wave
    constexpr int per_col = TOK / CG;          // positions to a column group
    // The query heads a KV head serves (16 / per_col of them, or fewer: a column group's columns
    // past per_col group repeat its last real one, computed alike and never stored).
    const int group = a.heads / a.kv_heads;
    const int used = per_col * group;
    static_assert(CG <= 2, "two column groups a wave at most: more spill");
    constexpr int CHUNK = attention_chunk(D);  // positions a stage holds
    constexpr int PT = CHUNK / 16, KS = PT / 2, DS = D / 32, DT = D / 16;
    constexpr int KF = PT * DS, VF = DT * KS;  // a chunk's key and value fragments
    static_assert(KF == 8 && VF == 8, "a chunk is 8 key and 8 value fragments");
    constexpr int TILE_ELEMS = kv_tile(D);
    constexpr int NS = ATTN_STAGES;
    constexpr int LOADS = ATTN_STAGE / 64 / WAVES;  // 1 KiB loads a wave makes of a stage
    static_assert(LOADS * 64 * WAVES == ATTN_STAGE, "a stage in whole 1 KiB loads");
    // The ring of NS stages, each a chunk's 8 key fragments then its 8 value fragments, then the
    // slot's block ids.
    extern __shared__ uint4 attn_ring[];
    uint32_t* block_ids = reinterpret_cast<uint32_t*>(attn_ring + NS * ATTN_STAGE);
    // Workgroup KV t + kv takes tile t for KV head kv: a tile's heads are dispatched together, in
    // the tiles' order (the longest first), so that the last workgroups to start are short ones.
    const int kv = (int)(blockIdx.x % (uint32_t)a.kv_heads);
    const PrefillTile tile = tiles[blockIdx.x / (uint32_t)a.kv_heads];
    // A tile that leaves the tensors (1 to TILE positions, of a slot of the table, inside the
    // cache's capacity and the M_pad rows) is skipped by the whole workgroup before any barrier:
    // the host builds valid ones, and a caller's own tiles in device memory cannot be checked there.
    if (tile.count == 0 || tile.count > (uint32_t)TILE || tile.slot >= (uint32_t)a.nslots || tile.count > (uint32_t)a.capacity ||
        tile.pos0 > (uint32_t)a.capacity - tile.count || tile.count > (uint32_t)a.M_pad || tile.row0 > (uint32_t)a.M_pad - tile.count)
        return;
    // The wave's index, uniform: the branches on it below are the whole wave's.
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    const int lane = threadIdx.x % WAVE;
    const int H = a.heads, KV = a.kv_heads;
    const int col = lane % 16;
    const uint32_t last = tile.pos0 + tile.count - 1;
    const int blocks = (int)(last / BLOCK_TOKENS) + 1;
    const int chunks = (int)(last / CHUNK) + 1;

    // The slot's blocks 0 .. blocks - 1 (a block the slot does not hold reads as block 0, never
    // reached by a position the run holds).
    for (int i = threadIdx.x; i < blocks; i += THREADS) {
        const uint32_t blk = a.table[(size_t)tile.slot * a.max_blocks + i];
        block_ids[i] = blk < (uint32_t)a.nblocks ? blk : 0u;
    }
    uint4 qf[CG][DS];
    uint32_t cpos[CG];
    const int colr = min(col, used - 1);  // the real column this one computes
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        const int tok = w * TOK + cg * per_col + colr / group;  // within the tile
        const int head = kv * group + colr % group;
        const size_t row = tile.row0 + (tok < (int)tile.count ? tok : 0);
        cpos[cg] = tile.pos0 + tok;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) qf[cg][ds] = load16(q + (row * H + head) * D + ds * 32 + (lane / 16) * 8);
    }
    // The ids and q in place (this wait and barrier are the compiler's own: no load to LDS is in
    // flight yet).
    __syncthreads();

    // Chunk ci into stage ci % NS, straight from the cache into LDS: wave w copies the stage's
    // fragments LOADS w .. LOADS w + LOADS - 1 (of 16: the chunk's keys, a run of its block's key
    // tile from fragment 8 half, then its values, fragments (dt, half + ks) of the value tile), lane
    // l its 16 bytes 16 l. Past the last chunk the last is loaded again (never read), so that every
    // wave makes LOADS loads a chunk and its count in flight says which stages have landed. The
    // block id is read by an LDS read of its own, which the compiler does not order behind the
    // loads to LDS in flight.
    auto fetch = [&](int ci) __attribute__((always_inline)) {
        const int c = min(ci, chunks - 1);
        const uint32_t* at = block_ids + c * CHUNK / BLOCK_TOKENS;
        uint32_t id;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(id) : "v"(lds_offset(at)) : "memory");
        const uint32_t blk = __builtin_amdgcn_readfirstlane(id);
        const int half = (c * CHUNK % BLOCK_TOKENS) / 32;
        const uint16_t* src = kvpool + ((size_t)blk * KV + kv) * 2 * TILE_ELEMS;
        uint4* dst = attn_ring + (ci % NS) * ATTN_STAGE;
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const int f = w * LOADS + j;  // the stage's fragment
            const int from = f < KF ? half * KF + f : TILE_ELEMS / 512 + ((f - KF) / KS) * 2 + half + (f - KF) % KS;
            load_to_lds(src + (size_t)from * 512 + lane * 8, dst + f * 64);
        }
    };

    LazySoftmax<PT, DT> sm[CG];
    // The wave's first position: chunks wholly at or below it need no mask.
    const uint32_t first = tile.pos0 + w * TOK;
    // Chunks 0 .. nfull - 1 need no mask: they end at or before the wave's first position and the
    // tile's last (a wave past the tile's count has a first position past its last).
    const int nfull = (int)((min(first, last) + 1) / CHUNK);

    // The ring: chunk ci's keys are in registers when step ci starts. Its values are read from
    // LDS while the score MFMAs run; then chunk ci + 1's stage is waited for (the barrier also says
    // every wave is done with stage ci - 1, which chunk ci + NS - 1 takes) and, once the softmax has
    // read every score, its keys read while the exponentials and the value MFMAs of chunk ci run.
    // Fragment i of a stage is 1 KiB i on, lane l's 16 bytes 16 l on: its LDS address is the lane's
    // base plus a constant.
    constexpr int STAGE_BYTES = ATTN_STAGE * 16;
    constexpr int VALUES = KF * 1024;  // the values' bytes from the stage's start
    const uint32_t ring0 = lds_offset(attn_ring) + lane * 16;
#pragma unroll
    for (int ci = 0; ci < NS - 1; ++ci) fetch(ci);
    wait_vm<LOADS * (NS - 2)>();
    stage_barrier();
    uint4 kf[KF], vf[VF];
    lds_read16_x8<0, 1024>(ring0, kf);
    lds_landed(kf);
    // Step ci, its softmax half as MASK (keys past a column's position count for nothing, and the
    // values past the tile's last position read as zero) and FIRST (chunk 0). Past the last chunk
    // the keys of a stage the ring has already waited for are read and never used.
    auto step = [&](int ci, auto mask_tag, auto first_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value, FIRST = decltype(first_tag)::value;
        lds_read16_x8<VALUES, 1024>(ring0 + (uint32_t)(ci % NS) * STAGE_BYTES, vf);
        // The first k-block of every tile's product before any later one: the MFMAs a tile's
        // next k-block waits on are done by the time it issues.
        f32x4 s[CG][PT];
#pragma unroll
        for (int cg = 0; cg < CG; ++cg)
#pragma unroll
            for (int pt = 0; pt < PT; ++pt) s[cg][pt] = mfma16(kf[pt * DS], qf[cg][0], sm[cg].neg_r);
#pragma unroll
        for (int ds = 1; ds < DS; ++ds)
#pragma unroll
            for (int cg = 0; cg < CG; ++cg)
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) s[cg][pt] = mfma16(kf[pt * DS + ds], qf[cg][ds], s[cg][pt]);
        // Stage ci + 1 landed for every wave: no more than the NS - 3 chunks fetched after it in
        // flight for this one, then the barrier.
        wait_vm<LOADS * (NS - 3)>();
        stage_barrier();
        fetch(ci + NS - 1);  // its id's LDS read waits for every LDS read before it: vf has landed
        lds_arrived(vf);
        const uint32_t p0 = (uint32_t)ci * CHUNK;
        float mx[CG];
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) mx[cg] = sm[cg].template peak<MASK>(s[cg], p0, cpos[cg]);
        // The keys' reads may take registers the compiler counts free once an MFMA has issued, and
        // an MFMA reads its accumulator input late in its passes, past the wait states the
        // compiler would give its own loads (it does not look into asm): the reads come after the
        // maxima, whose reads of every score wait for every score MFMA to finish.
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) asm volatile("" ::"v"(mx[cg]));
        lds_read16_x8<0, 1024>(ring0 + (uint32_t)((ci + 1) % NS) * STAGE_BYTES, kf);
        // Values past the tile's last position read as zero (attention_rows.comp:1-13): every
        // position up to it was written by this run or before it; the cache may hold anything
        // past it, NaN included, and 0 NaN is NaN. A chunk with no mask ends at or before the
        // tile's last position.
        if (MASK && p0 + CHUNK - 1 > last) zero_values_past<KS, DT>(vf, p0, last);
        // One check for the wave's column groups (the rescale is rare past chunk 0), so that the
        // exponentials and value MFMAs below are one stretch of code: the compiler runs a group's
        // exponentials beside the previous group's MFMAs (a wave's VALU work runs beside its own
        // MFMAs when they do not depend on it).
        float peak_all = mx[0];
#pragma unroll
        for (int cg = 1; cg < CG; ++cg) peak_all = fmaxf(peak_all, mx[cg]);
        if (FIRST || __builtin_amdgcn_ballot_w64(peak_all > LAZY_SHIFT) != 0) {
#pragma unroll
            for (int cg = 0; cg < CG; ++cg) sm[cg].template rescale<FIRST>(s[cg], mx[cg]);
        }
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
            uint4 pf[KS];
            LazySoftmax<PT, DT>::probs(s[cg], pf);
            sm[cg].accumulate(pf, vf);
        }
        lds_landed(kf);
    };
    using yes = std::true_type;
    using no = std::false_type;
    if (nfull > 0)
        step(0, no{}, yes{});
    else
        step(0, yes{}, yes{});
    int ci = 1;
    for (; ci < nfull; ++ci) step(ci, no{}, no{});
    for (; ci < chunks; ++ci) step(ci, yes{}, no{});
    // No load into this workgroup's LDS may still be in flight when its waves end.
    wait_vm<0>();
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        const int tok = w * TOK + cg * per_col + colr / group;
        if (col >= used || tok >= (int)tile.count) continue;
        const int head = kv * group + colr % group;
        const size_t row = tile.row0 + tok;
        const float inv = 1.0f / sm[cg].lsum[0];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int d = dt * 16 + (lane / 16) * 4;
            const f32x4 o = sm[cg].o[dt];
            uint2 packed = make_uint2(pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv));
            *reinterpret_cast<uint2*>(attended + act_index((int)row, head * D + d, H * D)) = packed;
        }
    }
}

// Each projection's X rows to a workgroup. 128 for all: with two workgroups to a CU, one's
// epilogue (10 bytes an output for o_proj and down_proj: the f32 residual in and out, the next
// norm's bf16 operand) and prologue run beside the other's products, which at 8 x 2048 positions
// beats one 256-row workgroup to a CU for every projection (gate/up by a tenth).
constexpr int QKV_TM = 128, O_TM = 128, GATE_UP_TM = 128, DOWN_TM = 128;

template <int EPI, int WR, int TM, int D = HEAD_DIM>
void gemm(const char* label, const PrefillArgs& a, const GemmArgs& g, hipStream_t stream, DispatchTimer* timer) {
    dispatch(label, prefill_gemm<EPI, WR, TM, D>, dim3(g.N / TN, a.M_pad / TM), dim3(GemmTile<TM>::THREADS), GemmTile<TM>::LDS,
             stream, timer, a, g);
}

// The attention's instance for `group` query heads to a KV head and heads of D dimensions.
template <int D>
hipError_t attention(const PrefillArgs& a, const uint16_t* q, const uint16_t* kv, uint16_t* attended, const PrefillTile* tiles,
                     int ntiles, size_t lds, hipStream_t stream, DispatchTimer* timer) {
    const dim3 grid((uint32_t)ntiles * (uint32_t)a.kv_heads);
    if (a.kv_heads <= 0 || a.heads % a.kv_heads != 0) return hipErrorInvalidValue;
    const int group = a.heads / a.kv_heads;
#define TGX_ATTENTION(TILE_, WAVES_, CG_) \
    dispatch("prefill_attention", prefill_attention<TILE_, WAVES_, CG_, D>, grid, dim3(WAVES_ * WAVE), lds, stream, timer, a, q, kv, attended, tiles)
    // At D 128 a wave holds one column group: two groups' outputs and scores would hold more than
    // its registers.
    if (group == 1)
        TGX_ATTENTION(ATTN_TILE, 2, 1);
    else if (group == 2)
        TGX_ATTENTION(ATTN_TILE, 4, 1);
    else if (group == 3) {
        if constexpr (D == 64) TGX_ATTENTION(ATTN_TILE_3, 4, 2);
        else TGX_ATTENTION(ATTN_TILE_3, 8, 1);
    } else if (group == 4)
        TGX_ATTENTION(ATTN_TILE, 8, 1);
    else if (group == 5) {
        if constexpr (D == 64) TGX_ATTENTION(ATTN_TILE_5, 4, 2);
        else TGX_ATTENTION(ATTN_TILE_5, 8, 1);
    } else if (group <= 8) {
        if constexpr (D == 64) TGX_ATTENTION(ATTN_TILE_8, 4, 2);
        else TGX_ATTENTION(ATTN_TILE_8, 8, 1);
    } else if (group <= 16) {
        // A position to a column group, eight waves of two at D 64, of one at D 128.
        if constexpr (D == 64) TGX_ATTENTION(ATTN_TILE_16, 8, 2);
        else TGX_ATTENTION(ATTN_TILE_16_D128, 8, 1);
    } else {
        return hipErrorInvalidValue;
    }
#undef TGX_ATTENTION
    return hipSuccess;
}

hipError_t allow(const void* kernel, size_t device_lds) {
    hipFuncAttributes attr{};
    hipError_t e = hipFuncGetAttributes(&attr, kernel);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(device_lds - attr.sharedSizeBytes));
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// The prefill's scratch for callers that cannot allocate (tgx_prefill_runs_noalloc): one array of
// PREFILL_SCRATCH_BYTES on each GPU the library runs on, held until the process ends. In host code
// `scratch` names a host-side stand-in, not the device's array: host code reaches the array only
// through the address prefill_scratch_address found for the device.
static __device__ __align__(256) unsigned char scratch[PREFILL_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_lock;
void* scratch_at[MAX_DEVICES] = {};
}  // namespace

hipError_t prefill_scratch_address(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> hold(scratch_lock);
    if (!scratch_at[device]) {
        int current = -1;
        hipError_t e = hipGetDevice(&current);
        if (e != hipSuccess) return e;
        if (current != device) return hipErrorInvalidDevice;  // the caller makes the device current
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        scratch_at[device] = p;
    }
    *out = scratch_at[device];
    return hipSuccess;
}

// Zeroes `count` 16-byte words at p: a kernel, not hipMemsetAsync, so that a caller may record it
// into a graph.
__global__ void __launch_bounds__(256) fill_zero(uint4* __restrict__ p, size_t count) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) p[i] = make_uint4(0, 0, 0, 0);
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
    if (bytes % 16 || (uintptr_t)p % 16) return hipErrorInvalidValue;
    const size_t count = bytes / 16;
    if (count == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((count + 255) / 256, 1024);
    fill_zero<<<blocks, 256, 0, stream>>>((uint4*)p, count);
    return hipGetLastError();
}

// Copies `count` 16-byte words from device memory to pinned host memory the device maps, by the
// compute queue's own stores: a copy engine's transfer queued behind a kernel starts only on a
// signal between the queues, which at 256 KiB took longer than the copy itself.
__global__ void __launch_bounds__(256) copy_words(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t count) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_copy_words(const void* src, void* dst, size_t bytes, hipStream_t stream) {
    if (bytes % 16 || (uintptr_t)src % 16 || (uintptr_t)dst % 16) return hipErrorInvalidValue;
    const size_t count = bytes / 16;
    if (count == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((count + 255) / 256, 256);
    copy_words<<<blocks, 256, 0, stream>>>((const uint4*)src, (uint4*)dst, count);
    return hipGetLastError();
}

// Copies the segments' 4-byte words in one launch (host staging the device maps, read over the
// bus, into device memory): the step's inputs reach the device on the compute queue, ahead of the
// step, with no signal between queues.
__global__ void __launch_bounds__(256) copy_segments(CopySegments c) {
    const uint32_t total = c.end[c.n - 1];
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
        int k = 0;
        while (i >= c.end[k]) ++k;
        const uint32_t j = i - (k ? c.end[k - 1] : 0u);
        c.dst[k][j] = c.src[k][j];
    }
}

hipError_t launch_copy_segments(const CopySegments& c, hipStream_t stream) {
    if (c.n <= 0) return hipSuccess;
    if (c.n > COPY_SEGMENTS) return hipErrorInvalidValue;
    for (int k = 0; k < c.n; ++k)
        if ((k ? c.end[k - 1] : 0u) > c.end[k]) return hipErrorInvalidValue;
    const uint32_t total = c.end[c.n - 1];
    if (total == 0) return hipSuccess;
    const unsigned blocks = std::min<unsigned>((total + 255) / 256, 256);
    copy_segments<<<blocks, 256, 0, stream>>>(c);
    return hipGetLastError();
}

int prefill_attention_tile(int group, int head_dim) { return attention_tile(group, head_dim); }

hipError_t prefill_prepare(size_t device_lds) {
    hipError_t e;
    if ((e = allow((const void*)prefill_gemm<EPI_QKV, QKV_ROWS, QKV_TM, 64>, device_lds)) != hipSuccess) return e;
    if ((e = allow((const void*)prefill_gemm<EPI_QKV, QKV_ROWS, QKV_TM, 128>, device_lds)) != hipSuccess) return e;
    if ((e = allow((const void*)prefill_gemm<EPI_RESIDUAL_IN, 4, O_TM>, device_lds)) != hipSuccess) return e;
    if ((e = allow((const void*)prefill_gemm<EPI_RESIDUAL_IN, 16, O_TM>, device_lds)) != hipSuccess) return e;
    if ((e = allow((const void*)prefill_gemm<EPI_RESIDUAL, 4, DOWN_TM>, device_lds)) != hipSuccess) return e;
    if ((e = allow((const void*)prefill_gemm<EPI_RESIDUAL, 16, DOWN_TM>, device_lds)) != hipSuccess) return e;
    for (const void* f : {(const void*)prefill_attention<ATTN_TILE, 2, 1, 64>, (const void*)prefill_attention<ATTN_TILE, 4, 1, 64>,
                          (const void*)prefill_attention<ATTN_TILE, 8, 1, 64>, (const void*)prefill_attention<ATTN_TILE_8, 4, 2, 64>,
                          (const void*)prefill_attention<ATTN_TILE, 2, 1, 128>, (const void*)prefill_attention<ATTN_TILE, 4, 1, 128>,
                          (const void*)prefill_attention<ATTN_TILE, 8, 1, 128>, (const void*)prefill_attention<ATTN_TILE_8, 8, 1, 128>,
                          (const void*)prefill_attention<ATTN_TILE_16, 8, 2, 64>, (const void*)prefill_attention<ATTN_TILE_16_D128, 8, 1, 128>,
                          (const void*)prefill_attention<ATTN_TILE_3, 4, 2, 64>, (const void*)prefill_attention<ATTN_TILE_3, 8, 1, 128>,
                          (const void*)prefill_attention<ATTN_TILE_5, 4, 2, 64>, (const void*)prefill_attention<ATTN_TILE_5, 8, 1, 128>})
        if ((e = allow(f, device_lds)) != hipSuccess) return e;
    return allow((const void*)prefill_gemm<EPI_SILU, QKV_ROWS, GATE_UP_TM>, device_lds);
}

size_t prefill_attention_lds(int max_blocks) {
    // The attention's ring and the slot's block ids.
    return (size_t)ATTN_STAGES * ATTN_STAGE * sizeof(uint4) + (size_t)max_blocks * sizeof(uint32_t);
}

hipError_t launch_prefill_gemm(const PrefillArgs& a, int epi, int strip_rows, const GemmArgs& g, hipStream_t stream,
                               DispatchTimer* timer) {
    if (g.K <= 0 || g.K % 1024 || g.N <= 0 || g.N % TN || a.M_pad % ROW_TILE_MAX) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_QKV:
            if (strip_rows != QKV_ROWS) return hipErrorInvalidValue;
            if (a.head_dim == 128)
                gemm<EPI_QKV, QKV_ROWS, QKV_TM, 128>("prefill_qkv", a, g, stream, timer);
            else if (a.head_dim == 64)
                gemm<EPI_QKV, QKV_ROWS, QKV_TM, 64>("prefill_qkv", a, g, stream, timer);
            else
                return hipErrorInvalidValue;
            break;
        case EPI_SILU:
            if (strip_rows != QKV_ROWS) return hipErrorInvalidValue;
            gemm<EPI_SILU, QKV_ROWS, GATE_UP_TM>("prefill_gate_up", a, g, stream, timer);
            break;
        case EPI_RESIDUAL_IN:
            if (strip_rows == 4)
                gemm<EPI_RESIDUAL_IN, 4, O_TM>("prefill_o", a, g, stream, timer);
            else if (strip_rows == 16)
                gemm<EPI_RESIDUAL_IN, 16, O_TM>("prefill_o", a, g, stream, timer);
            else
                return hipErrorInvalidValue;
            break;
        case EPI_RESIDUAL:
            if (strip_rows == 4)
                gemm<EPI_RESIDUAL, 4, DOWN_TM>("prefill_down", a, g, stream, timer);
            else if (strip_rows == 16)
                gemm<EPI_RESIDUAL, 16, DOWN_TM>("prefill_down", a, g, stream, timer);
            else
                return hipErrorInvalidValue;
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_prefill_attention(const PrefillArgs& a, const uint16_t* q, const uint16_t* kv, uint16_t* attended,
                                    const PrefillTile* tiles, int ntiles, hipStream_t stream, DispatchTimer* timer) {
    const size_t lds = prefill_attention_lds(a.max_blocks);
    hipError_t e = a.head_dim == 128 ? attention<128>(a, q, kv, attended, tiles, ntiles, lds, stream, timer)
                   : a.head_dim == 64 ? attention<64>(a, q, kv, attended, tiles, ntiles, lds, stream, timer)
                                      : hipErrorInvalidValue;
    return e != hipSuccess ? e : hipGetLastError();
}

hipError_t launch_prefill_norm(const PrefillArgs& a, bool final, const float* x, const float* gain, uint16_t* out_bf16,
                               float* out_f32, hipStream_t stream, DispatchTimer* timer) {
    const dim3 rows4((a.M_pad + 3) / 4);
    // hidden is 1024 or 2048 (the shape check's).
    if (a.hidden != 1024 && a.hidden != 2048) return hipErrorInvalidValue;
    const bool wide = a.hidden == 2048;
    if (final)
        dispatch("prefill_final_norm", wide ? prefill_norm<true, 32> : prefill_norm<true, 16>, rows4, dim3(256), 0, stream, timer, a, x,
                 gain, (uint16_t*)nullptr, out_f32);
    else
        dispatch("prefill_norm", wide ? prefill_norm<false, 32> : prefill_norm<false, 16>, rows4, dim3(256), 0, stream, timer, a, x, gain,
                 out_bf16, (float*)nullptr);
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, const PrefillLayer* layers, int nlayers, const float* final_norm,
                          const PrefillBuffers& b, hipStream_t stream, DispatchTimer* timer) {
    if (a.head_dim != 64 && a.head_dim != 128) return hipErrorInvalidValue;
    const int qkv_rows = (a.heads + 2 * a.kv_heads) * a.head_dim;
    hipError_t e = hipSuccess;
    // Layer 0's input norm; each later norm's input (the rows times the gain, and their sums of
    // squares) comes from the projection before it, the rows' scales applied by the GEMM after.
    if (nlayers > 0) e = launch_prefill_norm(a, false, b.x, layers[0].input_norm, b.normed, nullptr, stream, timer);
    const float* input = b.x;  // layer 0 reads the run's states, which stay as written
    for (int l = 0; l < nlayers && e == hipSuccess; ++l) {
        const PrefillLayer& L = layers[l];
        GemmArgs qkv{L.qkv, b.normed, a.hidden, qkv_rows, nullptr, nullptr, nullptr, b.q, L.kv,
                     l == 0 ? nullptr : b.row_sq, nullptr, nullptr, nullptr};
        e = launch_prefill_gemm(a, EPI_QKV, QKV_ROWS, qkv, stream, timer);
        if (e == hipSuccess) e = launch_prefill_attention(a, b.q, L.kv, b.attended, b.tiles, b.ntiles, stream, timer);
        GemmArgs o{L.o, b.attended, a.heads * a.head_dim, a.hidden, input, b.mid, nullptr, nullptr, nullptr,
                   nullptr, L.post_norm, b.normed, b.row_sq};
        if (e == hipSuccess) e = launch_prefill_gemm(a, EPI_RESIDUAL_IN, L.od_rows, o, stream, timer);
        GemmArgs gu{L.gate_up, b.normed, a.hidden, 2 * a.inner, nullptr, nullptr, b.mlp, nullptr, nullptr,
                    b.row_sq, nullptr, nullptr, nullptr};
        if (e == hipSuccess) e = launch_prefill_gemm(a, EPI_SILU, QKV_ROWS, gu, stream, timer);
        // The last layer's output goes to the final norm, which reads the f32 rows.
        GemmArgs down{L.down, b.mlp, a.inner, a.hidden, b.mid, b.h, nullptr, nullptr, nullptr,
                      nullptr, l + 1 < nlayers ? layers[l + 1].input_norm : nullptr, b.normed, b.row_sq};
        if (e == hipSuccess) e = launch_prefill_gemm(a, EPI_RESIDUAL, L.od_rows, down, stream, timer);
        input = b.h;
    }
    if (e == hipSuccess) e = launch_prefill_norm(a, true, input, final_norm, nullptr, b.out, stream, timer);
    return e;
}

}  // namespace tgx
