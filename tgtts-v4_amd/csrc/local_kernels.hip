// The local stack and the patch sampler on gfx950 (crates/graph/src/local/mod.rs:354-656 with
// local_{norm,qkv_rope,attention,partial,add_norm,gate_up}.comp; crates/graph/src/local/dit.rs
// with local_embed.comp, dit_euler.comp and cfm_noise.comp):
//
//   local_gemm      C = X W^T over a few hundred tokens, bf16 in, f32 accumulate, a 64-row by
//                   128-token tile to a workgroup of four waves, staged through LDS by direct
//                   global-to-LDS loads, with the epilogue fused: RoPE at each token's place in
//                   its sequence (local_qkv_rope.comp), SiLU(gate) up (local_gate_up.comp), or
//                   the f32 sums of one part of the columns (local_partial.comp)
//   local_attention every token of a sequence attends to every token of it, a wave to a
//                   sequence and query head, both products on MFMA (local_attention.comp)
//   local_add_norm  residual + the parts' sums in their order, then RMSNorm (local_add_norm.comp,
//                   local_norm.comp)
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

constexpr int LG_THREADS = 256;
constexpr int LG_TKB = 2;                             // k-blocks of 32 to a stage
constexpr int LG_W_STAGE = 4 * LG_TKB * 64;            // uint4 per stage: 4 strips, 8 KiB
constexpr int LG_X_STAGE = 8 * LG_TKB * 64;            // 8 token tiles, 16 KiB
constexpr int LG_FRAGS = (LG_W_STAGE + LG_X_STAGE) / 64 / 4;  // 1 KiB fragments a wave loads a stage
constexpr int LG_NBUF = 4;  // stages in the LDS ring: three in flight while one is multiplied
constexpr size_t LG_LDS = (size_t)LG_NBUF * (LG_W_STAGE + LG_X_STAGE) * sizeof(uint4);  // 96 KiB

enum LocalEpilogue { LEPI_QKV = 0, LEPI_PARTIAL = 1, LEPI_SILU = 2 };

struct LocalGemm {
    const uint16_t* w;  // 16-row tiles of [N][K]
    const uint16_t* x;  // bf16 [M_pad][K]
    int K, N;
    float* partial;     // LEPI_PARTIAL: f32 [parts][M_pad][N]
    uint16_t* mlp;      // LEPI_SILU: bf16 [M_pad][N / 2]
    uint16_t *q, *k, *v;
};

// Strip s (0, 1) of wave row wn of n-block nb: two strips of W in a row, or for the gate/up
// projection a strip of the gate and the same rows of up.
template <int EPI>
__device__ __forceinline__ int local_strip(int nb, int wn, int s, int N) {
    if (EPI == LEPI_SILU) {
        const int gate = nb * 2 + wn;
        return s == 0 ? gate : gate + N / 32;
    }
    return nb * 4 + wn * 2 + s;
}

// Grid (n-blocks, token blocks, parts): part z sums k-blocks z K/32/parts .. of every row.
template <int EPI>
__global__ void __launch_bounds__(LG_THREADS) local_gemm(LocalArgs a, LocalGemm g) {
    extern __shared__ uint4 lds[];
    uint4* ws = lds;                         // [LG_NBUF][LG_W_STAGE]
    uint4* xs = lds + LG_NBUF * LG_W_STAGE;  // [LG_NBUF][LG_X_STAGE]
    const int nb = blockIdx.x, m0 = blockIdx.y * LOCAL_TOKEN_TILE, part = blockIdx.z;
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int wn = w / 2, wm = w % 2;
    const int kblocks = g.K / 32;
    const int part_kb = kblocks / gridDim.z;
    const int kb0 = part * part_kb;
    const int stages = part_kb / LG_TKB;

    // Fragments 0..7 of a stage are W's (strip f / 2, k-block f % 2), 8..23 the tokens' (tile
    // (f - 8) / 2): lane l of a load writes bytes 16 l .. of the fragment, the MFMA operand order.
    // Each wave issues exactly LG_FRAGS loads a stage (the branch is uniform across the wave), so
    // its count of loads in flight says which stages have landed.
    auto fetch = [&](int st) {
        const int buf = st % LG_NBUF;
#pragma unroll
        for (int j = 0; j < LG_FRAGS; ++j) {
            const int f = w * LG_FRAGS + j;
            const int kb = kb0 + st * LG_TKB + f % 2;
            if (f < 8) {
                const int sl = f / 2;
                const uint16_t* src = g.w + weight_tile_index(local_strip<EPI>(nb, sl / 2, sl % 2, g.N), kb, kblocks, 16) + lane * 8;
                load_to_lds(src, &ws[buf * LG_W_STAGE + f * 64]);
            } else {
                const int mt = (f - 8) / 2;
                const uint16_t* src = g.x + (size_t)(m0 + mt * 16 + lane % 16) * g.K + kb * 32 + (lane / 16) * 8;
                load_to_lds(src, &xs[buf * LG_X_STAGE + (f - 8) * 64]);
            }
        }
    };

    f32x4 acc[2][4];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int p = 0; p < LG_NBUF - 1; ++p)
        if (p < stages) fetch(p);
    for (int st = 0; st < stages; ++st) {
        // Stage st has landed once no more than the later stages' loads are in flight; the barrier
        // makes it so for every wave, and says every wave is done with stage st - 1, whose buffer
        // the next fetch takes.
        const int ahead = min(LG_NBUF - 2, stages - 1 - st);
        if (ahead >= 2)
            wait_vm<2 * LG_FRAGS>();
        else if (ahead == 1)
            wait_vm<LG_FRAGS>();
        else
            wait_vm<0>();
        stage_barrier();
        if (st + LG_NBUF - 1 < stages) fetch(st + LG_NBUF - 1);
        const int buf = st % LG_NBUF;
        // fr[6 kbl + s]: W strip s; fr[6 kbl + 2 + t]: token tile t; of k-block kbl.
        uint4 fr[LG_TKB * 6];
#pragma unroll
        for (int kbl = 0; kbl < LG_TKB; ++kbl) {
#pragma unroll
            for (int s = 0; s < 2; ++s) fr[kbl * 6 + s] = lds_read16(&ws[buf * LG_W_STAGE + ((wn * 2 + s) * LG_TKB + kbl) * 64 + lane]);
#pragma unroll
            for (int t = 0; t < 4; ++t) fr[kbl * 6 + 2 + t] = lds_read16(&xs[buf * LG_X_STAGE + ((wm * 4 + t) * LG_TKB + kbl) * 64 + lane]);
        }
        lds_landed(fr);
#pragma unroll
        for (int kbl = 0; kbl < LG_TKB; ++kbl)
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int t = 0; t < 4; ++t) acc[s][t] = mfma16(fr[kbl * 6 + s], fr[kbl * 6 + 2 + t], acc[s][t]);
    }

    // Tile (s, t) holds W rows 16 strip + 4 (lane / 16) + i against token m0 + 16 (4 wm + t) + lane % 16.
    const int quad = lane / 16;
    if (EPI == LEPI_PARTIAL) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int n = local_strip<EPI>(nb, wn, s, g.N) * 16 + quad * 4;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int m = m0 + (wm * 4 + t) * 16 + lane % 16;
                *reinterpret_cast<float4*>(g.partial + ((size_t)part * a.M_pad + m) * g.N + n) =
                    make_float4(acc[s][t][0], acc[s][t][1], acc[s][t][2], acc[s][t][3]);
            }
        }
    } else if (EPI == LEPI_SILU) {
        const int inner = g.N / 2;
        const int n = local_strip<EPI>(nb, wn, 0, g.N) * 16 + quad * 4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int m = m0 + (wm * 4 + t) * 16 + lane % 16;
            if (m >= a.M) continue;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float gate = acc[0][t][i], up = acc[1][t][i];
                v[i] = gate / (1.0f + __expf(-gate)) * up;
            }
            *reinterpret_cast<uint2*>(g.mlp + (size_t)m * inner + n) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        }
    } else {  // LEPI_QKV: a strip's rows pair as r, r + 8 (lanes l and l ^ 32)
        const int H = a.heads, KV = a.kv_heads;
        const bool second = quad >= 2;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int strip = local_strip<EPI>(nb, wn, s, g.N);
            const int head = strip / 4, qtr = strip % 4;
            const int p0 = qtr * 8 + (quad % 2) * 4;  // the first of this lane's 4 pairs
            const int d0 = p0 + (second ? HEAD_DIM / 2 : 0);
            const bool rotate = head < H + KV && a.rope;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float own[4], other[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    own[i] = acc[s][t][i];
                    other[i] = lane_xor32(own[i]);
                }
                const int m = m0 + (wm * 4 + t) * 16 + lane % 16;
                if (m >= a.M) continue;
                float v[4];
                if (rotate) {
                    const int place = m % a.T;
                    const float4 co = *reinterpret_cast<const float4*>(a.cos + place * (HEAD_DIM / 2) + p0);
                    const float4 si = *reinterpret_cast<const float4*>(a.sin + place * (HEAD_DIM / 2) + p0);
                    const float c4[4] = {co.x, co.y, co.z, co.w}, s4[4] = {si.x, si.y, si.z, si.w};
                    // As upstream: x cos + rotate_half(x) sin (local_qkv_rope.comp:71-76).
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        v[i] = second ? own[i] * c4[i] + other[i] * s4[i] : own[i] * c4[i] - other[i] * s4[i];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = own[i];
                }
                const uint2 packed = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                if (head < H)
                    *reinterpret_cast<uint2*>(g.q + ((size_t)m * H + head) * HEAD_DIM + d0) = packed;
                else if (head < H + KV)
                    *reinterpret_cast<uint2*>(g.k + ((size_t)m * KV + head - H) * HEAD_DIM + d0) = packed;
                else
                    *reinterpret_cast<uint2*>(g.v + ((size_t)m * KV + head - H - KV) * HEAD_DIM + d0) = packed;
            }
        }
    }
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
    uint16_t* out = attended + ((size_t)(first + r) * H + head) * HEAD_DIM;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
        *reinterpret_cast<uint2*>(out + 16 * dt + 4 * g) =
            make_uint2(pack_bf16x2(o[dt][0] * inv, o[dt][1] * inv), pack_bf16x2(o[dt][2] * inv, o[dt][3] * inv));
}

// ---------------------------------------------------------------------------------------------
// local_add_norm: a wave to a token. sum = residual + the parts' sums in part order (written to
// `sum` when given), then RMSNorm with gain g: lane l squares its hidden / 64 values in order, the
// lanes added by a butterfly. FINAL writes the normed row in f32, else in bf16.
template <bool FINAL>
__global__ void __launch_bounds__(256) local_add_norm(LocalArgs a, const float* __restrict__ partial, int parts,
                                                      const float* __restrict__ residual, float* __restrict__ sum,
                                                      const float* __restrict__ gain, uint16_t* __restrict__ normed,
                                                      float* __restrict__ out) {
    const int m = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (m >= a.M) return;
    const int K = a.hidden, per = K / WAVE;  // 16 at hidden 1024
    float v[32];
    const int base = lane * per;
#pragma unroll
    for (int e = 0; e < 32; e += 4) {
        if (e >= per) break;
        float4 r = *reinterpret_cast<const float4*>(residual + (size_t)m * K + base + e);
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int p = 0; p < parts; ++p) {
            const float4 s = *reinterpret_cast<const float4*>(partial + ((size_t)p * a.M_pad + m) * K + base + e);
            acc.x += s.x;
            acc.y += s.y;
            acc.z += s.z;
            acc.w += s.w;
        }
        v[e] = r.x + acc.x;
        v[e + 1] = r.y + acc.y;
        v[e + 2] = r.z + acc.z;
        v[e + 3] = r.w + acc.w;
        if (sum) *reinterpret_cast<float4*>(sum + (size_t)m * K + base + e) = make_float4(v[e], v[e + 1], v[e + 2], v[e + 3]);
    }
    float squares = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        if (e >= per) break;
        squares += v[e] * v[e];
    }
    const float scale = 1.0f / sqrtf(wave_sum(squares) / (float)K + a.eps);
#pragma unroll
    for (int e = 0; e < 32; e += 8) {
        if (e >= per) break;
        float n[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) n[i] = v[e + i] * scale * gain[base + e + i];
        if (FINAL) {
            *reinterpret_cast<float4*>(out + (size_t)m * K + base + e) = make_float4(n[0], n[1], n[2], n[3]);
            *reinterpret_cast<float4*>(out + (size_t)m * K + base + e + 4) = make_float4(n[4], n[5], n[6], n[7]);
        } else {
            *reinterpret_cast<uint4*>(normed + (size_t)m * K + base + e) =
                make_uint4(pack_bf16x2(n[0], n[1]), pack_bf16x2(n[2], n[3]), pack_bf16x2(n[4], n[5]), pack_bf16x2(n[6], n[7]));
        }
    }
}

// ---------------------------------------------------------------------------------------------
// local_embed: grid (hidden / 256, rows); thread n of the row: acc_f = bias[n] + sum_c W[n][c]
// frame_f[c] in channel order, for each of the row's frames, written as tokens first + f of both
// of the row's sequences; and the copied tokens.
constexpr int EMBED_MAX = 1024;     // channels x frames a row's patch may hold
constexpr int EMBED_CHANNELS = 64;  // channels at most (a row of W in 16 float4 loads)

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
    for (int i = threadIdx.x; i < C * F; i += 256) {
        const int f = i / C, c = i % C;
        frames[i] = e.src[((size_t)row * C + c) * F + f];
    }
    __syncthreads();
    if (blockIdx.x * 256 + threadIdx.x >= a.hidden) return;
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
    const int K = a.hidden;
    for (int s = 0; s < e.seqs; ++s) {
        const size_t seq0 = (size_t)(row * e.seqs + s) * a.T;
#pragma unroll
        for (int f = 0; f < F; ++f) e.x0[(seq0 + e.first + f) * K + n] = acc[f];
        for (int t = 0; t < e.copies; ++t) {
            const float* src = e.copy_src + ((size_t)(e.shared ? 0 : row * e.copies) + t) * K;
            e.x0[(seq0 + e.copy_at + t) * K + n] = (e.guided && s > 0) ? 0.f : src[n];
        }
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
    const float* src = e.out + ((size_t)(row * 2 + tmc / F) * a.T + e.first + tmc % F) * K + (lane / 16) * 8;
    float4 lo[EULER_KB], hi[EULER_KB];
    uint4 wf[EULER_KB][EULER_STRIPS];
#pragma unroll
    for (int j = 0; j < EULER_KB; ++j) {
        const int kb = w * EULER_KB + j;
        lo[j] = *reinterpret_cast<const float4*>(src + kb * 32);
        hi[j] = *reinterpret_cast<const float4*>(src + kb * 32 + 4);
#pragma unroll
        for (int s = 0; s < EULER_STRIPS; ++s)
            wf[j][s] = *reinterpret_cast<const uint4*>(e.w + weight_tile_index(min(s, strips - 1), kb, KB, 16) + lane * 8);
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

hipError_t launch_local_stack(const LocalArgs& a, const LocalLayer* layers, int nlayers, const float* final_norm,
                              const LocalBuffers& b, hipStream_t stream, DispatchTimer* timer) {
    const dim3 block(LG_THREADS);
    const int mblocks = a.M_pad / LOCAL_TOKEN_TILE;
    const dim3 rows4((a.M + 3) / 4);
    const int H = a.heads, KV = a.kv_heads;
    const int qkv_rows = (H + 2 * KV) * HEAD_DIM;
    // The first layer's input norm.
    dispatch("local_norm", local_add_norm<false>, rows4, dim3(256), 0, stream, timer, a, (const float*)nullptr, 0, b.x0,
             (float*)nullptr, layers[0].input_norm, b.normed, (float*)nullptr);
    for (int l = 0; l < nlayers; ++l) {
        const LocalLayer& L = layers[l];
        const float* input = l == 0 ? b.x0 : b.x;
        LocalGemm qkv{L.qkv, b.normed, a.hidden, qkv_rows, nullptr, nullptr, b.q, b.k, b.v};
        dispatch("local_qkv_rope", local_gemm<LEPI_QKV>, dim3(qkv_rows / LOCAL_ROW_TILE, mblocks), block, LG_LDS, stream, timer, a, qkv);
        dispatch("local_attention", local_attention, dim3(a.M / a.T, H / 4), dim3(256), 0, stream, timer, a, (const uint16_t*)b.q,
                 (const uint16_t*)b.k, (const uint16_t*)b.v, b.attended);
        LocalGemm o{L.o, b.attended, H * HEAD_DIM, a.hidden, b.partial, nullptr, nullptr, nullptr, nullptr};
        dispatch("local_o_proj", local_gemm<LEPI_PARTIAL>, dim3(a.hidden / LOCAL_ROW_TILE, mblocks, b.o_parts), block, LG_LDS, stream,
                 timer, a, o);
        dispatch("local_o_add", local_add_norm<false>, rows4, dim3(256), 0, stream, timer, a, (const float*)b.partial, b.o_parts,
                 input, b.h, L.post_norm, b.normed, (float*)nullptr);
        LocalGemm gu{L.gate_up, b.normed, a.hidden, 2 * a.inner, nullptr, b.mlp, nullptr, nullptr, nullptr};
        dispatch("local_gate_up", local_gemm<LEPI_SILU>, dim3(a.inner / 32, mblocks), block, LG_LDS, stream, timer, a, gu);
        LocalGemm down{L.down, b.mlp, a.inner, a.hidden, b.partial, nullptr, nullptr, nullptr, nullptr};
        dispatch("local_down_proj", local_gemm<LEPI_PARTIAL>, dim3(a.hidden / LOCAL_ROW_TILE, mblocks, b.down_parts), block, LG_LDS,
                 stream, timer, a, down);
        if (l + 1 < nlayers)
            dispatch("local_down_add", local_add_norm<false>, rows4, dim3(256), 0, stream, timer, a, (const float*)b.partial,
                     b.down_parts, (const float*)b.h, b.x, layers[l + 1].input_norm, b.normed, (float*)nullptr);
        else
            dispatch("local_final_norm", local_add_norm<true>, rows4, dim3(256), 0, stream, timer, a, (const float*)b.partial,
                     b.down_parts, (const float*)b.h, b.x, final_norm, (uint16_t*)nullptr, b.out);
    }
    return hipGetLastError();
}

hipError_t local_prepare() {
    for (const void* k : {(const void*)local_gemm<LEPI_QKV>, (const void*)local_gemm<LEPI_PARTIAL>, (const void*)local_gemm<LEPI_SILU>}) {
        hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LG_LDS);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_local_embed(const LocalArgs& a, const EmbedArgs& e, int rows, hipStream_t stream, DispatchTimer* timer) {
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
