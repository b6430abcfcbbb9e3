// The decode step's kernels for gfx950 (crates/graph/src/decode.rs:456-736 and its GLSL kernels),
// rewritten around the MFMA unit: every projection is a bf16 16x16x32 MFMA GEMV over the batch
// padded to 16-column tiles, so that a row of the batch is summed in the same order whatever
// the batch (decode.rs:8-11): each output's products go through one chain of MFMAs along K, the
// same k-blocks in the same order for every batch size, and the chains are added in a fixed order.
//
//   gemv_qkv_rope     RMSNorm(x) -> [q; k; v] -> RoPE -> q, and k, v into the paged cache
//                     (gemv_qkv_rope.comp:51-107)
//   attention_decode  attention over the paged cache, a workgroup to each (row, KV head), its
//                     waves taking the 64-position blocks in turn with an online softmax and
//                     joined in wave order (attention_split.comp:52-111 + attention_combine.comp:29-57)
//   gemv_residual     out = residual + W x, o_proj and down_proj (gemv_residual.comp:28-45)
//   gemv_gate_up      RMSNorm(mid) -> gate, up -> SiLU(gate) up (gemv_gate_up.comp:31-52)
//   final_rmsnorm     the final norm (rmsnorm.comp:15-21)
//
// No workgroup waits for another: every output is finished by the workgroup that sums it, so
// that a kernel ends when its slowest workgroup does.
#include "decode_kernels.hpp"
#include "dispatch.hpp"

#include <math.h>

namespace tgx {

namespace {

// Projections: a workgroup of eight waves to a strip of R rows (two strips of 16 for gate/up)
// against one 16-row tile of the batch, the tile of blockIdx.y. R is 4 or 8 at small batches,
// so that the strips of a projection fill the 256 CUs, and 16 at large ones, whose tiles fill
// them instead; the workgroups of one strip sit on one XCD (their ids differ by a multiple of
// the strips, a multiple of 8) and read its weights from there after the first.
constexpr int GEMV_WAVES = 8;
constexpr int GEMV_THREADS = GEMV_WAVES * WAVE;
// K is taken in chunks of 32 k-blocks (1024 columns); wave w's chain runs over k-blocks
// 32 c + 4 w .. 32 c + 4 w + 3 of chunk c, chunk after chunk, whatever the batch and strip.
constexpr int CHUNK_KB = 32;
constexpr int CHUNK_COLS = CHUNK_KB * 32;
constexpr int PER_WAVE = CHUNK_KB / GEMV_WAVES;
constexpr int MAX_CHUNKS = 4;  // K up to 4096; kernels are built for 1 chunk and for up to 4

// Attention: a workgroup of eight waves to each (row, KV head).
constexpr int ATTN_WAVES = 8;
constexpr int ATTN_THREADS = ATTN_WAVES * WAVE;

__device__ __forceinline__ uint4 load16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// The B operand in LDS, one chunk of the tile's 16 rows: xs[kb 64 + 16 g + c] holds row c,
// columns 32 kb + 8 g .. + 7 of the chunk. col8 numbers the groups of 8 columns (0 .. 127).
__device__ __forceinline__ int xs_index(int c, int col8) { return (col8 / 4) * 64 + (col8 % 4) * 16 + c; }

// RMSNorm(x) gain of the tile's rows into xs, chunk by chunk through `each(chunk)` (norm.glsl:
// 12-53): a wave to a row; lane l sums the squares of its 16 elements of each chunk in order,
// chunk after chunk, and the lanes are added by a butterfly; the same arithmetic for a row
// whatever the batch. The rows of the tile past B are zero.
template <typename Each>
__device__ void stage_normed(const float* __restrict__ x, const float* __restrict__ gain, float eps, int B, int K,
                             int tile, uint4* xs, float* scales, Each each) {
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int chunks = K / CHUNK_COLS;
    if (chunks > 1) {
        for (int c = w; c < 16; c += GEMV_WAVES) {
            const int b = tile * 16 + c;
            if (b >= B) continue;
            float squares = 0.f;
            for (int ch = 0; ch < chunks; ++ch) {
                const float* row = x + (size_t)b * K + ch * CHUNK_COLS + lane * 16;
#pragma unroll
                for (int e = 0; e < 16; e += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(row + e);
                    squares += v.x * v.x;
                    squares += v.y * v.y;
                    squares += v.z * v.z;
                    squares += v.w * v.w;
                }
            }
            const float total = wave_sum(squares);
            if (lane == 0) scales[c] = 1.0f / sqrtf(total / (float)K + eps);
        }
        __syncthreads();
    }
    for (int ch = 0; ch < chunks; ++ch) {
        if (ch > 0) __syncthreads();
        float4 g[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) g[e] = *reinterpret_cast<const float4*>(gain + ch * CHUNK_COLS + lane * 16 + 4 * e);
        for (int c = w; c < 16; c += GEMV_WAVES) {
            const int b = tile * 16 + c;
            uint4 packed[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
            if (b < B) {
                const float* row = x + (size_t)b * K + ch * CHUNK_COLS + lane * 16;
                float4 v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = *reinterpret_cast<const float4*>(row + 4 * e);
                float scale;
                if (chunks == 1) {
                    float squares = 0.f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        squares += v[e].x * v[e].x;
                        squares += v[e].y * v[e].y;
                        squares += v[e].z * v[e].z;
                        squares += v[e].w * v[e].w;
                    }
                    scale = 1.0f / sqrtf(wave_sum(squares) / (float)K + eps);
                } else {
                    scale = scales[c];
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float4 a = v[2 * h], e2 = v[2 * h + 1], ga = g[2 * h], gb = g[2 * h + 1];
                    packed[h].x = pack_bf16x2(a.x * scale * ga.x, a.y * scale * ga.y);
                    packed[h].y = pack_bf16x2(a.z * scale * ga.z, a.w * scale * ga.w);
                    packed[h].z = pack_bf16x2(e2.x * scale * gb.x, e2.y * scale * gb.y);
                    packed[h].w = pack_bf16x2(e2.z * scale * gb.z, e2.w * scale * gb.w);
                }
            }
            xs[xs_index(c, 2 * lane)] = packed[0];
            xs[xs_index(c, 2 * lane + 1)] = packed[1];
        }
        __syncthreads();
        each(ch);
    }
}

// Bf16 vectors [B][K] of the tile's rows into xs, chunk by chunk through `each(chunk)`. Every
// chunk's vectors are loaded first (MAXC chunks at most), so that the chunks cost one round trip
// to memory, not one each.
template <int MAXC, typename Each>
__device__ void stage_raw(const uint16_t* __restrict__ xb, int B, int K, int tile, uint4* xs, Each each) {
    constexpr int per_thread = 16 * (CHUNK_COLS / 8) / GEMV_THREADS;  // uint4 per chunk
    const int chunks = K / CHUNK_COLS;
    uint4 v[MAXC][per_thread];
#pragma unroll
    for (int ch = 0; ch < MAXC; ++ch)
#pragma unroll
        for (int j = 0; j < per_thread; ++j) {
            const int i = threadIdx.x + j * GEMV_THREADS;
            const int c = i / (CHUNK_COLS / 8), g8 = i % (CHUNK_COLS / 8);
            const int b = tile * 16 + c;
            v[ch][j] = make_uint4(0, 0, 0, 0);
            if (ch < chunks && b < B) v[ch][j] = load16(xb + (size_t)b * K + (size_t)ch * CHUNK_COLS + g8 * 8);
        }
#pragma unroll
    for (int ch = 0; ch < MAXC; ++ch) {
        if (ch >= chunks) break;
        if (ch > 0) __syncthreads();
#pragma unroll
        for (int j = 0; j < per_thread; ++j) {
            const int i = threadIdx.x + j * GEMV_THREADS;
            xs[xs_index(i / (CHUNK_COLS / 8), i % (CHUNK_COLS / 8))] = v[ch][j];
        }
        __syncthreads();
        each(ch);
    }
}

// One wave's chains for strips `strip[s]` (R rows each) of W [N][K] against the tile, over every
// chunk. The weights of all its k-blocks are loaded first, so that they are in flight while the
// vectors are staged; the products of chunk c follow its staging.
template <int S, int R, int MAXC>
struct Gemv {
    f32x4 acc[S];
    uint4 wf[MAXC][PER_WAVE][S];

    __device__ void load(const uint16_t* __restrict__ w, const int (&strip)[S], int kblocks) {
        const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
        const int chunks = kblocks / CHUNK_KB;
        const bool live = lane % 16 < R;
#pragma unroll
        for (int c = 0; c < MAXC; ++c)
#pragma unroll
            for (int j = 0; j < PER_WAVE; ++j)
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    wf[c][j][s] = make_uint4(0, 0, 0, 0);
                    if (c < chunks && live)
                        wf[c][j][s] = load16(w + weight_tile_index(strip[s], c * CHUNK_KB + wave * PER_WAVE + j, kblocks, R) +
                                             weight_lane_offset(lane, R));
                }
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // The products of chunk c, once it is staged.
    __device__ void chunk(int c, const uint4* xs) {
        const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
#pragma unroll
        for (int cc = 0; cc < MAXC; ++cc) {
            if (cc != c) continue;  // registers indexed by constants only
#pragma unroll
            for (int j = 0; j < PER_WAVE; ++j) {
                const uint4 xv = xs[(wave * PER_WAVE + j) * 64 + lane];
#pragma unroll
                for (int s = 0; s < S; ++s) acc[s] = mfma16(wf[cc][j][s], xv, acc[s]);
            }
        }
    }
};

// Every wave's chains into red, [wave][s][lane] as f32x4, behind barriers (red shares memory
// with the staged vectors).
template <int S>
__device__ void spill(const f32x4 (&acc)[S], f32x4* red) {
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < S; ++s) red[(w * S + s) * 64 + lane] = acc[s];
    __syncthreads();
}

// Row r of strip s against row c of the tile: the waves' chains added in wave order.
template <int S>
__device__ __forceinline__ float reduced(const f32x4* red, int s, int r, int c) {
    const int lane = (r / 4) * 16 + c, i = r % 4;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < GEMV_WAVES; ++w) v += red[(w * S + s) * 64 + lane][i];
    return v;
}

__device__ __forceinline__ bool placed(const DecodeArgs& a, int b, uint32_t& pos, uint32_t& slot) {
    pos = a.positions[b];
    slot = a.slots[b];
    return pos < (uint32_t)a.capacity && slot < (uint32_t)a.nslots;
}

// The cache block holding `pos` of `slot`, or -1 when the slot has none there.
__device__ __forceinline__ long block_of(const DecodeArgs& a, uint32_t slot, uint32_t pos) {
    const uint32_t blk = a.table[(size_t)slot * a.max_blocks + pos / BLOCK_TOKENS];
    return blk < (uint32_t)a.nblocks ? (long)blk : -1;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// gemv_qkv_rope: workgroup (strip, tile): a strip of R permuted rows (R/2 RoPE pairs of a head).
template <int R, int MAXC>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_qkv_rope(DecodeArgs a, LayerArgs l) {
    __shared__ uint4 xs[CHUNK_KB * 64];
    __shared__ float scales[16];
    const int K = a.hidden, kblocks = K / 32;
    const int strip_id = blockIdx.x, tile = blockIdx.y;
    const int strip[1] = {strip_id};
    Gemv<1, R, MAXC> g;
    g.load(l.qkv, strip, kblocks);
    stage_normed(l.x, l.input_norm, a.eps, a.rows, K, tile, xs, scales, [&](int ch) { g.chunk(ch, xs); });
    f32x4* red = reinterpret_cast<f32x4*>(xs);
    spill<1>(g.acc, red);

    const int per_head = HEAD_DIM / R;  // strips to a head
    const int head = strip_id / per_head;
    const int H = a.heads, KV = a.kv_heads;
    for (int idx = threadIdx.x; idx < (R / 2) * 16; idx += GEMV_THREADS) {
        const int p = idx % (R / 2), c = idx / (R / 2);
        const int b = tile * 16 + c;
        uint32_t pos, slot;
        if (b >= a.rows || !placed(a, b, pos, slot)) continue;
        const int i = (strip_id % per_head) * (R / 2) + p;  // the pair's first dimension in the head
        float va = reduced<1>(red, 0, p, c);
        float vc = reduced<1>(red, 0, p + R / 2, c);
        if (head < H + KV && a.rope) {
            // As upstream: x cos + rotate_half(x) sin (gemv_qkv_rope.comp:88-94).
            const float co = a.cos[(size_t)pos * (HEAD_DIM / 2) + i];
            const float si = a.sin[(size_t)pos * (HEAD_DIM / 2) + i];
            const float ra = va * co - vc * si;
            const float rc = vc * co + va * si;
            va = ra;
            vc = rc;
        }
        if (head < H) {
            uint16_t* q = l.q + ((size_t)b * H + head) * HEAD_DIM;
            q[i] = (uint16_t)bf16_bits(va);
            q[i + HEAD_DIM / 2] = (uint16_t)bf16_bits(vc);
            continue;
        }
        const long blk = block_of(a, slot, pos);
        if (blk < 0) continue;
        const int kv = head < H + KV ? head - H : head - H - KV;
        uint16_t* tl = l.kv + ((size_t)blk * KV + kv) * 2 * KV_TILE;
        const int pp = (int)(pos % BLOCK_TOKENS);
        if (head < H + KV) {
            tl[key_index(pp, i)] = (uint16_t)bf16_bits(va);
            tl[key_index(pp, i + HEAD_DIM / 2)] = (uint16_t)bf16_bits(vc);
        } else {
            tl[KV_TILE + value_index(pp, i)] = (uint16_t)bf16_bits(va);
            tl[KV_TILE + value_index(pp, i + HEAD_DIM / 2)] = (uint16_t)bf16_bits(vc);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// gemv_gate_up: workgroup (s, tile): strip s (16 rows) of the gate and the same strip of up.
template <int MAXC>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_gate_up(DecodeArgs a, LayerArgs l) {
    __shared__ uint4 xs[CHUNK_KB * 64];
    __shared__ float scales[16];
    const int K = a.hidden, kblocks = K / 32;
    const int s = blockIdx.x, tile = blockIdx.y;
    const int strip[2] = {s, s + a.inner / 16};
    Gemv<2, 16, MAXC> g;
    g.load(l.gate_up, strip, kblocks);
    stage_normed(l.mid, l.post_norm, a.eps, a.rows, K, tile, xs, scales, [&](int ch) { g.chunk(ch, xs); });
    f32x4* red = reinterpret_cast<f32x4*>(xs);
    spill<2>(g.acc, red);
    for (int idx = threadIdx.x; idx < 16 * 16; idx += GEMV_THREADS) {
        const int r = idx % 16, c = idx / 16;
        const int b = tile * 16 + c;
        if (b >= a.rows) continue;
        const float gate = reduced<2>(red, 0, r, c);
        const float up = reduced<2>(red, 1, r, c);
        l.mlp[(size_t)b * a.inner + s * 16 + r] = (uint16_t)bf16_bits(gate / (1.0f + __expf(-gate)) * up);
    }
}

// ---------------------------------------------------------------------------------------------
// gemv_residual: out = residual + W x; workgroup (strip, tile) over the whole of K.
template <int R, int MAXC>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_residual(DecodeArgs a, ResidualArgs r) {
    __shared__ uint4 xs[CHUNK_KB * 64];
    const int kblocks = r.K / 32;
    const int strip_id = blockIdx.x, tile = blockIdx.y;
    const int strip[1] = {strip_id};
    Gemv<1, R, MAXC> g;
    g.load(r.w, strip, kblocks);
    stage_raw<MAXC>(r.x, a.rows, r.K, tile, xs, [&](int ch) { g.chunk(ch, xs); });
    f32x4* red = reinterpret_cast<f32x4*>(xs);
    spill<1>(g.acc, red);
    for (int idx = threadIdx.x; idx < R * 16; idx += GEMV_THREADS) {
        const int row = idx % R, c = idx / R;
        const int b = tile * 16 + c;
        if (b >= a.rows) continue;
        const size_t at = (size_t)b * r.N + strip_id * R + row;
        r.out[at] = r.residual[at] + reduced<1>(red, 0, row, c);
    }
}

// ---------------------------------------------------------------------------------------------
// attention_decode: workgroup (kv, b) attends the `group` query heads KV head kv serves of row b
// over its slot's positions 0..pos; wave w takes blocks w, w + 8, ... with an online softmax, the
// next block's keys and values loaded while the current one is taken.
// Per block, S^T = K Q^T (keys as rows, heads as columns) and O^T += V^T P, P in bf16 straight
// from the registers S^T left it in.
__global__ void __launch_bounds__(ATTN_THREADS) attention_decode(DecodeArgs a, LayerArgs l) {
    extern __shared__ float attn_lds[];  // [waves][group][65] partial outputs
    __shared__ float sm_m[ATTN_WAVES][16];
    __shared__ float sm_l[ATTN_WAVES][16];
    const int kv = blockIdx.x, b = blockIdx.y;
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int H = a.heads, KV = a.kv_heads, group = H / KV;
    uint32_t pos, slot;
    if (!placed(a, b, pos, slot)) return;
    const int blocks = (int)(pos / BLOCK_TOKENS) + 1;
    const int h = lane % 16;

    uint4 qf[2];
#pragma unroll
    for (int ds = 0; ds < 2; ++ds) {
        qf[ds] = make_uint4(0, 0, 0, 0);
        if (h < group) qf[ds] = load16(l.q + ((size_t)b * H + kv * group + h) * HEAD_DIM + ds * 32 + (lane / 16) * 8);
    }
    float m = -INFINITY, total = 0.f;
    f32x4 o[4] = {};
    uint4 kf[8], vf[8], kn[8], vn[8];
    // Loads block bi's tiles into (k, v); false when the slot holds no block there.
    auto fetch = [&](int bi, uint4 (&k)[8], uint4 (&v)[8]) -> bool {
        if (bi >= blocks) return false;
        const long blk = block_of(a, slot, (uint32_t)bi * BLOCK_TOKENS);
        if (blk < 0) return false;
        const uint16_t* kt = l.kv + ((size_t)blk * KV + kv) * 2 * KV_TILE;
#pragma unroll
        for (int i = 0; i < 8; ++i) k[i] = load16(kt + (i * 64 + lane) * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = load16(kt + KV_TILE + (i * 64 + lane) * 8);
        return true;
    };
    bool have = fetch(w, kf, vf);
    for (int bi = w; have; bi += ATTN_WAVES) {
        const bool have_next = fetch(bi + ATTN_WAVES, kn, vn);
        const uint32_t p0 = (uint32_t)bi * BLOCK_TOKENS;
        f32x4 s[4];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) {
            s[pt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ds = 0; ds < 2; ++ds) s[pt] = mfma16(kf[pt * 2 + ds], qf[ds], s[pt]);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t p = p0 + pt * 16 + (lane / 16) * 4 + i;
                const float v = p <= pos ? s[pt][i] * a.scale : -INFINITY;
                s[pt][i] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
        mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
        const float m_new = fmaxf(m, mx);
        const float rescale = __expf(m - m_new);
        float sum = 0.f;
        uint4 pf[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            uint32_t words[4];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int pt = 2 * ks + half;
                // P rounded to bf16 for the product, the sum taken over the rounded values.
                words[half * 2] = pack_bf16x2(__expf(s[pt][0] - m_new), __expf(s[pt][1] - m_new));
                words[half * 2 + 1] = pack_bf16x2(__expf(s[pt][2] - m_new), __expf(s[pt][3] - m_new));
                sum += bf16_lo(words[half * 2]);
                sum += bf16_hi(words[half * 2]);
                sum += bf16_lo(words[half * 2 + 1]);
                sum += bf16_hi(words[half * 2 + 1]);
            }
            pf[ks] = make_uint4(words[0], words[1], words[2], words[3]);
        }
        sum += __shfl_xor(sum, 16, WAVE);
        sum += __shfl_xor(sum, 32, WAVE);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            o[dt] *= rescale;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) o[dt] = mfma16(vf[dt * 2 + ks], pf[ks], o[dt]);
        }
        total = total * rescale + sum;
        m = m_new;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            kf[i] = kn[i];
            vf[i] = vn[i];
        }
        have = have_next;
    }
    if (lane < 16) {
        sm_m[w][h] = m;
        sm_l[w][h] = total;
    }
    if (h < group) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) attn_lds[(w * group + h) * (HEAD_DIM + 1) + dt * 16 + (lane / 16) * 4 + i] = o[dt][i];
    }
    __syncthreads();
    // The waves joined in order (wave 0 holds block 0, so M is finite).
    const size_t head0 = (size_t)b * H + kv * group;
    for (int idx = threadIdx.x; idx < group * HEAD_DIM; idx += ATTN_THREADS) {
        const int hh = idx / HEAD_DIM, d = idx % HEAD_DIM;
        float M = -INFINITY;
        for (int j = 0; j < ATTN_WAVES; ++j) M = fmaxf(M, sm_m[j][hh]);
        float L = 0.f, O = 0.f;
        for (int j = 0; j < ATTN_WAVES; ++j) {
            const float f = sm_l[j][hh] > 0.f ? __expf(sm_m[j][hh] - M) : 0.f;
            L += sm_l[j][hh] * f;
            O += attn_lds[(j * group + hh) * (HEAD_DIM + 1) + d] * f;
        }
        l.attended[(head0 + hh) * HEAD_DIM + d] = (uint16_t)bf16_bits(O / L);
    }
}

// ---------------------------------------------------------------------------------------------
// final_rmsnorm: the final norm, a wave to a row; with `advance`, moves each placed row on by one
// position once the step is done with it.
__global__ void __launch_bounds__(WAVE) final_rmsnorm(DecodeArgs a, const float* __restrict__ x,
                                                      const float* __restrict__ gain, float* __restrict__ out,
                                                      uint32_t* positions, int advance) {
    const int b = blockIdx.x, lane = threadIdx.x;
    const int K = a.hidden, per_lane = K / WAVE;
    const float* row = x + (size_t)b * K + lane * per_lane;
    float squares = 0.f;
    for (int e = 0; e < per_lane; e += 4) {
        float4 v = *reinterpret_cast<const float4*>(row + e);
        squares += v.x * v.x;
        squares += v.y * v.y;
        squares += v.z * v.z;
        squares += v.w * v.w;
    }
    const float scale = 1.0f / sqrtf(wave_sum(squares) / (float)K + a.eps);
    for (int e = 0; e < per_lane; e += 4) {
        float4 v = *reinterpret_cast<const float4*>(row + e);
        float4 g = *reinterpret_cast<const float4*>(gain + lane * per_lane + e);
        float4 r = make_float4(v.x * scale * g.x, v.y * scale * g.y, v.z * scale * g.z, v.w * scale * g.w);
        *reinterpret_cast<float4*>(out + (size_t)b * K + lane * per_lane + e) = r;
    }
    if (advance && lane == 0) {
        const uint32_t pos = positions[b];
        if (pos < (uint32_t)a.capacity) positions[b] = pos + 1;
    }
}

// ---------------------------------------------------------------------------------------------
// Launchers.

namespace {


size_t attention_lds(const DecodeArgs& a) { return (size_t)ATTN_WAVES * (a.heads / a.kv_heads) * (HEAD_DIM + 1) * 4; }

template <int R>
hipError_t launch_layer_r(const DecodeArgs& a, const LayerArgs& l, const ResidualArgs& o,
                          const ResidualArgs& down, hipStream_t stream, DispatchTimer* timer) {
    const int tiles = decode_tiles(a.rows);
    const int qkv_strips = (a.heads + 2 * a.kv_heads) * HEAD_DIM / R;
    const bool wide = a.hidden > CHUNK_COLS;
    const dim3 block(GEMV_THREADS);
    if (wide)
        dispatch("gemv_qkv_rope", gemv_qkv_rope<R, MAX_CHUNKS>, dim3(qkv_strips, tiles), block, 0, stream, timer, a, l);
    else
        dispatch("gemv_qkv_rope", gemv_qkv_rope<R, 1>, dim3(qkv_strips, tiles), block, 0, stream, timer, a, l);
    dispatch("attention_decode", attention_decode, dim3(a.kv_heads, a.rows), dim3(ATTN_THREADS), attention_lds(a), stream, timer, a, l);
    if (o.K > CHUNK_COLS)
        dispatch("o_proj", gemv_residual<R, MAX_CHUNKS>, dim3(o.N / R, tiles), block, 0, stream, timer, a, o);
    else
        dispatch("o_proj", gemv_residual<R, 1>, dim3(o.N / R, tiles), block, 0, stream, timer, a, o);
    if (wide)
        dispatch("gemv_gate_up", gemv_gate_up<MAX_CHUNKS>, dim3(a.inner / 16, tiles), block, 0, stream, timer, a, l);
    else
        dispatch("gemv_gate_up", gemv_gate_up<1>, dim3(a.inner / 16, tiles), block, 0, stream, timer, a, l);
    if (down.K > CHUNK_COLS)
        dispatch("down_proj", gemv_residual<R, MAX_CHUNKS>, dim3(down.N / R, tiles), block, 0, stream, timer, a, down);
    else
        dispatch("down_proj", gemv_residual<R, 1>, dim3(down.N / R, tiles), block, 0, stream, timer, a, down);
    return hipGetLastError();
}

}  // namespace

int decode_tiles(int rows) { return (rows + 15) / 16; }

// Strips of 4 or 8 rows spread a small batch's projections over more CUs, but measured no faster
// than 16 on MI355X (each launch's time is set by its chain of memory round trips, not by how
// many CUs stream its weights), so every batch takes 16: one weight layout, the prefill's too.
int decode_strip_rows(int rows) {
    (void)rows;
    return 16;
}

int decode_max_k() { return MAX_CHUNKS * CHUNK_COLS; }

hipError_t decode_prepare(size_t device_lds) {
    hipFuncAttributes attr{};
    hipError_t e = hipFuncGetAttributes(&attr, (const void*)attention_decode);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute((const void*)attention_decode, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)(device_lds - attr.sharedSizeBytes));
}

size_t decode_attention_lds(int heads, int kv_heads) { return (size_t)ATTN_WAVES * (heads / kv_heads) * (HEAD_DIM + 1) * 4; }

hipError_t launch_decode_layer(const DecodeArgs& a, const LayerArgs& l, const ResidualArgs& o,
                               const ResidualArgs& down, hipStream_t stream, DispatchTimer* timer) {
    switch (decode_strip_rows(a.rows)) {
        case 4: return launch_layer_r<4>(a, l, o, down, stream, timer);
        case 8: return launch_layer_r<8>(a, l, o, down, stream, timer);
        default: return launch_layer_r<16>(a, l, o, down, stream, timer);
    }
}

hipError_t launch_final_norm(const DecodeArgs& a, const float* x, const float* gain, float* out,
                             uint32_t* positions, int advance, hipStream_t stream, DispatchTimer* timer) {
    dispatch("final_norm", final_rmsnorm, dim3(a.rows), dim3(WAVE), 0, stream, timer, a, x, gain, out, positions, advance);
    return hipGetLastError();
}

}  // namespace tgx
