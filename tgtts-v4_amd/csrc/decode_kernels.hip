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

#include <hip/hip_ext.h>
#include <math.h>

namespace tgx {

namespace {

// Projections: a workgroup of eight waves to a strip of 16 rows (two strips for gate/up).
constexpr int GEMV_WAVES = 8;
constexpr int GEMV_THREADS = GEMV_WAVES * WAVE;
// K is taken in chunks of 32 k-blocks (1024 columns); wave w's chain runs over k-blocks
// 32 c + 4 w .. 32 c + 4 w + 3 of chunk c, chunk after chunk, whatever the batch.
constexpr int CHUNK_KB = 32;
constexpr int PER_WAVE = CHUNK_KB / GEMV_WAVES;
constexpr int MAX_CHUNKS = 4;  // K up to 4096; kernels are built for 1 chunk and for up to 4

// Attention: a workgroup of eight waves to each (row, KV head).
constexpr int ATTN_WAVES = 8;
constexpr int ATTN_THREADS = ATTN_WAVES * WAVE;

__device__ __forceinline__ uint4 load16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// The B operand in LDS: xs[(t CHUNK_KB + kb) 64 + 16 g + c] holds batch row 16 t + c, columns
// 32 kb + 8 g .. + 7 of the chunk; rows past B are zero. col8 numbers the groups of 8 columns
// of the chunk (0 .. 127).
__device__ __forceinline__ int xs_index(int b, int col8) {
    return ((b / 16) * CHUNK_KB + col8 / 4) * 64 + (col8 % 4) * 16 + b % 16;
}

// The reciprocal root mean square of each of the batch's rows of x (norm.glsl:12-29), into
// scales[b]: a wave to a row, lane l summing elements [l K/64, (l+1) K/64) in order, the lanes
// added by a butterfly; the same arithmetic for a row whatever the batch.
__device__ void row_scales(const float* __restrict__ x, float eps, int B, int K, float* scales) {
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int per_lane = K / WAVE;
    for (int b = w; b < B; b += GEMV_WAVES) {
        const float* row = x + (size_t)b * K + lane * per_lane;
        float squares = 0.f;
        for (int e = 0; e < per_lane; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(row + e);
            squares += v.x * v.x;
            squares += v.y * v.y;
            squares += v.z * v.z;
            squares += v.w * v.w;
        }
        const float total = wave_sum(squares);
        if (lane == 0) scales[b] = 1.0f / sqrtf(total / (float)K + eps);
    }
}

// Chunk c of RMSNorm(x) gain, rows [0, NT 16), into xs (bf16).
template <int NT>
__device__ void stage_normed(const float* __restrict__ x, const float* __restrict__ gain, const float* scales,
                             int B, int K, int c, uint4* xs) {
    constexpr int groups = CHUNK_KB * 4;  // groups of 8 columns in a chunk
    for (int i = threadIdx.x; i < NT * 16 * groups; i += GEMV_THREADS) {
        const int b = i / groups, g8 = i % groups;
        uint4 packed = make_uint4(0, 0, 0, 0);
        if (b < B) {
            const int k0 = c * CHUNK_KB * 32 + g8 * 8;
            const float scale = scales[b];
            const float4 a = *reinterpret_cast<const float4*>(x + (size_t)b * K + k0);
            const float4 e = *reinterpret_cast<const float4*>(x + (size_t)b * K + k0 + 4);
            const float4 ga = *reinterpret_cast<const float4*>(gain + k0);
            const float4 gb = *reinterpret_cast<const float4*>(gain + k0 + 4);
            packed.x = pack_bf16x2(a.x * scale * ga.x, a.y * scale * ga.y);
            packed.y = pack_bf16x2(a.z * scale * ga.z, a.w * scale * ga.w);
            packed.z = pack_bf16x2(e.x * scale * gb.x, e.y * scale * gb.y);
            packed.w = pack_bf16x2(e.z * scale * gb.z, e.w * scale * gb.w);
        }
        xs[xs_index(b, g8)] = packed;
    }
}

// Chunk c of bf16 vectors [B][K], rows [0, NT 16), into xs.
template <int NT>
__device__ void stage_raw(const uint16_t* __restrict__ xb, int B, int K, int c, uint4* xs) {
    constexpr int groups = CHUNK_KB * 4;
    for (int i = threadIdx.x; i < NT * 16 * groups; i += GEMV_THREADS) {
        const int b = i / groups, g8 = i % groups;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (b < B) v = load16(xb + (size_t)b * K + (size_t)c * CHUNK_KB * 32 + g8 * 8);
        xs[xs_index(b, g8)] = v;
    }
}

// One wave's chains for strips `strip[s]` of W [N][K] against the batch, over every chunk.
// The weights of all its k-blocks are loaded first, so that they are in flight while the
// vectors are staged; the products of chunk c follow its staging.
template <int S, int NT, int MAXC>
struct Gemv {
    f32x4 acc[S][NT];
    uint4 wf[MAXC][PER_WAVE][S];
    int chunks;

    __device__ void load(const uint16_t* __restrict__ w, const int (&strip)[S], int kblocks) {
        const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
        chunks = kblocks / CHUNK_KB;
#pragma unroll
        for (int c = 0; c < MAXC; ++c)
#pragma unroll
            for (int j = 0; j < PER_WAVE; ++j)
#pragma unroll
                for (int s = 0; s < S; ++s)
                    if (c < chunks)
                        wf[c][j][s] = load16(w + weight_tile_index(strip[s], c * CHUNK_KB + wave * PER_WAVE + j, kblocks) + lane * 8);
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // The products of chunk c, once it is staged.
    __device__ void chunk(int c, const uint4* xs) {
        const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
#pragma unroll
        for (int cc = 0; cc < MAXC; ++cc) {
            if (cc != c) continue;  // registers indexed by constants only
#pragma unroll
            for (int j = 0; j < PER_WAVE; ++j) {
                const int kb = wave * PER_WAVE + j;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const uint4 xv = xs[(t * CHUNK_KB + kb) * 64 + lane];
#pragma unroll
                    for (int s = 0; s < S; ++s) acc[s][t] = mfma16(wf[cc][j][s], xv, acc[s][t]);
                }
            }
        }
    }
};

// Every wave's chains into red, [wave][s][t][lane] as f32x4, behind barriers (red shares memory
// with the staged vectors).
template <int S, int NT>
__device__ void spill(const f32x4 (&acc)[S][NT], f32x4* red) {
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int t = 0; t < NT; ++t) red[((w * S + s) * NT + t) * 64 + lane] = acc[s][t];
    __syncthreads();
}

// Row r of strip s against batch row b: the waves' chains added in wave order.
template <int S, int NT>
__device__ __forceinline__ float reduced(const f32x4* red, int s, int r, int b) {
    const int t = b / 16, lane = (r / 4) * 16 + b % 16, i = r % 4;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < GEMV_WAVES; ++w) v += red[((w * S + s) * NT + t) * 64 + lane][i];
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
// gemv_qkv_rope: a workgroup per strip of 16 permuted rows (8 RoPE pairs of one head).
template <int NT, int MAXC>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_qkv_rope(DecodeArgs a, LayerArgs l) {
    extern __shared__ uint4 smem[];
    __shared__ float scales[64];
    const int K = a.hidden, kblocks = K / 32;
    const int strip_id = blockIdx.x;
    const int strip[1] = {strip_id};
    Gemv<1, NT, MAXC> g;
    g.load(l.qkv, strip, kblocks);
    row_scales(l.x, a.eps, a.rows, K, scales);
    for (int c = 0; c < g.chunks; ++c) {
        __syncthreads();
        stage_normed<NT>(l.x, l.input_norm, scales, a.rows, K, c, smem);
        __syncthreads();
        g.chunk(c, smem);
    }
    f32x4* red = reinterpret_cast<f32x4*>(smem);
    spill<1, NT>(g.acc, red);

    const int quarters = HEAD_DIM / 16;
    const int head = strip_id / quarters;
    const int H = a.heads, KV = a.kv_heads;
    for (int idx = threadIdx.x; idx < 8 * a.rows; idx += GEMV_THREADS) {
        const int p = idx % 8, b = idx / 8;
        uint32_t pos, slot;
        if (!placed(a, b, pos, slot)) continue;
        const int i = (strip_id % quarters) * 8 + p;  // the pair's first dimension in the head
        float va = reduced<1, NT>(red, 0, p, b);
        float vc = reduced<1, NT>(red, 0, p + 8, b);
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
        uint16_t* tile = l.kv + ((size_t)blk * KV + kv) * 2 * KV_TILE;
        const int pp = (int)(pos % BLOCK_TOKENS);
        if (head < H + KV) {
            tile[key_index(pp, i)] = (uint16_t)bf16_bits(va);
            tile[key_index(pp, i + HEAD_DIM / 2)] = (uint16_t)bf16_bits(vc);
        } else {
            tile[KV_TILE + value_index(pp, i)] = (uint16_t)bf16_bits(va);
            tile[KV_TILE + value_index(pp, i + HEAD_DIM / 2)] = (uint16_t)bf16_bits(vc);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// gemv_gate_up: a workgroup per strip s of the gate and the same strip of up.
template <int NT, int MAXC>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_gate_up(DecodeArgs a, LayerArgs l) {
    extern __shared__ uint4 smem[];
    __shared__ float scales[64];
    const int K = a.hidden, kblocks = K / 32;
    const int s = blockIdx.x;
    const int strip[2] = {s, s + a.inner / 16};
    Gemv<2, NT, MAXC> g;
    g.load(l.gate_up, strip, kblocks);
    row_scales(l.mid, a.eps, a.rows, K, scales);
    for (int c = 0; c < g.chunks; ++c) {
        __syncthreads();
        stage_normed<NT>(l.mid, l.post_norm, scales, a.rows, K, c, smem);
        __syncthreads();
        g.chunk(c, smem);
    }
    f32x4* red = reinterpret_cast<f32x4*>(smem);
    spill<2, NT>(g.acc, red);
    for (int idx = threadIdx.x; idx < 16 * a.rows; idx += GEMV_THREADS) {
        const int r = idx % 16, b = idx / 16;
        const float gate = reduced<2, NT>(red, 0, r, b);
        const float up = reduced<2, NT>(red, 1, r, b);
        l.mlp[(size_t)b * a.inner + s * 16 + r] = (uint16_t)bf16_bits(gate / (1.0f + __expf(-gate)) * up);
    }
}

// ---------------------------------------------------------------------------------------------
// gemv_residual: out = residual + W x, a workgroup per strip of 16 rows over the whole of K.
template <int NT, int MAXC>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_residual(DecodeArgs a, ResidualArgs r) {
    extern __shared__ uint4 smem[];
    const int kblocks = r.K / 32;
    const int strip_id = blockIdx.x;
    const int strip[1] = {strip_id};
    Gemv<1, NT, MAXC> g;
    g.load(r.w, strip, kblocks);
    for (int c = 0; c < g.chunks; ++c) {
        __syncthreads();
        stage_raw<NT>(r.x, a.rows, r.K, c, smem);
        __syncthreads();
        g.chunk(c, smem);
    }
    f32x4* red = reinterpret_cast<f32x4*>(smem);
    spill<1, NT>(g.acc, red);
    for (int idx = threadIdx.x; idx < 16 * a.rows; idx += GEMV_THREADS) {
        const int row = idx % 16, b = idx / 16;
        const size_t at = (size_t)b * r.N + strip_id * 16 + row;
        r.out[at] = r.residual[at] + reduced<1, NT>(red, 0, row, b);
    }
}

// ---------------------------------------------------------------------------------------------
// attention_decode: workgroup (kv, b) attends the `group` query heads KV head kv serves of row b
// over its slot's positions 0..pos; wave w takes blocks w, w + 8, ... with an online softmax.
// Per block, S^T = K Q^T (keys as rows, heads as columns) and O^T += V^T P, P in bf16 straight
// from the registers S^T left it in.
__global__ void __launch_bounds__(ATTN_THREADS) attention_decode(DecodeArgs a, LayerArgs l) {
    __shared__ float sm_m[ATTN_WAVES][16];
    __shared__ float sm_l[ATTN_WAVES][16];
    __shared__ float sm_o[ATTN_WAVES][16][HEAD_DIM + 1];
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
    for (int bi = w; bi < blocks; bi += ATTN_WAVES) {
        const long blk = block_of(a, slot, (uint32_t)bi * BLOCK_TOKENS);
        if (blk < 0) break;
        const uint16_t* kt = l.kv + ((size_t)blk * KV + kv) * 2 * KV_TILE;
        uint4 kf[8], vf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) kf[i] = load16(kt + (i * 64 + lane) * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) vf[i] = load16(kt + KV_TILE + (i * 64 + lane) * 8);
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
                float e[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    e[i] = __uint_as_float(bf16_bits(__expf(s[pt][i] - m_new)) << 16);
                    sum += e[i];
                }
                words[half * 2] = pack_bf16x2(e[0], e[1]);
                words[half * 2 + 1] = pack_bf16x2(e[2], e[3]);
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
    }
    if (lane < 16) {
        sm_m[w][h] = m;
        sm_l[w][h] = total;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm_o[w][h][dt * 16 + (lane / 16) * 4 + i] = o[dt][i];
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
            O += sm_o[j][hh][d] * f;
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

// LDS of a projection: one chunk of the batch's vectors, or the waves' chains, the larger.
template <int NT>
size_t stage_bytes(int strips) {
    const size_t xs = (size_t)NT * 16 * CHUNK_KB * 32 * 2;
    const size_t red = (size_t)GEMV_WAVES * strips * NT * 64 * sizeof(f32x4);
    return xs > red ? xs : red;
}

// Launches `kernel`, timed by the next pair of the timer's events when there is a timer.
template <typename... KernelArgs, typename... Args>
void dispatch(const char* label, void (*kernel)(KernelArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t stream,
              DispatchTimer* timer, Args... args) {
    if (timer && timer->used < timer->capacity) {
        const int i = timer->used++;
        timer->labels[i] = label;
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, timer->start[i], timer->stop[i], 0, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
}

template <int NT>
hipError_t launch_layer_nt(const DecodeArgs& a, const LayerArgs& l, const ResidualArgs& o,
                           const ResidualArgs& down, hipStream_t stream, DispatchTimer* timer) {
    const int qkv_strips = (a.heads + 2 * a.kv_heads) * HEAD_DIM / 16;
    const bool wide = a.hidden > CHUNK_KB * 32;
    if (wide)
        dispatch("gemv_qkv_rope", gemv_qkv_rope<NT, MAX_CHUNKS>, dim3(qkv_strips), dim3(GEMV_THREADS), stage_bytes<NT>(1), stream, timer, a, l);
    else
        dispatch("gemv_qkv_rope", gemv_qkv_rope<NT, 1>, dim3(qkv_strips), dim3(GEMV_THREADS), stage_bytes<NT>(1), stream, timer, a, l);
    dispatch("attention_decode", attention_decode, dim3(a.kv_heads, a.rows), dim3(ATTN_THREADS), 0, stream, timer, a, l);
    if (o.K > CHUNK_KB * 32)
        dispatch("o_proj", gemv_residual<NT, MAX_CHUNKS>, dim3(o.N / 16), dim3(GEMV_THREADS), stage_bytes<NT>(1), stream, timer, a, o);
    else
        dispatch("o_proj", gemv_residual<NT, 1>, dim3(o.N / 16), dim3(GEMV_THREADS), stage_bytes<NT>(1), stream, timer, a, o);
    if (wide)
        dispatch("gemv_gate_up", gemv_gate_up<NT, MAX_CHUNKS>, dim3(a.inner / 16), dim3(GEMV_THREADS), stage_bytes<NT>(2), stream, timer, a, l);
    else
        dispatch("gemv_gate_up", gemv_gate_up<NT, 1>, dim3(a.inner / 16), dim3(GEMV_THREADS), stage_bytes<NT>(2), stream, timer, a, l);
    if (down.K > CHUNK_KB * 32)
        dispatch("down_proj", gemv_residual<NT, MAX_CHUNKS>, dim3(down.N / 16), dim3(GEMV_THREADS), stage_bytes<NT>(1), stream, timer, a, down);
    else
        dispatch("down_proj", gemv_residual<NT, 1>, dim3(down.N / 16), dim3(GEMV_THREADS), stage_bytes<NT>(1), stream, timer, a, down);
    return hipGetLastError();
}

// Lets `kernel` take dynamic LDS up to what the device allows a workgroup beside its static LDS.
hipError_t allow_lds_for(const void* kernel, size_t device_most) {
    hipFuncAttributes attr{};
    hipError_t e = hipFuncGetAttributes(&attr, kernel);
    if (e != hipSuccess) return e;
    const int most = (int)(device_most - attr.sharedSizeBytes);
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, most);
}

template <int NT>
hipError_t allow_lds(size_t device_most) {
    const void* kernels[] = {
        (const void*)gemv_qkv_rope<NT, 1>, (const void*)gemv_qkv_rope<NT, MAX_CHUNKS>,
        (const void*)gemv_gate_up<NT, 1>,  (const void*)gemv_gate_up<NT, MAX_CHUNKS>,
        (const void*)gemv_residual<NT, 1>, (const void*)gemv_residual<NT, MAX_CHUNKS>,
    };
    for (const void* k : kernels) {
        hipError_t e = allow_lds_for(k, device_most);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
}  // namespace

int decode_tiles(int rows) { return (rows + 15) / 16; }

size_t decode_lds_bytes(int rows) {
    switch (decode_tiles(rows)) {
        case 1: return stage_bytes<1>(2);
        case 2: return stage_bytes<2>(2);
        case 3: return stage_bytes<3>(2);
        default: return stage_bytes<4>(2);
    }
}

int decode_max_k() { return MAX_CHUNKS * CHUNK_KB * 32; }

hipError_t decode_prepare(size_t device_lds) {
    hipError_t e;
    if ((e = allow_lds<1>(device_lds)) != hipSuccess) return e;
    if ((e = allow_lds<2>(device_lds)) != hipSuccess) return e;
    if ((e = allow_lds<3>(device_lds)) != hipSuccess) return e;
    return allow_lds<4>(device_lds);
}

hipError_t launch_decode_layer(const DecodeArgs& a, const LayerArgs& l, const ResidualArgs& o,
                               const ResidualArgs& down, hipStream_t stream, DispatchTimer* timer) {
    switch (decode_tiles(a.rows)) {
        case 1: return launch_layer_nt<1>(a, l, o, down, stream, timer);
        case 2: return launch_layer_nt<2>(a, l, o, down, stream, timer);
        case 3: return launch_layer_nt<3>(a, l, o, down, stream, timer);
        case 4: return launch_layer_nt<4>(a, l, o, down, stream, timer);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_final_norm(const DecodeArgs& a, const float* x, const float* gain, float* out,
                             uint32_t* positions, int advance, hipStream_t stream, DispatchTimer* timer) {
    dispatch("final_norm", final_rmsnorm, dim3(a.rows), dim3(WAVE), 0, stream, timer, a, x, gain, out, positions, advance);
    return hipGetLastError();
}

}  // namespace tgx
