// The prefill's kernels for gfx950 (crates/graph/src/prefill.rs:218-413 with norm_rows.comp,
// add_norm_rows.comp, rope_rows.comp, attention_rows.comp, silu_mul_rows.comp and the MLIR GEMM
// kernels/gpu/gemm.mlir), rewritten for the MFMA unit:
//
//   prefill_norm       RMSNorm of each row of the f32 stream into bf16 (norm_rows.comp, and the
//                      norm half of add_norm_rows.comp; the residual add is the GEMM's epilogue)
//   prefill_gemm       C = X W^T, bf16 in, f32 accumulate, a 256 x 128 tile to a workgroup of
//                      four waves staged through LDS twice buffered, with the epilogue fused:
//                      RoPE and the cache write (rope_rows.comp), the residual add
//                      (add_norm_rows.comp), or SiLU(gate) up (silu_mul_rows.comp)
//   prefill_attention  causal attention over the paged cache, 32 positions of a run to a
//                      workgroup, keys and values staged through LDS a 64-position block at a time
//                      with an online softmax (attention_rows.comp)
#include "prefill_kernels.hpp"

#include <hip/hip_ext.h>
#include <math.h>

namespace tgx {

namespace {

constexpr int PF_WAVES = 4;
constexpr int PF_THREADS = PF_WAVES * WAVE;
// The GEMM's workgroup tile: 256 rows of W (16 strips) by 128 rows of X, K 64 at a time (two
// k-blocks); wave (wn, wm) takes W rows 128 wn .. + 127 (8 strips) by X rows 64 wm .. + 63.
constexpr int TN = 256, TM = 128, TKB = 2;
constexpr int W_STRIPS = TN / 16;   // 16
constexpr int X_TILES = TM / 16;    // 8
constexpr int W_STAGE = W_STRIPS * TKB * 64;  // uint4 per stage: 32 KiB
constexpr int X_STAGE = X_TILES * TKB * 64;   // 16 KiB

enum Epilogue { EPI_QKV = 0, EPI_RESIDUAL = 1, EPI_SILU = 2 };

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

struct GemmArgs {
    const uint16_t* w;  // 16-row tiles of [N][K]
    const uint16_t* x;  // bf16 [M_pad][K]
    int K, N;
    // epilogues
    const float* residual;  // EPI_RESIDUAL: f32 [M_pad][N]
    float* out;             // EPI_RESIDUAL: f32 [M_pad][N]
    uint16_t* mlp;          // EPI_SILU: bf16 [M_pad][N / 2]
    uint16_t* q;            // EPI_QKV
    uint16_t* kv;           // EPI_QKV: the layer's cache pool
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

template <int EPI>
__global__ void __launch_bounds__(PF_THREADS) prefill_gemm(PrefillArgs a, GemmArgs g) {
    extern __shared__ uint4 lds[];
    uint4* ws = lds;                  // [2][W_STAGE]
    uint4* xs = lds + 2 * W_STAGE;    // [2][X_STAGE]
    const int nb = blockIdx.x, mb = blockIdx.y;
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int wn = w / 2, wm = w % 2;
    const int kblocks = g.K / 32;
    const int stages = kblocks / TKB;
    const int m0 = mb * TM;

    uint4 wreg[W_STAGE / PF_THREADS], xreg[X_STAGE / PF_THREADS];
    auto fetch = [&](int st) {
#pragma unroll
        for (int j = 0; j < W_STAGE / PF_THREADS; ++j) {
            const int i = threadIdx.x + j * PF_THREADS;
            const int sl = i / (TKB * 64), kbl = (i / 64) % TKB, ln = i % 64;
            wreg[j] = load16(g.w + weight_tile_index(stage_strip<EPI>(nb, sl, g.N), st * TKB + kbl, kblocks, 16) + ln * 8);
        }
#pragma unroll
        for (int j = 0; j < X_STAGE / PF_THREADS; ++j) {
            const int i = threadIdx.x + j * PF_THREADS;
            const int m = i / (TKB * 4), c8 = i % (TKB * 4);
            xreg[j] = load16(g.x + (size_t)(m0 + m) * g.K + st * TKB * 32 + c8 * 8);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < W_STAGE / PF_THREADS; ++j) ws[buf * W_STAGE + threadIdx.x + j * PF_THREADS] = wreg[j];
#pragma unroll
        for (int j = 0; j < X_STAGE / PF_THREADS; ++j) {
            const int i = threadIdx.x + j * PF_THREADS;
            const int m = i / (TKB * 4), c8 = i % (TKB * 4);
            const int mt = m / 16, kbl = c8 / 4, gq = c8 % 4;
            xs[buf * X_STAGE + (mt * TKB + kbl) * 64 + gq * 16 + m % 16] = xreg[j];
        }
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    fetch(0);
    store(0);
    __syncthreads();
    for (int st = 0; st < stages; ++st) {
        const int buf = st % 2;
        if (st + 1 < stages) fetch(st + 1);
#pragma unroll
        for (int kbl = 0; kbl < TKB; ++kbl) {
            uint4 af[8], bf[4];
#pragma unroll
            for (int s = 0; s < 8; ++s) af[s] = ws[buf * W_STAGE + ((wn * 8 + s) * TKB + kbl) * 64 + lane];
#pragma unroll
            for (int t = 0; t < 4; ++t) bf[t] = xs[buf * X_STAGE + ((wm * 4 + t) * TKB + kbl) * 64 + lane];
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int t = 0; t < 4; ++t) acc[s][t] = mfma16(af[s], bf[t], acc[s][t]);
        }
        if (st + 1 < stages) store(1 - buf);
        __syncthreads();
    }

    // Epilogue: tile (s, t) holds W rows 16 strip + 4 (lane / 16) + i against X row
    // m0 + 64 wm + 16 t + lane % 16.
    const int quad = lane / 16;
    if (EPI == EPI_RESIDUAL) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int n = strip_of<EPI>(nb, wn, s, g.N) * 16 + quad * 4;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int m = m0 + wm * 64 + t * 16 + lane % 16;
                if (m >= a.M) continue;
                const float4 r = *reinterpret_cast<const float4*>(g.residual + (size_t)m * g.N + n);
                float4 o;
                o.x = r.x + acc[s][t][0];
                o.y = r.y + acc[s][t][1];
                o.z = r.z + acc[s][t][2];
                o.w = r.w + acc[s][t][3];
                *reinterpret_cast<float4*>(g.out + (size_t)m * g.N + n) = o;
            }
        }
    } else if (EPI == EPI_SILU) {
        const int inner = g.N / 2;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int n = strip_of<EPI>(nb, wn, s, g.N) * 16 + quad * 4;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int m = m0 + wm * 64 + t * 16 + lane % 16;
                if (m >= a.M) continue;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float gate = acc[s][t][i], up = acc[s + 4][t][i];
                    v[i] = gate / (1.0f + __expf(-gate)) * up;
                }
                uint2 packed = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                *reinterpret_cast<uint2*>(g.mlp + (size_t)m * inner + n) = packed;
            }
        }
    } else {  // EPI_QKV: rows of a strip pair as r, r + 8 (lanes l and l ^ 32)
        const int H = a.heads, KV = a.kv_heads;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int strip = strip_of<EPI>(nb, wn, s, g.N);
            const int head = strip / 4, qtr = strip % 4;
            const bool second = quad >= 2;  // rows 8..15: the pairs' second halves
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int m = m0 + wm * 64 + t * 16 + lane % 16;
                float own[4], other[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    own[i] = acc[s][t][i];
                    other[i] = __shfl_xor(own[i], 32, WAVE);
                }
                if (m >= a.M) continue;
                const uint32_t pos = a.tok_pos[m];
                const uint32_t slot = a.tok_slot[m];
                if (pos >= (uint32_t)a.capacity || slot >= (uint32_t)a.nslots) continue;
                const int p0 = qtr * 8 + (quad % 2) * 4;  // the first of this lane's 4 pairs
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] = own[i];
                    if (head < H + KV && a.rope) {
                        const float co = a.cos[(size_t)pos * (HEAD_DIM / 2) + p0 + i];
                        const float si = a.sin[(size_t)pos * (HEAD_DIM / 2) + p0 + i];
                        // As upstream: x cos + rotate_half(x) sin (rope_rows.comp:52-59).
                        v[i] = second ? own[i] * co + other[i] * si : own[i] * co - other[i] * si;
                    }
                }
                const int d0 = p0 + (second ? HEAD_DIM / 2 : 0);
                if (head < H) {
                    uint2 packed = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
                    *reinterpret_cast<uint2*>(g.q + ((size_t)m * H + head) * HEAD_DIM + d0) = packed;
                    continue;
                }
                const uint32_t blk = a.table[(size_t)slot * a.max_blocks + pos / BLOCK_TOKENS];
                if (blk >= (uint32_t)a.nblocks) continue;
                const int kv = head < H + KV ? head - H : head - H - KV;
                uint16_t* tl = g.kv + ((size_t)blk * KV + kv) * 2 * KV_TILE;
                const int pp = (int)(pos % BLOCK_TOKENS);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint16_t bits = (uint16_t)bf16_bits(v[i]);
                    if (head < H + KV)
                        tl[key_index(pp, d0 + i)] = bits;
                    else
                        tl[KV_TILE + value_index(pp, d0 + i)] = bits;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// prefill_norm: a wave to a row: lane l sums the squares of its K/64 elements in order, the lanes
// added by a butterfly (norm.glsl:12-29); rows past M are written zero.
template <bool FINAL>
__global__ void __launch_bounds__(256) prefill_norm(PrefillArgs a, const float* __restrict__ x, const float* __restrict__ gain,
                                                    uint16_t* __restrict__ out_bf16, float* __restrict__ out_f32) {
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (row >= a.M_pad) return;
    const int K = a.hidden, per_lane = K / WAVE;
    if (row >= a.M) {
        if (!FINAL)
            for (int e = 0; e < per_lane; e += 8)
                *reinterpret_cast<uint4*>(out_bf16 + (size_t)row * K + lane * per_lane + e) = make_uint4(0, 0, 0, 0);
        return;
    }
    const float* r = x + (size_t)row * K + lane * per_lane;
    float squares = 0.f;
    for (int e = 0; e < per_lane; e += 4) {
        const float4 v = *reinterpret_cast<const float4*>(r + e);
        squares += v.x * v.x;
        squares += v.y * v.y;
        squares += v.z * v.z;
        squares += v.w * v.w;
    }
    const float scale = 1.0f / sqrtf(wave_sum(squares) / (float)K + a.eps);
    for (int e = 0; e < per_lane; e += 8) {
        const float4 v0 = *reinterpret_cast<const float4*>(r + e);
        const float4 v1 = *reinterpret_cast<const float4*>(r + e + 4);
        const float4 g0 = *reinterpret_cast<const float4*>(gain + lane * per_lane + e);
        const float4 g1 = *reinterpret_cast<const float4*>(gain + lane * per_lane + e + 4);
        const float n[8] = {v0.x * scale * g0.x, v0.y * scale * g0.y, v0.z * scale * g0.z, v0.w * scale * g0.w,
                            v1.x * scale * g1.x, v1.y * scale * g1.y, v1.z * scale * g1.z, v1.w * scale * g1.w};
        if (FINAL) {
            *reinterpret_cast<float4*>(out_f32 + (size_t)row * K + lane * per_lane + e) = make_float4(n[0], n[1], n[2], n[3]);
            *reinterpret_cast<float4*>(out_f32 + (size_t)row * K + lane * per_lane + e + 4) = make_float4(n[4], n[5], n[6], n[7]);
        } else {
            *reinterpret_cast<uint4*>(out_bf16 + (size_t)row * K + lane * per_lane + e) =
                make_uint4(pack_bf16x2(n[0], n[1]), pack_bf16x2(n[2], n[3]), pack_bf16x2(n[4], n[5]), pack_bf16x2(n[6], n[7]));
        }
    }
}

// ---------------------------------------------------------------------------------------------
// prefill_attention: workgroup (tile, kv): the tile's positions (up to 32, eight to a wave) for
// the `group` query heads KV head kv serves. Columns of the MFMA are (position, head) pairs,
// 16 / group positions to a column group, CG = group / 2 column groups to a wave. The slot's
// blocks from 0 to the tile's last position are staged through LDS in turn; each column keeps
// its running maximum, sum and output (attention_rows.comp:71-116).
template <int CG>
__global__ void __launch_bounds__(PF_THREADS) prefill_attention(PrefillArgs a, const uint16_t* __restrict__ q,
                                                                const uint16_t* __restrict__ kvpool,
                                                                uint16_t* __restrict__ attended,
                                                                const PrefillTile* __restrict__ tiles) {
    __shared__ uint4 stage[2][2 * KV_TILE / 8];  // two blocks of keys then values
    constexpr int group = 2 * CG;
    constexpr int per_col = 16 / group;  // positions to a column group
    const PrefillTile tile = tiles[blockIdx.x];
    const int kv = blockIdx.y;
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int H = a.heads, KV = a.kv_heads;
    const int col = lane % 16;
    const uint32_t last = tile.pos0 + tile.count - 1;
    const int blocks = (int)(last / BLOCK_TOKENS) + 1;

    uint4 qf[CG][2];
    uint32_t cpos[CG];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        const int tok = w * 8 + cg * per_col + col / group;  // within the tile
        const int head = kv * group + col % group;
        const size_t row = tile.row0 + (tok < (int)tile.count ? tok : 0);
        cpos[cg] = tile.pos0 + tok;
#pragma unroll
        for (int ds = 0; ds < 2; ++ds) qf[cg][ds] = load16(q + (row * H + head) * HEAD_DIM + ds * 32 + (lane / 16) * 8);
    }
    float m[CG], l[CG];
    f32x4 o[CG][4];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        m[cg] = -INFINITY;
        l[cg] = 0.f;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[cg][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    auto fetch = [&](int bi, uint4 (&r)[4]) {
        const uint32_t blk = a.table[(size_t)tile.slot * a.max_blocks + bi];
        const uint16_t* src = kvpool + ((size_t)(blk < (uint32_t)a.nblocks ? blk : 0) * KV + kv) * 2 * KV_TILE;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = load16(src + (size_t)(threadIdx.x + j * PF_THREADS) * 8);
    };
    uint4 reg[4];
    fetch(0, reg);
#pragma unroll
    for (int j = 0; j < 4; ++j) stage[0][threadIdx.x + j * PF_THREADS] = reg[j];
    __syncthreads();
    for (int bi = 0; bi < blocks; ++bi) {
        const int buf = bi % 2;
        if (bi + 1 < blocks) fetch(bi + 1, reg);
        uint4 kf[8], vf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) kf[i] = stage[buf][i * 64 + lane];
#pragma unroll
        for (int i = 0; i < 8; ++i) vf[i] = stage[buf][KV_TILE / 8 + i * 64 + lane];
        const uint32_t p0 = (uint32_t)bi * BLOCK_TOKENS;
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
            f32x4 s[4];
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                s[pt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ds = 0; ds < 2; ++ds) s[pt] = mfma16(kf[pt * 2 + ds], qf[cg][ds], s[pt]);
            }
            float mx = -INFINITY;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t p = p0 + pt * 16 + (lane / 16) * 4 + i;
                    const float v = p <= cpos[cg] ? s[pt][i] * a.scale : -INFINITY;
                    s[pt][i] = v;
                    mx = fmaxf(mx, v);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
            mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
            // Block 0 holds position 0, which every column sees, so m is finite after it.
            const float m_new = fmaxf(m[cg], mx);
            const float rescale = __expf(m[cg] - m_new);
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
                o[cg][dt] *= rescale;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) o[cg][dt] = mfma16(vf[dt * 2 + ks], pf[ks], o[cg][dt]);
            }
            l[cg] = l[cg] * rescale + sum;
            m[cg] = m_new;
        }
        if (bi + 1 < blocks) {
#pragma unroll
            for (int j = 0; j < 4; ++j) stage[1 - buf][threadIdx.x + j * PF_THREADS] = reg[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        const int tok = w * 8 + cg * per_col + col / group;
        if (tok >= (int)tile.count) continue;
        const int head = kv * group + col % group;
        const size_t row = tile.row0 + tok;
        const float inv = 1.0f / l[cg];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d = dt * 16 + (lane / 16) * 4;
            uint2 packed = make_uint2(pack_bf16x2(o[cg][dt][0] * inv, o[cg][dt][1] * inv),
                                      pack_bf16x2(o[cg][dt][2] * inv, o[cg][dt][3] * inv));
            *reinterpret_cast<uint2*>(attended + (row * H + head) * HEAD_DIM + d) = packed;
        }
    }
}

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

constexpr size_t GEMM_LDS = (size_t)2 * (W_STAGE + X_STAGE) * sizeof(uint4);

hipError_t allow(const void* kernel, size_t device_lds) {
    hipFuncAttributes attr{};
    hipError_t e = hipFuncGetAttributes(&attr, kernel);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(device_lds - attr.sharedSizeBytes));
}

}  // namespace

hipError_t prefill_prepare(size_t device_lds) {
    hipError_t e;
    if ((e = allow((const void*)prefill_gemm<EPI_QKV>, device_lds)) != hipSuccess) return e;
    if ((e = allow((const void*)prefill_gemm<EPI_RESIDUAL>, device_lds)) != hipSuccess) return e;
    return allow((const void*)prefill_gemm<EPI_SILU>, device_lds);
}

hipError_t launch_prefill(const PrefillArgs& a, const PrefillLayer* layers, int nlayers, const float* final_norm,
                          const PrefillBuffers& b, hipStream_t stream, DispatchTimer* timer) {
    const int mblocks = a.M_pad / TM;
    const dim3 rows4((a.M_pad + 3) / 4);
    const int group = a.heads / a.kv_heads;
    const int qkv_rows = (a.heads + 2 * a.kv_heads) * HEAD_DIM;
    // Layer 0's input norm; each later norm follows the down projection that feeds it.
    if (nlayers > 0)
        dispatch("prefill_norm", prefill_norm<false>, rows4, dim3(256), 0, stream, timer, a, b.x,
                 layers[0].input_norm, b.normed, (float*)nullptr);
    const float* input = b.x;  // layer 0 reads the run's states, which stay as written
    for (int l = 0; l < nlayers; ++l) {
        const PrefillLayer& L = layers[l];
        GemmArgs qkv{L.qkv, b.normed, a.hidden, qkv_rows, nullptr, nullptr, nullptr, b.q, L.kv};
        dispatch("prefill_qkv", prefill_gemm<EPI_QKV>, dim3(qkv_rows / TN, mblocks), dim3(PF_THREADS), GEMM_LDS, stream, timer, a, qkv);
        switch (group) {
            case 2: dispatch("prefill_attention", prefill_attention<1>, dim3(b.ntiles, a.kv_heads), dim3(PF_THREADS), 0, stream, timer, a, (const uint16_t*)b.q, (const uint16_t*)L.kv, b.attended, b.tiles); break;
            case 4: dispatch("prefill_attention", prefill_attention<2>, dim3(b.ntiles, a.kv_heads), dim3(PF_THREADS), 0, stream, timer, a, (const uint16_t*)b.q, (const uint16_t*)L.kv, b.attended, b.tiles); break;
            case 8: dispatch("prefill_attention", prefill_attention<4>, dim3(b.ntiles, a.kv_heads), dim3(PF_THREADS), 0, stream, timer, a, (const uint16_t*)b.q, (const uint16_t*)L.kv, b.attended, b.tiles); break;
            case 16: dispatch("prefill_attention", prefill_attention<8>, dim3(b.ntiles, a.kv_heads), dim3(PF_THREADS), 0, stream, timer, a, (const uint16_t*)b.q, (const uint16_t*)L.kv, b.attended, b.tiles); break;
            default: return hipErrorInvalidValue;
        }
        GemmArgs o{L.o, b.attended, a.heads * HEAD_DIM, a.hidden, input, b.mid, nullptr, nullptr, nullptr};
        dispatch("prefill_o", prefill_gemm<EPI_RESIDUAL>, dim3(a.hidden / TN, mblocks), dim3(PF_THREADS), GEMM_LDS, stream, timer, a, o);
        dispatch("prefill_norm", prefill_norm<false>, rows4, dim3(256), 0, stream, timer, a, (const float*)b.mid, L.post_norm,
                 b.normed, (float*)nullptr);
        GemmArgs gu{L.gate_up, b.normed, a.hidden, 2 * a.inner, nullptr, nullptr, b.mlp, nullptr, nullptr};
        dispatch("prefill_gate_up", prefill_gemm<EPI_SILU>, dim3(2 * a.inner / TN, mblocks), dim3(PF_THREADS), GEMM_LDS, stream, timer, a, gu);
        GemmArgs down{L.down, b.mlp, a.inner, a.hidden, b.mid, b.h, nullptr, nullptr, nullptr};
        dispatch("prefill_down", prefill_gemm<EPI_RESIDUAL>, dim3(a.hidden / TN, mblocks), dim3(PF_THREADS), GEMM_LDS, stream, timer, a, down);
        input = b.h;
        if (l + 1 < nlayers)
            dispatch("prefill_norm", prefill_norm<false>, rows4, dim3(256), 0, stream, timer, a, (const float*)b.h,
                     layers[l + 1].input_norm, b.normed, (float*)nullptr);
    }
    dispatch("prefill_final_norm", prefill_norm<true>, rows4, dim3(256), 0, stream, timer, a, input, final_norm,
             (uint16_t*)nullptr, b.out);
    return hipGetLastError();
}

}  // namespace tgx
