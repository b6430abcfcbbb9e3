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
//   gemv_residual     out = residual + W x, o_proj and down_proj (gemv_residual.comp:28-45), which
//                     also leave out as the next norm takes it (out gain in bf16, sums of squares)
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

// Projections: a workgroup of eight waves to a strip of W (16 rows for q/k/v, 2 x 16 for gate/up,
// 4 or 16 for o_proj and down_proj) against one 16-row tile of the batch, the tile of blockIdx.y;
// the workgroups of one strip sit on one XCD (their ids differ by a multiple of the strips, a
// multiple of 8) and read its weights from there after the first. A workgroup issues every load
// it makes at its start, so that it waits for memory once.
constexpr int GEMV_WAVES = 8;
constexpr int GEMV_THREADS = GEMV_WAVES * WAVE;
// K is taken in chunks of 32 k-blocks (1024 columns); wave w's chain runs over k-blocks
// 32 c + 4 w .. 32 c + 4 w + 3 of chunk c, chunk after chunk, whatever the batch and strip.
constexpr int CHUNK_KB = 32;
constexpr int CHUNK_COLS = CHUNK_KB * 32;
constexpr int PER_WAVE = CHUNK_KB / GEMV_WAVES;
constexpr int MAX_CHUNKS = 6;  // K up to 6144 (down_proj's inner); kernels are built for 1 to 6 chunks
// hidden up to 2048 (VoxCPM2's LMs): the norms, q/k/v and gate/up. Past it layer 0's q/k/v, which
// reads the f32 rows, would hold more than a wave's registers.
constexpr int MAX_HIDDEN_CHUNKS = 2;
// A norm's input carries a sum of squares for each SQ_COLS columns of a row, or for each
// SQ_WIDE_COLS where the projection that wrote it took strips of that many rows.
constexpr int SQ_COLS = 4;
constexpr int SQ_WIDE_COLS = 16;

// Attention: a workgroup of eight waves to each (row, KV head).
constexpr int ATTN_WAVES = 8;
constexpr int ATTN_THREADS = ATTN_WAVES * WAVE;

__device__ __forceinline__ uint4 load16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ float4 load_f4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Loads below are never branched around per lane: rows past the batch are read from the last row
// instead, and the chunk counts are template parameters. What such rows give lands in MFMA rows
// or columns that nothing reads (a row of C depends on that row of A alone, a column on that
// column of B alone).
//
// all_issued() ends the issue of a kernel's loads: the scheduler may move nothing across it, so
// that every load is in flight before the first value is used (left to itself it interleaves the
// loads with the MFMAs to save registers, one memory round trip after another).
__device__ __forceinline__ void all_issued() { __builtin_amdgcn_sched_barrier(0); }

// The MFMA's B operand straight from memory, no LDS: wave w's k-blocks are 32 c + 4 w + j of
// chunk c (j < 4), and lane 16 g + t of a k-block holds row t of the tile (batch row
// 16 tile + t), columns 32 kb + 8 g .. + 7. Each wave reads only the columns of its own
// k-blocks, so the vectors need no sharing between waves.
template <int CH>
struct Operand {
    static constexpr int KB = CH * PER_WAVE;  // k-blocks to a wave
    uint4 xf[KB];

    __device__ static int kblock(int i) { return (i / PER_WAVE) * CHUNK_KB + (int)(threadIdx.x / WAVE) * PER_WAVE + i % PER_WAVE; }
    __device__ static int column(int i) { return kblock(i) * 32 + ((threadIdx.x % WAVE) / 16) * 8; }
    __device__ static int row(int B, int tile) { return min(tile * 16 + (int)(threadIdx.x % 16), B - 1); }
};

// Where the projections' bf16 operands keep row b, column k: k-block by k-block, the batch's rows
// one after another in each, [K / 32][B][32]. A k-block of a tile's 16 rows is then 1 KiB in one
// piece (every cache line read whole), and a tile of one row the same 64 bytes 16 times over.
__device__ __forceinline__ size_t operand_index(int b, int k, int B) { return ((size_t)(k / 32) * B + b) * 32 + k % 32; }

// Bf16 rows [B][K] in operand order.
template <int CH>
struct RawRows : Operand<CH> {
    using Operand<CH>::KB;

    __device__ void load(const uint16_t* __restrict__ x, int B, int tile) {
        const int b = Operand<CH>::row(B, tile);
#pragma unroll
        for (int i = 0; i < KB; ++i) this->xf[i] = load16(x + operand_index(b, Operand<CH>::column(i), B));
    }
};

// RMSNorm's rows (norm.glsl:12-53) from the f32 rows: x gain in bf16, the row's scale 1 / rms(x)
// applied to the products afterwards, RMSNorm(x) W^T = s (x gain) W^T. `squares` is the lane's
// sum of x^2 over its columns, in k-block order; row_scales adds the lanes' in a fixed order.
template <int CH>
struct NormedRows : Operand<CH> {
    using Operand<CH>::KB;
    float4 xr[KB][2], gr[KB][2];
    float squares;

    __device__ void load(const float* __restrict__ x, const float* __restrict__ gain, int B, int tile) {
        const float* row = x + (size_t)Operand<CH>::row(B, tile) * (CH * CHUNK_COLS);
#pragma unroll
        for (int i = 0; i < KB; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) xr[i][h] = load_f4(row + Operand<CH>::column(i) + 4 * h);
#pragma unroll
        for (int i = 0; i < KB; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) gr[i][h] = load_f4(gain + Operand<CH>::column(i) + 4 * h);
    }
    __device__ void finish() {
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < KB; ++i) {
            const float4 a = xr[i][0], c = xr[i][1], ga = gr[i][0], gc = gr[i][1];
            sq += a.x * a.x;
            sq += a.y * a.y;
            sq += a.z * a.z;
            sq += a.w * a.w;
            sq += c.x * c.x;
            sq += c.y * c.y;
            sq += c.z * c.z;
            sq += c.w * c.w;
            this->xf[i] = make_uint4(pack_bf16x2(a.x * ga.x, a.y * ga.y), pack_bf16x2(a.z * ga.z, a.w * ga.w),
                                     pack_bf16x2(c.x * gc.x, c.y * gc.y), pack_bf16x2(c.z * gc.z, c.w * gc.w));
        }
        squares = sq;
    }
};

// The tile's rows' scales 1 / sqrt(sum / K + eps) from their sums of squares, sq [B][K / cols]
// (K = CH 1024; cols = SQ_COLS, or SQ_WIDE_COLS when WIDE): wave w takes tile rows
// RPW w .. RPW w + RPW - 1; lane l of chunk c takes its columns c 1024 + 16 l .. + 15, four
// 4-column sums added in column order or the one 16-column sum the strip made so; the chunks'
// are added in chunk order and the lanes' totals in a fixed order (wave_sum). The same arithmetic
// for a row whatever the batch and whichever width its sums span.
template <int CH, bool WIDE>
struct RowSquares {
    static constexpr int RPW = 16 / GEMV_WAVES;  // rows to a wave
    float4 part[RPW][CH];                        // four 4-column sums, or (WIDE) a 16-column sum in .x

    __device__ void load(const float* __restrict__ sq, int B, int tile) {
        const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
#pragma unroll
        for (int h = 0; h < RPW; ++h) {
            const int b = min(tile * 16 + RPW * w + h, B - 1);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                if constexpr (WIDE)
                    part[h][c].x = sq[(size_t)b * (CH * 64) + c * 64 + lane];
                else
                    part[h][c] = load_f4(sq + (size_t)b * (CH * 256) + c * 256 + lane * 4);
            }
        }
    }
    // scale[RPW w + h], behind the caller's next barrier.
    __device__ void finish(float eps, float* scale) {
        const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
#pragma unroll
        for (int h = 0; h < RPW; ++h) {
            float t = 0.f;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                float u = part[h][c].x;
                if constexpr (!WIDE) {
                    u += part[h][c].y;
                    u += part[h][c].z;
                    u += part[h][c].w;
                }
                t = c == 0 ? u : t + u;
            }
            const float total = wave_sum(t);
            if (lane == 0) scale[RPW * w + h] = 1.0f / sqrtf(total / (float)(CH * CHUNK_COLS) + eps);
        }
    }
};

// One wave's chains for strips `strip[s]` (R rows each, in MFMA rows 0..R-1) of W [N][CH chunks]
// against its k-blocks of the tile, k-block after k-block.
template <int S, int CH, int R = 16>
struct Gemv {
    static constexpr int KB = CH * PER_WAVE;
    f32x4 acc[S];
    uint4 wf[KB][S];

    __device__ void load(const uint16_t* __restrict__ w, const int (&strip)[S]) {
        constexpr int kblocks = CH * CHUNK_KB;
        const int lane = threadIdx.x % WAVE;
        // Lanes past the strip's rows read its last row again.
        const int off = weight_lane_offset((lane / 16) * 16 + min(lane % 16, R - 1), R);
#pragma unroll
        for (int i = 0; i < KB; ++i)
#pragma unroll
            for (int s = 0; s < S; ++s) wf[i][s] = load16(w + weight_tile_index(strip[s], Operand<CH>::kblock(i), kblocks, R) + off);
    }

    __device__ void run(const uint4 (&xf)[KB]) {
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < KB; ++i)
#pragma unroll
            for (int s = 0; s < S; ++s) acc[s] = mfma16(wf[i][s], xf[i], acc[s]);
    }
};

// Every wave's chains into red, [wave][s][lane] as f32x4 (and, when sq is set, every lane's
// squares into sq), behind a barrier.
template <int S>
__device__ void spill(const f32x4 (&acc)[S], f32x4* red, float* sq = nullptr, float squares = 0.f) {
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
#pragma unroll
    for (int s = 0; s < S; ++s) red[(w * S + s) * 64 + lane] = acc[s];
    if (sq) sq[threadIdx.x] = squares;
    __syncthreads();
}

// The tile's rows' scales from every lane's squares in sq (lane 16 g + t of wave w: row t), added
// wave by wave, g within a wave, into scale[t] = 1 / sqrt(sum / K + eps), behind a barrier.
__device__ void row_scales(const float* sq, int K, float eps, float* scale) {
    if (threadIdx.x < 16) {
        float total = 0.f;
        for (int w = 0; w < GEMV_WAVES; ++w)
#pragma unroll
            for (int g = 0; g < 4; ++g) total += sq[w * WAVE + g * 16 + threadIdx.x];
        scale[threadIdx.x] = 1.0f / sqrtf(total / (float)K + eps);
    }
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
// gemv_qkv_rope: workgroup (strip, tile): a strip of 16 permuted rows (8 RoPE pairs of a head of
// D = head_dim dimensions, the pairs (i, i + D / 2)).
// PRENORMED: the input comes as x input_norm in bf16 with its sums of squares (every layer past
// the first), else as the f32 rows. The epilogue's thread (p, c) (pair p, tile row c; the first
// 128 threads) loads its row's position and slot first of all, and the RoPE factors and cache
// block that hang on them while the products' operands are on their way.
template <int CH, bool PRENORMED, int D, bool WIDE = false>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_qkv_rope(DecodeArgs a, LayerArgs l) {
    constexpr int R = QKV_ROWS;
    constexpr int EPI = (R / 2) * 16;  // epilogue threads
    __shared__ f32x4 red[GEMV_WAVES * 64];
    __shared__ float sq[GEMV_THREADS], scale[16];
    const int strip_id = blockIdx.x, tile = blockIdx.y;
    const int strip[1] = {strip_id};
    const int p = threadIdx.x % (R / 2), c = (threadIdx.x / (R / 2)) % 16;
    const int b = tile * 16 + c;
    const int per_head = D / R;  // strips to a head
    const int head = strip_id / per_head;
    const int i = (strip_id % per_head) * (R / 2) + p;  // the pair's first dimension in the head
    uint32_t pos = 0, slot = 0;
    if (threadIdx.x < EPI) {  // whole waves
        pos = a.positions[min(b, a.rows - 1)];
        slot = a.slots[min(b, a.rows - 1)];
    }
    RowSquares<CH, WIDE> squares;
    RawRows<CH> xb;
    NormedRows<CH> xn;
    if constexpr (PRENORMED) {
        squares.load(l.x_sq, a.rows, tile);
        xb.load(l.xn, a.rows, tile);
    } else {
        xn.load(l.x, l.input_norm, a.rows, tile);
    }
    Gemv<1, CH, R> g;
    g.load(l.qkv, strip);
    if (PRENORMED || CH <= 2) all_issued();  // past two chunks the f32 rows would take too many registers
    float co = 1.f, si = 0.f;
    uint32_t entry = UINT32_MAX;
    if (threadIdx.x < EPI) {
        // 32-bit indexes (the tables hold far fewer than 2^32 entries)
        const uint32_t pc = min(pos, (uint32_t)a.capacity - 1), sc = min(slot, (uint32_t)a.nslots - 1);
        const uint32_t at = pc * (D / 2) + (uint32_t)i;
        co = a.cos[at];
        si = a.sin[at];
        // The product kept apart from the add: fused, they make a 64-bit multiply-add whose unused
        // high half the register allocator takes from a register a load in flight is to fill, so
        // that it waits for every load before this one.
        uint32_t row = sc * (uint32_t)a.max_blocks;
        asm volatile("" : "+v"(row));
        entry = a.table[row + pc / BLOCK_TOKENS];
    }
    if constexpr (PRENORMED) {
        squares.finish(a.eps, scale);
        g.run(xb.xf);
        spill<1>(g.acc, red);
    } else {
        xn.finish();
        g.run(xn.xf);
        spill<1>(g.acc, red, sq, xn.squares);
        row_scales(sq, a.hidden, a.eps, scale);
    }

    const int H = a.heads, KV = a.kv_heads;
    if (threadIdx.x >= EPI || b >= a.rows || pos >= (uint32_t)a.capacity || slot >= (uint32_t)a.nslots) return;
    float va = reduced<1>(red, 0, 2 * p, c) * scale[c];      // strip rows 2 p, 2 p + 1: the pair (qkv_row_of)
    float vc = reduced<1>(red, 0, 2 * p + 1, c) * scale[c];
    if (head < H + KV && a.rope) {
        // As upstream: x cos + rotate_half(x) sin (gemv_qkv_rope.comp:88-94).
        const float ra = va * co - vc * si;
        const float rc = vc * co + va * si;
        va = ra;
        vc = rc;
    }
    if (head < H) {
        uint16_t* q = l.q + ((size_t)b * H + head) * D;
        q[i] = (uint16_t)bf16_bits(va);
        q[i + D / 2] = (uint16_t)bf16_bits(vc);
        return;
    }
    if (entry >= (uint32_t)a.nblocks) return;  // the slot holds no block there
    const int kv = head < H + KV ? head - H : head - H - KV;
    constexpr int TILE = kv_tile(D);
    uint16_t* tl = l.kv + ((size_t)entry * KV + kv) * 2 * TILE;
    const int pp = (int)(pos % BLOCK_TOKENS);
    if (head < H + KV) {
        tl[key_index(pp, i, D)] = (uint16_t)bf16_bits(va);
        tl[key_index(pp, i + D / 2, D)] = (uint16_t)bf16_bits(vc);
    } else {
        tl[TILE + value_index(pp, i)] = (uint16_t)bf16_bits(va);
        tl[TILE + value_index(pp, i + D / 2)] = (uint16_t)bf16_bits(vc);
    }
}

// ---------------------------------------------------------------------------------------------
// gemv_gate_up: workgroup (s, group): strip s (16 rows) of the gate and the same strip of up,
// against TT 16-row tiles of mid post_norm in bf16 (tiles TT group .. TT group + TT - 1) and mid's
// sums of squares. The strips' weights are read once for the TT tiles, and each tile's products
// are the same chains as with one tile to a workgroup; the tiles' partial sums go through LDS two
// at a time.
template <int CH, int TT, bool WIDE = false>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_gate_up(DecodeArgs a, LayerArgs l) {
    constexpr int TS = TT < 2 ? TT : 2;  // tiles reduced at once
    __shared__ f32x4 red[TS][GEMV_WAVES * 2 * 64];
    __shared__ float scale[TT][16];
    const int s = blockIdx.x, tile0 = blockIdx.y * TT;
    const int strip[2] = {s, s + a.inner / 16};
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    RowSquares<CH, WIDE> squares[TT];
    RawRows<CH> x[TT];
    Gemv<2, CH> g;
#pragma unroll
    for (int t = 0; t < TT; ++t) squares[t].load(l.mid_sq, a.rows, tile0 + t);
#pragma unroll
    for (int t = 0; t < TT; ++t) x[t].load(l.mid_n, a.rows, tile0 + t);
    g.load(l.gate_up, strip);
    all_issued();
#pragma unroll
    for (int t = 0; t < TT; ++t) squares[t].finish(a.eps, scale[t]);
    f32x4 acc[TT][2];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        g.run(x[t].xf);
        acc[t][0] = g.acc[0];
        acc[t][1] = g.acc[1];
    }
#pragma unroll
    for (int t0 = 0; t0 < TT; t0 += TS) {
        if (t0) __syncthreads();  // the last tiles' sums are read
#pragma unroll
        for (int t = 0; t < TS; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h) red[t][(w * 2 + h) * 64 + lane] = acc[t0 + t][h];
        __syncthreads();
        for (int idx = threadIdx.x; idx < TS * 16 * 16; idx += GEMV_THREADS) {
            const int r = idx % 16, c = (idx / 16) % 16, t = idx / 256;
            const int b = (tile0 + t0 + t) * 16 + c;
            if (b >= a.rows) continue;
            const float sc = scale[t0 + t][c];
            const float gate = reduced<2>(red[t], 0, r, c) * sc;
            const float up = reduced<2>(red[t], 1, r, c) * sc;
            l.mlp[operand_index(b, s * 16 + r, a.rows)] = (uint16_t)bf16_bits(silu(gate) * up);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// gemv_residual: out = residual + W x, workgroup (strip, tile): a strip of R rows over the whole
// of K. The epilogue's thread (c, q) (tile row c, rows 4 q .. 4 q + 3 of the strip; the first
// 4 R threads) loads its residual and next-norm gains first of all, and with next_norm set also
// writes out next_norm in bf16 and the sum of squares of the strip's R columns of row c: its 4 in
// order, and at R = 16 the four threads' sums added in column order (the order a 4-column reader
// adds them in).
template <int CH, int R>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_residual(DecodeArgs a, ResidualArgs r) {
    constexpr int EPI = 16 * (R / SQ_COLS);
    constexpr int LOADERS = EPI < WAVE ? WAVE : EPI;  // whole waves load (past EPI, the same again)
    static_assert(LOADERS % WAVE == 0, "whole waves");
    __shared__ f32x4 red[GEMV_WAVES * 64];
    const int strip_id = blockIdx.x, tile = blockIdx.y;
    const int strip[1] = {strip_id};
    const int c = threadIdx.x % 16, q = (threadIdx.x / 16) % (R / SQ_COLS);
    const int b = tile * 16 + c;
    const int n0 = strip_id * R + q * SQ_COLS;
    float4 res = make_float4(0.f, 0.f, 0.f, 0.f), gain = res;
    if (threadIdx.x < LOADERS) {
        res = load_f4(r.residual + (size_t)min(b, a.rows - 1) * r.N + n0);
        gain = load_f4((r.next_norm ? r.next_norm : r.residual) + n0);
    }
    RawRows<CH> x;
    Gemv<1, CH, R> g;
    x.load(r.x, a.rows, tile);
    g.load(r.w, strip);
    all_issued();
    g.run(x.xf);
    spill<1>(g.acc, red);
    if (threadIdx.x >= EPI) return;  // whole waves stay (EPI is 16 or 64): the shuffles below read every lane
    const float4 v = make_float4(res.x + reduced<1>(red, 0, q * 4, c), res.y + reduced<1>(red, 0, q * 4 + 1, c),
                                 res.z + reduced<1>(red, 0, q * 4 + 2, c), res.w + reduced<1>(red, 0, q * 4 + 3, c));
    float s2 = v.x * v.x;
    s2 += v.y * v.y;
    s2 += v.z * v.z;
    s2 += v.w * v.w;
    if constexpr (R == SQ_WIDE_COLS) {
        // Lanes c, c + 16, c + 32 and c + 48 hold row c's sums of the strip's columns 0-3, 4-7,
        // 8-11 and 12-15.
        static_assert(EPI == WAVE, "the strip's four sums of a row in one wave");
        const float s4 = __shfl_down(s2, 16), s8 = __shfl_down(s2, 32), s12 = __shfl_down(s2, 48);
        s2 += s4;
        s2 += s8;
        s2 += s12;
    }
    if (b >= a.rows) return;
    const size_t at = (size_t)b * r.N + n0;
    *reinterpret_cast<float4*>(r.out + at) = v;
    if (r.next_norm) {
        *reinterpret_cast<uint2*>(r.out_n + operand_index(b, n0, a.rows)) =
            make_uint2(pack_bf16x2(v.x * gain.x, v.y * gain.y), pack_bf16x2(v.z * gain.z, v.w * gain.w));
        if (q == 0) r.out_sq[(size_t)b * (r.N / R) + strip_id] = s2;
    }
}

// ---------------------------------------------------------------------------------------------
// attention_decode: workgroup (kv, b) attends the `group` query heads KV head kv serves of row b
// over its slot's positions 0..pos; wave w takes turns w, w + 8, ... (a turn: TURN = 32 positions,
// half a cache block, D / 16 key and D / 16 value fragments; at 256 positions all eight waves have
// one, where whole-block turns left four idle) with an online softmax, two turns' keys and values
// in flight at once. Per turn, S^T = K Q^T (keys as rows, heads as columns) and O^T += V^T P, P in
// bf16 straight from the registers S^T left it in.
// Two memory round trips before the first product: the row's position, the cache blocks of the
// wave's turns (lane j of register r: the block of turn w + 8 (j + 64 r), from the row's copy of
// its slot's table) and q together, then the first two turns' keys and values.
constexpr int attention_turn(int /* head_dim: either width */) { return BLOCK_TOKENS / 2; }
// The positions a row may reach: 32768 at head_dim 64, 16384 at 128 (the block ids of a wave's
// turns in two registers and one).
constexpr int attention_capacity(int head_dim) { return head_dim == 64 ? 32768 : 16384; }

template <int D>
__global__ void __launch_bounds__(ATTN_THREADS) attention_decode(DecodeArgs a, LayerArgs l) {
    constexpr int TURN = attention_turn(D);
    constexpr int PT = TURN / 16, KS = PT / 2, DT = D / 16, DS = D / 32;
    constexpr int KF = PT * DS, VF = DT * KS;  // a turn's key and value fragments
    static_assert(KF == D / 16 && VF == D / 16, "a turn is D / 16 key and D / 16 value fragments");
    constexpr int BREGS = attention_capacity(D) / (ATTN_WAVES * WAVE * TURN);  // block-id registers
    static_assert(BREGS == 1 || BREGS == 2, "one or two registers of a wave's turns' blocks");
    constexpr int TILE = kv_tile(D);
    extern __shared__ float attn_lds[];  // [waves][group][D + 1] partial outputs
    __shared__ float sm_m[ATTN_WAVES][16];
    __shared__ float sm_l[ATTN_WAVES][16];
    const int kv = blockIdx.x, b = blockIdx.y;
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int H = a.heads, KV = a.kv_heads, group = H / KV;
    const int h = lane % 16;
    const uint32_t pos = a.positions[b];
    uint32_t turn_block[BREGS];
#pragma unroll
    for (int r = 0; r < BREGS; ++r)
        turn_block[r] = a.row_table[(uint32_t)b * (uint32_t)a.max_blocks +
                                    (uint32_t)min((w + ATTN_WAVES * (lane + WAVE * r)) * TURN / BLOCK_TOKENS, a.max_blocks - 1)];
    // Columns past the group read its last head again; nothing reads what they give.
    uint4 qf[DS];
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) qf[ds] = load16(l.q + ((size_t)b * H + kv * group + min(h, group - 1)) * D + ds * 32 + (lane / 16) * 8);
    all_issued();
    if (pos >= (uint32_t)a.capacity) return;  // a spare row
    const int turns = (int)(pos / TURN) + 1;

    // Turn j's block, and whether the wave has it (the slot may hold no block there).
    auto block_of_turn = [&](int j) {
        if constexpr (BREGS == 1)
            return (uint32_t)__builtin_amdgcn_readlane((int)turn_block[0], min(j, WAVE - 1));
        else
            return (uint32_t)(j < WAVE ? __builtin_amdgcn_readlane((int)turn_block[0], j)
                                       : __builtin_amdgcn_readlane((int)turn_block[1], min(j - WAVE, WAVE - 1)));
    };
    auto has = [&](int j) { return w + ATTN_WAVES * j < turns && block_of_turn(j) < (uint32_t)a.nblocks; };
    // Turn j's keys and values: its positions' key fragments are one run of the block's key tile
    // (8 of them from fragment 8 half), its value fragments (dt, ks) those of dimensions 16 dt and
    // positions 32 (half + ks) of the value tile. Without the turn (`real` false) every lane reads
    // the pool's first 16 bytes instead, one cache line an instruction from the caches: the loads
    // are made either way, so that the waits for them can be counted exactly (a load under a branch
    // makes the compiler wait for every load before its first use).
    auto fetch = [&](int j, bool real, uint4 (&k)[KF], uint4 (&v)[VF]) {
        const int half = ((w + ATTN_WAVES * j) * TURN % BLOCK_TOKENS) / 32;
        const uint16_t* kt = real ? l.kv + ((size_t)block_of_turn(j) * KV + kv) * 2 * TILE : l.kv;
        const int at = real ? lane * 8 : 0;
        const int k0 = real ? half * KF * 512 : 0, kstride = real ? 512 : 0;
        const int v0 = real ? TILE + half * 512 : 0;
#pragma unroll
        for (int i = 0; i < KF; ++i) k[i] = load16(kt + k0 + i * kstride + at);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) v[dt * KS + ks] = load16(kt + v0 + (dt * 2 + ks) * kstride + at);
    };
    OnlineSoftmax<PT, DT> sm;
    const float scale_log2 = log2_scale(a.scale);
    // S^T = K Q^T for a turn's keys, then its softmax step (masked only in the turn holding the
    // position).
    auto take = [&](const uint4 (&k)[KF], const uint4 (&v)[VF], int j) __attribute__((always_inline)) {
        f32x4 s[PT];
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
            s[pt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) s[pt] = mfma16(k[pt * DS + ds], qf[ds], s[pt]);
        }
        const uint32_t p0 = (uint32_t)(w + ATTN_WAVES * j) * TURN;
        if (p0 + TURN - 1 <= pos)
            sm.template block<false>(s, v, p0, pos, pos, scale_log2);
        else
            sm.template block<true>(s, v, p0, pos, pos, scale_log2);
    };
    // Two buffers: the first two turns straight (every context up to 16 turns), then the rest
    // two at a time, each pair's loads issued once the last pair is taken.
    uint4 ka[KF], va[VF], kb[KF], vb[VF];
    const bool t0 = has(0), t1 = has(1);
    fetch(0, t0, ka, va);
    fetch(1, t1, kb, vb);
    if (t0) take(ka, va, 0);
    if (t1) take(kb, vb, 1);
    for (int j = 2; t1 && has(j); j += 2) {
        const bool next = has(j + 1);
        fetch(j, true, ka, va);
        fetch(j + 1, next, kb, vb);
        take(ka, va, j);
        if (!next) break;
        take(kb, vb, j + 1);
    }
    if (lane < 16) {
        sm_m[w][h] = sm.m;
        sm_l[w][h] = sm.l;
    }
    if (h < group) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) attn_lds[(w * group + h) * (D + 1) + dt * 16 + (lane / 16) * 4 + i] = sm.o[dt][i];
    }
    __syncthreads();
    // The waves joined in order (wave 0 holds turn 0, so M is finite).
    for (int idx = threadIdx.x; idx < group * D; idx += ATTN_THREADS) {
        const int hh = idx / D, d = idx % D;
        float M = -INFINITY;
        for (int j = 0; j < ATTN_WAVES; ++j) M = fmaxf(M, sm_m[j][hh]);
        float L = 0.f, O = 0.f;
        for (int j = 0; j < ATTN_WAVES; ++j) {
            const float f = sm_l[j][hh] > 0.f ? __builtin_amdgcn_exp2f(sm_m[j][hh] - M) : 0.f;
            L += sm_l[j][hh] * f;
            O += attn_lds[(j * group + hh) * (D + 1) + d] * f;
        }
        l.attended[operand_index(b, (kv * group + hh) * D + d, a.rows)] = (uint16_t)bf16_bits(O / L);
    }
}

// ---------------------------------------------------------------------------------------------
// final_rmsnorm: the final norm, a wave to a row, for hidden = CH 1024; with `advance`, moves each
// placed row on by one position once the step is done with it.
template <int CH>
__global__ void __launch_bounds__(WAVE) final_rmsnorm(DecodeArgs a, const float* __restrict__ x, const float* __restrict__ gain,
                                                      float* __restrict__ out, uint32_t* positions, int advance) {
    constexpr int K = CH * CHUNK_COLS, V = K / WAVE / 4;  // float4 to a lane
    const int b = blockIdx.x, lane = threadIdx.x;
    const size_t at = (size_t)b * K + lane * (K / WAVE);
    float4 v[V], g[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
        v[e] = *reinterpret_cast<const float4*>(x + at + 4 * e);
        g[e] = *reinterpret_cast<const float4*>(gain + lane * (K / WAVE) + 4 * e);
    }
    float squares = 0.f;
#pragma unroll
    for (int e = 0; e < V; ++e) {
        squares += v[e].x * v[e].x;
        squares += v[e].y * v[e].y;
        squares += v[e].z * v[e].z;
        squares += v[e].w * v[e].w;
    }
    const float scale = 1.0f / sqrtf(wave_sum(squares) / (float)K + a.eps);
#pragma unroll
    for (int e = 0; e < V; ++e)
        *reinterpret_cast<float4*>(out + at + 4 * e) =
            make_float4(v[e].x * scale * g[e].x, v[e].y * scale * g[e].y, v[e].z * scale * g[e].z, v[e].w * scale * g[e].w);
    if (advance && lane == 0) {
        const uint32_t pos = positions[b];
        if (pos < (uint32_t)a.capacity) positions[b] = pos + 1;
    }
}

// ---------------------------------------------------------------------------------------------
// Launchers: each kernel's instance, grid, block and LDS for a shape, shared by the step's
// launchers below and by the program API, so that a dispatch made either way runs the same code.

namespace {

size_t attention_lds(const DecodeArgs& a) { return (size_t)ATTN_WAVES * (a.heads / a.kv_heads) * (a.head_dim + 1) * 4; }

// The kernel instantiated for `chunks` chunks of K (1 to MAX_CHUNKS, checked by the shape).
template <template <int> class Pick>
auto by_chunks(int chunks) -> decltype(Pick<1>::get()) {
    switch (chunks) {
        case 2: return Pick<2>::get();
        case 3: return Pick<3>::get();
        case 4: return Pick<4>::get();
        case 5: return Pick<5>::get();
        case 6: return Pick<6>::get();
        default: return Pick<1>::get();
    }
}
// Kernels whose K is hidden are built for up to MAX_HIDDEN_CHUNKS chunks (the shape check refuses
// more); past that the picks name the largest, never launched.
constexpr int hidden_ch(int ch) { return ch < MAX_HIDDEN_CHUNKS ? ch : MAX_HIDDEN_CHUNKS; }
template <int D>
struct Qkv {
    template <int CH> struct Plain { static auto get() { return gemv_qkv_rope<hidden_ch(CH), false, D>; } };
    template <int CH> struct Normed { static auto get() { return gemv_qkv_rope<hidden_ch(CH), true, D>; } };
    template <int CH> struct NormedWide { static auto get() { return gemv_qkv_rope<hidden_ch(CH), true, D, true>; } };
};
template <int CH> struct PickGateUp { static auto get() { return gemv_gate_up<hidden_ch(CH), 1>; } };
template <int CH> struct PickGateUpWide { static auto get() { return gemv_gate_up<hidden_ch(CH), 1, true>; } };
template <int CH> struct PickResidual4 { static auto get() { return gemv_residual<CH, 4>; } };
template <int CH> struct PickResidual16 { static auto get() { return gemv_residual<CH, 16>; } };
template <int CH> struct PickFinal { static auto get() { return final_rmsnorm<hidden_ch(CH)>; } };

// The kernel of `launch` with its arguments `params`, timed by the timer's next events when given.
hipError_t dispatch_launch(const char* label, const KernelLaunch& k, void** params, hipStream_t stream, DispatchTimer* timer) {
    if (timer && timer->used < timer->capacity) {
        const int i = timer->used++;
        timer->labels[i] = label;
        return hipExtLaunchKernel(k.func, k.grid, k.block, params, k.lds, stream, timer->start[i], timer->stop[i], 0);
    }
    return hipLaunchKernel(k.func, k.grid, k.block, params, k.lds, stream);
}

}  // namespace

KernelLaunch qkv_launch(const DecodeArgs& a, bool prenormed, bool wide) {
    const int chunks = a.hidden / CHUNK_COLS;
    KernelLaunch k;
    if (a.head_dim == 128)
        k.func = !prenormed ? (const void*)by_chunks<Qkv<128>::Plain>(chunks)
                 : wide     ? (const void*)by_chunks<Qkv<128>::NormedWide>(chunks)
                            : (const void*)by_chunks<Qkv<128>::Normed>(chunks);
    else
        k.func = !prenormed ? (const void*)by_chunks<Qkv<64>::Plain>(chunks)
                 : wide     ? (const void*)by_chunks<Qkv<64>::NormedWide>(chunks)
                            : (const void*)by_chunks<Qkv<64>::Normed>(chunks);
    k.grid = dim3((a.heads + 2 * a.kv_heads) * a.head_dim / QKV_ROWS, decode_tiles(a.rows));
    k.block = dim3(GEMV_THREADS);
    return k;
}

KernelLaunch attention_launch(const DecodeArgs& a) {
    KernelLaunch k;
    k.func = a.head_dim == 128 ? (const void*)attention_decode<128> : (const void*)attention_decode<64>;
    k.grid = dim3(a.kv_heads, a.rows);
    k.block = dim3(ATTN_THREADS);
    k.lds = (uint32_t)attention_lds(a);
    return k;
}

KernelLaunch residual_launch(const DecodeArgs& a, const ResidualArgs& r) {
    const int chunks = r.K / CHUNK_COLS;
    KernelLaunch k;
    if (r.R == 4)
        k.func = (const void*)by_chunks<PickResidual4>(chunks);
    else if (r.R == 16)
        k.func = (const void*)by_chunks<PickResidual16>(chunks);
    else
        return k;
    k.grid = dim3(r.N / r.R, decode_tiles(a.rows));
    k.block = dim3(GEMV_THREADS);
    return k;
}

KernelLaunch gate_up_launch(const DecodeArgs& a, bool wide) {
    const int tiles = decode_tiles(a.rows);
    const int hidden_chunks = a.hidden / CHUNK_COLS;
    // Past one tile a workgroup takes two or four, reading the strips' weights once for them (for a
    // hidden size of one chunk: more would not fit the registers).
    const int per = hidden_chunks > 1 || tiles == 1 ? 1 : tiles == 2 ? 2 : 4;
    KernelLaunch k;
    if (wide)
        k.func = per == 1 ? (const void*)by_chunks<PickGateUpWide>(hidden_chunks)
                 : per == 2 ? (const void*)gemv_gate_up<1, 2, true>
                            : (const void*)gemv_gate_up<1, 4, true>;
    else
        k.func = per == 1 ? (const void*)by_chunks<PickGateUp>(hidden_chunks)
                 : per == 2 ? (const void*)gemv_gate_up<1, 2>
                            : (const void*)gemv_gate_up<1, 4>;
    k.grid = dim3(a.inner / 16, (tiles + per - 1) / per);
    k.block = dim3(GEMV_THREADS);
    return k;
}

KernelLaunch final_norm_launch(const DecodeArgs& a) {
    KernelLaunch k;
    k.func = (const void*)by_chunks<PickFinal>(a.hidden / CHUNK_COLS);
    k.grid = dim3(a.rows);
    k.block = dim3(WAVE);
    return k;
}

hipError_t launch_decode_layer(const DecodeArgs& a, const LayerArgs& l, const ResidualArgs& o, const ResidualArgs& down,
                               hipStream_t stream, DispatchTimer* timer) {
    DecodeArgs aa = a;
    LayerArgs ll = l;
    ResidualArgs oo = o, dd = down;
    void* layer_params[] = {&aa, &ll};
    // The squares o_proj and down_proj leave span their strips' rows: 16 columns at 16-row strips.
    const bool wide = o.R == SQ_WIDE_COLS;
    hipError_t e = dispatch_launch("gemv_qkv_rope", qkv_launch(a, l.xn != nullptr, wide), layer_params, stream, timer);
    if (e == hipSuccess) e = dispatch_launch("attention_decode", attention_launch(a), layer_params, stream, timer);
    const KernelLaunch ko = residual_launch(a, o), kd = residual_launch(a, down);
    if (!ko.func || !kd.func) return hipErrorInvalidValue;
    void* o_params[] = {&aa, &oo};
    if (e == hipSuccess) e = dispatch_launch("o_proj", ko, o_params, stream, timer);
    if (e == hipSuccess) e = dispatch_launch("gemv_gate_up", gate_up_launch(a, wide), layer_params, stream, timer);
    void* down_params[] = {&aa, &dd};
    if (e == hipSuccess) e = dispatch_launch("down_proj", kd, down_params, stream, timer);
    return e != hipSuccess ? e : hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// stream_read: the bandwidth the decode kernels are held to (kernels/glsl/stream_read.comp:1-23):
// every thread reads STREAM_LOADS 16-byte pieces a grid's width apart, all issued before any is
// used, and each wave writes one word of their XOR, so that no read can be left out.
constexpr int STREAM_THREADS = 256;
constexpr int STREAM_LOADS = 8;

__global__ void __launch_bounds__(STREAM_THREADS) stream_read(const uint4* __restrict__ data, uint32_t* __restrict__ out) {
    const size_t stride = (size_t)gridDim.x * STREAM_THREADS;
    const size_t at = (size_t)blockIdx.x * STREAM_THREADS + threadIdx.x;
    uint4 v[STREAM_LOADS];
#pragma unroll
    for (int i = 0; i < STREAM_LOADS; ++i) v[i] = data[at + i * stride];
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < STREAM_LOADS; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    for (int off = 32; off >= 1; off >>= 1) x ^= (uint32_t)__shfl_xor((int)x, off, WAVE);
    if (threadIdx.x % WAVE == 0) out[blockIdx.x * (STREAM_THREADS / WAVE) + threadIdx.x / WAVE] = x;
}

size_t stream_read_unit() { return (size_t)STREAM_THREADS * STREAM_LOADS * sizeof(uint4); }

KernelLaunch stream_read_launch(size_t bytes) {
    KernelLaunch k;
    k.func = (const void*)stream_read;
    k.grid = dim3((unsigned)(bytes / stream_read_unit()));
    k.block = dim3(STREAM_THREADS);
    return k;
}

namespace {
__global__ void __launch_bounds__(WAVE) read_clock(uint64_t* out) {
    if (threadIdx.x == 0) *out = wall_clock64();
}
}  // namespace

hipError_t launch_read_clock(uint64_t* out, hipStream_t stream) {
    hipLaunchKernelGGL(read_clock, dim3(1), dim3(WAVE), 0, stream, out);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void* data, size_t bytes, uint32_t* out, hipStream_t stream) {
    if (bytes == 0 || bytes % stream_read_unit()) return hipErrorInvalidValue;
    const uint4* d = (const uint4*)data;
    void* params[] = {&d, &out};
    return dispatch_launch("stream_read", stream_read_launch(bytes), params, stream, nullptr);
}

int decode_tiles(int rows) { return (rows + 15) / 16; }

int decode_residual_rows(int rows) { return rows <= 16 ? 4 : 16; }

int decode_max_k() { return MAX_CHUNKS * CHUNK_COLS; }

int decode_max_hidden() { return MAX_HIDDEN_CHUNKS * CHUNK_COLS; }

int decode_max_capacity(int head_dim) { return attention_capacity(head_dim); }

hipError_t decode_prepare(size_t device_lds) {
    for (const void* f : {(const void*)attention_decode<64>, (const void*)attention_decode<128>}) {
        hipFuncAttributes attr{};
        hipError_t e = hipFuncGetAttributes(&attr, f);
        if (e != hipSuccess) return e;
        e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(device_lds - attr.sharedSizeBytes));
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

size_t decode_attention_lds(int heads, int kv_heads, int head_dim) {
    return (size_t)ATTN_WAVES * (heads / kv_heads) * (head_dim + 1) * 4;
}

hipError_t launch_final_norm(const DecodeArgs& a, const float* x, const float* gain, float* out, uint32_t* positions,
                             int advance, hipStream_t stream, DispatchTimer* timer) {
    DecodeArgs aa = a;
    void* params[] = {&aa, &x, &gain, &out, &positions, &advance};
    const hipError_t e = dispatch_launch("final_norm", final_norm_launch(a), params, stream, timer);
    return e != hipSuccess ? e : hipGetLastError();
}

}  // namespace tgx
