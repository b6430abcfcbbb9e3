// The prefill's host side (Prefill::run, crates/graph/src/prefill.rs:473-503): runs of positions
// laid out as rows of one set of tensors, the cache blocks they write handed to their slots, the
// attention's tiles, and the kernels launched over the decoder's weights and cache.
#include <algorithm>
#include <cstring>
#include <type_traits>
#include <vector>

#include "runtime.hpp"

namespace tgx {

namespace {

constexpr int ROW_TILE = 256;  // the GEMM's rows per workgroup

template <typename T>
tgx_status prefill_alloc(Decoder* d, T** out, size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count, 1) * sizeof(T);
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(TGX_E_HIP, "hipMalloc of " + std::to_string(bytes) + " bytes: " + hipGetErrorString(e));
    d->pf.allocations.push_back({p, bytes});
    *out = (T*)p;
    return TGX_OK;
}

void prefill_free(Decoder* d) {
    for (auto& b : d->pf.allocations) hipFree(b.ptr);
    d->pf.allocations.clear();
    d->pf.rows_held = 0;
}

// Tensors for `rows` rows (a multiple of ROW_TILE), kept until a longer prefill needs more.
tgx_status hold_rows(Decoder* d, int rows, int tiles) {
    if (rows <= d->pf.rows_held && tiles <= d->pf.tiles_held) return TGX_OK;
    TGX_HIP(hipStreamSynchronize(d->ctx->stream));
    prefill_free(d);
    const Shape& s = d->shape;
    const size_t h = s.hidden, att = (size_t)s.heads * s.head_dim;
    PrefillState& p = d->pf;
    TGX_TRY(prefill_alloc(d, &p.x, rows * h));
    TGX_TRY(prefill_alloc(d, &p.h, rows * h));
    TGX_TRY(prefill_alloc(d, &p.mid, rows * h));
    TGX_TRY(prefill_alloc(d, &p.out, rows * h));
    TGX_TRY(prefill_alloc(d, &p.normed, rows * h));
    TGX_TRY(prefill_alloc(d, &p.row_sq, rows * h / 128));
    TGX_TRY(prefill_alloc(d, &p.q, rows * att));
    TGX_TRY(prefill_alloc(d, &p.attended, rows * att));
    TGX_TRY(prefill_alloc(d, &p.mlp, rows * (size_t)s.inner));
    TGX_TRY(prefill_alloc(d, &p.tok_pos, (size_t)rows));
    TGX_TRY(prefill_alloc(d, &p.tok_slot, (size_t)rows));
    TGX_TRY(prefill_alloc(d, &p.tiles, (size_t)tiles));
    // Rows past a run's are read by the GEMMs: keep them zero.
    TGX_HIP(hipMemset(p.x, 0, rows * h * 4));
    TGX_HIP(hipMemset(p.h, 0, rows * h * 4));
    TGX_HIP(hipMemset(p.mid, 0, rows * h * 4));
    TGX_HIP(hipMemset(p.normed, 0, rows * h * 2));
    TGX_HIP(hipMemset(p.row_sq, 0, rows * h / 128 * 4));
    TGX_HIP(hipMemset(p.attended, 0, rows * att * 2));
    TGX_HIP(hipMemset(p.mlp, 0, rows * (size_t)s.inner * 2));
    p.rows_held = rows;
    p.tiles_held = tiles;
    return TGX_OK;
}

// The prefill's kernels over the tensors p points at.
tgx_status launch(Decoder* d, const PrefillState& p) {
    const Shape& s = d->shape;
    PrefillArgs a{};
    a.M = p.M;
    a.M_pad = p.M_pad;
    a.hidden = s.hidden;
    a.inner = s.inner;
    a.heads = s.heads;
    a.kv_heads = s.kv_heads;
    a.capacity = s.capacity;
    a.nslots = d->slots;
    a.max_blocks = d->max_blocks;
    a.nblocks = d->nblocks;
    a.eps = s.eps;
    a.head_dim = s.head_dim;
    a.scale = 1.0f / std::sqrt((float)s.head_dim);
    a.rope = s.rope ? 1 : 0;
    a.tok_pos = p.tok_pos;
    a.tok_slot = p.tok_slot;
    a.table = d->table;
    a.cos = d->cos;
    a.sin = d->sin;
    std::vector<PrefillLayer> layers(s.layers);
    for (int l = 0; l < s.layers; ++l) {
        const Layer& L = d->layers[l];
        layers[l] = PrefillLayer{L.qkv, L.o, L.gate_up, L.down, L.input_norm, L.post_norm,
                                 d->kv + (size_t)l * d->nblocks * s.kv_heads * 2 * kv_tile(s.head_dim), d->od_rows};
    }
    PrefillBuffers b{p.x, p.h, p.mid, p.normed, p.q, p.attended, p.mlp, p.row_sq, p.out, p.tiles, p.ntiles};
    if (d->timed) d->timer.used = 0;
    hipError_t e = launch_prefill(a, layers.data(), s.layers, d->final_norm, b, d->ctx->stream, d->timed ? &d->timer : nullptr);
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string("launching the prefill: ") + hipGetErrorString(e));
    return TGX_OK;
}

}  // namespace

void prefill_release(Decoder* d) { prefill_free(d); }

tgx_status prefill_runs(Decoder* d, const tgx_run* runs, int nruns, const float* x, float* out) {
    if (!out) return fail(TGX_E_ARG, "null out");
    TGX_TRY(prefill_device(d, runs, nruns, x, false));
    TGX_HIP(hipMemcpyAsync(out, d->pf.out, (size_t)d->pf.M * d->shape.hidden * 4, hipMemcpyDeviceToHost, d->ctx->stream));
    TGX_HIP(hipStreamSynchronize(d->ctx->stream));
    return TGX_OK;
}

namespace {

// The rows and the attention's tiles of `runs`, checked against the decoder: each run's positions
// as rows one after another (M of them, M_pad padded to the GEMM's rows), the tiles later in a run,
// which attend to more, first.
struct Plan {
    size_t M = 0;
    int M_pad = 0;
    std::vector<uint32_t> pos, slot;
    std::vector<PrefillTile> tiles;
};

tgx_status make_plan(Decoder* d, const tgx_run* runs, int nruns, Plan& plan) {
    if (!d || !runs) return fail(TGX_E_ARG, "null decoder or runs");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (nruns <= 0) return fail(TGX_E_SHAPE, "no runs");
    const Shape& s = d->shape;
    std::vector<char> taken(d->slots, 0);
    size_t M = 0;
    for (int r = 0; r < nruns; ++r) {
        const tgx_run& run = runs[r];
        if (run.len == 0 || run.slot >= (uint32_t)d->slots || taken[run.slot] ||
            (uint64_t)run.start + run.len > (uint64_t)s.capacity)
            return fail(TGX_E_SHAPE, "run " + std::to_string(r) + ": " + std::to_string(run.len) + " positions from " +
                                         std::to_string(run.start) + " in slot " + std::to_string(run.slot) + " of " +
                                         std::to_string(d->slots) + ", a cache of " + std::to_string(s.capacity));
        taken[run.slot] = 1;
        M += run.len;
    }
    plan.M = M;
    plan.M_pad = (int)((M + ROW_TILE - 1) / ROW_TILE * ROW_TILE);
    plan.pos.assign(plan.M_pad, TGX_SPARE);
    plan.slot.assign(plan.M_pad, TGX_SPARE);
    plan.tiles.clear();
    const uint32_t tile = (uint32_t)prefill_attention_tile(s.heads / s.kv_heads, s.head_dim);  // positions a workgroup
    size_t row = 0;
    for (int r = 0; r < nruns; ++r) {
        const tgx_run& run = runs[r];
        for (uint32_t i = 0; i < run.len; ++i) {
            plan.pos[row + i] = run.start + i;
            plan.slot[row + i] = run.slot;
        }
        for (uint32_t t0 = 0; t0 < run.len; t0 += tile)
            plan.tiles.push_back(PrefillTile{(uint32_t)(row + t0), run.start + t0, std::min<uint32_t>(tile, run.len - t0), run.slot});
        row += run.len;
    }
    std::stable_sort(plan.tiles.begin(), plan.tiles.end(), [](const PrefillTile& a, const PrefillTile& b) {
        return a.pos0 + a.count > b.pos0 + b.count;
    });
    return TGX_OK;
}

tgx_status hold_runs(Decoder* d, const tgx_run* runs, int nruns) {
    for (int r = 0; r < nruns; ++r) TGX_TRY(hold_slot(d, runs[r].slot, runs[r].start + runs[r].len));
    return TGX_OK;
}

// The plan's tokens and tiles and the input into the tensors p points at, the padding rows the
// kernels read before they write cleared (the input's; the attention writes only the runs' rows of
// its output), then the kernels; on the context's stream, without waiting.
tgx_status enqueue(Decoder* d, const Plan& plan, const PrefillState& p, const float* x, bool x_on_device) {
    const size_t h = d->shape.hidden, att = (size_t)d->shape.heads * d->shape.head_dim, M = plan.M, pad = plan.M_pad - M;
    hipStream_t st = d->ctx->stream;
    TGX_TRY(sync_slots(d));
    TGX_HIP(hipMemcpyAsync(p.x, x, M * h * 4, x_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st));
    TGX_HIP(launch_fill_zero(p.x + M * h, pad * h * 4, st));
    TGX_HIP(launch_fill_zero(p.attended + M * att, pad * att * 2, st));
    TGX_HIP(hipMemcpyAsync(p.tok_pos, plan.pos.data(), plan.M_pad * 4, hipMemcpyHostToDevice, st));
    TGX_HIP(hipMemcpyAsync(p.tok_slot, plan.slot.data(), plan.M_pad * 4, hipMemcpyHostToDevice, st));
    TGX_HIP(hipMemcpyAsync(p.tiles, plan.tiles.data(), plan.tiles.size() * sizeof(PrefillTile), hipMemcpyHostToDevice, st));
    TGX_HIP(hipEventRecord(d->ev_start, st));
    TGX_TRY(launch(d, p));
    TGX_HIP(hipEventRecord(d->ev_end, st));
    return TGX_OK;
}

size_t whole(size_t bytes) { return (bytes + 255) / 256 * 256; }

// The bytes of a prefill's tensors for `rows` rows and `tiles` tiles, each 256-byte aligned.
size_t tensor_bytes(const Shape& s, size_t rows, size_t tiles) {
    const size_t h = s.hidden, att = (size_t)s.heads * s.head_dim;
    return 4 * whole(rows * h * 4) + whole(rows * h * 2) + whole(rows * h / 128 * 4) + 2 * whole(rows * att * 2) +
           whole(rows * (size_t)s.inner * 2) + 2 * whole(rows * 4) + whole(tiles * sizeof(PrefillTile));
}

// The tensors laid one after another from `base`.
void carve(const Shape& s, size_t rows, size_t tiles, unsigned char* base, PrefillState& p) {
    const size_t h = s.hidden, att = (size_t)s.heads * s.head_dim;
    size_t at = 0;
    auto take = [&](auto*& ptr, size_t bytes) {
        ptr = reinterpret_cast<std::remove_reference_t<decltype(ptr)>>(base + at);
        at += whole(bytes);
    };
    take(p.x, rows * h * 4);
    take(p.h, rows * h * 4);
    take(p.mid, rows * h * 4);
    take(p.out, rows * h * 4);
    take(p.normed, rows * h * 2);
    take(p.row_sq, rows * h / 128 * 4);
    take(p.q, rows * att * 2);
    take(p.attended, rows * att * 2);
    take(p.mlp, rows * (size_t)s.inner * 2);
    take(p.tok_pos, rows * 4);
    take(p.tok_slot, rows * 4);
    take(p.tiles, tiles * sizeof(PrefillTile));
}

}  // namespace

size_t prefill_bytes(const Decoder* d) {
    size_t n = 0;
    for (const auto& b : d->pf.allocations) n += b.bytes;
    return n;
}

tgx_status prefill_device(Decoder* d, const tgx_run* runs, int nruns, const float* x, bool x_on_device) {
    if (!x) return fail(TGX_E_ARG, "null x");
    Plan plan;
    TGX_TRY(make_plan(d, runs, nruns, plan));
    TGX_TRY(hold_runs(d, runs, nruns));
    TGX_TRY(hold_rows(d, plan.M_pad, (int)plan.tiles.size()));
    PrefillState& p = d->pf;
    p.M = (int)plan.M;
    p.M_pad = plan.M_pad;
    p.ntiles = (int)plan.tiles.size();
    return enqueue(d, plan, p, x, x_on_device);
}

tgx_status prefill_runs_noalloc(Decoder* d, const tgx_run* runs, int nruns, const float* x, float* out) {
    if (!x || !out) return fail(TGX_E_ARG, "null x or out");
    Plan plan;
    TGX_TRY(make_plan(d, runs, nruns, plan));
    void* base = d->ctx->scratch;
    if (!base) return fail(TGX_E_HIP, "the device has no prefill scratch");
    const Shape& s = d->shape;
    const size_t need = tensor_bytes(s, plan.M_pad, plan.tiles.size());
    if (need > PREFILL_SCRATCH_BYTES) {
        size_t most = 0;  // positions a call of one run takes at this shape
        const size_t tile = (size_t)prefill_attention_tile(s.heads / s.kv_heads, s.head_dim);
        for (size_t rows = ROW_TILE; tensor_bytes(s, rows, rows / tile + 1) <= PREFILL_SCRATCH_BYTES; rows += ROW_TILE) most = rows;
        return fail(TGX_E_SHAPE, std::to_string(plan.M) + " positions take " + std::to_string(need) +
                                     " bytes of tensors, past the scratch's " + std::to_string(PREFILL_SCRATCH_BYTES) +
                                     " (up to " + std::to_string(most) + " positions a call at this shape)");
    }
    TGX_TRY(hold_runs(d, runs, nruns));
    PrefillState p;
    carve(s, plan.M_pad, plan.tiles.size(), (unsigned char*)base, p);
    p.M = (int)plan.M;
    p.M_pad = plan.M_pad;
    p.ntiles = (int)plan.tiles.size();
    TGX_TRY(enqueue(d, plan, p, x, false));
    hipStream_t st = d->ctx->stream;
    TGX_HIP(hipMemcpyAsync(out, p.out, plan.M * s.hidden * 4, hipMemcpyDeviceToHost, st));
    TGX_HIP(hipStreamSynchronize(st));
    return TGX_OK;
}

tgx_status prefill_launch(Decoder* d, int times) {
    if (!d) return fail(TGX_E_ARG, "null decoder");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (d->pf.M == 0) return fail(TGX_E_SHAPE, "no prefill has run to launch again");
    if (times <= 0) return fail(TGX_E_ARG, "times");
    hipStream_t st = d->ctx->stream;
    TGX_HIP(hipEventRecord(d->ev_start, st));
    for (int i = 0; i < times; ++i) TGX_TRY(launch(d, d->pf));
    TGX_HIP(hipEventRecord(d->ev_end, st));
    TGX_HIP(hipEventRecord(d->ev_done, st));
    d->pending = true;
    return TGX_OK;
}

}  // namespace tgx
