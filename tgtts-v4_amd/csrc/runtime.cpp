// The host side of the runtime (runtime.hpp): device selection, the decoder's memory, weight
// tiling, the paged cache's block allocator, and the decode step recorded once as a HIP graph
// and launched every step (crates/graph/src/step.rs:111-149 records a command buffer once; a
// HIP graph is the MI355X counterpart).
#include "runtime.hpp"

#include "heads_kernels.hpp"
#include "local_kernels.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <functional>
#include <thread>
#include <tuple>

namespace tgx {

namespace {
thread_local std::string last_error_message;
}

tgx_status fail(tgx_status status, const std::string& message) {
    last_error_message = message;
    return status;
}

void clear_error() { last_error_message.clear(); }

const char* last_error() { return last_error_message.c_str(); }

// ---- numerics on the host ----

float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t u;
    if (exp == 0x1f) {
        u = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {  // subnormal: normalise
            int e = -1;
            do {
                man <<= 1;
                ++e;
            } while (!(man & 0x400u));
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else {
        u = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint16_t f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void rope_tables(const Shape& s, std::vector<float>& cos, std::vector<float>& sin) {
    // decode.rs:146-168: inv = 1 / theta^(i / dim) for even i, in f32; r = 1 / factor in f32;
    // angle = t * r * inv, in that order.
    const int half = s.head_dim / 2;
    cos.assign((size_t)s.capacity * half, 0.f);
    sin.assign((size_t)s.capacity * half, 0.f);
    std::vector<float> inv(half), r(half);
    for (int j = 0; j < half; ++j) {
        inv[j] = 1.0f / std::pow(s.rope_theta, (float)(2 * j) / (float)s.head_dim);
        r[j] = 1.0f / (float)(s.factors.empty() ? 1.0 : s.factors[j]);
    }
    for (int t = 0; t < s.capacity; ++t)
        for (int j = 0; j < half; ++j) {
            const float f = (float)t * r[j] * inv[j];
            cos[(size_t)t * half + j] = std::cos(f);
            sin[(size_t)t * half + j] = std::sin(f);
        }
}

tgx_status upload_graph(hipGraphExec_t exec, hipStream_t stream) {
    TGX_HIP(hipGraphUpload(exec, stream));
    TGX_HIP(hipStreamSynchronize(stream));
    return TGX_OK;
}

// ---- context ----

tgx_status context_create(int device, Context** out) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(TGX_E_NO_DEVICE, "no HIP device");
    if (device < 0 || device >= count)
        return fail(TGX_E_NO_DEVICE, "device " + std::to_string(device) + " of " + std::to_string(count));
    auto* ctx = new Context();
    ctx->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipGetDeviceProperties(&ctx->prop, device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return fail(TGX_E_HIP, std::string("context: ") + hipGetErrorString(e));
    }
    ctx->lds_bytes = ctx->prop.sharedMemPerBlock;
    int clock_khz = 0;
    if (hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, device) == hipSuccess && clock_khz > 0)
        ctx->tick_ns = 1e6 / (double)clock_khz;
    e = decode_prepare(ctx->lds_bytes);
    if (e == hipSuccess) e = prefill_prepare(ctx->lds_bytes);
    if (e == hipSuccess) e = heads_prepare(ctx->lds_bytes);
    if (e == hipSuccess) e = local_prepare();
    // The device is current: the prefill scratch's address on it, kept for the process.
    if (e == hipSuccess) e = prefill_scratch_address(device, &ctx->scratch);
    if (e != hipSuccess) {
        hipStreamDestroy(ctx->stream);
        delete ctx;
        return fail(TGX_E_HIP, std::string("preparing the kernels (") + std::to_string(ctx->prop.sharedMemPerBlock) +
                                   " bytes of LDS, the prefill scratch): " + hipGetErrorString(e));
    }
    if (std::strncmp(ctx->prop.gcnArchName, "gfx950", 6) != 0) {
        std::string arch = ctx->prop.gcnArchName;
        hipStreamDestroy(ctx->stream);
        delete ctx;
        return fail(TGX_E_KERNELS, "the kernels are built for gfx950, not " + arch);
    }
    *out = ctx;
    return TGX_OK;
}

void context_destroy(Context* ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    if (ctx->stream) hipStreamDestroy(ctx->stream);
    if (ctx->clock_host) hipHostFree(ctx->clock_host);
    delete ctx;
}

tgx_status wait_event(const Context* ctx, hipEvent_t ev, const char* what) {
    const auto begin = std::chrono::steady_clock::now();
    const auto spin = std::chrono::nanoseconds(ctx ? ctx->fence_spin_ns.load(std::memory_order_relaxed) : 0);
    while (true) {
        const hipError_t q = hipEventQuery(ev);
        if (q == hipSuccess) return TGX_OK;
        if (q != hipErrorNotReady) return fail(TGX_E_HIP, std::string(what) + ": " + hipGetErrorString(q));
        const auto waited = std::chrono::steady_clock::now() - begin;
        if (waited > std::chrono::seconds(60)) return fail(TGX_E_TIMEOUT, std::string(what) + " did not finish in 60 s");
        if (waited >= spin) std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
}

// ---- shapes ----

tgx_status check_shape(const tgx_shape* in, Shape* s) {
    auto refuse = [](const std::string& why) { return fail(TGX_E_SHAPE, why); };
    if (!in) return fail(TGX_E_ARG, "null shape");
    s->hidden = in->hidden;
    s->inner = in->inner;
    s->heads = in->heads;
    s->kv_heads = in->kv_heads;
    s->head_dim = in->head_dim;
    s->layers = in->layers;
    s->capacity = in->capacity;
    s->eps = in->eps;
    s->rope_theta = in->rope_theta;
    s->rope = in->rope != 0;
    s->factors.clear();
    if (in->rope_factors) s->factors.assign(in->rope_factors, in->rope_factors + in->head_dim / 2);
    // Head widths 64 (the backbone's) and 128 (VoxCPM2's LMs, decode.rs:919-933).
    if (s->head_dim != 64 && s->head_dim != 128)
        return refuse("head_dim " + std::to_string(s->head_dim) + ": the kernels take 64 or 128");
    if (s->layers < 0 || s->capacity <= 0) return refuse("layers " + std::to_string(s->layers) + ", capacity " + std::to_string(s->capacity));
    if (s->capacity > decode_max_capacity(s->head_dim))
        return refuse("capacity " + std::to_string(s->capacity) + " past the attention's " +
                      std::to_string(decode_max_capacity(s->head_dim)) + " at head_dim " + std::to_string(s->head_dim));
    // Query heads to a KV head: any group of 1 to 16 (the reference takes any group,
    // attention_split.comp:24-27): the decode attention's 16 MFMA columns hold up to 16 heads, and
    // a prefill attention column group 16 / group positions of them.
    if (s->kv_heads <= 0 || s->heads % s->kv_heads != 0 || s->heads / s->kv_heads > 16)
        return refuse(std::to_string(s->heads) + " heads over " + std::to_string(s->kv_heads) +
                      " KV heads: a whole group of 1 to 16 query heads a KV head");
    // The prefill GEMM takes q/k/v's rows in tiles of 256.
    if ((s->heads + 2 * s->kv_heads) * s->head_dim % 256 != 0)
        return refuse(std::to_string(s->heads) + " + 2 x " + std::to_string(s->kv_heads) + " heads of " + std::to_string(s->head_dim) +
                      ": q/k/v's rows are not a multiple of 256");
    // The projections take K in chunks of 1024 columns: hidden (the norms', q/k/v's and gate/up's
    // K) up to 2048, inner (down_proj's) and heads x head_dim (o_proj's) up to 6144
    // (decode_kernels.hip): VoxCPM2's LMs are 2048 wide with an FFN of 6144.
    for (auto [what, k, most] : {std::tuple<const char*, int, int>{"hidden", s->hidden, decode_max_hidden()},
                                 {"inner", s->inner, decode_max_k()},
                                 {"heads x head_dim", s->heads * s->head_dim, decode_max_k()}})
        if (k <= 0 || k % 1024 != 0 || k > most)
            return refuse(std::string(what) + " " + std::to_string(k) + ": a multiple of 1024 up to " + std::to_string(most));
    if (s->inner % 16 != 0 || s->hidden % 16 != 0) return refuse("rows in strips of 16");
    if (!(s->eps >= 0.f)) return refuse("eps");
    return TGX_OK;
}

tgx_status check_batch(const Shape& s, const tgx_batch* batch) {
    if (!batch) return fail(TGX_E_ARG, "null batch");
    const int block_tokens = batch->block_tokens == 0 ? BLOCK_TOKENS : batch->block_tokens;
    if (batch->rows <= 0 || batch->rows > 64 || batch->rows > batch->slots)
        return fail(TGX_E_SHAPE, std::to_string(batch->rows) + " rows in " + std::to_string(batch->slots) +
                                     " slots (1 to 64 rows, no more than the slots)");
    if (block_tokens != BLOCK_TOKENS)
        return fail(TGX_E_SHAPE, "blocks of " + std::to_string(block_tokens) + " positions: the kernels take 64");
    if (batch->blocks < 0) return fail(TGX_E_SHAPE, "a pool of " + std::to_string(batch->blocks) + " blocks");
    if (decode_attention_lds(s.heads, s.kv_heads, s.head_dim) > 160 * 1024)
        return fail(TGX_E_SHAPE, "the attention of " + std::to_string(s.heads / s.kv_heads) + " heads to a KV head takes past 160 KiB of LDS");
    return TGX_OK;
}

tgx_status placement(int slots, int capacity, const tgx_row* rows, int nrows, uint32_t* words) {
    // Batch::placement (decode.rs:198-227): positions, then slots; a spare row past every position.
    std::vector<char> taken(slots > 0 ? slots : 0, 0);
    for (int b = 0; b < nrows; ++b) {
        const tgx_row r = rows[b];
        words[b] = TGX_SPARE;
        words[nrows + b] = TGX_SPARE;
        if (r.position == TGX_SPARE) continue;
        if (r.position >= (uint32_t)capacity || r.slot >= (uint32_t)slots || taken[r.slot]) {
            return fail(TGX_E_SHAPE, "row " + std::to_string(b) + " at position " + std::to_string(r.position) + " of " +
                                         std::to_string(capacity) + " in slot " + std::to_string(r.slot) + " of " +
                                         std::to_string(slots) + ", taken: " +
                                         (r.slot < (uint32_t)slots && taken[r.slot] ? "true" : "false"));
        }
        taken[r.slot] = 1;
        words[b] = r.position;
        words[nrows + b] = r.slot;
    }
    return TGX_OK;
}

// ---- the decoder ----

DecodeArgs Decoder::args() const {
    DecodeArgs a{};
    a.hidden = shape.hidden;
    a.inner = shape.inner;
    a.heads = shape.heads;
    a.kv_heads = shape.kv_heads;
    a.head_dim = shape.head_dim;
    a.rows = rows;
    a.capacity = shape.capacity;
    a.nslots = slots;
    a.max_blocks = max_blocks;
    a.nblocks = nblocks;
    a.eps = shape.eps;
    a.scale = 1.0f / std::sqrt((float)shape.head_dim);
    a.rope = shape.rope ? 1 : 0;
    a.positions = positions;
    a.slots = slot_of_row;
    a.table = table;
    a.row_table = row_table;
    a.cos = cos;
    a.sin = sin;
    return a;
}

LayerArgs Decoder::layer_args(int l) const {
    LayerArgs la{};
    la.x = l == 0 ? x_in : h_a;
    la.xn = l == 0 ? nullptr : xn_a;
    la.x_sq = sq_a;
    la.input_norm = layers[l].input_norm;
    la.qkv = layers[l].qkv;
    la.q = q;
    la.kv = kv + (size_t)l * nblocks * shape.kv_heads * 2 * kv_tile(shape.head_dim);
    la.attended = attended;
    la.mid_n = xn_b;
    la.mid_sq = sq_b;
    la.gate_up = layers[l].gate_up;
    la.mlp = mlp;
    return la;
}

ResidualArgs Decoder::o_args(int l) const {
    ResidualArgs r{};
    r.w = layers[l].o;
    r.x = attended;
    r.K = shape.heads * shape.head_dim;
    r.N = shape.hidden;
    r.R = od_rows;
    r.residual = l == 0 ? x_in : h_a;
    r.out = h_b;
    r.next_norm = layers[l].post_norm;
    r.out_n = xn_b;
    r.out_sq = sq_b;
    return r;
}

ResidualArgs Decoder::down_args(int l) const {
    ResidualArgs r{};
    r.w = layers[l].down;
    r.x = mlp;
    r.K = shape.inner;
    r.N = shape.hidden;
    r.R = od_rows;
    r.residual = h_b;
    r.out = h_a;
    // The next layer's input norm; the last layer's output goes to the final norm, which takes the
    // f32 rows.
    r.next_norm = l + 1 < shape.layers ? layers[l + 1].input_norm : nullptr;
    r.out_n = xn_a;
    r.out_sq = sq_a;
    return r;
}

namespace {

template <typename T>
tgx_status alloc(Decoder* d, T** out, size_t count, bool zero = true) {
    void* p = nullptr;
    const size_t bytes = count * sizeof(T);
    if (bytes == 0) {
        *out = nullptr;
        return TGX_OK;
    }
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(TGX_E_HIP, "hipMalloc of " + std::to_string(bytes) + " bytes: " + hipGetErrorString(e));
    d->allocations.push_back({p, bytes});
    d->device_bytes += bytes;
    if (zero) {
        e = hipMemset(p, 0, bytes);
        if (e != hipSuccess) return fail(TGX_E_HIP, std::string("hipMemset: ") + hipGetErrorString(e));
    }
    *out = (T*)p;
    return TGX_OK;
}

// The step's dispatches on the context's stream, in order (decode_batch_graph's ops,
// decode.rs:630-723): five a layer, then the final norm.
hipError_t enqueue_step(Decoder* d, int advance, DispatchTimer* timer, int* dispatches) {
    hipStream_t s = d->ctx->stream;
    const DecodeArgs a = d->args();
    hipError_t err = hipSuccess;
    int n = 0;
    for (int l = 0; l < d->shape.layers && err == hipSuccess; ++l) {
        // layer 0 reads x_in, which stays as written
        err = launch_decode_layer(a, d->layer_args(l), d->o_args(l), d->down_args(l), s, timer);
        n += 5;
    }
    const float* x = d->shape.layers > 0 ? d->h_a : d->x_in;
    if (err == hipSuccess) {
        err = launch_final_norm(a, x, d->final_norm, d->out, d->positions, advance, s, timer);
        n += 1;
    }
    if (dispatches) *dispatches = n;
    return err;
}

tgx_status record(Decoder* d, int advance, hipGraphExec_t* exec) {
    *exec = nullptr;
    hipStream_t s = d->ctx->stream;
    TGX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int dispatches = 0;
    hipError_t err = enqueue_step(d, advance, nullptr, &dispatches);
    hipGraph_t graph = nullptr;
    hipError_t end = hipStreamEndCapture(s, &graph);
    if (err != hipSuccess) {
        if (graph) hipGraphDestroy(graph);
        return fail(TGX_E_HIP, std::string("recording the step: ") + hipGetErrorString(err));
    }
    if (end != hipSuccess) return fail(TGX_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(end));
    hipError_t e = hipGraphInstantiate(exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    TGX_TRY(upload_graph(*exec, s));
    d->dispatches = dispatches;
    return TGX_OK;
}

// The program of d->rows rows as the current one, recorded if it has not been.
tgx_status use_program(Decoder* d) {
    auto it = d->programs.find(d->rows);
    if (it == d->programs.end()) {
        Decoder::Program p;
        tgx_status st = record(d, 0, &p.step);
        if (st == TGX_OK) st = record(d, 1, &p.advance);
        if (st != TGX_OK) {
            if (p.step) hipGraphExecDestroy(p.step);
            return st;
        }
        p.dispatches = d->dispatches;
        it = d->programs.emplace(d->rows, p).first;
    }
    d->step_exec = it->second.step;
    d->advance_exec = it->second.advance;
    d->dispatches = it->second.dispatches;
    return TGX_OK;
}

tgx_status create_inner(Decoder* d, const tgx_batch* batch) {
    const Shape& s = d->shape;
    TGX_TRY(check_batch(s, batch));
    if (decode_attention_lds(s.heads, s.kv_heads, s.head_dim) + 4096 > d->ctx->lds_bytes)
        return fail(TGX_E_SHAPE, "the attention's LDS is past the device's " + std::to_string(d->ctx->lds_bytes));
    d->rows = batch->rows;
    d->max_rows = batch->rows;
    d->od_rows = decode_residual_rows(batch->rows);
    d->slots = batch->slots;
    d->block_tokens = batch->block_tokens == 0 ? BLOCK_TOKENS : batch->block_tokens;
    d->max_blocks = (s.capacity + BLOCK_TOKENS - 1) / BLOCK_TOKENS;
    d->nblocks = batch->blocks > 0 ? batch->blocks : d->slots * d->max_blocks;

    const int h = s.hidden, I = s.inner, H = s.heads, KV = s.kv_heads, D = s.head_dim;
    const size_t qkv_rows = (size_t)(H + 2 * KV) * D;
    d->layers.resize(s.layers);
    for (auto& L : d->layers) {
        TGX_TRY(alloc(d, &L.qkv, qkv_rows * h));
        TGX_TRY(alloc(d, &L.o, (size_t)h * H * D));
        TGX_TRY(alloc(d, &L.gate_up, (size_t)2 * I * h));
        TGX_TRY(alloc(d, &L.down, (size_t)h * I));
        TGX_TRY(alloc(d, &L.input_norm, (size_t)h));
        TGX_TRY(alloc(d, &L.post_norm, (size_t)h));
    }
    TGX_TRY(alloc(d, &d->final_norm, (size_t)h));
    const int R = d->rows;
    TGX_TRY(alloc(d, &d->x_in, (size_t)R * h));
    TGX_TRY(alloc(d, &d->h_a, (size_t)R * h));
    TGX_TRY(alloc(d, &d->h_b, (size_t)R * h));
    TGX_TRY(alloc(d, &d->xn_a, (size_t)R * h));
    TGX_TRY(alloc(d, &d->xn_b, (size_t)R * h));
    TGX_TRY(alloc(d, &d->sq_a, (size_t)R * h / 4));
    TGX_TRY(alloc(d, &d->sq_b, (size_t)R * h / 4));
    TGX_TRY(alloc(d, &d->out, (size_t)R * h));
    TGX_TRY(alloc(d, &d->q, (size_t)R * H * D));
    TGX_TRY(alloc(d, &d->attended, (size_t)R * H * D));
    TGX_TRY(alloc(d, &d->mlp, (size_t)R * I));
    TGX_TRY(alloc(d, &d->kv, (size_t)s.layers * d->nblocks * KV * 2 * kv_tile(D)));
    TGX_TRY(alloc(d, &d->positions, (size_t)R));
    TGX_TRY(alloc(d, &d->slot_of_row, (size_t)R));
    TGX_TRY(alloc(d, &d->table, (size_t)d->slots * d->max_blocks));
    TGX_TRY(alloc(d, &d->row_table, (size_t)R * d->max_blocks));
    TGX_TRY(alloc(d, &d->cos, (size_t)s.capacity * D / 2));
    TGX_TRY(alloc(d, &d->sin, (size_t)s.capacity * D / 2));
    // Norm gains start at one, so that an unloaded stack still runs finite.
    std::vector<float> ones(h, 1.0f);
    for (auto& L : d->layers) {
        TGX_HIP(hipMemcpy(L.input_norm, ones.data(), h * 4, hipMemcpyHostToDevice));
        TGX_HIP(hipMemcpy(L.post_norm, ones.data(), h * 4, hipMemcpyHostToDevice));
    }
    TGX_HIP(hipMemcpy(d->final_norm, ones.data(), h * 4, hipMemcpyHostToDevice));
    std::vector<float> cos, sin;
    rope_tables(s, cos, sin);
    TGX_HIP(hipMemcpy(d->cos, cos.data(), cos.size() * 4, hipMemcpyHostToDevice));
    TGX_HIP(hipMemcpy(d->sin, sin.data(), sin.size() * 4, hipMemcpyHostToDevice));

    TGX_HIP(hipHostMalloc((void**)&d->x_host, (size_t)R * h * 4, hipHostMallocCoherent));
    TGX_HIP(hipHostGetDevicePointer((void**)&d->x_mapped, d->x_host, 0));
    // The step's output is stored into it by a kernel (launch_copy_words), through its device
    // address: coherent, so that the stores reach host memory past the GPU's caches.
    TGX_HIP(hipHostMalloc((void**)&d->out_host, (size_t)R * h * 4, hipHostMallocCoherent));
    TGX_HIP(hipHostGetDevicePointer((void**)&d->out_mapped, d->out_host, 0));
    TGX_HIP(hipHostMalloc((void**)&d->placement_stage, (size_t)2 * R * 4, hipHostMallocCoherent));
    TGX_HIP(hipHostMalloc((void**)&d->table_stage, (size_t)d->slots * d->max_blocks * 4, hipHostMallocCoherent));
    TGX_HIP(hipHostMalloc((void**)&d->row_table_host, (size_t)R * d->max_blocks * 4, hipHostMallocCoherent));
    TGX_HIP(hipHostGetDevicePointer((void**)&d->placement_mapped, d->placement_stage, 0));
    TGX_HIP(hipHostGetDevicePointer((void**)&d->table_mapped, d->table_stage, 0));
    TGX_HIP(hipHostGetDevicePointer((void**)&d->row_table_mapped, d->row_table_host, 0));
    std::memset(d->x_host, 0, (size_t)R * h * 4);
    std::memset(d->out_host, 0, (size_t)R * h * 4);
    d->placement_host.assign(2 * (size_t)R, TGX_SPARE);
    d->table_host.assign((size_t)d->slots * d->max_blocks, TGX_SPARE);
    TGX_HIP(hipMemcpy(d->positions, d->placement_host.data(), R * 4, hipMemcpyHostToDevice));
    TGX_HIP(hipMemcpy(d->slot_of_row, d->placement_host.data() + R, R * 4, hipMemcpyHostToDevice));
    TGX_HIP(hipMemcpy(d->table, d->table_host.data(), (size_t)d->slots * d->max_blocks * 4, hipMemcpyHostToDevice));
    d->table_dirty = false;
    d->rows_dirty = true;
    d->slot_blocks.assign(d->slots, 0);
    d->free_list.clear();
    for (int b = d->nblocks - 1; b >= 0; --b) d->free_list.push_back((uint32_t)b);

    const int dispatches = 7 * s.layers + 2;  // the prefill's, the most a run dispatches
    d->timer_start.assign(dispatches, nullptr);
    d->timer_stop.assign(dispatches, nullptr);
    d->timer_labels.assign(dispatches, nullptr);
    for (int i = 0; i < dispatches; ++i) {
        TGX_HIP(hipEventCreate(&d->timer_start[i]));
        TGX_HIP(hipEventCreate(&d->timer_stop[i]));
    }
    d->timer.start = d->timer_start.data();
    d->timer.stop = d->timer_stop.data();
    d->timer.labels = d->timer_labels.data();
    d->timer.capacity = dispatches;
    TGX_HIP(hipEventCreate(&d->ev_start));
    TGX_HIP(hipEventCreate(&d->ev_end));
    TGX_HIP(hipEventCreateWithFlags(&d->ev_done, hipEventDisableTiming));
    TGX_HIP(hipEventCreateWithFlags(&d->ev_staged, hipEventDisableTiming));
    TGX_HIP(hipDeviceSynchronize());
    return use_program(d);
}

}  // namespace

hipError_t decoder_enqueue(Decoder* d, int advance, DispatchTimer* timer, int* dispatches) {
    return enqueue_step(d, advance, timer, dispatches);
}

tgx_status hold_slot(Decoder* d, uint32_t slot, uint32_t positions) {
    const int need = (int)((positions + BLOCK_TOKENS - 1) / BLOCK_TOKENS);
    while (d->slot_blocks[slot] < need) {
        if (d->free_list.empty())
            return fail(TGX_E_SHAPE, "the cache's " + std::to_string(d->nblocks) + " blocks are all taken");
        const uint32_t blk = d->free_list.back();
        d->free_list.pop_back();
        d->table_host[(size_t)slot * d->max_blocks + d->slot_blocks[slot]] = blk;
        d->slot_blocks[slot] += 1;
        d->table_dirty = true;
    }
    return TGX_OK;
}

tgx_status hold_ahead(Decoder* d, int times, int advance) {
    // Each placed row writes its key and value at its position, and with `advance` at the next
    // times - 1 after it too: its slot must hold blocks for all of them (decode.rs:198-227 refuses
    // a placement past the cache on the host; here the blocks are held, the capacity refused).
    const uint64_t reach = advance ? (uint64_t)times : 1;
    for (int b = 0; b < d->rows; ++b) {
        const uint32_t pos = d->placement_host[b];
        if (pos == TGX_SPARE) continue;
        if ((uint64_t)pos + reach > (uint64_t)d->shape.capacity)
            return fail(TGX_E_SHAPE, "row " + std::to_string(b) + " at position " + std::to_string(pos) + " run " +
                                         std::to_string(reach) + " steps on passes a capacity of " + std::to_string(d->shape.capacity));
        TGX_TRY(hold_slot(d, d->placement_host[d->rows + b], (uint32_t)(pos + reach)));
    }
    return TGX_OK;
}

void moved_on(Decoder* d, int times) {
    for (int b = 0; b < d->rows; ++b)
        if (d->placement_host[b] != TGX_SPARE) d->placement_host[b] += (uint32_t)times;
}

namespace {

// Before the host fills any pinned staging buffer: the copies queued from them before have run.
tgx_status staging_wait(Decoder* d) {
    if (d->staged) {
        TGX_HIP(hipEventSynchronize(d->ev_staged));
        d->staged = false;
    }
    return TGX_OK;
}

// The staged copies launched (one kernel on the context's stream), the event after them.
tgx_status staging_queued(Decoder* d) {
    const hipError_t e = launch_copy_segments(d->copies, d->ctx->stream);
    d->copies.n = 0;
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string("copying the step's inputs: ") + hipGetErrorString(e));
    TGX_HIP(hipEventRecord(d->ev_staged, d->ctx->stream));
    d->staged = true;
    return TGX_OK;
}

// A copy of `bytes` (whole 4-byte words) from a staging buffer's device address to device memory,
// staged for the next staging_queued (the ones before launched first when the list is full).
tgx_status stage_copy(Decoder* d, const void* mapped, void* dst, size_t bytes) {
    CopySegments& c = d->copies;
    if (c.n == COPY_SEGMENTS) {
        const hipError_t e = launch_copy_segments(c, d->ctx->stream);
        c.n = 0;
        if (e != hipSuccess) return fail(TGX_E_HIP, std::string("copying the step's inputs: ") + hipGetErrorString(e));
    }
    const uint32_t before = c.n ? c.end[c.n - 1] : 0u;
    c.src[c.n] = static_cast<const uint32_t*>(mapped);
    c.dst[c.n] = static_cast<uint32_t*>(dst);
    c.end[c.n] = before + (uint32_t)(bytes / 4);
    c.n += 1;
    return TGX_OK;
}

// The block table (when it changed) and the rows' copies of their slots' rows of it, staged and
// queued for the device; the caller has waited for the staging (staging_wait).
tgx_status queue_slots(Decoder* d) {
    const size_t mb = (size_t)d->max_blocks;
    if (d->table_dirty) {
        std::memcpy(d->table_stage, d->table_host.data(), d->slots * mb * 4);
        TGX_TRY(stage_copy(d, d->table_mapped, d->table, d->slots * mb * 4));
    }
    for (int b = 0; b < d->rows; ++b) {
        const uint32_t slot = d->placement_host[d->rows + b];
        for (size_t i = 0; i < mb; ++i)
            d->row_table_host[b * mb + i] = slot < (uint32_t)d->slots ? d->table_host[slot * mb + i] : TGX_SPARE;
    }
    TGX_TRY(stage_copy(d, d->row_table_mapped, d->row_table, d->rows * mb * 4));
    d->table_dirty = false;
    d->rows_dirty = false;
    return TGX_OK;
}

// The placement's words staged and queued for the device (the caller has waited for the staging).
tgx_status queue_placement(Decoder* d) {
    const size_t R = (size_t)d->rows;
    std::memcpy(d->placement_stage, d->placement_host.data(), 2 * R * 4);
    TGX_TRY(stage_copy(d, d->placement_mapped, d->positions, R * 4));
    return stage_copy(d, d->placement_mapped + R, d->slot_of_row, R * 4);
}

}  // namespace

tgx_status sync_slots(Decoder* d) {
    if (!d->table_dirty && !d->rows_dirty) return TGX_OK;
    TGX_TRY(staging_wait(d));
    TGX_TRY(queue_slots(d));
    return staging_queued(d);
}

tgx_status decoder_create(Context* ctx, const tgx_shape* shape, const tgx_batch* batch, Decoder** out) {
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or output");
    Shape s;
    TGX_TRY(check_shape(shape, &s));
    TGX_HIP(hipSetDevice(ctx->device));
    auto* d = new Decoder();
    d->ctx = ctx;
    d->shape = s;
    tgx_status st = create_inner(d, batch);
    if (st != TGX_OK) {
        std::string msg = last_error_message;
        decoder_destroy(d);
        return fail(st, msg);
    }
    *out = d;
    return TGX_OK;
}

void decoder_destroy(Decoder* d) {
    if (!d) return;
    hipSetDevice(d->ctx->device);
    hipStreamSynchronize(d->ctx->stream);
    prefill_release(d);
    for (auto& [rows, p] : d->programs) {
        if (p.step) hipGraphExecDestroy(p.step);
        if (p.advance) hipGraphExecDestroy(p.advance);
    }
    if (d->ev_start) hipEventDestroy(d->ev_start);
    if (d->ev_end) hipEventDestroy(d->ev_end);
    if (d->ev_done) hipEventDestroy(d->ev_done);
    for (auto e : d->timer_start)
        if (e) hipEventDestroy(e);
    for (auto e : d->timer_stop)
        if (e) hipEventDestroy(e);
    for (auto& b : d->allocations) hipFree(b.ptr);
    if (d->x_host) hipHostFree(d->x_host);
    if (d->out_host) hipHostFree(d->out_host);
    if (d->ev_staged) hipEventDestroy(d->ev_staged);
    if (d->placement_stage) hipHostFree(d->placement_stage);
    if (d->table_stage) hipHostFree(d->table_stage);
    if (d->row_table_host) hipHostFree(d->row_table_host);
    delete d;
}

// The weight's values as f32, `count` of `dtype`.
std::vector<float> as_f32(const void* data, tgx_dtype dtype, size_t count) {
    std::vector<float> v(count);
    if (dtype == TGX_F32) {
        std::memcpy(v.data(), data, count * 4);
    } else {
        const uint16_t* h = (const uint16_t*)data;
        for (size_t i = 0; i < count; ++i) v[i] = dtype == TGX_BF16 ? bf16_to_f32(h[i]) : f16_to_f32(h[i]);
    }
    return v;
}

std::vector<uint16_t> tile_rows(const std::vector<float>& w, int n, int k, int R,
                                const std::function<int(int, int)>& row_of) {
    std::vector<uint16_t> t((size_t)n * k);
    const int kblocks = k / 32;
    for (int strip = 0; strip < n / R; ++strip)
        for (int kb = 0; kb < kblocks; ++kb) {
            uint16_t* dst = t.data() + weight_tile_index(strip, kb, kblocks, R);
            for (int lane = 0; lane < 64; ++lane) {
                if (lane % 16 >= R) continue;
                const int src_row = row_of(strip, lane % 16);
                const float* src = w.data() + (size_t)src_row * k + kb * 32 + (lane / 16) * 8;
                uint16_t* out = dst + weight_lane_offset(lane, R);
                for (int j = 0; j < 8; ++j) out[j] = f32_to_bf16(src[j]);
            }
        }
    return t;
}

tgx_status load_layer_tensor(Layer& L, const Shape& s, const std::string& name, const std::string& what,
                             const void* data, tgx_dtype dtype, size_t count, int o_rows, int down_rows) {
    const int h = s.hidden, I = s.inner, H = s.heads, KV = s.kv_heads, D = s.head_dim;
    const int qkv_rows = (H + 2 * KV) * D;
    auto want = [&](size_t expect) -> tgx_status {
        if (count != expect)
            return fail(TGX_E_WEIGHTS, name + ": " + std::to_string(count) + " values, not " + std::to_string(expect));
        return TGX_OK;
    };
    auto upload = [&](void* dst, const void* src, size_t bytes) -> tgx_status {
        TGX_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
        return TGX_OK;
    };
    if (what == "input_layernorm" || what == "post_attention_layernorm") {
        TGX_TRY(want(h));
        auto v = as_f32(data, dtype, count);
        return upload(what == "input_layernorm" ? L.input_norm : L.post_norm, v.data(), (size_t)h * 4);
    }
    if (what == "qkv_proj") {
        TGX_TRY(want((size_t)qkv_rows * h));
        auto t = tile_rows(as_f32(data, dtype, count), qkv_rows, h, QKV_ROWS,
                           [D](int strip, int r) { return qkv_row_of(strip, r, D, QKV_ROWS); });
        return upload(L.qkv, t.data(), t.size() * 2);
    }
    if (what == "o_proj") {
        TGX_TRY(want((size_t)h * H * D));
        auto t = tile_rows(as_f32(data, dtype, count), h, H * D, o_rows, [o_rows](int strip, int r) { return strip * o_rows + r; });
        return upload(L.o, t.data(), t.size() * 2);
    }
    if (what == "gate_up_proj") {
        TGX_TRY(want((size_t)2 * I * h));
        auto t = tile_rows(as_f32(data, dtype, count), 2 * I, h, 16, [](int strip, int r) { return strip * 16 + r; });
        return upload(L.gate_up, t.data(), t.size() * 2);
    }
    if (what == "down_proj") {
        TGX_TRY(want((size_t)h * I));
        auto t = tile_rows(as_f32(data, dtype, count), h, I, down_rows,
                           [down_rows](int strip, int r) { return strip * down_rows + r; });
        return upload(L.down, t.data(), t.size() * 2);
    }
    return fail(TGX_E_WEIGHTS, name + ": no such tensor");
}

tgx_status decoder_load(Decoder* d, const char* name, const void* data, tgx_dtype dtype, size_t count) {
    if (!d || !name || !data) return fail(TGX_E_ARG, "null decoder, name or data");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (dtype != TGX_F32 && dtype != TGX_BF16 && dtype != TGX_F16) return fail(TGX_E_ARG, "dtype");
    const Shape& s = d->shape;
    std::string n = name;
    if (n == "norm") {
        if (count != (size_t)s.hidden)
            return fail(TGX_E_WEIGHTS, n + ": " + std::to_string(count) + " values, not " + std::to_string(s.hidden));
        auto v = as_f32(data, dtype, count);
        TGX_HIP(hipMemcpy(d->final_norm, v.data(), (size_t)s.hidden * 4, hipMemcpyHostToDevice));
        return TGX_OK;
    }
    int l = -1;
    char what[128] = {0};
    if (std::sscanf(name, "layers.%d.%127s", &l, what) != 2 || l < 0 || l >= s.layers)
        return fail(TGX_E_WEIGHTS, n + ": no such tensor in a stack of " + std::to_string(s.layers) + " layers");
    return load_layer_tensor(d->layers[l], s, n, what, data, dtype, count, d->od_rows, d->od_rows);
}

namespace {

// The rows placed (checked, their slots' blocks held) and their placement and block tables
// queued for the device; the caller waits for the staging before and marks it after.
tgx_status place_rows(Decoder* d, const tgx_row* rows, int nrows) {
    if (!d || !rows) return fail(TGX_E_ARG, "null decoder or rows");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (nrows != d->rows)
        return fail(TGX_E_SHAPE, std::to_string(nrows) + " rows for a batch of " + std::to_string(d->rows));
    std::vector<uint32_t> words(2 * (size_t)nrows);
    TGX_TRY(placement(d->slots, d->shape.capacity, rows, nrows, words.data()));
    for (int b = 0; b < nrows; ++b) {
        const tgx_row r = rows[b];
        if (r.position == TGX_SPARE) continue;
        TGX_TRY(hold_slot(d, r.slot, r.position + 1));
    }
    std::copy(words.begin(), words.end(), d->placement_host.begin());
    d->rows_dirty = true;
    TGX_TRY(queue_slots(d));
    return queue_placement(d);
}

}  // namespace

tgx_status decoder_place(Decoder* d, const tgx_row* rows, int nrows) {
    if (!d) return fail(TGX_E_ARG, "null decoder");
    TGX_TRY(staging_wait(d));
    const tgx_status st = place_rows(d, rows, nrows);
    // Whatever was queued before a refusal is marked too.
    TGX_TRY(staging_queued(d));
    return st;
}

tgx_status decoder_use_rows(Decoder* d, int rows) {
    if (!d) return fail(TGX_E_ARG, "null decoder");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (rows < 1 || rows > d->max_rows)
        return fail(TGX_E_SHAPE, std::to_string(rows) + " rows in a batch of " + std::to_string(d->max_rows));
    if (rows == d->rows) return TGX_OK;
    const int before = d->rows;
    d->rows = rows;
    tgx_status st = use_program(d);
    if (st != TGX_OK) {
        d->rows = before;  // the program it had stays
        return st;
    }
    // Every row spare until placed again.
    std::fill(d->placement_host.begin(), d->placement_host.begin() + 2 * rows, TGX_SPARE);
    d->rows_dirty = true;
    TGX_TRY(staging_wait(d));
    TGX_TRY(queue_placement(d));
    return staging_queued(d);
}

tgx_status decoder_set_rows(Decoder* d, const tgx_row* rows, int nrows, const float* x) {
    if (!d || !rows || !x) return fail(TGX_E_ARG, "null decoder, rows or x");
    // One wait for the staging, then the placement, the tables and x queued behind one mark: the
    // step's own launch and wait follow them on the stream, so a step through host arrays makes
    // one round trip to the device.
    TGX_TRY(staging_wait(d));
    tgx_status st = place_rows(d, rows, nrows);
    if (st == TGX_OK) {
        std::memcpy(d->x_host, x, (size_t)nrows * d->shape.hidden * 4);
        st = stage_copy(d, d->x_mapped, d->x_in, (size_t)nrows * d->shape.hidden * 4);
    }
    TGX_TRY(staging_queued(d));
    return st;
}

tgx_status decoder_start(Decoder* d) {
    if (!d) return fail(TGX_E_ARG, "null decoder");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    hipStream_t s = d->ctx->stream;
    TGX_TRY(hold_ahead(d, 1, 0));
    TGX_TRY(sync_slots(d));
    TGX_HIP(hipEventRecord(d->ev_start, s));
    if (d->timed || !d->use_graph) {
        // Launched dispatch by dispatch, each timed by its own events when timed (Decoder::timings).
        d->timer.used = 0;
        hipError_t e = enqueue_step(d, 0, d->timed ? &d->timer : nullptr, nullptr);
        if (e != hipSuccess) return fail(TGX_E_HIP, std::string("launching the step: ") + hipGetErrorString(e));
    } else {
        TGX_HIP(hipGraphLaunch(d->step_exec, s));
    }
    TGX_HIP(hipEventRecord(d->ev_end, s));
    TGX_HIP(launch_copy_words(d->out, d->out_mapped, (size_t)d->rows * d->shape.hidden * 4, s));
    TGX_HIP(hipEventRecord(d->ev_done, s));
    d->pending = true;
    return TGX_OK;
}

tgx_status decoder_wait(Decoder* d) {
    if (!d) return fail(TGX_E_ARG, "null decoder");
    if (!d->pending) return TGX_OK;
    const tgx_status r = wait_event(d->ctx, d->ev_done, "the step");
    if (r != TGX_E_TIMEOUT) d->pending = false;
    return r;
}

tgx_status decoder_output(Decoder* d, float* out) {
    if (!d || !out) return fail(TGX_E_ARG, "null decoder or out");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    std::memcpy(out, d->out_host, (size_t)d->rows * d->shape.hidden * 4);
    return TGX_OK;
}

tgx_status decoder_release_slot(Decoder* d, uint32_t slot) {
    if (!d) return fail(TGX_E_ARG, "null decoder");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (slot >= (uint32_t)d->slots) return fail(TGX_E_SHAPE, "slot " + std::to_string(slot) + " of " + std::to_string(d->slots));
    for (int i = d->slot_blocks[slot] - 1; i >= 0; --i) {
        uint32_t& e = d->table_host[(size_t)slot * d->max_blocks + i];
        d->free_list.push_back(e);
        e = TGX_SPARE;
    }
    d->slot_blocks[slot] = 0;
    d->table_dirty = true;
    return TGX_OK;
}

tgx_status decoder_reserve(Decoder* d, uint32_t slot, uint32_t positions) {
    if (!d) return fail(TGX_E_ARG, "null decoder");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (slot >= (uint32_t)d->slots) return fail(TGX_E_SHAPE, "slot " + std::to_string(slot) + " of " + std::to_string(d->slots));
    if (positions > (uint32_t)d->shape.capacity)
        return fail(TGX_E_SHAPE, std::to_string(positions) + " positions past a capacity of " + std::to_string(d->shape.capacity));
    TGX_TRY(hold_slot(d, slot, positions));
    return sync_slots(d);
}

tgx_status decoder_launch(Decoder* d, int times, int advance) {
    if (!d) return fail(TGX_E_ARG, "null decoder");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (times <= 0) return fail(TGX_E_ARG, "times");
    hipStream_t s = d->ctx->stream;
    TGX_TRY(hold_ahead(d, times, advance));
    TGX_TRY(sync_slots(d));
    TGX_HIP(hipEventRecord(d->ev_start, s));
    for (int i = 0; i < times; ++i) {
        if (d->timed || !d->use_graph) {
            d->timer.used = 0;
            hipError_t e = enqueue_step(d, advance, d->timed ? &d->timer : nullptr, nullptr);
            if (e != hipSuccess) return fail(TGX_E_HIP, std::string("launching the step: ") + hipGetErrorString(e));
        } else {
            TGX_HIP(hipGraphLaunch(advance ? d->advance_exec : d->step_exec, s));
        }
        if (advance) moved_on(d, 1);
    }
    TGX_HIP(hipEventRecord(d->ev_end, s));
    TGX_HIP(hipEventRecord(d->ev_done, s));
    d->pending = true;
    return TGX_OK;
}

tgx_status decoder_read_cache(Decoder* d, uint32_t slot, uint32_t positions, float* k, float* v) {
    if (!d || !k || !v) return fail(TGX_E_ARG, "null argument");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (slot >= (uint32_t)d->slots || positions > (uint32_t)d->slot_blocks[slot] * BLOCK_TOKENS)
        return fail(TGX_E_SHAPE, "slot " + std::to_string(slot) + " holds fewer than " + std::to_string(positions) + " positions");
    const Shape& s = d->shape;
    const int KV = s.kv_heads, D = s.head_dim, TILE = kv_tile(D);
    std::vector<uint16_t> tilebuf(2 * TILE);
    TGX_HIP(hipStreamSynchronize(d->ctx->stream));
    for (int l = 0; l < s.layers; ++l)
        for (int kv = 0; kv < KV; ++kv)
            for (uint32_t p0 = 0; p0 < positions; p0 += BLOCK_TOKENS) {
                const uint32_t blk = d->table_host[(size_t)slot * d->max_blocks + p0 / BLOCK_TOKENS];
                const uint16_t* src = d->kv + (((size_t)l * d->nblocks + blk) * KV + kv) * 2 * TILE;
                TGX_HIP(hipMemcpy(tilebuf.data(), src, 2 * TILE * 2, hipMemcpyDeviceToHost));
                for (uint32_t p = p0; p < positions && p < p0 + BLOCK_TOKENS; ++p)
                    for (int dd = 0; dd < D; ++dd) {
                        const size_t at = (((size_t)l * KV + kv) * positions + p) * D + dd;
                        k[at] = bf16_to_f32(tilebuf[key_index((int)(p - p0), dd, D)]);
                        v[at] = bf16_to_f32(tilebuf[TILE + value_index((int)(p - p0), dd)]);
                    }
            }
    return TGX_OK;
}

tgx_status decoder_timings(Decoder* d, int max, tgx_timing* out, int* n) {
    if (!d || !n) return fail(TGX_E_ARG, "null decoder or count");
    if (d->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (!d->timed) {
        *n = 0;
        return TGX_OK;
    }
    const int used = d->timer.used;
    *n = used;
    for (int i = 0; i < used && i < max && out; ++i) {
        float ms = 0.f;
        TGX_HIP(hipEventElapsedTime(&ms, d->timer.start[i], d->timer.stop[i]));
        std::snprintf(out[i].label, sizeof out[i].label, "%s", d->timer.labels[i]);
        out[i].ms = ms;
    }
    return TGX_OK;
}

}  // namespace tgx
