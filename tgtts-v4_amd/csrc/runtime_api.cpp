// The runtime beneath the models (include/tgx.h, tgx_alloc .. tgx_copy_regions): memory in a
// residence (crates/vulkan/src/memory.rs), the decode step's kernels by name with their bindings
// in order (crates/graph/src/kernels.rs:27-161), and programs of dispatches recorded as HIP graphs
// and run as often as needed (crates/vulkan/src/recording.rs:116-760).
//
// A dispatch is checked on the host before anything is recorded: every binding it must have is
// there, of its kernel's element size and alignment, and holds every byte the kernel reaches for
// the dispatch's constants, so that no recorded kernel reads or writes past a binding.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "handles.hpp"
#include "runtime.hpp"

struct tgx_memory {
    tgx::Context* ctx = nullptr;
    void* ptr = nullptr;
    uint64_t bytes = 0;
    tgx_residence residence = TGX_DEVICE;
    int programs = 0;  // programs that bind it
    int running = 0;   // of those, started and not yet waited for
};

namespace tgx {
namespace {

struct BindingInfo {
    const char* name;
    tgx_access access;
    tgx_dtype element;
    bool optional;
};

// A dispatch's bindings, resolved: each one's address and bytes (null and 0 when left out).
struct Bound {
    void* ptr = nullptr;
    uint64_t bytes = 0;
};

// A dispatch ready to launch: the kernel, its grid and LDS, and the arguments it takes, kept where
// `params` points for as long as the program lives.
struct Launch {
    const char* name = nullptr;
    KernelLaunch k;
    DecodeArgs a{};
    LayerArgs l{};
    ResidualArgs r{};
    const void* in0 = nullptr;
    const void* in1 = nullptr;
    void* out0 = nullptr;
    void* out1 = nullptr;
    int advance = 0;
    void* params[6] = {};
};

using Builder = tgx_status (*)(const Bound* b, const uint32_t* c, Launch* out);

struct KernelDesc {
    const char* name;
    std::vector<BindingInfo> bindings;
    std::vector<const char*> constants;
    Builder build;
};

size_t element_bytes(tgx_dtype e) { return e == TGX_BF16 || e == TGX_F16 ? 2 : 4; }

float as_float(uint32_t bits) {
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// The constants every decode kernel takes first, in order.
constexpr int C_HIDDEN = 0, C_INNER = 1, C_HEADS = 2, C_KV = 3, C_ROWS = 4, C_CAPACITY = 5, C_SLOTS = 6, C_MAX_BLOCKS = 7,
              C_BLOCKS = 8, C_EPS = 9, C_ROPE = 10, C_HEAD_DIM = 11, C_COMMON = 12;
std::vector<const char*> decode_constants(std::vector<const char*> own = {}) {
    std::vector<const char*> c = {"hidden", "inner", "heads", "kv_heads", "rows", "capacity", "slots", "max_blocks", "blocks",
                                  "eps", "rope", "head_dim"};
    c.insert(c.end(), own.begin(), own.end());
    return c;
}

// The shape and placement constants as the kernels take them, refused as tgx_decoder_create
// refuses a shape and a batch; the placement's tables are bound by the kernels that read them.
tgx_status decode_args(const uint32_t* c, DecodeArgs* a) {
    tgx_shape in{};
    in.hidden = (int)c[C_HIDDEN];
    in.inner = (int)c[C_INNER];
    in.heads = (int)c[C_HEADS];
    in.kv_heads = (int)c[C_KV];
    in.head_dim = (int)c[C_HEAD_DIM];
    in.layers = 1;
    in.capacity = (int)c[C_CAPACITY];
    in.eps = as_float(c[C_EPS]);
    in.rope_theta = 10000.f;
    in.rope = c[C_ROPE] != 0;
    Shape s;
    TGX_TRY(check_shape(&in, &s));
    tgx_batch batch{(int)c[C_ROWS], (int)c[C_SLOTS], BLOCK_TOKENS, (int)c[C_BLOCKS]};
    if ((int)c[C_ROWS] <= 0 || c[C_ROWS] > 64) return fail(TGX_E_SHAPE, "rows " + std::to_string(c[C_ROWS]) + ": 1 to 64");
    TGX_TRY(check_batch(s, &batch));
    const uint32_t need = (c[C_CAPACITY] + BLOCK_TOKENS - 1) / BLOCK_TOKENS;
    if (c[C_MAX_BLOCKS] < need || c[C_BLOCKS] == 0 || c[C_SLOTS] == 0 || c[C_MAX_BLOCKS] > (1u << 20) || c[C_BLOCKS] > (1u << 24) ||
        c[C_SLOTS] > (1u << 16))
        return fail(TGX_E_SHAPE, std::to_string(c[C_SLOTS]) + " slots of " + std::to_string(c[C_MAX_BLOCKS]) +
                                     " blocks in a pool of " + std::to_string(c[C_BLOCKS]) + " (a slot's table holds " +
                                     std::to_string(need) + " blocks at the capacity)");
    if (c[C_ROPE] > 1) return fail(TGX_E_SHAPE, "rope is 0 or 1");
    *a = DecodeArgs{};
    a->hidden = s.hidden;
    a->inner = s.inner;
    a->heads = s.heads;
    a->kv_heads = s.kv_heads;
    a->head_dim = s.head_dim;
    a->rows = (int)c[C_ROWS];
    a->capacity = s.capacity;
    a->nslots = (int)c[C_SLOTS];
    a->max_blocks = (int)c[C_MAX_BLOCKS];
    a->nblocks = (int)c[C_BLOCKS];
    a->eps = s.eps;
    a->scale = 1.0f / std::sqrt((float)s.head_dim);
    a->rope = (int)c[C_ROPE];
    return TGX_OK;
}

// Refuses binding `i` (`what`) when it holds fewer than `need` bytes.
tgx_status holds(const Bound* b, int i, const char* what, uint64_t need) {
    if (b[i].bytes < need)
        return fail(TGX_E_SHAPE, std::string(what) + ": a binding of " + std::to_string(b[i].bytes) + " bytes where the kernel reaches " +
                                     std::to_string(need));
    return TGX_OK;
}

uint64_t pool_bytes(const DecodeArgs& a) { return (uint64_t)a.nblocks * a.kv_heads * 2 * kv_tile(a.head_dim) * 2; }
uint64_t qkv_rows(const DecodeArgs& a) { return (uint64_t)(a.heads + 2 * a.kv_heads) * a.head_dim; }

// gemv_qkv_rope (gemv_qkv_rope.comp): x | (xn, x_sq), gain, W, cos, sin, positions, slots, table
// -> q, cache pool.
tgx_status build_qkv(const Bound* b, const uint32_t* c, Launch* L) {
    DecodeArgs a;
    TGX_TRY(decode_args(c, &a));
    const uint64_t R = a.rows, h = a.hidden;
    const bool prenormed = b[1].ptr != nullptr;
    if (prenormed == (b[0].ptr != nullptr) || prenormed != (b[2].ptr != nullptr))
        return fail(TGX_E_SHAPE, "gemv_qkv_rope takes x, or xn with x_sq");
    if (prenormed) {
        TGX_TRY(holds(b, 1, "xn", R * h * 2));
        TGX_TRY(holds(b, 2, "x_sq", R * (h / 4) * 4));
    } else {
        TGX_TRY(holds(b, 0, "x", R * h * 4));
    }
    TGX_TRY(holds(b, 3, "gain", h * 4));
    TGX_TRY(holds(b, 4, "w", qkv_rows(a) * h * 2));
    TGX_TRY(holds(b, 5, "cos", (uint64_t)a.capacity * (a.head_dim / 2) * 4));
    TGX_TRY(holds(b, 6, "sin", (uint64_t)a.capacity * (a.head_dim / 2) * 4));
    TGX_TRY(holds(b, 7, "positions", R * 4));
    TGX_TRY(holds(b, 8, "slots", R * 4));
    TGX_TRY(holds(b, 9, "table", (uint64_t)a.nslots * a.max_blocks * 4));
    TGX_TRY(holds(b, 10, "q", R * a.heads * a.head_dim * 2));
    TGX_TRY(holds(b, 11, "kv", pool_bytes(a)));
    a.positions = (const uint32_t*)b[7].ptr;
    a.slots = (const uint32_t*)b[8].ptr;
    a.table = (const uint32_t*)b[9].ptr;
    a.cos = (const float*)b[5].ptr;
    a.sin = (const float*)b[6].ptr;
    LayerArgs l{};
    l.x = (const float*)b[0].ptr;
    l.xn = (const uint16_t*)b[1].ptr;
    l.x_sq = (const float*)b[2].ptr;
    l.input_norm = (const float*)b[3].ptr;
    l.qkv = (const uint16_t*)b[4].ptr;
    l.q = (uint16_t*)b[10].ptr;
    l.kv = (uint16_t*)b[11].ptr;
    L->a = a;
    L->l = l;
    L->k = qkv_launch(a, prenormed);
    L->params[0] = &L->a;
    L->params[1] = &L->l;
    return TGX_OK;
}

// attention_decode (attention_split.comp + attention_combine.comp): q, cache pool, positions,
// row_table -> attended.
tgx_status build_attention(const Bound* b, const uint32_t* c, Launch* L) {
    DecodeArgs a;
    TGX_TRY(decode_args(c, &a));
    const uint64_t R = a.rows;
    TGX_TRY(holds(b, 0, "q", R * a.heads * a.head_dim * 2));
    TGX_TRY(holds(b, 1, "kv", pool_bytes(a)));
    TGX_TRY(holds(b, 2, "positions", R * 4));
    TGX_TRY(holds(b, 3, "row_table", R * a.max_blocks * 4));
    TGX_TRY(holds(b, 4, "attended", R * a.heads * a.head_dim * 2));
    a.positions = (const uint32_t*)b[2].ptr;
    a.row_table = (const uint32_t*)b[3].ptr;
    LayerArgs l{};
    l.q = (uint16_t*)b[0].ptr;
    l.kv = (uint16_t*)b[1].ptr;
    l.attended = (uint16_t*)b[4].ptr;
    L->a = a;
    L->l = l;
    L->k = attention_launch(a);
    L->params[0] = &L->a;
    L->params[1] = &L->l;
    return TGX_OK;
}

// gemv_residual (gemv_residual.comp): x, W, residual [, next_gain] -> out [, out_n, out_sq];
// constants K, N, strip_rows (4 or 16: W's tiles) past the common ones.
tgx_status build_residual(const Bound* b, const uint32_t* c, Launch* L) {
    DecodeArgs a;
    TGX_TRY(decode_args(c, &a));
    const int K = (int)c[C_COMMON], N = (int)c[C_COMMON + 1], Rs = (int)c[C_COMMON + 2];
    if (K <= 0 || K % 1024 != 0 || K > decode_max_k() || N <= 0 || N % 16 != 0 || N > (1 << 16) || (Rs != 4 && Rs != 16))
        return fail(TGX_E_SHAPE, "gemv_residual: K " + std::to_string(K) + " (a multiple of 1024 up to " +
                                     std::to_string(decode_max_k()) + "), N " + std::to_string(N) + " (a multiple of 16), strips of " +
                                     std::to_string(Rs) + " rows (4 or 16)");
    const bool norm = b[3].ptr != nullptr;
    if (norm != (b[5].ptr != nullptr) || norm != (b[6].ptr != nullptr))
        return fail(TGX_E_SHAPE, "gemv_residual takes next_gain, out_n and out_sq together or none of them");
    const uint64_t R = a.rows;
    TGX_TRY(holds(b, 0, "x", R * K * 2));
    TGX_TRY(holds(b, 1, "w", (uint64_t)N * K * 2));
    TGX_TRY(holds(b, 2, "residual", R * N * 4));
    TGX_TRY(holds(b, 4, "out", R * N * 4));
    if (norm) {
        TGX_TRY(holds(b, 3, "next_gain", (uint64_t)N * 4));
        TGX_TRY(holds(b, 5, "out_n", R * N * 2));
        TGX_TRY(holds(b, 6, "out_sq", R * (N / 4) * 4));
    }
    ResidualArgs r{};
    r.x = (const uint16_t*)b[0].ptr;
    r.w = (const uint16_t*)b[1].ptr;
    r.residual = (const float*)b[2].ptr;
    r.next_norm = (const float*)b[3].ptr;
    r.out = (float*)b[4].ptr;
    r.out_n = (uint16_t*)b[5].ptr;
    r.out_sq = (float*)b[6].ptr;
    r.K = K;
    r.N = N;
    r.R = Rs;
    L->a = a;
    L->r = r;
    L->k = residual_launch(a, r);
    L->params[0] = &L->a;
    L->params[1] = &L->r;
    return TGX_OK;
}

// gemv_gate_up (gemv_gate_up.comp): mid_n, mid_sq, W -> mlp.
tgx_status build_gate_up(const Bound* b, const uint32_t* c, Launch* L) {
    DecodeArgs a;
    TGX_TRY(decode_args(c, &a));
    const uint64_t R = a.rows, h = a.hidden;
    TGX_TRY(holds(b, 0, "mid_n", R * h * 2));
    TGX_TRY(holds(b, 1, "mid_sq", R * (h / 4) * 4));
    TGX_TRY(holds(b, 2, "w", 2 * (uint64_t)a.inner * h * 2));
    TGX_TRY(holds(b, 3, "mlp", R * a.inner * 2));
    LayerArgs l{};
    l.mid_n = (const uint16_t*)b[0].ptr;
    l.mid_sq = (const float*)b[1].ptr;
    l.gate_up = (const uint16_t*)b[2].ptr;
    l.mlp = (uint16_t*)b[3].ptr;
    L->a = a;
    L->l = l;
    L->k = gate_up_launch(a);
    L->params[0] = &L->a;
    L->params[1] = &L->l;
    return TGX_OK;
}

// rmsnorm (rmsnorm.comp): x, gain -> out [, positions moved on by one]; constant advance.
tgx_status build_rmsnorm(const Bound* b, const uint32_t* c, Launch* L) {
    DecodeArgs a;
    TGX_TRY(decode_args(c, &a));
    const uint64_t R = a.rows, h = a.hidden;
    const uint32_t advance = c[C_COMMON];
    if (advance > 1) return fail(TGX_E_SHAPE, "advance is 0 or 1");
    if (advance && !b[3].ptr) return fail(TGX_E_SHAPE, "rmsnorm moves the rows on only with their positions bound");
    TGX_TRY(holds(b, 0, "x", R * h * 4));
    TGX_TRY(holds(b, 1, "gain", h * 4));
    TGX_TRY(holds(b, 2, "out", R * h * 4));
    if (b[3].ptr) TGX_TRY(holds(b, 3, "positions", R * 4));
    L->a = a;
    L->in0 = b[0].ptr;
    L->in1 = b[1].ptr;
    L->out0 = b[2].ptr;
    L->out1 = b[3].ptr;
    L->advance = (int)advance;
    L->k = final_norm_launch(a);
    L->params[0] = &L->a;
    L->params[1] = &L->in0;
    L->params[2] = &L->in1;
    L->params[3] = &L->out0;
    L->params[4] = &L->out1;
    L->params[5] = &L->advance;
    return TGX_OK;
}

// stream_read (stream_read.comp): data -> one word a wave; the data binding's bytes, a multiple
// of the kernel's unit, are what it reads.
tgx_status build_stream_read(const Bound* b, const uint32_t*, Launch* L) {
    const uint64_t unit = stream_read_unit();
    if (b[0].bytes == 0 || b[0].bytes % unit != 0 || b[0].bytes / unit > (1u << 31))
        return fail(TGX_E_SHAPE, "stream_read reads a multiple of " + std::to_string(unit) + " bytes, not " + std::to_string(b[0].bytes));
    const KernelLaunch k = stream_read_launch(b[0].bytes);
    TGX_TRY(holds(b, 1, "out", (uint64_t)k.grid.x * (k.block.x / 64) * 4));
    L->in0 = b[0].ptr;
    L->out0 = b[1].ptr;
    L->k = k;
    L->params[0] = &L->in0;
    L->params[1] = &L->out0;
    return TGX_OK;
}

constexpr tgx_access RD = TGX_READ, WR = TGX_WRITE;

const std::vector<KernelDesc>& kernels() {
    static const std::vector<KernelDesc> table = {
        {"gemv_qkv_rope",
         {{"x", RD, TGX_F32, true},
          {"xn", RD, TGX_BF16, true},
          {"x_sq", RD, TGX_F32, true},
          {"gain", RD, TGX_F32, false},
          {"w", RD, TGX_BF16, false},
          {"cos", RD, TGX_F32, false},
          {"sin", RD, TGX_F32, false},
          {"positions", RD, TGX_U32, false},
          {"slots", RD, TGX_U32, false},
          {"table", RD, TGX_U32, false},
          {"q", WR, TGX_BF16, false},
          {"kv", WR, TGX_BF16, false}},
         decode_constants(),
         build_qkv},
        {"attention_decode",
         {{"q", RD, TGX_BF16, false},
          {"kv", RD, TGX_BF16, false},
          {"positions", RD, TGX_U32, false},
          {"row_table", RD, TGX_U32, false},
          {"attended", WR, TGX_BF16, false}},
         decode_constants(),
         build_attention},
        {"gemv_residual",
         {{"x", RD, TGX_BF16, false},
          {"w", RD, TGX_BF16, false},
          {"residual", RD, TGX_F32, false},
          {"next_gain", RD, TGX_F32, true},
          {"out", WR, TGX_F32, false},
          {"out_n", WR, TGX_BF16, true},
          {"out_sq", WR, TGX_F32, true}},
         decode_constants({"K", "N", "strip_rows"}),
         build_residual},
        {"gemv_gate_up",
         {{"mid_n", RD, TGX_BF16, false}, {"mid_sq", RD, TGX_F32, false}, {"w", RD, TGX_BF16, false}, {"mlp", WR, TGX_BF16, false}},
         decode_constants(),
         build_gate_up},
        {"rmsnorm",
         {{"x", RD, TGX_F32, false}, {"gain", RD, TGX_F32, false}, {"out", WR, TGX_F32, false}, {"positions", WR, TGX_U32, true}},
         decode_constants({"advance"}),
         build_rmsnorm},
        {"stream_read", {{"data", RD, TGX_U32, false}, {"out", WR, TGX_U32, false}}, {}, build_stream_read},
    };
    return table;
}

const KernelDesc* kernel_at(int i) { return i >= 0 && i < (int)kernels().size() ? &kernels()[i] : nullptr; }

// What the weights' tiles take: strips of 16 (or 4) rows, 32 columns a k-block.
int tile_height(tgx_tiles t) { return t == TGX_TILES_4 ? 4 : 16; }
// The head width of q/k/v rows in tiles of `t`: 64 or 128, 0 for rows of no heads.
int tiles_head_dim(tgx_tiles t) { return t == TGX_TILES_QKV ? 64 : t == TGX_TILES_QKV128 ? 128 : 0; }
bool tiles_hold(tgx_tiles t, int rows, int cols) {
    if (t != TGX_TILES_16 && t != TGX_TILES_4 && t != TGX_TILES_QKV && t != TGX_TILES_QKV128) return false;
    if (rows <= 0 || cols <= 0 || rows % tile_height(t) != 0 || cols % 32 != 0) return false;
    if (tiles_head_dim(t) && rows % tiles_head_dim(t) != 0) return false;
    return (uint64_t)rows * cols <= (1ull << 31);
}

}  // namespace

// A program: its dispatches as launches, the graph they are recorded into, and how it runs.
struct Program {
    Context* ctx = nullptr;
    bool timed = false, ended = false, pending = false;
    std::vector<std::unique_ptr<Launch>> launches;
    std::vector<tgx_memory*> memories;  // one entry per binding of a dispatch
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<hipGraphNode_t> nodes, frontier, after;  // after: what every dispatch now waits for
    hipEvent_t ev_start = nullptr, ev_end = nullptr;
    std::vector<hipEvent_t> t_start, t_stop;
    bool timings_valid = false;
};

}  // namespace tgx

struct tgx_program {
    tgx::Program* p;
};

using namespace tgx;

extern "C" {

tgx_status tgx_alloc(tgx_context* ctx, uint64_t bytes, tgx_residence residence, tgx_memory** out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or out");
    *out = nullptr;
    if (bytes == 0) return fail(TGX_E_SHAPE, "memory of 0 bytes");
    if (residence != TGX_DEVICE && residence != TGX_UPLOAD && residence != TGX_READBACK) return fail(TGX_E_ARG, "residence");
    void* p = nullptr;
    if (residence == TGX_DEVICE) {
        TGX_HIP(hipMalloc(&p, bytes));
        hipError_t e = hipMemset(p, 0, bytes);
        if (e != hipSuccess) {
            hipFree(p);
            return fail(TGX_E_HIP, std::string("hipMemset: ") + hipGetErrorString(e));
        }
    } else {
        TGX_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault));
        std::memset(p, 0, bytes);
    }
    auto* m = new tgx_memory();
    m->ctx = ctx->ctx;
    m->ptr = p;
    m->bytes = bytes;
    m->residence = residence;
    *out = m;
    return TGX_OK;
}

tgx_status tgx_free(tgx_memory* mem) {
    clear_error();
    if (!mem) return TGX_OK;
    if (mem->programs > 0)
        return fail(TGX_E_BUSY, std::to_string(mem->programs) + " program(s) bind this memory: destroy them first");
    hipError_t e = mem->residence == TGX_DEVICE ? hipFree(mem->ptr) : hipHostFree(mem->ptr);
    delete mem;
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string("freeing memory: ") + hipGetErrorString(e));
    return TGX_OK;
}

tgx_status tgx_memory_info(const tgx_memory* mem, uint64_t* bytes, tgx_residence* residence) {
    clear_error();
    if (!mem) return fail(TGX_E_ARG, "null memory");
    if (bytes) *bytes = mem->bytes;
    if (residence) *residence = mem->residence;
    return TGX_OK;
}

static tgx_status host_access(tgx_memory* mem, uint64_t offset, const void* host, uint64_t bytes) {
    if (!mem || (!host && bytes)) return fail(TGX_E_ARG, "null memory or host array");
    if (offset > mem->bytes || bytes > mem->bytes - offset)
        return fail(TGX_E_SHAPE, std::to_string(bytes) + " bytes at " + std::to_string(offset) + " of memory of " +
                                     std::to_string(mem->bytes));
    if (mem->running > 0) return fail(TGX_E_BUSY, "a program that binds this memory runs");
    return TGX_OK;
}

tgx_status tgx_write(tgx_memory* mem, uint64_t offset, const void* src, uint64_t bytes) {
    clear_error();
    TGX_TRY(host_access(mem, offset, src, bytes));
    if (bytes == 0) return TGX_OK;
    hipStream_t s = mem->ctx->stream;
    TGX_HIP(hipStreamSynchronize(s));  // what the context's stream has queued may read it
    if (mem->residence == TGX_DEVICE) {
        TGX_HIP(hipMemcpyAsync((char*)mem->ptr + offset, src, bytes, hipMemcpyHostToDevice, s));
        TGX_HIP(hipStreamSynchronize(s));
    } else {
        std::memcpy((char*)mem->ptr + offset, src, bytes);
    }
    return TGX_OK;
}

tgx_status tgx_read(tgx_memory* mem, uint64_t offset, void* dst, uint64_t bytes) {
    clear_error();
    TGX_TRY(host_access(mem, offset, dst, bytes));
    if (bytes == 0) return TGX_OK;
    hipStream_t s = mem->ctx->stream;
    TGX_HIP(hipStreamSynchronize(s));
    if (mem->residence == TGX_DEVICE) {
        TGX_HIP(hipMemcpyAsync(dst, (const char*)mem->ptr + offset, bytes, hipMemcpyDeviceToHost, s));
        TGX_HIP(hipStreamSynchronize(s));
    } else {
        std::memcpy(dst, (const char*)mem->ptr + offset, bytes);
    }
    return TGX_OK;
}

uint64_t tgx_tiles_bytes(tgx_tiles tiles, int rows, int cols) {
    return tiles_hold(tiles, rows, cols) ? (uint64_t)rows * cols * 2 : 0;
}

tgx_status tgx_write_tiles(tgx_memory* mem, uint64_t offset, const void* src, tgx_dtype dtype, tgx_tiles tiles, int rows,
                           int cols) {
    clear_error();
    if (!mem || !src) return fail(TGX_E_ARG, "null memory or source");
    if (dtype != TGX_F32 && dtype != TGX_BF16 && dtype != TGX_F16) return fail(TGX_E_ARG, "dtype");
    if (!tiles_hold(tiles, rows, cols))
        return fail(TGX_E_SHAPE, std::to_string(rows) + " x " + std::to_string(cols) + " in tiles of " +
                                     std::to_string(tile_height(tiles)) + "-row strips and 32-column k-blocks" +
                                     (tiles_head_dim(tiles) ? " (rows a multiple of " + std::to_string(tiles_head_dim(tiles)) + ")"
                                                            : std::string()));
    const int R = tile_height(tiles), D = tiles_head_dim(tiles);
    std::vector<uint16_t> t;
    if (D)
        t = tile_rows(as_f32(src, dtype, (size_t)rows * cols), rows, cols, R,
                      [D](int strip, int r) { return qkv_row_of(strip, r, D, QKV_ROWS); });
    else
        t = tile_rows(as_f32(src, dtype, (size_t)rows * cols), rows, cols, R, [R](int strip, int r) { return strip * R + r; });
    return tgx_write(mem, offset, t.data(), (uint64_t)t.size() * 2);
}

tgx_status tgx_rope_tables(const tgx_shape* shape, float* cos, float* sin) {
    clear_error();
    if (!cos || !sin) return fail(TGX_E_ARG, "null tables");
    Shape s;
    TGX_TRY(check_shape(shape, &s));
    std::vector<float> c, si;
    rope_tables(s, c, si);
    std::memcpy(cos, c.data(), c.size() * 4);
    std::memcpy(sin, si.data(), si.size() * 4);
    return TGX_OK;
}

int tgx_kernel_count(void) { return (int)kernels().size(); }

tgx_status tgx_kernel_find(const char* name, int* kernel) {
    clear_error();
    if (!name || !kernel) return fail(TGX_E_ARG, "null name or out");
    for (int i = 0; i < (int)kernels().size(); ++i)
        if (std::strcmp(kernels()[i].name, name) == 0) {
            *kernel = i;
            return TGX_OK;
        }
    return fail(TGX_E_KERNELS, std::string("no kernel called ") + name);
}

tgx_status tgx_kernel_info(int kernel, const char** name, int* bindings, int* constants) {
    clear_error();
    const KernelDesc* k = kernel_at(kernel);
    if (!k) return fail(TGX_E_KERNELS, "kernel " + std::to_string(kernel) + " of " + std::to_string(kernels().size()));
    if (name) *name = k->name;
    if (bindings) *bindings = (int)k->bindings.size();
    if (constants) *constants = (int)k->constants.size();
    return TGX_OK;
}

tgx_status tgx_kernel_binding(int kernel, int i, tgx_binding_info* out) {
    clear_error();
    const KernelDesc* k = kernel_at(kernel);
    if (!k || !out || i < 0 || i >= (int)k->bindings.size()) return fail(TGX_E_ARG, "no such kernel or binding");
    const BindingInfo& b = k->bindings[i];
    std::memset(out, 0, sizeof(*out));
    std::strncpy(out->name, b.name, sizeof(out->name) - 1);
    out->access = b.access;
    out->element = b.element;
    out->optional = b.optional ? 1 : 0;
    return TGX_OK;
}

tgx_status tgx_kernel_constant(int kernel, int i, const char** name) {
    clear_error();
    const KernelDesc* k = kernel_at(kernel);
    if (!k || !name || i < 0 || i >= (int)k->constants.size()) return fail(TGX_E_ARG, "no such kernel or constant");
    *name = k->constants[i];
    return TGX_OK;
}

tgx_status tgx_program_begin(tgx_context* ctx, int timed, tgx_program** out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or out");
    *out = nullptr;
    auto* p = new Program();
    p->ctx = ctx->ctx;
    p->timed = timed != 0;
    hipError_t e = hipGraphCreate(&p->graph, 0);
    if (e == hipSuccess) e = hipEventCreate(&p->ev_start);
    if (e == hipSuccess) e = hipEventCreate(&p->ev_end);
    if (e != hipSuccess) {
        if (p->ev_start) hipEventDestroy(p->ev_start);
        if (p->graph) hipGraphDestroy(p->graph);
        delete p;
        return fail(TGX_E_HIP, std::string("starting a program: ") + hipGetErrorString(e));
    }
    *out = new tgx_program{p};
    return TGX_OK;
}

tgx_status tgx_program_launch(tgx_program* prog, const tgx_dispatch* d) {
    clear_error();
    if (!prog || !d) return fail(TGX_E_ARG, "null program or dispatch");
    Program* p = prog->p;
    if (p->ended) return fail(TGX_E_BUSY, "the program is recorded: it takes no more dispatches");
    const KernelDesc* k = kernel_at(d->kernel);
    if (!k) return fail(TGX_E_KERNELS, "kernel " + std::to_string(d->kernel) + " of " + std::to_string(kernels().size()));
    const std::string who = std::string(k->name) + ": ";
    if (d->nbindings != (int)k->bindings.size() || (d->nbindings && !d->bindings))
        return fail(TGX_E_SHAPE, who + std::to_string(d->nbindings) + " bindings for a kernel that binds " + std::to_string(k->bindings.size()));
    if (d->nconstants != (int)k->constants.size() || (d->nconstants && !d->constants))
        return fail(TGX_E_SHAPE, who + std::to_string(d->nconstants) + " constants for a kernel that takes " + std::to_string(k->constants.size()));
    // recording.rs binding_range: inside the memory, aligned to the element and not empty.
    std::vector<Bound> bound(k->bindings.size());
    std::vector<tgx_memory*> used;
    for (size_t i = 0; i < k->bindings.size(); ++i) {
        const tgx_binding& b = d->bindings[i];
        const BindingInfo& info = k->bindings[i];
        if (!b.memory) {
            if (!info.optional) return fail(TGX_E_SHAPE, who + "binding " + info.name + " is not optional");
            continue;
        }
        if (b.memory->ctx != p->ctx) return fail(TGX_E_ARG, who + "binding " + info.name + ": memory of another context");
        const uint64_t size = b.size ? b.size : (b.offset < b.memory->bytes ? b.memory->bytes - b.offset : 0);
        const uint64_t align = std::max<uint64_t>(element_bytes(info.element), 16);
        if (size == 0 || b.offset > b.memory->bytes || size > b.memory->bytes - b.offset)
            return fail(TGX_E_SHAPE, who + "binding " + info.name + ": " + std::to_string(size) + " bytes from " +
                                         std::to_string(b.offset) + " of a memory of " + std::to_string(b.memory->bytes));
        if (b.offset % align != 0)
            return fail(TGX_E_SHAPE, who + "binding " + info.name + " at offset " + std::to_string(b.offset) + ", not a multiple of " +
                                         std::to_string(align));
        bound[i] = {(char*)b.memory->ptr + b.offset, size};
        used.push_back(b.memory);
    }
    auto L = std::make_unique<Launch>();
    L->name = k->name;
    TGX_TRY(k->build(bound.data(), d->constants, L.get()));
    if (!L->k.func) return fail(TGX_E_KERNELS, who + "no instance for these constants");
    const bool derive = d->groups[0] == 0 && d->groups[1] == 0 && d->groups[2] == 0;
    if (!derive && (d->groups[0] != L->k.grid.x || d->groups[1] != L->k.grid.y || d->groups[2] != L->k.grid.z))
        return fail(TGX_E_SHAPE, who + "a grid of " + std::to_string(d->groups[0]) + " x " + std::to_string(d->groups[1]) + " x " +
                                     std::to_string(d->groups[2]) + " where the kernel takes " + std::to_string(L->k.grid.x) + " x " +
                                     std::to_string(L->k.grid.y) + " x " + std::to_string(L->k.grid.z));
    if (L->k.lds > p->ctx->lds_bytes) return fail(TGX_E_SHAPE, who + std::to_string(L->k.lds) + " bytes of LDS");
    // The graph: a barrier waits for everything recorded so far, every dispatch for what the last
    // barrier waited for (recording.rs Dispatch::barrier).
    if (d->barrier) {
        p->after = p->frontier;
        p->frontier.clear();
    }
    hipKernelNodeParams np{};
    np.func = const_cast<void*>(L->k.func);
    np.gridDim = L->k.grid;
    np.blockDim = L->k.block;
    np.sharedMemBytes = L->k.lds;
    np.kernelParams = L->params;
    np.extra = nullptr;
    hipGraphNode_t node = nullptr;
    TGX_HIP(hipGraphAddKernelNode(&node, p->graph, p->after.data(), p->after.size(), &np));
    p->nodes.push_back(node);
    p->frontier.push_back(node);
    for (tgx_memory* m : used) {
        ++m->programs;
        p->memories.push_back(m);
    }
    p->launches.push_back(std::move(L));
    return TGX_OK;
}

tgx_status tgx_program_end(tgx_program* prog) {
    clear_error();
    if (!prog) return fail(TGX_E_ARG, "null program");
    Program* p = prog->p;
    if (p->ended) return TGX_OK;
    if (p->launches.empty()) return fail(TGX_E_SHAPE, "a program of no dispatches");
    if (!p->timed) {
        TGX_HIP(hipGraphInstantiate(&p->exec, p->graph, nullptr, nullptr, 0));
        TGX_TRY(upload_graph(p->exec, p->ctx->stream));
    }
    if (p->timed) {
        p->t_start.assign(p->launches.size(), nullptr);
        p->t_stop.assign(p->launches.size(), nullptr);
        for (size_t i = 0; i < p->launches.size(); ++i) {
            TGX_HIP(hipEventCreate(&p->t_start[i]));
            TGX_HIP(hipEventCreate(&p->t_stop[i]));
        }
    }
    p->ended = true;
    return TGX_OK;
}

tgx_status tgx_program_start(tgx_program* prog) {
    clear_error();
    if (!prog) return fail(TGX_E_ARG, "null program");
    Program* p = prog->p;
    if (!p->ended) return fail(TGX_E_BUSY, "the program is still recording: tgx_program_end first");
    if (p->pending) return fail(TGX_E_BUSY, "the program runs");
    hipStream_t s = p->ctx->stream;
    TGX_HIP(hipEventRecord(p->ev_start, s));
    if (p->timed) {
        // Dispatch by dispatch in order, each between events of its own.
        for (size_t i = 0; i < p->launches.size(); ++i) {
            const Launch& L = *p->launches[i];
            TGX_HIP(hipExtLaunchKernel(L.k.func, L.k.grid, L.k.block, const_cast<void**>(L.params), L.k.lds, s, p->t_start[i],
                                       p->t_stop[i], 0));
        }
        p->timings_valid = true;
    } else {
        TGX_HIP(hipGraphLaunch(p->exec, s));
    }
    TGX_HIP(hipEventRecord(p->ev_end, s));
    for (tgx_memory* m : p->memories) ++m->running;
    p->pending = true;
    return TGX_OK;
}

tgx_status tgx_program_wait(tgx_program* prog) {
    clear_error();
    if (!prog) return fail(TGX_E_ARG, "null program");
    Program* p = prog->p;
    if (!p->pending) return TGX_OK;
    // Spin, then sleep, for at most 60 s (crates/vulkan/src/context.rs:24,120-136).
    const auto begin = std::chrono::steady_clock::now();
    for (int i = 0;; ++i) {
        hipError_t e = hipEventQuery(p->ev_end);
        if (e == hipSuccess) break;
        if (e != hipErrorNotReady) {
            for (tgx_memory* m : p->memories) --m->running;
            p->pending = false;
            return fail(TGX_E_HIP, std::string("waiting for the program: ") + hipGetErrorString(e));
        }
        if (std::chrono::steady_clock::now() - begin > std::chrono::seconds(60))
            return fail(TGX_E_TIMEOUT, "the program did not finish in 60 s");
        if (i > 1000) std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    for (tgx_memory* m : p->memories) --m->running;
    p->pending = false;
    return TGX_OK;
}

tgx_status tgx_program_run(tgx_program* prog) {
    TGX_TRY(tgx_program_start(prog));
    return tgx_program_wait(prog);
}

tgx_status tgx_program_timings(tgx_program* prog, int max, tgx_timing* out, int* n) {
    clear_error();
    if (!prog || !n) return fail(TGX_E_ARG, "null program or n");
    Program* p = prog->p;
    if (p->pending) return fail(TGX_E_BUSY, "the program runs");
    *n = 0;
    if (!p->timed || !p->timings_valid) return TGX_OK;
    *n = (int)p->launches.size();
    for (int i = 0; i < *n && i < max && out; ++i) {
        std::memset(out[i].label, 0, sizeof(out[i].label));
        std::strncpy(out[i].label, p->launches[i]->name, sizeof(out[i].label) - 1);
        TGX_HIP(hipEventElapsedTime(&out[i].ms, p->t_start[i], p->t_stop[i]));
    }
    return TGX_OK;
}

tgx_status tgx_program_elapsed_ms(tgx_program* prog, float* ms) {
    clear_error();
    if (!prog || !ms) return fail(TGX_E_ARG, "null program or out");
    Program* p = prog->p;
    if (p->pending) return fail(TGX_E_BUSY, "the program runs");
    TGX_HIP(hipEventElapsedTime(ms, p->ev_start, p->ev_end));
    return TGX_OK;
}

tgx_status tgx_program_destroy(tgx_program* prog) {
    clear_error();
    if (!prog) return TGX_OK;
    Program* p = prog->p;
    // A program's drop waits for it (recording.rs:730-760).
    tgx_status st = tgx_program_wait(prog);
    if (st == TGX_E_TIMEOUT) return st;  // still running: nothing it uses may go
    for (tgx_memory* m : p->memories) --m->programs;
    if (p->exec) hipGraphExecDestroy(p->exec);
    if (p->graph) hipGraphDestroy(p->graph);
    for (hipEvent_t e : p->t_start) if (e) hipEventDestroy(e);
    for (hipEvent_t e : p->t_stop) if (e) hipEventDestroy(e);
    hipEventDestroy(p->ev_start);
    hipEventDestroy(p->ev_end);
    delete p;
    delete prog;
    return st;
}

tgx_status tgx_copy_regions(tgx_context* ctx, tgx_memory* dst, tgx_memory* src, const tgx_region* regions, int n) {
    clear_error();
    if (!ctx || !dst || !src || (n > 0 && !regions) || n < 0) return fail(TGX_E_ARG, "null context, memory or regions");
    if (dst->ctx != ctx->ctx || src->ctx != ctx->ctx) return fail(TGX_E_ARG, "memory of another context");
    if (dst->running || src->running) return fail(TGX_E_BUSY, "a program that binds the memory runs");
    for (int i = 0; i < n; ++i) {
        const tgx_region& r = regions[i];
        if (r.src_offset > src->bytes || r.bytes > src->bytes - r.src_offset || r.dst_offset > dst->bytes ||
            r.bytes > dst->bytes - r.dst_offset)
            return fail(TGX_E_SHAPE, "region " + std::to_string(i) + ": " + std::to_string(r.bytes) + " bytes from " +
                                         std::to_string(r.src_offset) + " of " + std::to_string(src->bytes) + " to " +
                                         std::to_string(r.dst_offset) + " of " + std::to_string(dst->bytes));
    }
    hipStream_t s = ctx->ctx->stream;
    for (int i = 0; i < n; ++i)
        if (regions[i].bytes)
            TGX_HIP(hipMemcpyAsync((char*)dst->ptr + regions[i].dst_offset, (const char*)src->ptr + regions[i].src_offset,
                                   regions[i].bytes, hipMemcpyDefault, s));
    TGX_HIP(hipStreamSynchronize(s));
    return TGX_OK;
}

}  // extern "C"
