// The runtime beneath the models (include/tgx.h, tgx_alloc .. tgx_copy_regions): memory in a
// residence (crates/vulkan/src/memory.rs), the kernels by name with their bindings in order (the
// decode step's, crates/graph/src/kernels.rs:27-161; the prefill's, prefill.rs:32-116; the local
// stacks' and the sampler's, local/mod.rs:28-113; the LM side's and the prompt's, lm_side.rs:28-38
// and prompt.rs:42-67), and programs of dispatches recorded as HIP graphs and run as often as
// needed (crates/vulkan/src/recording.rs:116-760). Past the decode step a kernel's launch is the
// one the models' own launcher makes for the same arguments, captured instead of made.
//
// A dispatch is checked on the host before anything is recorded: every binding it must have is
// there, of its kernel's element size and alignment, and holds every byte the kernel reaches for
// the dispatch's constants, so that no recorded kernel reads or writes past a binding.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <ctime>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "dispatch.hpp"
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
// `params` points for as long as the program lives; or, for a kernel whose launch is captured
// from the models' own launcher (capture_one), each argument's bytes as captured, `captured`
// pointing at them.
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
    std::vector<std::vector<unsigned char>> args;
    std::vector<void*> captured;
    void** kernel_params() { return captured.empty() ? params : captured.data(); }
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

// A stack's shape from constants, refused as tgx_decoder_create refuses it.
tgx_status shape_of(uint32_t hidden, uint32_t inner, uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t capacity,
                    uint32_t eps, uint32_t rope, Shape* s) {
    if (rope > 1) return fail(TGX_E_SHAPE, "rope is 0 or 1");
    if (hidden > (1u << 20) || inner > (1u << 20) || heads > 1024 || kv_heads > 1024 || head_dim > 1024 || capacity > (1u << 24))
        return fail(TGX_E_SHAPE, "a shape past the kernels' sizes");
    tgx_shape in{};
    in.hidden = (int)hidden;
    in.inner = (int)inner;
    in.heads = (int)heads;
    in.kv_heads = (int)kv_heads;
    in.head_dim = (int)head_dim;
    in.layers = 1;
    in.capacity = (int)capacity;
    in.eps = as_float(eps);
    in.rope_theta = 10000.f;
    in.rope = rope != 0;
    return check_shape(&in, s);
}

// A placement: `slots` slot tables of `max_blocks` entries each, enough for `capacity` positions,
// into a pool of `blocks` cache blocks.
tgx_status check_placement(uint32_t capacity, uint32_t slots, uint32_t max_blocks, uint32_t blocks) {
    const uint32_t need = (capacity + BLOCK_TOKENS - 1) / BLOCK_TOKENS;
    if (max_blocks < need || blocks == 0 || slots == 0 || max_blocks > (1u << 20) || blocks > (1u << 24) || slots > (1u << 16))
        return fail(TGX_E_SHAPE, std::to_string(slots) + " slots of " + std::to_string(max_blocks) + " blocks in a pool of " +
                                     std::to_string(blocks) + " (a slot's table holds " + std::to_string(need) +
                                     " blocks at the capacity)");
    return TGX_OK;
}

// The shape and placement constants as the kernels take them, refused as tgx_decoder_create
// refuses a shape and a batch; the placement's tables are bound by the kernels that read them.
tgx_status decode_args(const uint32_t* c, DecodeArgs* a) {
    Shape s;
    TGX_TRY(shape_of(c[C_HIDDEN], c[C_INNER], c[C_HEADS], c[C_KV], c[C_HEAD_DIM], c[C_CAPACITY], c[C_EPS], c[C_ROPE], &s));
    tgx_batch batch{(int)c[C_ROWS], (int)c[C_SLOTS], BLOCK_TOKENS, (int)c[C_BLOCKS]};
    if ((int)c[C_ROWS] <= 0 || c[C_ROWS] > 64) return fail(TGX_E_SHAPE, "rows " + std::to_string(c[C_ROWS]) + ": 1 to 64");
    TGX_TRY(check_batch(s, &batch));
    TGX_TRY(check_placement(c[C_CAPACITY], c[C_SLOTS], c[C_MAX_BLOCKS], c[C_BLOCKS]));
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

// The columns one of a norm's input's sums of squares spans, as gemv_residual's strip_rows made
// them: 4 or 16.
tgx_status sq_cols_of(uint32_t v, const char* who, uint32_t* cols) {
    if (v != 4 && v != 16) return fail(TGX_E_SHAPE, std::string(who) + ": sq_cols " + std::to_string(v) + " (4 or 16)");
    *cols = v;
    return TGX_OK;
}

// gemv_qkv_rope (gemv_qkv_rope.comp): x | (xn, x_sq), gain, W, cos, sin, positions, slots, table
// -> q, cache pool; constant sq_cols (the columns each of x_sq's sums spans: 4, or 16 where
// gemv_residual took 16-row strips).
tgx_status build_qkv(const Bound* b, const uint32_t* c, Launch* L) {
    DecodeArgs a;
    TGX_TRY(decode_args(c, &a));
    uint32_t cols;
    TGX_TRY(sq_cols_of(c[C_COMMON], "gemv_qkv_rope", &cols));
    const uint64_t R = a.rows, h = a.hidden;
    const bool prenormed = b[1].ptr != nullptr;
    if (prenormed == (b[0].ptr != nullptr) || prenormed != (b[2].ptr != nullptr))
        return fail(TGX_E_SHAPE, "gemv_qkv_rope takes x, or xn with x_sq");
    if (prenormed) {
        TGX_TRY(holds(b, 1, "xn", R * h * 2));
        TGX_TRY(holds(b, 2, "x_sq", R * (h / cols) * 4));
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
    L->k = qkv_launch(a, prenormed, cols == 16);
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
// constants K, N, strip_rows (4 or 16: W's tiles, and the columns each of out_sq's sums of squares
// spans) past the common ones.
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
        TGX_TRY(holds(b, 6, "out_sq", R * (N / Rs) * 4));
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

// gemv_gate_up (gemv_gate_up.comp): mid_n, mid_sq, W -> mlp; constant sq_cols (as gemv_qkv_rope's).
tgx_status build_gate_up(const Bound* b, const uint32_t* c, Launch* L) {
    DecodeArgs a;
    TGX_TRY(decode_args(c, &a));
    uint32_t cols;
    TGX_TRY(sq_cols_of(c[C_COMMON], "gemv_gate_up", &cols));
    const uint64_t R = a.rows, h = a.hidden;
    TGX_TRY(holds(b, 0, "mid_n", R * h * 2));
    TGX_TRY(holds(b, 1, "mid_sq", R * (h / cols) * 4));
    TGX_TRY(holds(b, 2, "w", 2 * (uint64_t)a.inner * h * 2));
    TGX_TRY(holds(b, 3, "mlp", R * a.inner * 2));
    LayerArgs l{};
    l.mid_n = (const uint16_t*)b[0].ptr;
    l.mid_sq = (const float*)b[1].ptr;
    l.gate_up = (const uint16_t*)b[2].ptr;
    l.mlp = (uint16_t*)b[3].ptr;
    L->a = a;
    L->l = l;
    L->k = gate_up_launch(a, cols == 16);
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

// The one launch `launcher` makes, captured instead of made (capture_launches): the kernel, grid,
// LDS and arguments the models' own launch takes for the same arguments.
template <typename F>
tgx_status capture_one(const char* who, F&& launcher, Launch* L) {
    hipError_t e = hipSuccess;
    std::vector<CapturedLaunch> c = capture_launches([&] { e = launcher(); });
    if (c.size() != 1) return fail(TGX_E_SHAPE, std::string(who) + ": no instance takes these constants");
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string(who) + ": " + hipGetErrorString(e));
    L->k = KernelLaunch{c[0].func, c[0].grid, c[0].block, c[0].lds};
    L->args = std::move(c[0].args);
    L->captured.clear();
    for (auto& a : L->args) L->captured.push_back(a.data());
    return TGX_OK;
}

uint64_t round_up(uint64_t v, uint64_t to) { return (v + to - 1) / to * to; }

// ---- the prefill's kernels (prefill.rs:32-81) ----

// The constants every prefill kernel takes first, in order: the run's rows (positions over every
// run, laid one after another), the stack's shape and the cache's placement. Tensors of rows hold
// rows_pad of them, rows rounded up to 256 (the GEMM's tile), except where a kernel says.
constexpr int P_ROWS = 0, P_HIDDEN = 1, P_INNER = 2, P_HEADS = 3, P_KV = 4, P_HEAD_DIM = 5, P_CAPACITY = 6, P_SLOTS = 7,
              P_MAX_BLOCKS = 8, P_BLOCKS = 9, P_EPS = 10, P_ROPE = 11, P_COMMON = 12;
constexpr uint32_t PREFILL_MAX_ROWS = 1u << 20;
std::vector<const char*> prefill_constants(std::vector<const char*> own = {}) {
    std::vector<const char*> c = {"rows", "hidden", "inner", "heads", "kv_heads", "head_dim", "capacity", "slots", "max_blocks",
                                  "blocks", "eps", "rope"};
    c.insert(c.end(), own.begin(), own.end());
    return c;
}

tgx_status prefill_args(const uint32_t* c, PrefillArgs* a) {
    Shape s;
    TGX_TRY(shape_of(c[P_HIDDEN], c[P_INNER], c[P_HEADS], c[P_KV], c[P_HEAD_DIM], c[P_CAPACITY], c[P_EPS], c[P_ROPE], &s));
    if (c[P_ROWS] == 0 || c[P_ROWS] > PREFILL_MAX_ROWS)
        return fail(TGX_E_SHAPE, "rows " + std::to_string(c[P_ROWS]) + ": 1 to " + std::to_string(PREFILL_MAX_ROWS));
    TGX_TRY(check_placement(c[P_CAPACITY], c[P_SLOTS], c[P_MAX_BLOCKS], c[P_BLOCKS]));
    *a = PrefillArgs{};
    a->M = (int)c[P_ROWS];
    a->M_pad = (int)round_up(c[P_ROWS], 256);
    a->hidden = s.hidden;
    a->inner = s.inner;
    a->heads = s.heads;
    a->kv_heads = s.kv_heads;
    a->head_dim = s.head_dim;
    a->capacity = s.capacity;
    a->nslots = (int)c[P_SLOTS];
    a->max_blocks = (int)c[P_MAX_BLOCKS];
    a->nblocks = (int)c[P_BLOCKS];
    a->eps = s.eps;
    a->scale = 1.0f / std::sqrt((float)s.head_dim);
    a->rope = (int)c[P_ROPE];
    return TGX_OK;
}

uint64_t prefill_pool_bytes(const PrefillArgs& a) { return (uint64_t)a.nblocks * a.kv_heads * 2 * kv_tile(a.head_dim) * 2; }

// norm_rows (norm_rows.comp): x, gain -> out. The first layer's input norm: x [rows][hidden] f32
// into bf16 rows in fragment order (rows_pad of them, zero past rows), as the GEMMs read them.
tgx_status build_norm_rows(const Bound* b, const uint32_t* c, Launch* L) {
    PrefillArgs a;
    TGX_TRY(prefill_args(c, &a));
    const uint64_t h = a.hidden;
    TGX_TRY(holds(b, 0, "x", (uint64_t)a.M * h * 4));
    TGX_TRY(holds(b, 1, "gain", h * 4));
    TGX_TRY(holds(b, 2, "out", (uint64_t)a.M_pad * h * 2));
    return capture_one("norm_rows", [&] {
        return launch_prefill_norm(a, false, (const float*)b[0].ptr, (const float*)b[1].ptr, (uint16_t*)b[2].ptr, nullptr, nullptr, nullptr);
    }, L);
}

// final_norm_rows (norm_rows.comp as the last step): x, gain -> out, f32 [rows][hidden] both.
tgx_status build_final_norm_rows(const Bound* b, const uint32_t* c, Launch* L) {
    PrefillArgs a;
    TGX_TRY(prefill_args(c, &a));
    const uint64_t h = a.hidden;
    TGX_TRY(holds(b, 0, "x", (uint64_t)a.M * h * 4));
    TGX_TRY(holds(b, 1, "gain", h * 4));
    TGX_TRY(holds(b, 2, "out", (uint64_t)a.M * h * 4));
    return capture_one("final_norm_rows", [&] {
        return launch_prefill_norm(a, true, (const float*)b[0].ptr, (const float*)b[1].ptr, nullptr, (float*)b[2].ptr, nullptr, nullptr);
    }, L);
}

// gemm_rope_rows (the q/k/v GEMM with rope_rows.comp fused): x, W, [row_sq,] cos, sin, positions,
// slots, table -> q, cache pool. x: bf16 [rows_pad][hidden] in fragment order, an RMSNorm's output,
// or with row_sq its input times the gain and the rows' sums of squares over each 128 columns
// ([rows_pad][hidden / 128] f32); W: q/k/v rows in tiles of TGX_TILES_QKV (head_dim 64) or
// TGX_TILES_QKV128; positions and slots: [rows] u32 (a position past the capacity or a slot past
// the table's is a spare row: nothing written).
tgx_status build_gemm_rope_rows(const Bound* b, const uint32_t* c, Launch* L) {
    PrefillArgs a;
    TGX_TRY(prefill_args(c, &a));
    const uint64_t h = a.hidden, D = a.head_dim, Mp = a.M_pad, N = (uint64_t)(a.heads + 2 * a.kv_heads) * D;
    TGX_TRY(holds(b, 0, "x", Mp * h * 2));
    TGX_TRY(holds(b, 1, "w", N * h * 2));
    if (b[2].ptr) TGX_TRY(holds(b, 2, "row_sq", Mp * (h / 128) * 4));
    TGX_TRY(holds(b, 3, "cos", (uint64_t)a.capacity * (D / 2) * 4));
    TGX_TRY(holds(b, 4, "sin", (uint64_t)a.capacity * (D / 2) * 4));
    TGX_TRY(holds(b, 5, "positions", (uint64_t)a.M * 4));
    TGX_TRY(holds(b, 6, "slots", (uint64_t)a.M * 4));
    TGX_TRY(holds(b, 7, "table", (uint64_t)a.nslots * a.max_blocks * 4));
    TGX_TRY(holds(b, 8, "q", Mp * a.heads * D * 2));
    TGX_TRY(holds(b, 9, "kv", prefill_pool_bytes(a)));
    a.cos = (const float*)b[3].ptr;
    a.sin = (const float*)b[4].ptr;
    a.tok_pos = (const uint32_t*)b[5].ptr;
    a.tok_slot = (const uint32_t*)b[6].ptr;
    a.table = (const uint32_t*)b[7].ptr;
    GemmArgs g{};
    g.w = (const uint16_t*)b[1].ptr;
    g.x = (const uint16_t*)b[0].ptr;
    g.K = a.hidden;
    g.N = (int)N;
    g.row_sq = (const float*)b[2].ptr;
    g.q = (uint16_t*)b[8].ptr;
    g.kv = (uint16_t*)b[9].ptr;
    return capture_one("gemm_rope_rows", [&] { return launch_prefill_gemm(a, EPI_QKV, QKV_ROWS, g, nullptr, nullptr); }, L);
}

// attention_rows (attention_rows.comp): q, cache pool, table, tiles -> attended, constant tiles.
// Each tile is 4 u32: row0, pos0, count, slot: rows row0 .. row0 + count - 1 are positions
// pos0 .. of the slot, every position of a run up to its own attending to the slot's cache. A tile
// holds at most 32 positions (16 at 8 or 16 query heads a KV head, 8 at 16 of 128 dimensions); one
// that leaves the tensors is skipped. attended: bf16 [rows_pad][heads head_dim] in fragment order, written at the tiles' rows
// only (the GEMM after it reads every row: keep the rest zero).
tgx_status build_attention_rows(const Bound* b, const uint32_t* c, Launch* L) {
    PrefillArgs a;
    TGX_TRY(prefill_args(c, &a));
    const uint32_t ntiles = c[P_COMMON];
    if (ntiles == 0 || ntiles > PREFILL_MAX_ROWS)
        return fail(TGX_E_SHAPE, "attention_rows: " + std::to_string(ntiles) + " tiles (1 to " + std::to_string(PREFILL_MAX_ROWS) + ")");
    const uint64_t Mp = a.M_pad, att = (uint64_t)a.heads * a.head_dim;
    TGX_TRY(holds(b, 0, "q", Mp * att * 2));
    TGX_TRY(holds(b, 1, "kv", prefill_pool_bytes(a)));
    TGX_TRY(holds(b, 2, "table", (uint64_t)a.nslots * a.max_blocks * 4));
    TGX_TRY(holds(b, 3, "tiles", (uint64_t)ntiles * sizeof(PrefillTile)));
    TGX_TRY(holds(b, 4, "attended", Mp * att * 2));
    a.table = (const uint32_t*)b[2].ptr;
    return capture_one("attention_rows", [&] {
        return launch_prefill_attention(a, (const uint16_t*)b[0].ptr, (const uint16_t*)b[1].ptr, (uint16_t*)b[4].ptr,
                                        (const PrefillTile*)b[3].ptr, (int)ntiles, nullptr, nullptr);
    }, L);
}

// gemm_add_norm_rows (o_proj or down_proj with add_norm_rows.comp fused): x, W, residual
// [, next_gain] -> out [, out_n, out_sq]; constants K, N, strip_rows (W's tiles: 4 or 16) and
// residual_in (1: the accumulators start at the residual, as the prefill does for o_proj; 0: it
// is added after the products, as for down_proj; the same sums either way). x: bf16
// [rows_pad][K] in fragment order; residual and out: f32 [rows][N]; with next_gain the next
// norm's input, out next_gain in bf16 in fragment order ([rows_pad][N]), and out's sums of
// squares over each 128 columns ([rows][N / 128] f32).
tgx_status build_gemm_add_norm_rows(const Bound* b, const uint32_t* c, Launch* L) {
    PrefillArgs a;
    TGX_TRY(prefill_args(c, &a));
    const uint32_t K = c[P_COMMON], N = c[P_COMMON + 1], Rs = c[P_COMMON + 2], in = c[P_COMMON + 3];
    if (K == 0 || K % 1024 || K > (uint32_t)decode_max_k() || N == 0 || N % 256 || N > (1u << 16) || (Rs != 4 && Rs != 16) || in > 1)
        return fail(TGX_E_SHAPE, "gemm_add_norm_rows: K " + std::to_string(K) + " (a multiple of 1024 up to " +
                                     std::to_string(decode_max_k()) + "), N " + std::to_string(N) + " (a multiple of 256), strips of " +
                                     std::to_string(Rs) + " rows (4 or 16), residual_in " + std::to_string(in) + " (0 or 1)");
    if ((b[3].ptr != nullptr) != (b[5].ptr != nullptr) || (b[3].ptr != nullptr) != (b[6].ptr != nullptr))
        return fail(TGX_E_SHAPE, "gemm_add_norm_rows takes next_gain, out_n and out_sq together or none of them");
    const uint64_t M = a.M, Mp = a.M_pad;
    TGX_TRY(holds(b, 0, "x", Mp * K * 2));
    TGX_TRY(holds(b, 1, "w", (uint64_t)N * K * 2));
    TGX_TRY(holds(b, 2, "residual", M * N * 4));
    TGX_TRY(holds(b, 4, "out", M * N * 4));
    if (b[3].ptr) {
        TGX_TRY(holds(b, 3, "next_gain", (uint64_t)N * 4));
        TGX_TRY(holds(b, 5, "out_n", Mp * N * 2));
        TGX_TRY(holds(b, 6, "out_sq", M * (N / 128) * 4));
    }
    GemmArgs g{};
    g.w = (const uint16_t*)b[1].ptr;
    g.x = (const uint16_t*)b[0].ptr;
    g.K = (int)K;
    g.N = (int)N;
    g.residual = (const float*)b[2].ptr;
    g.out = (float*)b[4].ptr;
    g.next_gain = (const float*)b[3].ptr;
    g.out_n = (uint16_t*)b[5].ptr;
    g.out_sq = (float*)b[6].ptr;
    const int epi = in ? EPI_RESIDUAL_IN : EPI_RESIDUAL;
    return capture_one("gemm_add_norm_rows", [&] { return launch_prefill_gemm(a, epi, (int)Rs, g, nullptr, nullptr); }, L);
}

// gemm_silu_mul_rows (gate/up with silu_mul_rows.comp fused): x, W [, row_sq] -> mlp; constants
// K, N (gate's rows then up's: N / 2 outputs). x as gemm_rope_rows takes it ([rows_pad][K]); mlp:
// bf16 [rows_pad][N / 2] in fragment order.
tgx_status build_gemm_silu_mul_rows(const Bound* b, const uint32_t* c, Launch* L) {
    PrefillArgs a;
    TGX_TRY(prefill_args(c, &a));
    const uint32_t K = c[P_COMMON], N = c[P_COMMON + 1];
    if (K == 0 || K % 1024 || K > 4096 || N == 0 || N % 256 || N > (1u << 16))
        return fail(TGX_E_SHAPE, "gemm_silu_mul_rows: K " + std::to_string(K) + " (a multiple of 1024 up to 4096), N " +
                                     std::to_string(N) + " (a multiple of 256)");
    const uint64_t Mp = a.M_pad;
    TGX_TRY(holds(b, 0, "x", Mp * K * 2));
    TGX_TRY(holds(b, 1, "w", (uint64_t)N * K * 2));
    if (b[2].ptr) TGX_TRY(holds(b, 2, "row_sq", Mp * (K / 128) * 4));
    TGX_TRY(holds(b, 3, "mlp", Mp * (N / 2) * 2));
    GemmArgs g{};
    g.w = (const uint16_t*)b[1].ptr;
    g.x = (const uint16_t*)b[0].ptr;
    g.K = (int)K;
    g.N = (int)N;
    g.row_sq = (const float*)b[2].ptr;
    g.mlp = (uint16_t*)b[3].ptr;
    return capture_one("gemm_silu_mul_rows", [&] { return launch_prefill_gemm(a, EPI_SILU, QKV_ROWS, g, nullptr, nullptr); }, L);
}

// ---- the local stacks' and the patch sampler's kernels (local/mod.rs:28-113) ----

// The constants every local-stack kernel takes first: tokens in sequences of seq_tokens (token m
// at place m % seq_tokens of its sequence) and the stack's shape (head_dim 64, hidden 1024).
// Tensors of tokens hold tokens_pad of them (tokens rounded up to 16 up to 64 tokens, to 64
// past that) where a GEMM reads them, `tokens` elsewhere, as each kernel says.
constexpr int L_TOKENS = 0, L_SEQ = 1, L_HIDDEN = 2, L_INNER = 3, L_HEADS = 4, L_KV = 5, L_EPS = 6, L_ROPE = 7, L_COMMON = 8;
constexpr uint32_t LOCAL_MAX_TOKENS = 1u << 16;
std::vector<const char*> local_constants(std::vector<const char*> own = {}) {
    std::vector<const char*> c = {"tokens", "seq_tokens", "hidden", "inner", "heads", "kv_heads", "eps", "rope"};
    c.insert(c.end(), own.begin(), own.end());
    return c;
}

tgx_status local_args(const uint32_t* c, LocalArgs* a) {
    const uint32_t M = c[L_TOKENS], T = c[L_SEQ];
    if (T == 0 || T > (uint32_t)LOCAL_MAX_T || M == 0 || M > LOCAL_MAX_TOKENS || M % T)
        return fail(TGX_E_SHAPE, std::to_string(M) + " tokens in sequences of " + std::to_string(T) + " (1 to " +
                                     std::to_string(LOCAL_MAX_T) + " tokens a sequence, whole sequences, " +
                                     std::to_string(LOCAL_MAX_TOKENS) + " tokens at most)");
    Shape s;
    TGX_TRY(shape_of(c[L_HIDDEN], c[L_INNER], c[L_HEADS], c[L_KV], HEAD_DIM, T, c[L_EPS], c[L_ROPE], &s));
    if (s.hidden != 1024 || s.heads % 4 || s.inner % 64)
        return fail(TGX_E_SHAPE, "a local stack " + std::to_string(s.hidden) + " wide of " + std::to_string(s.heads) +
                                     " heads with an FFN " + std::to_string(s.inner) +
                                     " wide (the kernels take 1024, heads a multiple of 4, an FFN a multiple of 64)");
    *a = LocalArgs{};
    a->M = (int)M;
    a->M_pad = local_rows_padded((int)M);
    a->T = (int)T;
    a->hidden = s.hidden;
    a->inner = s.inner;
    a->heads = s.heads;
    a->kv_heads = s.kv_heads;
    a->eps = s.eps;
    a->scale = 1.0f / std::sqrt((float)HEAD_DIM);
    a->rope = s.rope ? 1 : 0;
    return TGX_OK;
}

constexpr uint64_t LOCAL_SQ = 1024 / LOCAL_SQ_COLS;  // a token's sums of squares

// local_norm (local_norm.comp): x, gain -> normed, row_sq. The first layer's input norm as the
// GEMMs after it read it: x [tokens][1024] f32; normed = x gain in bf16, [tokens_pad][1024] in
// fragment order (written at the tokens' rows); row_sq: each 64 columns' sum of squares of x,
// [tokens][16] f32 (the GEMM applies the rows' scales).
tgx_status build_local_norm(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint64_t M = a.M, h = a.hidden;
    TGX_TRY(holds(b, 0, "x", M * h * 4));
    TGX_TRY(holds(b, 1, "gain", h * 4));
    TGX_TRY(holds(b, 2, "normed", (uint64_t)a.M_pad * h * 2));
    TGX_TRY(holds(b, 3, "row_sq", M * LOCAL_SQ * 4));
    return capture_one("local_norm", [&] {
        return launch_local_add_norm(a, false, nullptr, 0, (const float*)b[0].ptr, nullptr, (const float*)b[1].ptr, (uint16_t*)b[2].ptr,
                                     (float*)b[3].ptr, nullptr, nullptr, nullptr);
    }, L);
}

// local_qkv_rope (local_qkv_rope.comp): x, W, row_sq, cos, sin -> q, k, v. x and row_sq as
// local_norm writes them ([tokens_pad] rows each); W in tiles of TGX_TILES_QKV; cos and sin
// [seq_tokens][32] (the rotation at each place of a sequence); q [tokens][heads][64], k and v
// [tokens][kv_heads][64], bf16.
tgx_status build_local_qkv_rope(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint64_t M = a.M, Mp = a.M_pad, h = a.hidden, N = (uint64_t)(a.heads + 2 * a.kv_heads) * HEAD_DIM;
    TGX_TRY(holds(b, 0, "x", Mp * h * 2));
    TGX_TRY(holds(b, 1, "w", N * h * 2));
    TGX_TRY(holds(b, 2, "row_sq", Mp * LOCAL_SQ * 4));
    TGX_TRY(holds(b, 3, "cos", (uint64_t)a.T * (HEAD_DIM / 2) * 4));
    TGX_TRY(holds(b, 4, "sin", (uint64_t)a.T * (HEAD_DIM / 2) * 4));
    TGX_TRY(holds(b, 5, "q", M * a.heads * HEAD_DIM * 2));
    TGX_TRY(holds(b, 6, "k", M * a.kv_heads * HEAD_DIM * 2));
    TGX_TRY(holds(b, 7, "v", M * a.kv_heads * HEAD_DIM * 2));
    a.cos = (const float*)b[3].ptr;
    a.sin = (const float*)b[4].ptr;
    LocalGemm g{};
    g.w = (const uint16_t*)b[1].ptr;
    g.x = (const uint16_t*)b[0].ptr;
    g.K = a.hidden;
    g.N = (int)N;
    g.row_sq = (const float*)b[2].ptr;
    g.q = (uint16_t*)b[5].ptr;
    g.k = (uint16_t*)b[6].ptr;
    g.v = (uint16_t*)b[7].ptr;
    return capture_one("local_qkv_rope", [&] { return launch_local_qkv(a, g, nullptr, nullptr); }, L);
}

// local_attention (local_attention.comp): q, k, v -> attended, every token of a sequence
// attending to every token of it; attended bf16 [tokens_pad][heads 64] in fragment order, written
// at the tokens' rows.
tgx_status build_local_attention(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint64_t M = a.M;
    TGX_TRY(holds(b, 0, "q", M * a.heads * HEAD_DIM * 2));
    TGX_TRY(holds(b, 1, "k", M * a.kv_heads * HEAD_DIM * 2));
    TGX_TRY(holds(b, 2, "v", M * a.kv_heads * HEAD_DIM * 2));
    TGX_TRY(holds(b, 3, "attended", (uint64_t)a.M_pad * a.heads * HEAD_DIM * 2));
    return capture_one("local_attention", [&] {
        return launch_local_attention(a, (const uint16_t*)b[0].ptr, (const uint16_t*)b[1].ptr, (const uint16_t*)b[2].ptr,
                                      (uint16_t*)b[3].ptr, nullptr, nullptr);
    }, L);
}

// local_partial (local_partial.comp): x, W -> partial; constants K, N, parts. Up to 64 tokens:
// the products over each of `parts` equal spans of K (16 or 32 k-blocks of 32 columns each),
// f32 [parts][tokens_pad][N]; x bf16 [tokens_pad][K] in fragment order.
tgx_status build_local_partial(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint32_t K = c[L_COMMON], N = c[L_COMMON + 1], parts = c[L_COMMON + 2];
    if (K == 0 || K > 8192 || N == 0 || N > 8192 || parts == 0 || parts > (uint32_t)LOCAL_MAX_PARTS)
        return fail(TGX_E_SHAPE, "local_partial: K " + std::to_string(K) + ", N " + std::to_string(N) + " in " + std::to_string(parts) +
                                     " parts");
    const uint64_t Mp = a.M_pad;
    TGX_TRY(holds(b, 0, "x", Mp * K * 2));
    TGX_TRY(holds(b, 1, "w", (uint64_t)N * K * 2));
    TGX_TRY(holds(b, 2, "partial", parts * Mp * N * 4));
    LocalGemm g{};
    g.w = (const uint16_t*)b[1].ptr;
    g.x = (const uint16_t*)b[0].ptr;
    g.K = (int)K;
    g.N = (int)N;
    g.partial = (float*)b[2].ptr;
    return capture_one("local_partial", [&] { return launch_local_partial(a, g, (int)parts, nullptr, nullptr); }, L);
}

// The add-norm kernels' checks: `parts` of partial ([parts][tokens_pad][1024] f32, bound when
// parts > 0), the residual [tokens][1024] f32 and the gain.
tgx_status add_norm_inputs(const Bound* b, const LocalArgs& a, uint32_t parts, const char* who) {
    if (parts > (uint32_t)LOCAL_MAX_PARTS || (parts > 0) != (b[0].ptr != nullptr))
        return fail(TGX_E_SHAPE, std::string(who) + ": " + std::to_string(parts) + " parts (0 to " + std::to_string(LOCAL_MAX_PARTS) +
                                     ", partial bound when more than 0)");
    const uint64_t M = a.M, h = a.hidden;
    if (parts) TGX_TRY(holds(b, 0, "partial", parts * (uint64_t)a.M_pad * h * 4));
    TGX_TRY(holds(b, 1, "residual", M * h * 4));
    TGX_TRY(holds(b, 2, "gain", h * 4));
    if (b[3].ptr) TGX_TRY(holds(b, 3, "sum", M * h * 4));
    return TGX_OK;
}

// local_add_norm (local_add_norm.comp): [partial,] residual, gain -> [sum,] normed, row_sq;
// constant parts. sum = residual + the parts' sums in part order; then the next norm's input as
// local_norm writes it.
tgx_status build_local_add_norm(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint32_t parts = c[L_COMMON];
    TGX_TRY(add_norm_inputs(b, a, parts, "local_add_norm"));
    TGX_TRY(holds(b, 4, "normed", (uint64_t)a.M_pad * a.hidden * 2));
    TGX_TRY(holds(b, 5, "row_sq", (uint64_t)a.M * LOCAL_SQ * 4));
    return capture_one("local_add_norm", [&] {
        return launch_local_add_norm(a, false, (const float*)b[0].ptr, (int)parts, (const float*)b[1].ptr, (float*)b[3].ptr,
                                     (const float*)b[2].ptr, (uint16_t*)b[4].ptr, (float*)b[5].ptr, nullptr, nullptr, nullptr);
    }, L);
}

// local_final_norm (local_norm.comp as a stack's last step): [partial,] residual, gain ->
// [sum,] out; constant parts. out = RMSNorm(residual + the parts' sums) gain, f32 [tokens][1024].
tgx_status build_local_final_norm(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint32_t parts = c[L_COMMON];
    TGX_TRY(add_norm_inputs(b, a, parts, "local_final_norm"));
    TGX_TRY(holds(b, 4, "out", (uint64_t)a.M * a.hidden * 4));
    return capture_one("local_final_norm", [&] {
        return launch_local_add_norm(a, true, (const float*)b[0].ptr, (int)parts, (const float*)b[1].ptr, (float*)b[3].ptr,
                                     (const float*)b[2].ptr, nullptr, nullptr, (float*)b[4].ptr, nullptr, nullptr);
    }, L);
}

// local_gemm_add_norm (local_partial.comp and local_add_norm.comp fused, past 64 tokens): x, W,
// residual [, next_gain] -> sum [, normed, row_sq]; constants K, N (1024), parts (2 or 4 spans of
// 16 or 32 k-blocks, added in part order as local_add_norm adds them). residual: f32
// [tokens_pad][1024]; sum [tokens][1024]; with next_gain the next norm's input as local_norm
// writes it.
tgx_status build_local_gemm_add_norm(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint32_t K = c[L_COMMON], N = c[L_COMMON + 1], parts = c[L_COMMON + 2];
    if (K == 0 || K > 8192 || N != (uint32_t)a.hidden || parts == 0 || parts > (uint32_t)LOCAL_MAX_PARTS)
        return fail(TGX_E_SHAPE, "local_gemm_add_norm: K " + std::to_string(K) + ", N " + std::to_string(N) + " (the hidden width) in " +
                                     std::to_string(parts) + " parts");
    if ((b[3].ptr != nullptr) != (b[5].ptr != nullptr) || (b[3].ptr != nullptr) != (b[6].ptr != nullptr))
        return fail(TGX_E_SHAPE, "local_gemm_add_norm takes next_gain, normed and row_sq together or none of them");
    const uint64_t M = a.M, Mp = a.M_pad;
    TGX_TRY(holds(b, 0, "x", Mp * K * 2));
    TGX_TRY(holds(b, 1, "w", (uint64_t)N * K * 2));
    TGX_TRY(holds(b, 2, "residual", Mp * N * 4));
    TGX_TRY(holds(b, 4, "sum", M * N * 4));
    if (b[3].ptr) {
        TGX_TRY(holds(b, 3, "next_gain", (uint64_t)N * 4));
        TGX_TRY(holds(b, 5, "normed", Mp * N * 2));
        TGX_TRY(holds(b, 6, "row_sq", M * LOCAL_SQ * 4));
    }
    LocalGemm g{};
    g.w = (const uint16_t*)b[1].ptr;
    g.x = (const uint16_t*)b[0].ptr;
    g.K = (int)K;
    g.N = (int)N;
    g.residual = (const float*)b[2].ptr;
    g.next_gain = (const float*)b[3].ptr;
    g.sum = (float*)b[4].ptr;
    g.normed = (uint16_t*)b[5].ptr;
    g.sum_sq = (float*)b[6].ptr;
    return capture_one("local_gemm_add_norm", [&] { return launch_local_add(a, g, (int)parts, nullptr, nullptr); }, L);
}

// local_gate_up (local_gate_up.comp): x, W, row_sq -> mlp. x and row_sq as local_norm writes them
// ([tokens_pad] rows each); W: the gate's rows then the up's, 2 inner x 1024 in tiles of
// TGX_TILES_16; mlp = SiLU(gate) up, bf16 [tokens_pad][inner] in fragment order.
tgx_status build_local_gate_up(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint64_t Mp = a.M_pad, h = a.hidden;
    TGX_TRY(holds(b, 0, "x", Mp * h * 2));
    TGX_TRY(holds(b, 1, "w", 2 * (uint64_t)a.inner * h * 2));
    TGX_TRY(holds(b, 2, "row_sq", Mp * LOCAL_SQ * 4));
    TGX_TRY(holds(b, 3, "mlp", Mp * a.inner * 2));
    LocalGemm g{};
    g.w = (const uint16_t*)b[1].ptr;
    g.x = (const uint16_t*)b[0].ptr;
    g.K = a.hidden;
    g.N = 2 * a.inner;
    g.row_sq = (const float*)b[2].ptr;
    g.mlp = (uint16_t*)b[3].ptr;
    return capture_one("local_gate_up", [&] { return launch_local_gate_up(a, g, nullptr, nullptr); }, L);
}

// local_embed (local_embed.comp): frames, W, bias, tokens [, gain] -> x0 [, normed, row_sq];
// constants past the stack's: patch_rows, channels, frames, first, copy_at, copies, guided,
// shared, seqs. Each patch row's frames [channels][frames] f32 through the linear layer (W f32
// [1024][channels], bias [1024]) into tokens first .. first + frames - 1 of each of its `seqs`
// sequences, and `copies` tokens of `tokens` ([patch_rows][copies][1024] f32, or [copies][1024]
// when shared) at copy_at .. (zero in the second sequence when guided); with gain, each token
// written is also the first layer's norm input as local_norm writes it. x0: f32 [tokens][1024].
tgx_status build_local_embed(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint32_t* o = c + L_COMMON;
    const uint32_t rows = o[0], C = o[1], F = o[2], first = o[3], copy_at = o[4], copies = o[5], guided = o[6], shared = o[7],
                   seqs = o[8];
    const uint64_t T = a.T;
    if (rows == 0 || seqs == 0 || seqs > 2 || (uint64_t)rows * seqs * T > (uint64_t)a.M || C == 0 || C % 4 || C > 64 || F == 0 ||
        F > 4 || C * F > 1024 || first + F > T || copies == 0 || copies > 2 || copy_at + copies > T || guided > 1 || shared > 1)
        return fail(TGX_E_SHAPE, "local_embed: " + std::to_string(rows) + " patch rows of " + std::to_string(seqs) +
                                     " sequences, frames of " + std::to_string(C) + " channels x " + std::to_string(F) +
                                     " at token " + std::to_string(first) + ", " + std::to_string(copies) + " tokens copied at " +
                                     std::to_string(copy_at) + " (channels a multiple of 4 up to 64, 1 to 4 frames, 1 or 2 "
                                     "sequences and copies, within a sequence of " + std::to_string(T) + " and the tokens)");
    if ((b[4].ptr != nullptr) != (b[6].ptr != nullptr) || (b[4].ptr != nullptr) != (b[7].ptr != nullptr))
        return fail(TGX_E_SHAPE, "local_embed takes gain, normed and row_sq together or none of them");
    const uint64_t h = a.hidden;
    TGX_TRY(holds(b, 0, "frames", (uint64_t)rows * C * F * 4));
    TGX_TRY(holds(b, 1, "w", h * C * 4));
    TGX_TRY(holds(b, 2, "bias", h * 4));
    TGX_TRY(holds(b, 3, "tokens", (uint64_t)(shared ? 1 : rows) * copies * h * 4));
    TGX_TRY(holds(b, 5, "x0", (uint64_t)a.M * h * 4));
    if (b[4].ptr) {
        TGX_TRY(holds(b, 4, "gain", h * 4));
        TGX_TRY(holds(b, 6, "normed", (uint64_t)a.M_pad * h * 2));
        TGX_TRY(holds(b, 7, "row_sq", (uint64_t)a.M * LOCAL_SQ * 4));
    }
    EmbedArgs e{};
    e.src = (const float*)b[0].ptr;
    e.w = (const float*)b[1].ptr;
    e.bias = (const float*)b[2].ptr;
    e.copy_src = (const float*)b[3].ptr;
    e.x0 = (float*)b[5].ptr;
    e.channels = (int)C;
    e.frames = (int)F;
    e.first = (int)first;
    e.copy_at = (int)copy_at;
    e.copies = (int)copies;
    e.guided = (int)guided;
    e.shared = (int)shared;
    e.seqs = (int)seqs;
    e.gain = (const float*)b[4].ptr;
    e.normed = (uint16_t*)b[6].ptr;
    e.row_sq = (float*)b[7].ptr;
    return capture_one("local_embed", [&] { return launch_local_embed(a, e, (int)rows, nullptr, nullptr); }, L);
}

// cfm_noise (cfm_noise.comp): noise, sampling -> state; constants rows, len. state[r][i] =
// sampling[r][0] (the row's temperature) noise[r][i], f32 [rows][len].
tgx_status build_cfm_noise(const Bound* b, const uint32_t* c, Launch* L) {
    const uint32_t rows = c[0], len = c[1];
    if (rows == 0 || len == 0 || (uint64_t)rows * len > (1u << 30))
        return fail(TGX_E_SHAPE, "cfm_noise: " + std::to_string(rows) + " rows of " + std::to_string(len));
    const uint64_t n = (uint64_t)rows * len;
    TGX_TRY(holds(b, 0, "noise", n * 4));
    TGX_TRY(holds(b, 1, "sampling", (uint64_t)rows * 2 * 4));
    TGX_TRY(holds(b, 2, "state", n * 4));
    return capture_one("cfm_noise", [&] {
        return launch_cfm_noise((const float*)b[0].ptr, (const float*)b[1].ptr, (float*)b[2].ptr, (int)rows, (int)len, nullptr, nullptr);
    }, L);
}

// dit_euler (dit_euler.comp): x, row_sq, gain, W, bias, sampling -> state (read and written);
// constants past the stack's: patch_rows, channels, frames, first, dt (f32 bits). The stack's
// last residual x [tokens][1024] and its sums of squares [tokens][16], normed with the final
// gain; out_proj (W [channels][1024] in tiles of TGX_TILES_16, bias [channels]) over tokens
// first .. first + frames - 1 of each patch row's two sequences (the conditional, then the
// unconditional); CFG-Zero* with the row's guidance scale (sampling [rows][2]: temperature,
// scale), and state [rows][channels][frames] -= dt guided.
tgx_status build_dit_euler(const Bound* b, const uint32_t* c, Launch* L) {
    LocalArgs a;
    TGX_TRY(local_args(c, &a));
    const uint32_t* o = c + L_COMMON;
    const uint32_t rows = o[0], C = o[1], F = o[2], first = o[3];
    const float dt = as_float(o[4]);
    if (rows == 0 || (uint64_t)rows * 2 * a.T > (uint64_t)a.M || C == 0 || C % 16 || C > 64 || F == 0 || F > 4 || C * F > 512 ||
        first + F > (uint32_t)a.T || !std::isfinite(dt))
        return fail(TGX_E_SHAPE, "dit_euler: " + std::to_string(rows) + " patch rows, frames of " + std::to_string(C) + " channels x " +
                                     std::to_string(F) + " at token " + std::to_string(first) +
                                     " (channels a multiple of 16 up to 64, 1 to 4 frames, two sequences a row within the tokens, "
                                     "a finite dt)");
    const uint64_t M = a.M, h = a.hidden;
    TGX_TRY(holds(b, 0, "x", M * h * 4));
    TGX_TRY(holds(b, 1, "row_sq", M * LOCAL_SQ * 4));
    TGX_TRY(holds(b, 2, "gain", h * 4));
    TGX_TRY(holds(b, 3, "w", (uint64_t)C * h * 2));
    TGX_TRY(holds(b, 4, "bias", (uint64_t)C * 4));
    TGX_TRY(holds(b, 5, "sampling", (uint64_t)rows * 2 * 4));
    TGX_TRY(holds(b, 6, "state", (uint64_t)rows * C * F * 4));
    EulerArgs e{};
    e.x = (const float*)b[0].ptr;
    e.row_sq = (const float*)b[1].ptr;
    e.gain = (const float*)b[2].ptr;
    e.w = (const uint16_t*)b[3].ptr;
    e.bias = (const float*)b[4].ptr;
    e.sampling = (const float*)b[5].ptr;
    e.state = (float*)b[6].ptr;
    e.channels = (int)C;
    e.frames = (int)F;
    e.first = (int)first;
    e.dt = dt;
    return capture_one("dit_euler", [&] { return launch_dit_euler(a, e, (int)rows, nullptr, nullptr); }, L);
}

// ---- the layers between VoxCPM2's LMs (lm_side.rs:28-38) ----

// gemv_linear (gemv_linear.comp): x0 [, x1], W, bias -> out; constants rows, K0, K1, N, offset,
// stride, act (0 none, 1 SiLU, 2 the scalar quantizer's levels), levels (f32 bits). out[r][offset
// + n] = act(W [x0[r]; x1[r]] + bias)[n]: x0 [rows][K0] and x1 [rows][K1] f32 (K1 0 without x1,
// K0 + K1 up to 4096, each a multiple of 32), W in tiles of TGX_TILES_16 of N rows rounded up to
// 16 (rows past N zero), out rows `stride` floats apart.
tgx_status build_gemv_linear(const Bound* b, const uint32_t* c, Launch* L) {
    const uint32_t rows = c[0], K0 = c[1], K1 = c[2], N = c[3], offset = c[4], stride = c[5], act = c[6];
    const float levels = as_float(c[7]);
    if (rows == 0 || rows > (1u << 16) || K0 == 0 || K0 % 32 || K1 % 32 || K0 + K1 > (uint32_t)LINEAR_MAX_K || N == 0 ||
        N > (1u << 16) || (uint64_t)offset + N > stride || stride > (1u << 20) || act > 2 || (K1 > 0) != (b[1].ptr != nullptr) ||
        (act == ACT_LEVELS && !(levels > 0.f && std::isfinite(levels))))
        return fail(TGX_E_SHAPE, "gemv_linear: " + std::to_string(rows) + " rows of " + std::to_string(K0) + " + " + std::to_string(K1) +
                                     " columns into " + std::to_string(N) + " at " + std::to_string(offset) + " of rows " +
                                     std::to_string(stride) + " apart, act " + std::to_string(act) +
                                     " (columns multiples of 32 up to " + std::to_string(LINEAR_MAX_K) +
                                     " in all, x1 bound when K1 > 0, levels positive)");
    const uint64_t K = K0 + K1;
    TGX_TRY(holds(b, 0, "x0", (uint64_t)rows * K0 * 4));
    if (K1) TGX_TRY(holds(b, 1, "x1", (uint64_t)rows * K1 * 4));
    TGX_TRY(holds(b, 2, "w", round_up(N, 16) * K * 2));
    TGX_TRY(holds(b, 3, "bias", (uint64_t)N * 4));
    TGX_TRY(holds(b, 4, "out", ((uint64_t)(rows - 1) * stride + offset + N) * 4));
    LinearArgs l{};
    l.w = (const uint16_t*)b[2].ptr;
    l.bias = (const float*)b[3].ptr;
    l.x0 = (const float*)b[0].ptr;
    l.x1 = (const float*)b[1].ptr;
    l.out = (float*)b[4].ptr;
    l.K0 = (int)K0;
    l.K1 = (int)K1;
    l.N = (int)N;
    l.rows = (int)rows;
    l.offset = (int)offset;
    l.stride = (int)stride;
    l.act = (int)act;
    l.levels = levels;
    return capture_one("gemv_linear", [&] { return launch_linear("gemv_linear", l, nullptr, nullptr); }, L);
}

// select_rows (select_rows.comp): flags, a, b -> out; constants rows, K. out[r] = flags[r] ? a[r]
// : b[r], rows of K f32 values (K a multiple of 4).
tgx_status build_select_rows(const Bound* b, const uint32_t* c, Launch* L) {
    const uint32_t rows = c[0], K = c[1];
    if (rows == 0 || K == 0 || K % 4 || (uint64_t)rows * K > (1u << 30))
        return fail(TGX_E_SHAPE, "select_rows: " + std::to_string(rows) + " rows of " + std::to_string(K) + " (a multiple of 4)");
    const uint64_t n = (uint64_t)rows * K * 4;
    TGX_TRY(holds(b, 0, "flags", (uint64_t)rows * 4));
    TGX_TRY(holds(b, 1, "a", n));
    TGX_TRY(holds(b, 2, "b", n));
    TGX_TRY(holds(b, 3, "out", n));
    return capture_one("select_rows", [&] {
        return launch_select_rows((const uint32_t*)b[0].ptr, (const float*)b[1].ptr, (const float*)b[2].ptr, (float*)b[3].ptr, (int)rows,
                                  (int)K, nullptr, nullptr);
    }, L);
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
         decode_constants({"sq_cols"}),
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
         decode_constants({"sq_cols"}),
         build_gate_up},
        {"rmsnorm",
         {{"x", RD, TGX_F32, false}, {"gain", RD, TGX_F32, false}, {"out", WR, TGX_F32, false}, {"positions", WR, TGX_U32, true}},
         decode_constants({"advance"}),
         build_rmsnorm},
        {"stream_read", {{"data", RD, TGX_U32, false}, {"out", WR, TGX_U32, false}}, {}, build_stream_read},
        // The prefill's (prefill.rs:32-81): the GEMMs carry rope_rows, add_norm_rows and
        // silu_mul_rows as their epilogues.
        {"norm_rows", {{"x", RD, TGX_F32, false}, {"gain", RD, TGX_F32, false}, {"out", WR, TGX_BF16, false}}, prefill_constants(),
         build_norm_rows},
        {"final_norm_rows", {{"x", RD, TGX_F32, false}, {"gain", RD, TGX_F32, false}, {"out", WR, TGX_F32, false}},
         prefill_constants(), build_final_norm_rows},
        {"gemm_rope_rows",
         {{"x", RD, TGX_BF16, false},
          {"w", RD, TGX_BF16, false},
          {"row_sq", RD, TGX_F32, true},
          {"cos", RD, TGX_F32, false},
          {"sin", RD, TGX_F32, false},
          {"positions", RD, TGX_U32, false},
          {"slots", RD, TGX_U32, false},
          {"table", RD, TGX_U32, false},
          {"q", WR, TGX_BF16, false},
          {"kv", WR, TGX_BF16, false}},
         prefill_constants(),
         build_gemm_rope_rows},
        {"attention_rows",
         {{"q", RD, TGX_BF16, false},
          {"kv", RD, TGX_BF16, false},
          {"table", RD, TGX_U32, false},
          {"tiles", RD, TGX_U32, false},
          {"attended", WR, TGX_BF16, false}},
         prefill_constants({"tiles"}),
         build_attention_rows},
        {"gemm_add_norm_rows",
         {{"x", RD, TGX_BF16, false},
          {"w", RD, TGX_BF16, false},
          {"residual", RD, TGX_F32, false},
          {"next_gain", RD, TGX_F32, true},
          {"out", WR, TGX_F32, false},
          {"out_n", WR, TGX_BF16, true},
          {"out_sq", WR, TGX_F32, true}},
         prefill_constants({"K", "N", "strip_rows", "residual_in"}),
         build_gemm_add_norm_rows},
        {"gemm_silu_mul_rows",
         {{"x", RD, TGX_BF16, false}, {"w", RD, TGX_BF16, false}, {"row_sq", RD, TGX_F32, true}, {"mlp", WR, TGX_BF16, false}},
         prefill_constants({"K", "N"}),
         build_gemm_silu_mul_rows},
        // The local stacks' and the sampler's (local/mod.rs:28-113).
        {"local_norm",
         {{"x", RD, TGX_F32, false}, {"gain", RD, TGX_F32, false}, {"normed", WR, TGX_BF16, false}, {"row_sq", WR, TGX_F32, false}},
         local_constants(),
         build_local_norm},
        {"local_qkv_rope",
         {{"x", RD, TGX_BF16, false},
          {"w", RD, TGX_BF16, false},
          {"row_sq", RD, TGX_F32, false},
          {"cos", RD, TGX_F32, false},
          {"sin", RD, TGX_F32, false},
          {"q", WR, TGX_BF16, false},
          {"k", WR, TGX_BF16, false},
          {"v", WR, TGX_BF16, false}},
         local_constants(),
         build_local_qkv_rope},
        {"local_attention",
         {{"q", RD, TGX_BF16, false}, {"k", RD, TGX_BF16, false}, {"v", RD, TGX_BF16, false}, {"attended", WR, TGX_BF16, false}},
         local_constants(),
         build_local_attention},
        {"local_partial", {{"x", RD, TGX_BF16, false}, {"w", RD, TGX_BF16, false}, {"partial", WR, TGX_F32, false}},
         local_constants({"K", "N", "parts"}), build_local_partial},
        {"local_add_norm",
         {{"partial", RD, TGX_F32, true},
          {"residual", RD, TGX_F32, false},
          {"gain", RD, TGX_F32, false},
          {"sum", WR, TGX_F32, true},
          {"normed", WR, TGX_BF16, false},
          {"row_sq", WR, TGX_F32, false}},
         local_constants({"parts"}),
         build_local_add_norm},
        {"local_final_norm",
         {{"partial", RD, TGX_F32, true},
          {"residual", RD, TGX_F32, false},
          {"gain", RD, TGX_F32, false},
          {"sum", WR, TGX_F32, true},
          {"out", WR, TGX_F32, false}},
         local_constants({"parts"}),
         build_local_final_norm},
        {"local_gemm_add_norm",
         {{"x", RD, TGX_BF16, false},
          {"w", RD, TGX_BF16, false},
          {"residual", RD, TGX_F32, false},
          {"next_gain", RD, TGX_F32, true},
          {"sum", WR, TGX_F32, false},
          {"normed", WR, TGX_BF16, true},
          {"row_sq", WR, TGX_F32, true}},
         local_constants({"K", "N", "parts"}),
         build_local_gemm_add_norm},
        {"local_gate_up",
         {{"x", RD, TGX_BF16, false}, {"w", RD, TGX_BF16, false}, {"row_sq", RD, TGX_F32, false}, {"mlp", WR, TGX_BF16, false}},
         local_constants(),
         build_local_gate_up},
        {"local_embed",
         {{"frames", RD, TGX_F32, false},
          {"w", RD, TGX_F32, false},
          {"bias", RD, TGX_F32, false},
          {"tokens", RD, TGX_F32, false},
          {"gain", RD, TGX_F32, true},
          {"x0", WR, TGX_F32, false},
          {"normed", WR, TGX_BF16, true},
          {"row_sq", WR, TGX_F32, true}},
         local_constants({"patch_rows", "channels", "frames", "first", "copy_at", "copies", "guided", "shared", "seqs"}),
         build_local_embed},
        {"cfm_noise", {{"noise", RD, TGX_F32, false}, {"sampling", RD, TGX_F32, false}, {"state", WR, TGX_F32, false}}, {"rows", "len"},
         build_cfm_noise},
        {"dit_euler",
         {{"x", RD, TGX_F32, false},
          {"row_sq", RD, TGX_F32, false},
          {"gain", RD, TGX_F32, false},
          {"w", RD, TGX_BF16, false},
          {"bias", RD, TGX_F32, false},
          {"sampling", RD, TGX_F32, false},
          {"state", WR, TGX_F32, false}},
         local_constants({"patch_rows", "channels", "frames", "first", "dt"}),
         build_dit_euler},
        // The layers between VoxCPM2's LMs (lm_side.rs:28-38) and the prompt's row select (prompt.rs:55-60).
        {"gemv_linear",
         {{"x0", RD, TGX_F32, false},
          {"x1", RD, TGX_F32, true},
          {"w", RD, TGX_BF16, false},
          {"bias", RD, TGX_F32, false},
          {"out", WR, TGX_F32, false}},
         {"rows", "K0", "K1", "N", "offset", "stride", "act", "levels"},
         build_gemv_linear},
        {"select_rows",
         {{"flags", RD, TGX_U32, false}, {"a", RD, TGX_F32, false}, {"b", RD, TGX_F32, false}, {"out", WR, TGX_F32, false}},
         {"rows", "K"},
         build_select_rows},
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
    bool ran = false;  // the last run has finished
    // The GPU clock's ticks at `origin`, an event recorded right after a one-wave kernel read the
    // clock into clock_host (re-taken by a start at most once a second): the run's events become
    // ticks from it (tgx_program_ends).
    hipEvent_t origin = nullptr;
    uint64_t* clock_host = nullptr;
    std::chrono::steady_clock::time_point origin_at{};
    bool origin_set = false;
};

// Drops what the program recorded: its launches, graph, timing events and the bindings it holds.
static void release_program(Program* p) {
    for (tgx_memory* m : p->memories) --m->programs;
    p->memories.clear();
    p->launches.clear();
    p->nodes.clear();
    p->frontier.clear();
    p->after.clear();
    if (p->exec) hipGraphExecDestroy(p->exec);
    if (p->graph) hipGraphDestroy(p->graph);
    p->exec = nullptr;
    p->graph = nullptr;
    for (hipEvent_t e : p->t_start) if (e) hipEventDestroy(e);
    for (hipEvent_t e : p->t_stop) if (e) hipEventDestroy(e);
    p->t_start.clear();
    p->t_stop.clear();
    p->timings_valid = false;
    p->ran = false;
    p->ended = false;
}

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

int tgx_attention_tile(int heads, int kv_heads, int head_dim) {
    if (kv_heads <= 0 || heads <= 0 || heads % kv_heads != 0 || heads / kv_heads > 16 || (head_dim != 64 && head_dim != 128)) return 0;
    return prefill_attention_tile(heads / kv_heads, head_dim);
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
    if (e == hipSuccess) e = hipEventCreate(&p->origin);
    if (e == hipSuccess) e = hipHostMalloc((void**)&p->clock_host, sizeof(uint64_t), hipHostMallocDefault);
    if (e != hipSuccess) {
        if (p->ev_start) hipEventDestroy(p->ev_start);
        if (p->ev_end) hipEventDestroy(p->ev_end);
        if (p->origin) hipEventDestroy(p->origin);
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
    np.kernelParams = L->kernel_params();
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
    const auto now = std::chrono::steady_clock::now();
    if (!p->origin_set || now - p->origin_at > std::chrono::seconds(1)) {
        // The clock's reading for tgx_program_ends, anchored close to the run (an event's time
        // relative to another is a float of milliseconds).
        TGX_HIP(launch_read_clock(p->clock_host, s));
        TGX_HIP(hipEventRecord(p->origin, s));
        p->origin_at = now;
        p->origin_set = true;
    }
    TGX_HIP(hipEventRecord(p->ev_start, s));
    p->ran = false;
    if (p->timed) {
        // Dispatch by dispatch in order, each between events of its own.
        for (size_t i = 0; i < p->launches.size(); ++i) {
            Launch& L = *p->launches[i];
            TGX_HIP(hipExtLaunchKernel(L.k.func, L.k.grid, L.k.block, L.kernel_params(), L.k.lds, s, p->t_start[i], p->t_stop[i], 0));
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
    const tgx_status r = wait_event(p->ctx, p->ev_end, "the program");
    if (r == TGX_E_TIMEOUT) return r;  // still running: it stays pending
    for (tgx_memory* m : p->memories) --m->running;
    p->pending = false;
    if (r == TGX_OK) p->ran = true;
    return r;
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
    release_program(p);
    hipEventDestroy(p->ev_start);
    hipEventDestroy(p->ev_end);
    hipEventDestroy(p->origin);
    hipHostFree(p->clock_host);
    delete p;
    delete prog;
    return st;
}

tgx_status tgx_program_ends(tgx_program* prog, uint64_t ends[2]) {
    clear_error();
    if (!prog || !ends) return fail(TGX_E_ARG, "null program or ends");
    Program* p = prog->p;
    if (p->pending || !p->ran) return fail(TGX_E_BUSY, "the ends of a program not run to the end");
    float ms[2] = {0.f, 0.f};
    TGX_HIP(hipEventElapsedTime(&ms[0], p->origin, p->ev_start));
    TGX_HIP(hipEventElapsedTime(&ms[1], p->origin, p->ev_end));
    for (int i = 0; i < 2; ++i) ends[i] = *p->clock_host + (uint64_t)std::llround((double)ms[i] * 1e6 / p->ctx->tick_ns);
    return TGX_OK;
}

tgx_status tgx_program_reset(tgx_program* prog, int timed) {
    clear_error();
    if (!prog) return fail(TGX_E_ARG, "null program");
    Program* p = prog->p;
    TGX_TRY(tgx_program_wait(prog));
    release_program(p);
    p->timed = timed != 0;
    TGX_HIP(hipGraphCreate(&p->graph, 0));
    return TGX_OK;
}

tgx_status tgx_context_dispatch(tgx_context* ctx, const tgx_dispatch* d, float* ms) {
    clear_error();
    if (!ctx || !d) return fail(TGX_E_ARG, "null context or dispatch");
    tgx_program* prog = nullptr;
    TGX_TRY(tgx_program_begin(ctx, 1, &prog));
    tgx_status st = tgx_program_launch(prog, d);
    if (st == TGX_OK) st = tgx_program_end(prog);
    if (st == TGX_OK) st = tgx_program_run(prog);
    tgx_timing t{};
    int n = 0;
    if (st == TGX_OK) st = tgx_program_timings(prog, 1, &t, &n);
    const std::string why = last_error();
    const tgx_status gone = tgx_program_destroy(prog);
    if (st != TGX_OK) return fail(st, why);
    if (gone != TGX_OK) return gone;
    if (ms) *ms = t.ms;
    return TGX_OK;
}

tgx_status tgx_context_set_fence_spin(tgx_context* ctx, uint64_t ns) {
    clear_error();
    if (!ctx) return fail(TGX_E_ARG, "null context");
    ctx->ctx->fence_spin_ns.store(ns, std::memory_order_relaxed);
    return TGX_OK;
}

tgx_status tgx_context_calibrate(tgx_context* ctx, tgx_calibration* out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or out");
    Context* c = ctx->ctx;
    if (!c->clock_host) TGX_HIP(hipHostMalloc((void**)&c->clock_host, sizeof(uint64_t), hipHostMallocDefault));
    hipStream_t s = c->stream;
    TGX_HIP(hipStreamSynchronize(s));  // nothing queued ahead of the reading
    auto monotonic = [] {
        timespec t{};
        clock_gettime(CLOCK_MONOTONIC, &t);
        return (uint64_t)t.tv_sec * 1000000000ull + (uint64_t)t.tv_nsec;
    };
    const uint64_t before = monotonic();
    TGX_HIP(launch_read_clock(c->clock_host, s));
    TGX_HIP(hipStreamSynchronize(s));
    const uint64_t after = monotonic();
    out->ticks = *c->clock_host;
    out->monotonic_ns = before + (after - before) / 2;
    out->deviation_ns = (after - before + 1) / 2;
    out->period_ns = (float)c->tick_ns;
    return TGX_OK;
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
