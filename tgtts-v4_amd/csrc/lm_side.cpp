// The LM side's host side (crates/graph/src/lm_side.rs:337-491): enc_to_lm_proj embeds the
// patch for the base LM; the scalar quantizer's in_proj rounds its output and out_proj widens it
// back; fusion_concat_proj joins that with the embedding for the residual LM, which runs without
// RoPE; mu is lm_to_dit_proj of the quantized output beside res_to_dit_proj of the residual LM's,
// and the stop logits stop_head of SiLU(stop_proj) of the quantized output. Both LMs are
// decoders over one batch; the whole step is recorded as one HIP graph.
#include <chrono>
#include <cmath>
#include <cstring>
#include <thread>

#include "patch.hpp"

namespace tgx {

namespace {

template <typename T>
tgx_status side_alloc(LmSide* s, T** out, size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count, 1) * sizeof(T);
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(TGX_E_HIP, "hipMalloc of " + std::to_string(bytes) + " bytes: " + hipGetErrorString(e));
    s->allocations.push_back({p, bytes});
    e = hipMemset(p, 0, bytes);
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string("hipMemset: ") + hipGetErrorString(e));
    *out = (T*)p;
    return TGX_OK;
}

tgx_status make_linear(LmSide* s, Linear& l, int n, int k, const char* name) {
    if (k % 32 || k > LINEAR_MAX_K || n <= 0)
        return fail(TGX_E_SHAPE, std::string(name) + ": " + std::to_string(n) + " x " + std::to_string(k) +
                                     " (columns a multiple of 32 up to " + std::to_string(LINEAR_MAX_K) + ")");
    l.N = n;
    l.K = k;
    const int n_pad = (n + 15) / 16 * 16;
    TGX_TRY(side_alloc(s, &l.w, (size_t)n_pad * k));
    return side_alloc(s, &l.b, (size_t)n);
}

struct Head {
    const char* name;
    Linear LmSide::*layer;
    bool bias;
};

// Heads::named (lm_side.rs:127-140).
const Head HEADS[] = {
    {"enc_to_lm_proj", &LmSide::enc_to_lm, true},   {"fsq_layer.in_proj", &LmSide::fsq_in, true},
    {"fsq_layer.out_proj", &LmSide::fsq_out, true}, {"fusion_concat_proj", &LmSide::fusion, true},
    {"lm_to_dit_proj", &LmSide::lm_to_dit, true},   {"res_to_dit_proj", &LmSide::res_to_dit, true},
    {"stop_proj", &LmSide::stop_proj, true},        {"stop_head", &LmSide::stop_head, false},
};

LinearArgs linear_args(const Linear& l, const float* x0, const float* x1, int k0, float* out, int rows, int offset,
                       int stride, int act, float levels) {
    LinearArgs a{};
    a.w = l.w;
    a.bias = l.b;
    a.x0 = x0;
    a.x1 = x1 ? x1 : x0;
    a.out = out;
    a.K0 = k0;
    a.K1 = l.K - k0;
    a.N = l.N;
    a.rows = rows;
    a.offset = offset;
    a.stride = stride;
    a.act = act;
    a.levels = levels;
    return a;
}

tgx_status side_record(LmSide* s, int advance, hipGraphExec_t* exec) {
    *exec = nullptr;
    hipStream_t st = s->ctx->stream;
    TGX_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int n = 0;
    hipError_t err = lm_side_enqueue(s, advance, nullptr, &n);
    hipGraph_t graph = nullptr;
    hipError_t end = hipStreamEndCapture(st, &graph);
    if (err != hipSuccess) {
        if (graph) hipGraphDestroy(graph);
        return fail(TGX_E_HIP, std::string("recording the LM side: ") + hipGetErrorString(err));
    }
    if (end != hipSuccess) return fail(TGX_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(end));
    hipError_t e = hipGraphInstantiate(exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    TGX_TRY(upload_graph(*exec, st));
    s->dispatches = n;
    return TGX_OK;
}

// The program of s->rows rows as the current one, recorded if it has not been.
tgx_status side_program(LmSide* s) {
    auto it = s->programs.find(s->rows);
    if (it == s->programs.end()) {
        RowProgram p;
        tgx_status st = side_record(s, 0, &p.exec);
        if (st == TGX_OK) st = side_record(s, 1, &p.advance);
        if (st != TGX_OK) {
            if (p.exec) hipGraphExecDestroy(p.exec);
            return st;
        }
        p.dispatches = s->dispatches;
        it = s->programs.emplace(s->rows, p).first;
    }
    s->exec = it->second.exec;
    s->advance_exec = it->second.advance;
    s->dispatches = it->second.dispatches;
    return TGX_OK;
}

}  // namespace

void destroy_programs(std::map<int, RowProgram>& programs) {
    for (auto& [rows, p] : programs) {
        if (p.exec) hipGraphExecDestroy(p.exec);
        if (p.advance) hipGraphExecDestroy(p.advance);
    }
    programs.clear();
}

tgx_status lm_side_use_rows(LmSide* s, int rows) {
    if (!s) return fail(TGX_E_ARG, "null LM side");
    if (s->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (rows < 1 || rows > s->max_rows)
        return fail(TGX_E_SHAPE, std::to_string(rows) + " rows in a batch of " + std::to_string(s->max_rows));
    if (rows == s->rows) return TGX_OK;
    const int before = s->rows;
    tgx_status st = decoder_use_rows(s->base, rows);
    if (st == TGX_OK) st = decoder_use_rows(s->residual, rows);
    if (st == TGX_OK) {
        s->rows = rows;
        st = side_program(s);
    }
    if (st != TGX_OK) {
        // Back to the program it had (recorded already), with its message kept.
        const std::string msg = last_error();
        s->rows = before;
        decoder_use_rows(s->base, before);
        decoder_use_rows(s->residual, before);
        side_program(s);
        return fail(st, msg);
    }
    return TGX_OK;
}

hipError_t lm_side_enqueue(LmSide* s, int advance, DispatchTimer* timer, int* dispatches) {
    hipStream_t st = s->ctx->stream;
    const int R = s->rows, h = s->hidden;
    Decoder* base = s->base;
    Decoder* res = s->residual;
    const float L = (float)s->levels;
    int n = 0, m = 0;
    hipError_t e = launch_linear("enc_to_lm_proj", linear_args(s->enc_to_lm, s->enc, nullptr, s->encoder, base->x_in, R, 0, h, ACT_NONE, L),
                                 st, timer);
    ++n;
    if (e == hipSuccess) e = decoder_enqueue(base, advance, timer, &m), n += m;
    if (e == hipSuccess)
        e = launch_linear("fsq_in_proj", linear_args(s->fsq_in, base->out, nullptr, h, s->levels_out, R, 0, s->latent, ACT_LEVELS, L), st, timer), ++n;
    if (e == hipSuccess)
        e = launch_linear("fsq_out_proj", linear_args(s->fsq_out, s->levels_out, nullptr, s->latent, s->lm_hidden, R, 0, h, ACT_NONE, L), st, timer), ++n;
    // The residual LM's input: fusion_concat_proj of [quantized output; embedding].
    if (e == hipSuccess)
        e = launch_linear("fusion_concat_proj", linear_args(s->fusion, s->lm_hidden, base->x_in, h, res->x_in, R, 0, h, ACT_NONE, L), st, timer), ++n;
    if (e == hipSuccess)
        e = launch_linear("lm_to_dit_proj", linear_args(s->lm_to_dit, s->lm_hidden, nullptr, h, s->mu, R, 0, 2 * s->dit, ACT_NONE, L), st, timer), ++n;
    if (e == hipSuccess)
        e = launch_linear("stop_proj", linear_args(s->stop_proj, s->lm_hidden, nullptr, h, s->stop_hidden, R, 0, h, ACT_SILU, L), st, timer), ++n;
    if (e == hipSuccess)
        e = launch_linear("stop_head", linear_args(s->stop_head, s->stop_hidden, nullptr, h, s->stop_logits, R, 0, 2, ACT_NONE, L), st, timer), ++n;
    if (e == hipSuccess) e = decoder_enqueue(res, advance, timer, &m), n += m;
    if (e == hipSuccess)
        e = launch_linear("res_to_dit_proj", linear_args(s->res_to_dit, res->out, nullptr, h, s->mu, R, s->dit, 2 * s->dit, ACT_NONE, L), st, timer), ++n;
    if (dispatches) *dispatches = n;
    return e;
}

tgx_status lm_side_create(Context* ctx, const tgx_shape* base, const tgx_shape* residual, const tgx_batch* batch,
                          const tgx_heads_shape* heads, LmSide** out) {
    if (!ctx || !base || !residual || !batch || !heads || !out) return fail(TGX_E_ARG, "null argument");
    *out = nullptr;
    if (residual->hidden != base->hidden || residual->capacity != base->capacity || residual->head_dim != base->head_dim)
        return fail(TGX_E_SHAPE, "a residual LM of " + std::to_string(residual->hidden) + " wide, " + std::to_string(residual->capacity) +
                                     " positions after a base LM of " + std::to_string(base->hidden) + ", " + std::to_string(base->capacity));
    if (heads->levels <= 0) return fail(TGX_E_SHAPE, "levels " + std::to_string(heads->levels));
    LmSide* s = new LmSide();
    s->ctx = ctx;
    auto done = [&](tgx_status st) {
        if (st != TGX_OK) lm_side_destroy(s);
        return st;
    };
    tgx_status r;
    if ((r = decoder_create(ctx, base, batch, &s->base)) != TGX_OK) return done(r);
    if ((r = decoder_create(ctx, residual, batch, &s->residual)) != TGX_OK) return done(r);
    s->rows = batch->rows;
    s->max_rows = batch->rows;
    s->hidden = base->hidden;
    s->encoder = heads->encoder;
    s->dit = heads->dit;
    s->latent = heads->latent;
    s->levels = heads->levels;
    const int h = s->hidden;
    if ((r = make_linear(s, s->enc_to_lm, h, s->encoder, "enc_to_lm_proj")) != TGX_OK) return done(r);
    if ((r = make_linear(s, s->fsq_in, s->latent, h, "fsq_layer.in_proj")) != TGX_OK) return done(r);
    if ((r = make_linear(s, s->fsq_out, h, s->latent, "fsq_layer.out_proj")) != TGX_OK) return done(r);
    if ((r = make_linear(s, s->fusion, h, 2 * h, "fusion_concat_proj")) != TGX_OK) return done(r);
    if ((r = make_linear(s, s->lm_to_dit, s->dit, h, "lm_to_dit_proj")) != TGX_OK) return done(r);
    if ((r = make_linear(s, s->res_to_dit, s->dit, h, "res_to_dit_proj")) != TGX_OK) return done(r);
    if ((r = make_linear(s, s->stop_proj, h, h, "stop_proj")) != TGX_OK) return done(r);
    if ((r = make_linear(s, s->stop_head, 2, h, "stop_head")) != TGX_OK) return done(r);
    const size_t R = s->rows;
    if ((r = side_alloc(s, &s->enc, R * s->encoder)) != TGX_OK) return done(r);
    if ((r = side_alloc(s, &s->levels_out, R * s->latent)) != TGX_OK) return done(r);
    if ((r = side_alloc(s, &s->lm_hidden, R * h)) != TGX_OK) return done(r);
    if ((r = side_alloc(s, &s->stop_hidden, R * h)) != TGX_OK) return done(r);
    if ((r = side_alloc(s, &s->mu, R * 2 * s->dit)) != TGX_OK) return done(r);
    if ((r = side_alloc(s, &s->stop_logits, R * 2)) != TGX_OK) return done(r);
    hipError_t e = hipEventCreate(&s->ev_start);
    if (e == hipSuccess) e = hipEventCreate(&s->ev_end);
    if (e != hipSuccess) return done(fail(TGX_E_HIP, std::string("hipEventCreate: ") + hipGetErrorString(e)));
    if ((r = side_program(s)) != TGX_OK) return done(r);
    *out = s;
    return TGX_OK;
}

void lm_side_destroy(LmSide* s) {
    if (!s) return;
    if (s->ctx) hipStreamSynchronize(s->ctx->stream);
    destroy_programs(s->programs);
    for (auto& b : s->allocations) hipFree(b.ptr);
    if (s->ev_start) hipEventDestroy(s->ev_start);
    if (s->ev_end) hipEventDestroy(s->ev_end);
    decoder_destroy(s->base);
    decoder_destroy(s->residual);
    delete s;
}

tgx_status lm_side_load(LmSide* s, const char* name, const void* data, tgx_dtype dtype, size_t count) {
    if (!s || !name || !data) return fail(TGX_E_ARG, "null LM side, name or data");
    if (s->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (dtype != TGX_F32 && dtype != TGX_BF16 && dtype != TGX_F16) return fail(TGX_E_ARG, "dtype");
    const std::string n = name;
    for (auto [prefix, dec] : {std::pair<const char*, Decoder*>{"base_lm.", s->base}, {"residual_lm.", s->residual}})
        if (n.compare(0, std::strlen(prefix), prefix) == 0) return decoder_load(dec, name + std::strlen(prefix), data, dtype, count);
    for (const Head& hd : HEADS) {
        const std::string stem = hd.name;
        if (n.compare(0, stem.size(), stem) != 0) continue;
        const std::string part = n.substr(stem.size());
        const Linear& l = s->*(hd.layer);
        if (part == ".weight") {
            if (count != (size_t)l.N * l.K)
                return fail(TGX_E_WEIGHTS, n + ": " + std::to_string(count) + " values, not " + std::to_string((size_t)l.N * l.K));
            std::vector<float> v = as_f32(data, dtype, count);
            const int n_pad = (l.N + 15) / 16 * 16;
            v.resize((size_t)n_pad * l.K, 0.f);
            auto t = tile_rows(v, n_pad, l.K, 16, [](int strip, int r) { return strip * 16 + r; });
            TGX_HIP(hipMemcpy(l.w, t.data(), t.size() * 2, hipMemcpyHostToDevice));
            return TGX_OK;
        }
        if (part == ".bias" && hd.bias) {
            if (count != (size_t)l.N)
                return fail(TGX_E_WEIGHTS, n + ": " + std::to_string(count) + " values, not " + std::to_string(l.N));
            std::vector<float> v = as_f32(data, dtype, count);
            TGX_HIP(hipMemcpy(l.b, v.data(), (size_t)l.N * 4, hipMemcpyHostToDevice));
            return TGX_OK;
        }
    }
    return fail(TGX_E_WEIGHTS, n + ": no such tensor of the LM side");
}

std::vector<LmHead> lm_side_heads() {
    std::vector<LmHead> out;
    for (const Head& h : HEADS) out.push_back({h.name, h.bias});
    return out;
}

tgx_status lm_side_set_rows(LmSide* s, const tgx_row* rows, int nrows, const float* enc) {
    if (!s || !rows) return fail(TGX_E_ARG, "null LM side or rows");
    if (s->pending) return fail(TGX_E_BUSY, "a step is under way");
    TGX_TRY(decoder_place(s->base, rows, nrows));
    TGX_TRY(decoder_place(s->residual, rows, nrows));
    if (enc) {
        TGX_HIP(hipMemcpyAsync(s->enc, enc, (size_t)s->rows * s->encoder * 4, hipMemcpyHostToDevice, s->ctx->stream));
        TGX_HIP(hipStreamSynchronize(s->ctx->stream));
    }
    return TGX_OK;
}

tgx_status lm_side_launch(LmSide* s, int times, int advance) {
    if (!s) return fail(TGX_E_ARG, "null LM side");
    if (s->pending || s->base->pending || s->residual->pending) return fail(TGX_E_BUSY, "a step is under way");
    if (times <= 0) return fail(TGX_E_ARG, "times");
    hipStream_t st = s->ctx->stream;
    TGX_TRY(hold_ahead(s->base, times, advance));
    TGX_TRY(hold_ahead(s->residual, times, advance));
    TGX_TRY(sync_slots(s->base));
    TGX_TRY(sync_slots(s->residual));
    TGX_HIP(hipEventRecord(s->ev_start, st));
    for (int i = 0; i < times; ++i) {
        if (s->use_graph) {
            TGX_HIP(hipGraphLaunch(advance ? s->advance_exec : s->exec, st));
        } else {
            hipError_t e = lm_side_enqueue(s, advance, nullptr, nullptr);
            if (e != hipSuccess) return fail(TGX_E_HIP, std::string("launching the LM side: ") + hipGetErrorString(e));
        }
        if (advance) {
            moved_on(s->base, 1);
            moved_on(s->residual, 1);
        }
    }
    TGX_HIP(hipEventRecord(s->ev_end, st));
    s->pending = true;
    return TGX_OK;
}

tgx_status lm_side_wait(LmSide* s) {
    if (!s) return fail(TGX_E_ARG, "null LM side");
    if (!s->pending) return TGX_OK;
    const tgx_status r = wait_event(s->ctx, s->ev_end, "the LM side");
    if (r != TGX_E_TIMEOUT) s->pending = false;
    return r;
}

tgx_status lm_side_read(LmSide* s, const char* tensor, float* out, size_t count) {
    if (!s || !tensor || !out) return fail(TGX_E_ARG, "null LM side, tensor or out");
    if (s->pending) return fail(TGX_E_BUSY, "a step is under way");
    const std::string n = tensor;
    const size_t R = s->rows, h = s->hidden;
    const float* src = nullptr;
    size_t len = 0;
    if (n == "embed") src = s->base->x_in, len = R * h;
    else if (n == "base_out") src = s->base->out, len = R * h;
    else if (n == "levels") src = s->levels_out, len = R * s->latent;
    else if (n == "lm_hidden") src = s->lm_hidden, len = R * h;
    else if (n == "residual_in") src = s->residual->x_in, len = R * h;
    else if (n == "residual_out") src = s->residual->out, len = R * h;
    else if (n == "stop_hidden") src = s->stop_hidden, len = R * h;
    else if (n == "mu") src = s->mu, len = R * 2 * s->dit;
    else if (n == "stop_logits") src = s->stop_logits, len = R * 2;
    else return fail(TGX_E_ARG, n + ": no such tensor of the LM side");
    if (count != len) return fail(TGX_E_SHAPE, n + ": " + std::to_string(len) + " values, not " + std::to_string(count));
    TGX_HIP(hipMemcpy(out, src, len * 4, hipMemcpyDeviceToHost));
    return TGX_OK;
}

}  // namespace tgx
