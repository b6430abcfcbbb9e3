// The local encoder (crates/graph/src/local/encoder.rs:42-198) and the patch step that chains it
// with the LM side and the sampler (crates/graph/src/patch.rs:98-166, 356-415).
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>

#include "patch.hpp"

namespace tgx {

namespace {

template <typename T>
tgx_status encoder_alloc(Encoder* e, T** out, size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count, 1) * sizeof(T);
    hipError_t err = hipMalloc(&p, bytes);
    if (err != hipSuccess) return fail(TGX_E_HIP, "hipMalloc of " + std::to_string(bytes) + " bytes: " + hipGetErrorString(err));
    e->allocations.push_back({p, bytes});
    e->device_bytes += bytes;
    err = hipMemset(p, 0, bytes);
    if (err != hipSuccess) return fail(TGX_E_HIP, std::string("hipMemset: ") + hipGetErrorString(err));
    *out = (T*)p;
    return TGX_OK;
}

tgx_status shape_fail(const std::string& why) { return fail(TGX_E_SHAPE, "encoder: " + why); }

// Records `enqueue`'s dispatches on `st` as a graph.
template <typename F>
tgx_status record(hipStream_t st, const char* what, F enqueue, hipGraphExec_t* exec) {
    if (*exec) {
        hipGraphExecDestroy(*exec);
        *exec = nullptr;
    }
    TGX_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    hipError_t err = enqueue();
    hipGraph_t graph = nullptr;
    hipError_t end = hipStreamEndCapture(st, &graph);
    if (err != hipSuccess) {
        if (graph) hipGraphDestroy(graph);
        return fail(TGX_E_HIP, std::string("recording ") + what + ": " + hipGetErrorString(err));
    }
    if (end != hipSuccess) return fail(TGX_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(end));
    hipError_t e = hipGraphInstantiate(exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    return upload_graph(*exec, st);
}

}  // namespace

LocalArgs Encoder::args() const {
    LocalArgs a{};
    a.M = M;
    a.M_pad = M_pad;
    a.T = T;
    a.hidden = shape.hidden;
    a.inner = shape.inner;
    a.heads = shape.heads;
    a.kv_heads = shape.kv_heads;
    a.eps = shape.eps;
    a.scale = 1.0f / std::sqrt((float)HEAD_DIM);
    a.rope = shape.rope ? 1 : 0;
    a.cos = cos;
    a.sin = sin;
    return a;
}

tgx_status encoder_create(Context* ctx, const tgx_shape* stack, const tgx_patch_shape* patch, Encoder** out) {
    if (!ctx || !stack || !patch || !out) return fail(TGX_E_ARG, "null context, shape, patch or out");
    *out = nullptr;
    const int F = patch->patch_size, C = patch->feat_dim;
    const int T = 1 + F;  // the learned token, then the frames (encoder.rs:47)
    tgx_shape st = *stack;
    st.capacity = T;
    Shape s;
    TGX_TRY(check_shape(&st, &s));
    const int H = s.heads, KV = s.kv_heads;
    if (patch->rows < 1) return shape_fail("no rows");
    if (F < 1 || F > 4) return shape_fail(std::to_string(F) + " frames to a patch (1 to 4)");
    if (C < 16 || C % 16 || C > 64) return shape_fail(std::to_string(C) + " channels (16, 32, 48 or 64)");
    // The local stacks' heads are 64 wide (VoxCPM2's encoder and DiT: 1024 wide over 16 heads).
    if (s.head_dim != HEAD_DIM) return shape_fail("a local stack of head_dim " + std::to_string(s.head_dim) + " (the kernels take 64)");
    if (T > LOCAL_MAX_T || H % 4) return shape_fail(std::to_string(T) + " tokens of " + std::to_string(H) + " heads");
    if (s.inner % 256 || !local_supported(s.hidden, s.inner, H, KV, LOCAL_O_PARTS, LOCAL_DOWN_PARTS))
        return shape_fail("a local stack " + std::to_string(s.hidden) + " wide with an FFN " + std::to_string(s.inner) + " wide");
    hipError_t pe = local_prepare();
    if (pe != hipSuccess) return fail(TGX_E_HIP, std::string("the local stack's LDS: ") + hipGetErrorString(pe));
    Encoder* e = new Encoder();
    e->ctx = ctx;
    e->shape = s;
    e->feat = C;
    e->frames = F;
    e->rows = patch->rows;
    e->max_rows = patch->rows;
    e->T = T;
    e->M = patch->rows * T;
    e->M_pad = local_rows_padded(e->M);
    auto done = [&](tgx_status r) {
        if (r != TGX_OK) encoder_destroy(e);
        return r;
    };
    const size_t h = s.hidden, Mp = e->M_pad, att = (size_t)H * HEAD_DIM, qkv_rows = (size_t)(H + 2 * KV) * HEAD_DIM;
    tgx_status r = TGX_OK;
    auto A = [&](auto** p, size_t n) {
        if (r == TGX_OK) r = encoder_alloc(e, p, n);
    };
    e->layers.resize(s.layers);
    for (auto& L : e->layers) {
        A(&L.qkv, qkv_rows * h);
        A(&L.o, h * att);
        A(&L.gate_up, 2 * (size_t)s.inner * h);
        A(&L.down, h * s.inner);
        A(&L.input_norm, h);
        A(&L.post_norm, h);
    }
    A(&e->final_norm, h);
    A(&e->in_w, h * C);
    A(&e->in_b, h);
    A(&e->special, h);
    A(&e->cos, (size_t)T * HEAD_DIM / 2);
    A(&e->sin, (size_t)T * HEAD_DIM / 2);
    A(&e->x0, Mp * h);
    A(&e->x, Mp * h);
    A(&e->h, Mp * h);
    A(&e->partial, (size_t)LOCAL_MAX_PARTS * Mp * h);
    A(&e->out, Mp * h);
    A(&e->normed, Mp * h);
    A(&e->row_sq, Mp * (h / LOCAL_SQ_COLS));
    A(&e->q, Mp * att);
    A(&e->k, Mp * KV * HEAD_DIM);
    A(&e->v, Mp * KV * HEAD_DIM);
    A(&e->attended, Mp * att);
    A(&e->mlp, Mp * s.inner);
    A(&e->patch, (size_t)e->rows * C * F);
    A(&e->embedding, (size_t)e->rows * h);
    if (r != TGX_OK) return done(r);
    std::vector<float> cs, sn;
    rope_tables(s, cs, sn);
    hipError_t err = hipMemcpy(e->cos, cs.data(), (size_t)T * HEAD_DIM / 2 * 4, hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemcpy(e->sin, sn.data(), (size_t)T * HEAD_DIM / 2 * 4, hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipEventCreate(&e->ev_start);
    if (err == hipSuccess) err = hipEventCreate(&e->ev_end);
    if (err != hipSuccess) return done(fail(TGX_E_HIP, std::string("encoder set-up: ") + hipGetErrorString(err)));
    *out = e;
    return TGX_OK;
}

void encoder_destroy(Encoder* e) {
    if (!e) return;
    if (e->ctx) hipStreamSynchronize(e->ctx->stream);
    destroy_programs(e->programs);
    for (auto& b : e->allocations) hipFree(b.ptr);
    if (e->ev_start) hipEventDestroy(e->ev_start);
    if (e->ev_end) hipEventDestroy(e->ev_end);
    delete e;
}

// load_encoder (encoder.rs:133-162): the stack's tensors as tgx_decoder_load names them,
// "special_token" [hidden], "in_proj.weight" [hidden][feat] and "in_proj.bias" [hidden].
tgx_status encoder_load(Encoder* e, const char* name, const void* data, tgx_dtype dtype, size_t count) {
    if (!e || !name || !data) return fail(TGX_E_ARG, "null encoder, name or data");
    if (e->pending) return fail(TGX_E_BUSY, "an encoding is under way");
    if (dtype != TGX_F32 && dtype != TGX_BF16 && dtype != TGX_F16) return fail(TGX_E_ARG, "dtype");
    const std::string n = name;
    const size_t h = e->shape.hidden, C = e->feat;
    auto upload = [&](float* dst, size_t expect) -> tgx_status {
        if (count != expect)
            return fail(TGX_E_WEIGHTS, n + ": " + std::to_string(count) + " values, not " + std::to_string(expect));
        auto v = as_f32(data, dtype, count);
        TGX_HIP(hipMemcpy(dst, v.data(), expect * 4, hipMemcpyHostToDevice));
        return TGX_OK;
    };
    if (n == "norm") return upload(e->final_norm, h);
    if (n == "special_token") return upload(e->special, h);
    if (n == "in_proj.weight") return upload(e->in_w, h * C);
    if (n == "in_proj.bias") return upload(e->in_b, h);
    int l = -1;
    char what[128] = {0};
    if (std::sscanf(name, "layers.%d.%127s", &l, what) == 2 && l >= 0 && l < e->shape.layers)
        return load_layer_tensor(e->layers[l], e->shape, n, what, data, dtype, count, 16, 16);
    return fail(TGX_E_WEIGHTS, n + ": no such tensor of the encoder");
}

hipError_t encoder_enqueue(Encoder* e, const float* patch, float* dst, int* dispatches) {
    hipStream_t st = e->ctx->stream;
    const LocalArgs a = e->args();
    const int C = e->feat, F = e->frames;
    // Token 0 of each row's sequence the learned token, tokens 1 .. F in_proj of its frames
    // (encoder.rs:92-111).
    // The embedding writes every token, and with them the first layer's norm input.
    EmbedArgs emb{patch, e->in_w, e->in_b, e->special, e->x0, C, F, 1, 0, 1, 0, 1, 1, e->layers[0].input_norm, e->normed, e->row_sq};
    hipError_t err = launch_local_embed(a, emb, e->rows, st, nullptr);
    std::vector<LocalLayer> layers(e->shape.layers);
    for (int l = 0; l < e->shape.layers; ++l) {
        const Layer& L = e->layers[l];
        layers[l] = LocalLayer{L.qkv, L.o, L.gate_up, L.down, L.input_norm, L.post_norm};
    }
    const LocalBuffers b{e->x0, e->x,        e->h,   e->normed,  e->row_sq, e->normed, e->row_sq,   e->q,
                         e->k,  e->v,        e->attended, e->mlp, e->partial, e->out,  e->o_parts, e->down_parts};
    if (err == hipSuccess) err = launch_local_stack(a, layers.data(), e->shape.layers, e->final_norm, b, st, nullptr);
    // The learned token's output, the first of each sequence (encoder.rs:113-114).
    const size_t row = (size_t)e->shape.hidden * sizeof(float);
    if (err == hipSuccess) err = hipMemcpy2DAsync(dst, row, e->out, (size_t)e->T * row, row, e->rows, hipMemcpyDeviceToDevice, st);
    if (dispatches) *dispatches = 1 + local_stack_dispatches(a, b, e->shape.layers);  // the embedding, the stack
    return err;
}

tgx_status encoder_encode(Encoder* e, const float* patch, float* out) {
    if (!e || !patch || !out) return fail(TGX_E_ARG, "null encoder, patch or output");
    if (e->pending) return fail(TGX_E_BUSY, "an encoding is under way");
    hipStream_t st = e->ctx->stream;
    const size_t len = (size_t)e->rows * e->feat * e->frames;
    TGX_HIP(hipMemcpyAsync(e->patch, patch, len * 4, hipMemcpyHostToDevice, st));
    if (!e->exec) {
        TGX_TRY(record(st, "the encoder", [&] { return encoder_enqueue(e, e->patch, e->embedding, &e->dispatches); }, &e->exec));
        RowProgram prog;
        prog.exec = e->exec;
        prog.dispatches = e->dispatches;
        e->programs[e->rows] = prog;
    }
    TGX_HIP(hipEventRecord(e->ev_start, st));
    TGX_HIP(hipGraphLaunch(e->exec, st));
    TGX_HIP(hipEventRecord(e->ev_end, st));
    TGX_TRY(wait_event(e->ctx, e->ev_end, "the encoding"));
    const size_t n = (size_t)e->rows * e->shape.hidden;
    TGX_HIP(hipMemcpy(out, e->embedding, n * 4, hipMemcpyDeviceToHost));
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(out[i])) return fail(TGX_E_NOT_FINITE, "the embedding is not finite");
    return TGX_OK;
}

tgx_status encoder_use_rows(Encoder* e, int rows) {
    if (!e) return fail(TGX_E_ARG, "null encoder");
    if (e->pending) return fail(TGX_E_BUSY, "an encoding is under way");
    if (rows < 1 || rows > e->max_rows)
        return fail(TGX_E_SHAPE, std::to_string(rows) + " rows in an encoder of " + std::to_string(e->max_rows));
    if (rows == e->rows) return TGX_OK;
    e->rows = rows;
    e->M = rows * e->T;
    e->M_pad = local_rows_padded(e->M);
    auto it = e->programs.find(rows);
    e->exec = it == e->programs.end() ? nullptr : it->second.exec;
    e->dispatches = it == e->programs.end() ? 0 : it->second.dispatches;
    return TGX_OK;
}

// ---- the patch step ----

std::vector<int> program_rows(int rows) {
    std::vector<int> out;
    for (int r = 1; r < rows; r *= 2) out.push_back(r);
    out.push_back(rows);
    return out;
}

int program_for(int rows, int n) {
    for (int r : program_rows(rows))
        if (r >= n) return r;
    return rows;
}

namespace {

// The current rows' embedding of the sampler's cond into the LM side's input, recorded if need be.
tgx_status step_encode_program(PatchStep* p) {
    Encoder* e = p->encoder;
    auto it = p->encodes.find(e->rows);
    if (it == p->encodes.end()) {
        RowProgram prog;
        TGX_TRY(record(p->side->ctx->stream, "the encoder",
                       [&] { return encoder_enqueue(e, p->sampler->cond, p->side->enc, &prog.dispatches); }, &prog.exec));
        it = p->encodes.emplace(e->rows, prog).first;
    }
    p->encode = it->second.exec;
    return TGX_OK;
}

}  // namespace

tgx_status patch_step_use_rows(PatchStep* p, int rows) {
    if (!p) return fail(TGX_E_ARG, "null patch step");
    if (p->pending) return fail(TGX_E_BUSY, "a step is under way");
    // The LM side first: it keeps its program when it cannot switch. Past it, a part that cannot
    // switch takes all three back to the program they had (recorded already), so that they never
    // run at different row counts.
    const int before = p->side->rows;
    TGX_TRY(lm_side_use_rows(p->side, rows));
    tgx_status st = encoder_use_rows(p->encoder, rows);
    if (st == TGX_OK) st = sampler_use_rows(p->sampler, rows);
    if (st == TGX_OK) st = step_encode_program(p);
    if (st != TGX_OK) {
        const std::string msg = last_error();
        lm_side_use_rows(p->side, before);
        encoder_use_rows(p->encoder, before);
        sampler_use_rows(p->sampler, before);
        step_encode_program(p);
        return fail(st, msg);
    }
    return TGX_OK;
}

tgx_status patch_step_create(Encoder* e, LmSide* side, Sampler* s, PatchStep** out) {
    if (!e || !side || !s || !out) return fail(TGX_E_ARG, "null encoder, LM side, sampler or out");
    *out = nullptr;
    if (e->ctx != side->ctx || s->ctx != side->ctx) return fail(TGX_E_ARG, "the three are on different contexts");
    if (e->max_rows != side->max_rows || s->max_rows != side->max_rows)
        return fail(TGX_E_SHAPE, "an encoder of " + std::to_string(e->max_rows) + " rows, an LM side of " +
                                     std::to_string(side->max_rows) + " and a sampler of " + std::to_string(s->max_rows));
    if (e->shape.hidden != side->encoder)
        return fail(TGX_E_SHAPE, "an encoder " + std::to_string(e->shape.hidden) + " wide for an LM side taking " +
                                     std::to_string(side->encoder));
    if (side->dit != s->shape.hidden)
        return fail(TGX_E_SHAPE, "mu " + std::to_string(side->dit) + " wide for a sampler " + std::to_string(s->shape.hidden) + " wide");
    if (e->feat != s->feat || e->frames != s->frames) return fail(TGX_E_SHAPE, "the encoder's patch is not the sampler's");
    PatchStep* p = new PatchStep();
    p->encoder = e;
    p->side = side;
    p->sampler = s;
    // The three at the same program: the LM side's.
    tgx_status r = encoder_use_rows(e, side->rows);
    if (r == TGX_OK) r = sampler_use_rows(s, side->rows);
    if (r == TGX_OK) r = step_encode_program(p);
    if (r == TGX_OK && hipEventCreate(&p->ev_start) != hipSuccess) r = fail(TGX_E_HIP, "hipEventCreate");
    if (r == TGX_OK && hipEventCreate(&p->ev_end) != hipSuccess) r = fail(TGX_E_HIP, "hipEventCreate");
    if (r != TGX_OK) {
        patch_step_destroy(p);
        return r;
    }
    *out = p;
    return TGX_OK;
}

void patch_step_destroy(PatchStep* p) {
    if (!p) return;
    if (p->side && p->side->ctx) hipStreamSynchronize(p->side->ctx->stream);
    destroy_programs(p->encodes);
    if (p->ev_start) hipEventDestroy(p->ev_start);
    if (p->ev_end) hipEventDestroy(p->ev_end);
    delete p;
}

tgx_status patch_step_launch(PatchStep* p, int times, int advance) {
    if (!p) return fail(TGX_E_ARG, "null patch step");
    if (times <= 0) return fail(TGX_E_ARG, "times");
    LmSide* l = p->side;
    Sampler* s = p->sampler;
    if (p->pending || l->pending || s->pending || p->encoder->pending) return fail(TGX_E_BUSY, "a step is under way");
    TGX_TRY(sampler_prepare(s));
    if (s->exec_dirty) TGX_TRY(sampler_record(s));
    hipStream_t st = l->ctx->stream;
    TGX_TRY(hold_ahead(l->base, times, advance));
    TGX_TRY(hold_ahead(l->residual, times, advance));
    TGX_TRY(sync_slots(l->base));
    TGX_TRY(sync_slots(l->residual));
    const size_t mu_bytes = (size_t)l->rows * 2 * l->dit * 4;
    TGX_HIP(hipEventRecord(p->ev_start, st));
    for (int i = 0; i < times; ++i) {
        // The patch before (the sampler's cond) embedded into the LM side's input, the LM side's
        // step, its mu to the sampler, the sample (patch.rs:107-156).
        TGX_HIP(hipGraphLaunch(p->encode, st));
        TGX_HIP(hipGraphLaunch(advance ? l->advance_exec : l->exec, st));
        TGX_HIP(hipMemcpyAsync(s->mu, l->mu, mu_bytes, hipMemcpyDeviceToDevice, st));
        TGX_HIP(hipGraphLaunch(s->exec, st));
        if (advance) {
            moved_on(l->base, 1);
            moved_on(l->residual, 1);
        }
    }
    TGX_HIP(hipEventRecord(p->ev_end, st));
    p->pending = true;
    return TGX_OK;
}

tgx_status patch_step_wait(PatchStep* p) {
    if (!p) return fail(TGX_E_ARG, "null patch step");
    if (!p->pending) return TGX_OK;
    tgx_status r = wait_event(p->side->ctx, p->ev_end, "the patch step");
    if (r != TGX_E_TIMEOUT) p->pending = false;
    return r;
}

tgx_status patch_step_run(PatchStep* p, const tgx_row* rows, int nrows, const float* cond, const float* noise,
                          const float* sampling, float* patch, float* stop_logits) {
    if (!p || !rows || !cond || !noise || !sampling || !patch || !stop_logits)
        return fail(TGX_E_ARG, "null patch step or array");
    if (p->pending) return fail(TGX_E_BUSY, "a step is under way");
    LmSide* l = p->side;
    Sampler* s = p->sampler;
    if (nrows < 1 || nrows > l->max_rows)
        return fail(TGX_E_SHAPE, std::to_string(nrows) + " rows for a step of " + std::to_string(l->max_rows));
    const int R = program_for(l->max_rows, nrows);
    TGX_TRY(patch_step_use_rows(p, R));
    // The program's rows past the given ones are spare: no cache written, nothing read back.
    const size_t len = (size_t)s->feat * s->frames;
    std::vector<tgx_row> all(rows, rows + nrows);
    all.resize(R, tgx_row{TGX_SPARE, 0});
    std::vector<float> c(cond, cond + nrows * len), z(noise, noise + nrows * len), g(sampling, sampling + nrows * 2);
    c.resize(R * len, 0.f);
    z.resize(R * len, 0.f);
    g.resize((size_t)R * 2, 0.f);
    TGX_TRY(lm_side_set_rows(l, all.data(), R, nullptr));
    TGX_TRY(sampler_set_inputs(s, nullptr, c.data(), z.data(), g.data()));
    TGX_TRY(patch_step_launch(p, 1, 0));
    TGX_TRY(patch_step_wait(p));
    std::vector<float> out(R * len), logits((size_t)R * 2);
    TGX_TRY(sampler_read(s, out.data()));
    TGX_TRY(lm_side_read(l, "stop_logits", logits.data(), logits.size()));
    std::copy(out.begin(), out.begin() + nrows * len, patch);
    std::copy(logits.begin(), logits.begin() + (size_t)nrows * 2, stop_logits);
    return TGX_OK;
}

}  // namespace tgx
