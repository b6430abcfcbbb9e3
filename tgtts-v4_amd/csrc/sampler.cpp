// The patch sampler's host side (crates/graph/src/local/dit.rs): its schedule, the time tokens
// computed from the time MLPs, the local DiT's weights and tensors, and the sample — noise,
// the condition's tokens, then each Euler step's embedding, DiT run and step — recorded as one
// HIP graph.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>

#include "patch.hpp"

namespace tgx {

// schedule (dit.rs:44-58): timesteps + 1 times from 1 to 0 as torch's linspace makes them in f32
// (from both ends towards the middle), each then swayed by t + (cos(pi t / 2) - 1 + t).
std::vector<float> euler_schedule(int timesteps) {
    const int steps = timesteps + 1;
    const float step = (0.0f - 1.0f) / (float)timesteps;
    std::vector<float> out(steps);
    for (int i = 0; i < steps; ++i) {
        const float t = i < steps / 2 ? 1.0f + step * (float)i : 0.0f - step * (float)(steps - i - 1);
        const float half_pi = 1.57079632679489661923f;
        out[i] = t + (std::cos(half_pi * t) - 1.0f + t);
    }
    return out;
}

// euler_steps (dit.rs:61-79): the first max(1, floor(0.04 (timesteps + 1))) steps run nothing;
// t and dt advance in f32 as solve_euler advances them.
void euler_steps(int timesteps, std::vector<float>& t_out, std::vector<float>& dt_out) {
    const std::vector<float> span = euler_schedule(std::max(timesteps, 1));
    const int n = (int)span.size();
    const int zero_init = std::max(1, (int)((double)n * 0.04));
    float t = span[0], dt = span[0] - span[1];
    t_out.clear();
    dt_out.clear();
    for (int step = 1; step < n; ++step) {
        if (step > zero_init) {
            t_out.push_back(t);
            dt_out.push_back(dt);
        }
        t -= dt;
        if (step < n - 1) dt = t - span[step + 1];
    }
}

namespace {

// SinusoidalPosEmb at scale 1000 (dit.rs:367-381): in f32, the sines then the cosines of 1000 t
// at frequencies exp(i rate), rate = -ln(10000) / (hidden / 2 - 1).
std::vector<double> time_embedding(float t, int hidden) {
    const int half = hidden / 2;
    const float rate = (float)(-(std::log(10000.0) / (double)(half - 1)));
    const float scaled = t * 1000.0f;
    std::vector<double> out(hidden);
    for (int i = 0; i < half; ++i) {
        const float angle = scaled * std::exp((float)i * rate);
        out[i] = (double)std::sin(angle);
        out[half + i] = (double)std::cos(angle);
    }
    return out;
}

template <typename T>
tgx_status sampler_alloc(Sampler* s, T** out, size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count, 1) * sizeof(T);
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(TGX_E_HIP, "hipMalloc of " + std::to_string(bytes) + " bytes: " + hipGetErrorString(e));
    s->allocations.push_back({p, bytes});
    s->device_bytes += bytes;
    e = hipMemset(p, 0, bytes);
    if (e != hipSuccess) return fail(TGX_E_HIP, std::string("hipMemset: ") + hipGetErrorString(e));
    *out = (T*)p;
    return TGX_OK;
}

tgx_status shape_fail(const std::string& why) { return fail(TGX_E_SHAPE, "sampler: " + why); }

}  // namespace

std::vector<double> TimeMlp::forward(const std::vector<double>& x, int hidden) const {
    std::vector<double> inner(hidden), out(hidden);
    for (int r = 0; r < hidden; ++r) {
        double acc = b1[r];
        for (int k = 0; k < hidden; ++k) acc += w1[(size_t)r * hidden + k] * x[k];
        inner[r] = acc / (1.0 + std::exp(-acc));
    }
    for (int r = 0; r < hidden; ++r) {
        double acc = b2[r];
        for (int k = 0; k < hidden; ++k) acc += w2[(size_t)r * hidden + k] * inner[k];
        out[r] = acc;
    }
    return out;
}

LocalArgs Sampler::args() const {
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

tgx_status sampler_create(Context* ctx, const tgx_shape* stack, const tgx_patch_shape* patch, Sampler** out) {
    if (!ctx || !stack || !patch || !out) return fail(TGX_E_ARG, "null context, shape, patch or out");
    *out = nullptr;
    const int F = patch->patch_size, C = patch->feat_dim;
    const int T = COND_AT + 2 * F;
    tgx_shape st = *stack;
    st.capacity = T;
    Shape s;
    TGX_TRY(check_shape(&st, &s));
    const int H = s.heads, KV = s.kv_heads;
    if (patch->rows < 1) return shape_fail("no rows");
    if (patch->timesteps < 1) return shape_fail("no timesteps");
    if (F < 1 || F > 4) return shape_fail(std::to_string(F) + " frames to a patch (1 to 4)");
    // dit_euler takes the channels as up to 4 MFMA strips of 16.
    if (C < 16 || C % 16 || C > 64)
        return shape_fail(std::to_string(C) + " channels of " + std::to_string(F) + " frames (16, 32, 48 or 64)");
    if (s.hidden != 1024) return shape_fail("a stack " + std::to_string(s.hidden) + " wide (the kernels take 1024)");
    // The local stacks' heads are 64 wide (VoxCPM2's encoder and DiT: 1024 wide over 16 heads).
    if (s.head_dim != HEAD_DIM) return shape_fail("a local stack of head_dim " + std::to_string(s.head_dim) + " (the kernels take 64)");
    // local_attention: a sequence's tokens as one MFMA tile, its query heads 4 to a workgroup.
    if (T > LOCAL_MAX_T || H % 4)
        return shape_fail(std::to_string(T) + " tokens of " + std::to_string(H) + " heads over " + std::to_string(KV));
    if (s.inner % 256 || !local_supported(s.hidden, s.inner, H, KV, LOCAL_O_PARTS, LOCAL_DOWN_PARTS))
        return shape_fail("a local stack " + std::to_string(s.hidden) + " wide with an FFN " + std::to_string(s.inner) + " wide");
    hipError_t pe = local_prepare();
    if (pe != hipSuccess) return fail(TGX_E_HIP, std::string("the local stack's LDS: ") + hipGetErrorString(pe));
    Sampler* smp = new Sampler();
    smp->ctx = ctx;
    smp->shape = s;
    smp->feat = C;
    smp->frames = F;
    smp->timesteps = patch->timesteps;
    smp->rows = patch->rows;
    smp->max_rows = patch->rows;
    smp->T = T;
    smp->M = patch->rows * 2 * T;
    smp->M_pad = local_rows_padded(smp->M);
    euler_steps(patch->timesteps, smp->step_t, smp->step_dt);
    auto done = [&](tgx_status st) {
        if (st != TGX_OK) sampler_destroy(smp);
        return st;
    };
    const size_t h = s.hidden, Mp = smp->M_pad, att = (size_t)H * HEAD_DIM, qkv_rows = (size_t)(H + 2 * KV) * HEAD_DIM;
    smp->layers.resize(s.layers);
    for (auto& L : smp->layers) {
        tgx_status r;
        if ((r = sampler_alloc(smp, &L.qkv, qkv_rows * h)) != TGX_OK) return done(r);
        if ((r = sampler_alloc(smp, &L.o, h * att)) != TGX_OK) return done(r);
        if ((r = sampler_alloc(smp, &L.gate_up, 2 * (size_t)s.inner * h)) != TGX_OK) return done(r);
        if ((r = sampler_alloc(smp, &L.down, h * s.inner)) != TGX_OK) return done(r);
        if ((r = sampler_alloc(smp, &L.input_norm, h)) != TGX_OK) return done(r);
        if ((r = sampler_alloc(smp, &L.post_norm, h)) != TGX_OK) return done(r);
    }
    tgx_status r = TGX_OK;
    auto A = [&](auto** p, size_t n) {
        if (r == TGX_OK) r = sampler_alloc(smp, p, n);
    };
    A(&smp->final_norm, h);
    A(&smp->in_w, h * C);
    A(&smp->in_b, h);
    A(&smp->cond_w, h * C);
    A(&smp->cond_b, h);
    A(&smp->out_w, (size_t)C * h);
    A(&smp->out_b, C);
    A(&smp->time_tokens, smp->step_t.size() * h + 1);
    A(&smp->cos, (size_t)T * HEAD_DIM / 2);
    A(&smp->sin, (size_t)T * HEAD_DIM / 2);
    A(&smp->x0, Mp * h);
    A(&smp->x, Mp * h);
    A(&smp->h, Mp * h);
    A(&smp->partial, (size_t)LOCAL_MAX_PARTS * Mp * h);
    A(&smp->normed, Mp * h);
    A(&smp->row_sq, Mp * (h / LOCAL_SQ_COLS));
    A(&smp->normed0, Mp * h);
    A(&smp->row_sq0, Mp * (h / LOCAL_SQ_COLS));
    A(&smp->q, Mp * att);
    A(&smp->k, Mp * KV * HEAD_DIM);
    A(&smp->v, Mp * KV * HEAD_DIM);
    A(&smp->attended, Mp * att);
    A(&smp->mlp, Mp * s.inner);
    A(&smp->mu, (size_t)smp->rows * MU_TOKENS * h);
    A(&smp->cond, (size_t)smp->rows * C * F);
    A(&smp->noise, (size_t)smp->rows * C * F);
    A(&smp->state, (size_t)smp->rows * C * F);
    A(&smp->sampling, (size_t)smp->rows * 2);
    if (r != TGX_OK) return done(r);
    for (TimeMlp* m : {&smp->time_mlp, &smp->delta_mlp}) {
        m->w1.assign(h * h, 0.0);
        m->w2.assign(h * h, 0.0);
        m->b1.assign(h, 0.0);
        m->b2.assign(h, 0.0);
    }
    std::vector<float> cs, sn;
    rope_tables(s, cs, sn);
    hipError_t e = hipMemcpy(smp->cos, cs.data(), (size_t)T * HEAD_DIM / 2 * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(smp->sin, sn.data(), (size_t)T * HEAD_DIM / 2 * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipEventCreate(&smp->ev_start);
    if (e == hipSuccess) e = hipEventCreate(&smp->ev_end);
    if (e != hipSuccess) return done(fail(TGX_E_HIP, std::string("sampler set-up: ") + hipGetErrorString(e)));
    *out = smp;
    return TGX_OK;
}

void sampler_destroy(Sampler* s) {
    if (!s) return;
    if (s->ctx) hipStreamSynchronize(s->ctx->stream);
    destroy_programs(s->programs);
    for (auto& b : s->allocations) hipFree(b.ptr);
    for (auto e : s->timer_start) hipEventDestroy(e);
    for (auto e : s->timer_stop) hipEventDestroy(e);
    if (s->ev_start) hipEventDestroy(s->ev_start);
    if (s->ev_end) hipEventDestroy(s->ev_end);
    delete s;
}

tgx_status sampler_load(Sampler* s, const char* name, const void* data, tgx_dtype dtype, size_t count) {
    if (!s || !name || !data) return fail(TGX_E_ARG, "null sampler, name or data");
    if (s->pending) return fail(TGX_E_BUSY, "a sample is under way");
    if (dtype != TGX_F32 && dtype != TGX_BF16 && dtype != TGX_F16) return fail(TGX_E_ARG, "dtype");
    const std::string n = name;
    const size_t h = s->shape.hidden, C = s->feat;
    auto want = [&](size_t expect) -> tgx_status {
        if (count != expect)
            return fail(TGX_E_WEIGHTS, n + ": " + std::to_string(count) + " values, not " + std::to_string(expect));
        return TGX_OK;
    };
    auto upload = [&](float* dst, size_t expect) -> tgx_status {
        TGX_TRY(want(expect));
        auto v = as_f32(data, dtype, count);
        TGX_HIP(hipMemcpy(dst, v.data(), expect * 4, hipMemcpyHostToDevice));
        return TGX_OK;
    };
    if (n == "norm") return upload(s->final_norm, h);
    if (n == "in_proj.weight") return upload(s->in_w, h * C);
    if (n == "in_proj.bias") return upload(s->in_b, h);
    if (n == "cond_proj.weight") return upload(s->cond_w, h * C);
    if (n == "cond_proj.bias") return upload(s->cond_b, h);
    if (n == "out_proj.weight") {
        TGX_TRY(want(C * h));
        auto t = tile_rows(as_f32(data, dtype, count), (int)C, (int)h, 16, [](int strip, int r) { return strip * 16 + r; });
        TGX_HIP(hipMemcpy(s->out_w, t.data(), t.size() * 2, hipMemcpyHostToDevice));
        return TGX_OK;
    }
    if (n == "out_proj.bias") return upload(s->out_b, C);
    for (int which = 0; which < 2; ++which) {
        const std::string prefix = which == 0 ? "time_mlp." : "delta_time_mlp.";
        if (n.compare(0, prefix.size(), prefix) != 0) continue;
        TimeMlp& m = which == 0 ? s->time_mlp : s->delta_mlp;
        const std::string part = n.substr(prefix.size());
        std::vector<double>* dst = nullptr;
        int bit = 0;
        if (part == "linear_1.weight") dst = &m.w1, bit = 1;
        else if (part == "linear_1.bias") dst = &m.b1, bit = 2;
        else if (part == "linear_2.weight") dst = &m.w2, bit = 4;
        else if (part == "linear_2.bias") dst = &m.b2, bit = 8;
        if (!dst) break;
        TGX_TRY(want(dst->size()));
        auto v = as_f32(data, dtype, count);
        for (size_t i = 0; i < v.size(); ++i) (*dst)[i] = (double)v[i];
        m.loaded |= bit;
        s->times_dirty = true;
        return TGX_OK;
    }
    int l = -1;
    char what[128] = {0};
    if (std::sscanf(name, "layers.%d.%127s", &l, what) == 2 && l >= 0 && l < s->shape.layers)
        return load_layer_tensor(s->layers[l], s->shape, n, what, data, dtype, count, 16, 16);
    return fail(TGX_E_WEIGHTS, n + ": no such tensor of the sampler");
}

// Each step's time token: time_mlp(emb(t)) + delta_time_mlp(emb(0)) in f64 (dit.rs:351-364; the
// step length is the DiT's input only in mean mode, which is refused, so the delta MLP sees 0).
tgx_status sampler_prepare(Sampler* s) {
    if (!s->times_dirty) return TGX_OK;
    if (s->time_mlp.loaded != 15 || s->delta_mlp.loaded != 15)
        return fail(TGX_E_WEIGHTS, "the time MLPs (time_mlp.*, delta_time_mlp.*) are not all loaded");
    const int h = s->shape.hidden;
    const std::vector<double> constant = s->delta_mlp.forward(time_embedding(0.0f, h), h);
    std::vector<float> tokens(s->step_t.size() * h);
    for (size_t i = 0; i < s->step_t.size(); ++i) {
        const std::vector<double> v = s->time_mlp.forward(time_embedding(s->step_t[i], h), h);
        for (int n = 0; n < h; ++n) tokens[i * h + n] = (float)(v[n] + constant[n]);
    }
    TGX_HIP(hipMemcpy(s->time_tokens, tokens.data(), tokens.size() * 4, hipMemcpyHostToDevice));
    s->times_dirty = false;
    return TGX_OK;
}

hipError_t sampler_enqueue(Sampler* s, const float* mu, DispatchTimer* timer, int* dispatches) {
    hipStream_t st = s->ctx->stream;
    const LocalArgs a = s->args();
    const int C = s->feat, F = s->frames, rows = s->rows;
    int n = 0;
    hipError_t e = launch_cfm_noise(s->noise, s->sampling, s->state, rows, C * F, st, timer);
    ++n;
    // The condition's tokens: cond_proj of the patch before at COND_AT, mu at 0 (zero in the
    // unconditional sequence), the same in every step (dit.rs:206-211).
    // Each embedding also writes its tokens' first-layer norm input into normed0 / row_sq0.
    const float* gain0 = s->layers[0].input_norm;
    EmbedArgs cond{s->cond, s->cond_w, s->cond_b, mu, s->x0, C, F, COND_AT, 0, MU_TOKENS, 1, 0, 2, gain0, s->normed0, s->row_sq0};
    if (e == hipSuccess) e = launch_local_embed(a, cond, rows, st, timer), ++n;
    std::vector<LocalLayer> layers(s->shape.layers);
    for (int l = 0; l < s->shape.layers; ++l) {
        const Layer& L = s->layers[l];
        layers[l] = LocalLayer{L.qkv, L.o, L.gate_up, L.down, L.input_norm, L.post_norm};
    }
    // No `out`: dit_euler takes the final norm of the tokens it reads.
    const LocalBuffers b{s->x0,       s->x,        s->h, s->normed, s->row_sq,   s->normed0, s->row_sq0, s->q, s->k,
                         s->v,        s->attended, s->mlp, s->partial, nullptr, s->o_parts, s->down_parts};
    const int x_at = COND_AT + F;
    for (size_t i = 0; i < s->step_t.size() && e == hipSuccess; ++i) {
        // in_proj of the patch so far at x_at, and the step's time token (dit.rs:213-219).
        EmbedArgs step{s->state, s->in_w, s->in_b, s->time_tokens + i * s->shape.hidden, s->x0, C, F, x_at, TIME_AT, 1, 0, 1, 2,
                       gain0, s->normed0, s->row_sq0};
        e = launch_local_embed(a, step, rows, st, timer);
        ++n;
        if (e == hipSuccess) e = launch_local_stack(a, layers.data(), s->shape.layers, s->final_norm, b, st, timer);
        n += local_stack_dispatches(a, b, s->shape.layers);
        EulerArgs eu{s->x, s->row_sq, s->final_norm, s->out_w, s->out_b, s->sampling, s->state, C, F, x_at, s->step_dt[i]};
        if (e == hipSuccess) e = launch_dit_euler(a, eu, rows, st, timer);
        ++n;
    }
    if (dispatches) *dispatches = n;
    return e;
}

tgx_status sampler_use_rows(Sampler* s, int rows) {
    if (!s) return fail(TGX_E_ARG, "null sampler");
    if (s->pending) return fail(TGX_E_BUSY, "a sample is under way");
    if (rows < 1 || rows > s->max_rows)
        return fail(TGX_E_SHAPE, std::to_string(rows) + " rows in a sampler of " + std::to_string(s->max_rows));
    if (rows == s->rows) return TGX_OK;
    s->rows = rows;
    s->M = rows * 2 * s->T;
    s->M_pad = local_rows_padded(s->M);
    auto it = s->programs.find(rows);
    s->exec = it == s->programs.end() ? nullptr : it->second.exec;
    s->dispatches = it == s->programs.end() ? 0 : it->second.dispatches;
    s->exec_dirty = it == s->programs.end();
    return TGX_OK;
}

tgx_status sampler_record(Sampler* s) {
    auto old = s->programs.find(s->rows);
    if (old != s->programs.end()) {
        hipGraphExecDestroy(old->second.exec);
        s->programs.erase(old);
    }
    s->exec = nullptr;
    hipStream_t st = s->ctx->stream;
    TGX_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int n = 0;
    hipError_t err = sampler_enqueue(s, s->mu, nullptr, &n);
    hipGraph_t graph = nullptr;
    hipError_t end = hipStreamEndCapture(st, &graph);
    if (err != hipSuccess) {
        if (graph) hipGraphDestroy(graph);
        return fail(TGX_E_HIP, std::string("recording the sample: ") + hipGetErrorString(err));
    }
    if (end != hipSuccess) return fail(TGX_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(end));
    hipError_t e = hipGraphInstantiate(&s->exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (e != hipSuccess) {
        s->exec = nullptr;
        return fail(TGX_E_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    }
    TGX_TRY(upload_graph(s->exec, st));
    s->dispatches = n;
    s->exec_dirty = false;
    RowProgram p;
    p.exec = s->exec;
    p.dispatches = n;
    s->programs[s->rows] = p;
    if ((int)s->timer_start.size() < n) {
        for (int i = (int)s->timer_start.size(); i < n; ++i) {
            hipEvent_t a = nullptr, b = nullptr;
            TGX_HIP(hipEventCreate(&a));
            TGX_HIP(hipEventCreate(&b));
            s->timer_start.push_back(a);
            s->timer_stop.push_back(b);
        }
        s->timer_labels.assign(n, nullptr);
        s->timer.start = s->timer_start.data();
        s->timer.stop = s->timer_stop.data();
        s->timer.labels = s->timer_labels.data();
        s->timer.capacity = n;
    }
    return TGX_OK;
}

tgx_status sampler_set_inputs(Sampler* s, const float* mu, const float* cond, const float* noise, const float* sampling) {
    if (!s) return fail(TGX_E_ARG, "null sampler");
    if (s->pending) return fail(TGX_E_BUSY, "a sample is under way");
    hipStream_t st = s->ctx->stream;
    const size_t rows = s->rows, len = (size_t)s->feat * s->frames;
    if (mu) TGX_HIP(hipMemcpyAsync(s->mu, mu, rows * MU_TOKENS * s->shape.hidden * 4, hipMemcpyHostToDevice, st));
    if (cond) TGX_HIP(hipMemcpyAsync(s->cond, cond, rows * len * 4, hipMemcpyHostToDevice, st));
    if (noise) TGX_HIP(hipMemcpyAsync(s->noise, noise, rows * len * 4, hipMemcpyHostToDevice, st));
    if (sampling) TGX_HIP(hipMemcpyAsync(s->sampling, sampling, rows * 2 * 4, hipMemcpyHostToDevice, st));
    TGX_HIP(hipStreamSynchronize(st));
    return TGX_OK;
}

tgx_status sampler_launch(Sampler* s, int times) {
    if (!s) return fail(TGX_E_ARG, "null sampler");
    if (s->pending) return fail(TGX_E_BUSY, "a sample is under way");
    if (times <= 0) return fail(TGX_E_ARG, "times");
    TGX_TRY(sampler_prepare(s));
    if (s->exec_dirty) TGX_TRY(sampler_record(s));
    hipStream_t st = s->ctx->stream;
    TGX_HIP(hipEventRecord(s->ev_start, st));
    for (int i = 0; i < times; ++i) {
        if (s->timed || !s->use_graph) {
            s->timer.used = 0;
            hipError_t e = sampler_enqueue(s, s->mu, s->timed ? &s->timer : nullptr, nullptr);
            if (e != hipSuccess) return fail(TGX_E_HIP, std::string("launching the sample: ") + hipGetErrorString(e));
        } else {
            TGX_HIP(hipGraphLaunch(s->exec, st));
        }
    }
    TGX_HIP(hipEventRecord(s->ev_end, st));
    s->pending = true;
    return TGX_OK;
}

tgx_status sampler_wait(Sampler* s) {
    if (!s) return fail(TGX_E_ARG, "null sampler");
    if (!s->pending) return TGX_OK;
    const tgx_status r = wait_event(s->ctx, s->ev_end, "the sample");
    if (r != TGX_E_TIMEOUT) s->pending = false;
    return r;
}

tgx_status sampler_read(Sampler* s, float* patch) {
    if (!s || !patch) return fail(TGX_E_ARG, "null sampler or patch");
    if (s->pending) return fail(TGX_E_BUSY, "a sample is under way");
    const size_t n = (size_t)s->rows * s->feat * s->frames;
    TGX_HIP(hipMemcpy(patch, s->state, n * 4, hipMemcpyDeviceToHost));
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(patch[i])) return fail(TGX_E_NOT_FINITE, "the sampled patch is not finite");
    return TGX_OK;
}

}  // namespace tgx
