// The C ABI of the patch sampler and the LM side (include/tgx.h): argument checks, the thread's
// error message, and nothing else.
#include <cmath>
#include <cstdio>
#include <string>

#include "handles.hpp"

namespace tgx {
const char* last_error();
}

using namespace tgx;

extern "C" {

// ---- the patch sampler ----

tgx_status tgx_euler_steps(int timesteps, int max, float* t, float* dt, int* n) {
    clear_error();
    if (!n) return fail(TGX_E_ARG, "null count");
    if (timesteps < 1) return fail(TGX_E_SHAPE, "no timesteps");
    std::vector<float> ts, dts;
    euler_steps(timesteps, ts, dts);
    *n = (int)ts.size();
    for (int i = 0; i < *n && i < max; ++i) {
        if (t) t[i] = ts[i];
        if (dt) dt[i] = dts[i];
    }
    return TGX_OK;
}

tgx_status tgx_sampler_create(tgx_context* ctx, const tgx_shape* stack, const tgx_patch_shape* patch, tgx_sampler** out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or output");
    Sampler* s = nullptr;
    TGX_TRY(sampler_create(ctx->ctx, stack, patch, &s));
    *out = new tgx_sampler{s};
    return TGX_OK;
}

void tgx_sampler_destroy(tgx_sampler* s) {
    if (!s) return;
    sampler_destroy(s->s);
    delete s;
}

#define SMP(p) ((p) ? (p)->s : nullptr)

tgx_status tgx_sampler_load(tgx_sampler* s, const char* name, const void* data, tgx_dtype dtype, size_t count) {
    clear_error();
    return sampler_load(SMP(s), name, data, dtype, count);
}

tgx_status tgx_sampler_sample(tgx_sampler* s, const float* mu, const float* cond, const float* noise, const float* sampling,
                              float* patch) {
    clear_error();
    if (!s || !mu || !cond || !noise || !sampling || !patch) return fail(TGX_E_ARG, "null sampler or array");
    // The whole batch: the program of all the rows (a patch step may have run fewer).
    TGX_TRY(sampler_use_rows(s->s, s->s->max_rows));
    TGX_TRY(sampler_set_inputs(s->s, mu, cond, noise, sampling));
    TGX_TRY(sampler_launch(s->s, 1));
    TGX_TRY(sampler_wait(s->s));
    return sampler_read(s->s, patch);
}

tgx_status tgx_sampler_launch(tgx_sampler* s, int times) {
    clear_error();
    return sampler_launch(SMP(s), times);
}

tgx_status tgx_sampler_wait(tgx_sampler* s) {
    clear_error();
    return sampler_wait(SMP(s));
}

tgx_status tgx_sampler_elapsed_ms(const tgx_sampler* s, float* out) {
    clear_error();
    if (!s || !out) return fail(TGX_E_ARG, "null sampler or output");
    if (s->s->pending) return fail(TGX_E_BUSY, "a sample is under way");
    TGX_HIP(hipEventElapsedTime(out, s->s->ev_start, s->s->ev_end));
    return TGX_OK;
}

tgx_status tgx_sampler_set_timed(tgx_sampler* s, int timed) {
    clear_error();
    if (!s) return fail(TGX_E_ARG, "null sampler");
    if (s->s->pending) return fail(TGX_E_BUSY, "a sample is under way");
    s->s->timed = timed != 0;
    return TGX_OK;
}

tgx_status tgx_sampler_timings(tgx_sampler* s, int max, tgx_timing* out, int* n) {
    clear_error();
    if (!s || !n) return fail(TGX_E_ARG, "null sampler or count");
    Sampler* p = s->s;
    if (p->pending) return fail(TGX_E_BUSY, "a sample is under way");
    if (!p->timed) {
        *n = 0;
        return TGX_OK;
    }
    *n = p->timer.used;
    for (int i = 0; i < p->timer.used && i < max && out; ++i) {
        float ms = 0.f;
        TGX_HIP(hipEventElapsedTime(&ms, p->timer.start[i], p->timer.stop[i]));
        std::snprintf(out[i].label, sizeof out[i].label, "%s", p->timer.labels[i]);
        out[i].ms = ms;
    }
    return TGX_OK;
}

tgx_status tgx_sampler_dispatches(const tgx_sampler* s, int* out) {
    clear_error();
    if (!s || !out) return fail(TGX_E_ARG, "null sampler or output");
    *out = s->s->dispatches;
    return TGX_OK;
}

// ---- the LM side ----

tgx_status tgx_lm_side_create(tgx_context* ctx, const tgx_shape* base, const tgx_shape* residual, const tgx_batch* batch,
                              const tgx_heads_shape* heads, tgx_lm_side** out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or output");
    LmSide* s = nullptr;
    TGX_TRY(lm_side_create(ctx->ctx, base, residual, batch, heads, &s));
    *out = new tgx_lm_side{s, tgx_decoder{s->base, true}, tgx_decoder{s->residual, true}};
    return TGX_OK;
}

void tgx_lm_side_destroy(tgx_lm_side* s) {
    if (!s) return;
    lm_side_destroy(s->s);
    delete s;
}

#define SIDE(p) ((p) ? (p)->s : nullptr)

tgx_status tgx_lm_side_load(tgx_lm_side* s, const char* name, const void* data, tgx_dtype dtype, size_t count) {
    clear_error();
    return lm_side_load(SIDE(s), name, data, dtype, count);
}

tgx_status tgx_lm_side_decoder(tgx_lm_side* s, int which, tgx_decoder** out) {
    clear_error();
    if (!s || !out) return fail(TGX_E_ARG, "null LM side or output");
    if (which != 0 && which != 1) return fail(TGX_E_ARG, "which: 0 (base LM) or 1 (residual LM)");
    *out = which == 0 ? &s->base : &s->residual;
    return TGX_OK;
}

tgx_status tgx_lm_side_set_rows(tgx_lm_side* s, const tgx_row* rows, int nrows, const float* enc) {
    clear_error();
    if (!s) return fail(TGX_E_ARG, "null LM side");
    // The whole batch: the program of all the rows (a patch step may have run fewer).
    TGX_TRY(lm_side_use_rows(s->s, s->s->max_rows));
    return lm_side_set_rows(s->s, rows, nrows, enc);
}

tgx_status tgx_lm_side_step(tgx_lm_side* s, const tgx_row* rows, int nrows, const float* enc, float* mu, float* stop_logits) {
    clear_error();
    if (!s || !rows || !enc || !mu || !stop_logits) return fail(TGX_E_ARG, "null LM side or array");
    LmSide* p = s->s;
    TGX_TRY(lm_side_use_rows(p, p->max_rows));
    TGX_TRY(lm_side_set_rows(p, rows, nrows, enc));
    TGX_TRY(lm_side_launch(p, 1, 0));
    TGX_TRY(lm_side_wait(p));
    const size_t n = (size_t)p->rows * 2 * p->dit;
    TGX_TRY(lm_side_read(p, "mu", mu, n));
    TGX_TRY(lm_side_read(p, "stop_logits", stop_logits, (size_t)p->rows * 2));
    for (int b = 0; b < nrows; ++b) {
        if (rows[b].position == TGX_SPARE) continue;
        for (int i = 0; i < 2 * p->dit; ++i)
            if (!std::isfinite(mu[(size_t)b * 2 * p->dit + i])) return fail(TGX_E_NOT_FINITE, "mu is not finite");
    }
    return TGX_OK;
}

tgx_status tgx_lm_side_launch(tgx_lm_side* s, int times, int advance) {
    clear_error();
    return lm_side_launch(SIDE(s), times, advance);
}

tgx_status tgx_lm_side_wait(tgx_lm_side* s) {
    clear_error();
    return lm_side_wait(SIDE(s));
}

tgx_status tgx_lm_side_elapsed_ms(const tgx_lm_side* s, float* out) {
    clear_error();
    if (!s || !out) return fail(TGX_E_ARG, "null LM side or output");
    if (s->s->pending) return fail(TGX_E_BUSY, "a step is under way");
    TGX_HIP(hipEventElapsedTime(out, s->s->ev_start, s->s->ev_end));
    return TGX_OK;
}

tgx_status tgx_lm_side_read(tgx_lm_side* s, const char* tensor, float* out, size_t count) {
    clear_error();
    return lm_side_read(SIDE(s), tensor, out, count);
}

tgx_status tgx_lm_side_dispatches(const tgx_lm_side* s, int* out) {
    clear_error();
    if (!s || !out) return fail(TGX_E_ARG, "null LM side or output");
    *out = s->s->dispatches;
    return TGX_OK;
}

// ---- a patch step ----

tgx_status tgx_patch_launch(tgx_lm_side* side, tgx_sampler* sampler, int times) {
    clear_error();
    if (!side || !sampler) return fail(TGX_E_ARG, "null LM side or sampler");
    LmSide* l = side->s;
    Sampler* s = sampler->s;
    if (l->ctx != s->ctx) return fail(TGX_E_ARG, "the LM side and the sampler are on different contexts");
    if (l->rows != s->rows || l->dit != s->shape.hidden)
        return fail(TGX_E_SHAPE, "an LM side of " + std::to_string(l->rows) + " rows and mu of " + std::to_string(l->dit) +
                                     " wide for a sampler of " + std::to_string(s->rows) + " rows " + std::to_string(s->shape.hidden) + " wide");
    if (times <= 0) return fail(TGX_E_ARG, "times");
    if (l->pending || s->pending) return fail(TGX_E_BUSY, "a step is under way");
    TGX_TRY(sampler_prepare(s));
    // The sampler's graph is recorded on its first launch; launch it once alone first if need be.
    if (s->exec_dirty) {
        TGX_TRY(sampler_launch(s, 1));
        TGX_TRY(sampler_wait(s));
    }
    hipStream_t st = l->ctx->stream;
    TGX_TRY(hold_ahead(l->base, times, 1));
    TGX_TRY(hold_ahead(l->residual, times, 1));
    TGX_TRY(sync_slots(l->base));
    TGX_TRY(sync_slots(l->residual));
    const size_t mu_bytes = (size_t)l->rows * 2 * l->dit * 4;
    TGX_HIP(hipEventRecord(l->ev_start, st));
    for (int i = 0; i < times; ++i) {
        TGX_HIP(hipGraphLaunch(l->advance_exec, st));
        TGX_HIP(hipMemcpyAsync(s->mu, l->mu, mu_bytes, hipMemcpyDeviceToDevice, st));
        TGX_HIP(hipGraphLaunch(s->exec, st));
        moved_on(l->base, 1);
        moved_on(l->residual, 1);
    }
    TGX_HIP(hipEventRecord(l->ev_end, st));
    l->pending = true;
    return TGX_OK;
}

tgx_status tgx_patch_elapsed_ms(const tgx_lm_side* side, float* out) { return tgx_lm_side_elapsed_ms(side, out); }

// ---- the encoder ----

tgx_status tgx_encoder_create(tgx_context* ctx, const tgx_shape* stack, const tgx_patch_shape* patch, tgx_encoder** out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or output");
    *out = nullptr;
    Encoder* e = nullptr;
    TGX_TRY(encoder_create(ctx->ctx, stack, patch, &e));
    *out = new tgx_encoder{e};
    return TGX_OK;
}

void tgx_encoder_destroy(tgx_encoder* e) {
    if (!e) return;
    encoder_destroy(e->e);
    delete e;
}

tgx_status tgx_encoder_load(tgx_encoder* e, const char* name, const void* data, tgx_dtype dtype, size_t count) {
    clear_error();
    if (!e) return fail(TGX_E_ARG, "null encoder");
    return encoder_load(e->e, name, data, dtype, count);
}

tgx_status tgx_encoder_encode(tgx_encoder* e, const float* patch, float* out) {
    clear_error();
    if (!e) return fail(TGX_E_ARG, "null encoder");
    TGX_TRY(encoder_use_rows(e->e, e->e->max_rows));
    return encoder_encode(e->e, patch, out);
}

tgx_status tgx_encoder_dispatches(const tgx_encoder* e, int* out) {
    clear_error();
    if (!e || !out) return fail(TGX_E_ARG, "null encoder or output");
    *out = e->e->dispatches;
    return TGX_OK;
}

// ---- the patch step with its encoder ----

tgx_status tgx_patch_step_create(tgx_encoder* e, tgx_lm_side* side, tgx_sampler* sampler, tgx_patch_step** out) {
    clear_error();
    if (!e || !side || !sampler || !out) return fail(TGX_E_ARG, "null encoder, LM side, sampler or output");
    *out = nullptr;
    PatchStep* p = nullptr;
    TGX_TRY(patch_step_create(e->e, side->s, sampler->s, &p));
    *out = new tgx_patch_step{p};
    return TGX_OK;
}

void tgx_patch_step_destroy(tgx_patch_step* p) {
    if (!p) return;
    patch_step_destroy(p->p);
    delete p;
}

tgx_status tgx_patch_step_run(tgx_patch_step* p, const tgx_row* rows, int nrows, const float* cond, const float* noise,
                              const float* sampling, float* patch, float* stop_logits) {
    clear_error();
    if (!p) return fail(TGX_E_ARG, "null patch step");
    return patch_step_run(p->p, rows, nrows, cond, noise, sampling, patch, stop_logits);
}

tgx_status tgx_patch_step_launch(tgx_patch_step* p, int times, int advance) {
    clear_error();
    if (!p) return fail(TGX_E_ARG, "null patch step");
    return patch_step_launch(p->p, times, advance);
}

tgx_status tgx_patch_step_wait(tgx_patch_step* p) {
    clear_error();
    if (!p) return fail(TGX_E_ARG, "null patch step");
    return patch_step_wait(p->p);
}

tgx_status tgx_patch_step_elapsed_ms(const tgx_patch_step* p, float* out) {
    clear_error();
    if (!p || !out) return fail(TGX_E_ARG, "null patch step or output");
    if (p->p->pending) return fail(TGX_E_BUSY, "a step is under way");
    TGX_HIP(hipEventElapsedTime(out, p->p->ev_start, p->p->ev_end));
    return TGX_OK;
}

}  // extern "C"
