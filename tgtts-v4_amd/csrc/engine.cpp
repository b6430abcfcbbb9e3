// The engine the service's GPU thread drives (crates/tgtts/src/rt.rs:92-111 Engine, 449-541
// Generating; crates/graph/src/generator.rs Generator): requests in slots, each started from its
// prompt (run into its slot of the caches from what the prompt cache keeps of its voice), then a
// patch of every request under way sampled in one patch step, until the stop head says to stop
// after one or the request's most are sampled. The patch step runs at the engine's rows, a row to a
// slot and free slots spare: a request's rows come out bit for bit as they would beside any others.
// The audio VAE is not part of the path: a request's sampled latent frames are handed back
// instead of decoded audio.
#include <cmath>
#include <cstring>
#include <memory>

#include "handles.hpp"
#include "prompt.hpp"

namespace tgx {

namespace {

// generator::Request (generator.rs:78-98), without the audio decoder's state.
struct Request {
    uint32_t position = 0;      // where the next step runs the patch before
    std::vector<float> before;  // the patch before, [feat_dim][patch_size] as the patch step takes it
    int left = 0;               // patches it may still sample
    int sampled = 0;
    float temperature = 1.f, cfg = 2.f;
    std::vector<float> frames;  // sampled and not yet taken, [frames][feat_dim]
};

}  // namespace

struct Engine {
    Context* ctx = nullptr;
    int slots = 0, capacity = 0, feat = 0, frames = 0;
    LmSide* side = nullptr;
    Encoder* encoder = nullptr;
    Sampler* sampler = nullptr;
    PatchStep* step = nullptr;
    Prompter* prompter = nullptr;
    PromptCache cache;
    const Checkpoint* checkpoint = nullptr;
    std::vector<std::unique_ptr<Request>> requests;
    std::vector<int> last_rows;  // the row each slot's request ran in at the last step, -1 if none
};

namespace {

// transposed (patch.rs): [a][b] -> [b][a].
std::vector<float> transposed(const float* v, int a, int b) {
    std::vector<float> out((size_t)a * b);
    for (int i = 0; i < a; ++i)
        for (int j = 0; j < b; ++j) out[(size_t)j * a + i] = v[(size_t)i * b + j];
    return out;
}

tgx_status no_request(int slot) { return fail(TGX_E_SHAPE, "no request under way in slot " + std::to_string(slot)); }

}  // namespace

void engine_destroy(Engine* e) {
    if (!e) return;
    prompter_destroy(e->prompter);
    patch_step_destroy(e->step);
    sampler_destroy(e->sampler);
    encoder_destroy(e->encoder);
    lm_side_destroy(e->side);
    delete e;
}

// Generator::new (generator.rs:130-193) over shapes the caller read from config.json, and weights
// from `ck`, which the engine reads token embeddings from and must outlive it.
tgx_status engine_create(Context* ctx, const Checkpoint* ck, const tgx_shape* base, const tgx_shape* residual,
                         const tgx_heads_shape* heads, const tgx_shape* encoder, const tgx_shape* dit, int feat_dim,
                         int patch_size, const tgx_engine_settings* settings, Engine** out) {
    if (!ctx || !ck || !base || !residual || !heads || !encoder || !dit || !settings || !out)
        return fail(TGX_E_ARG, "null context, checkpoint, shape, settings or output");
    *out = nullptr;
    const tgx_engine_settings& st = *settings;
    if (st.slots < 1 || st.capacity < 1 || st.max_rows < 1 || st.timesteps < 1)
        return fail(TGX_E_SHAPE, "settings of " + std::to_string(st.slots) + " slots, a cache of " + std::to_string(st.capacity) +
                                     ", runs of " + std::to_string(st.max_rows) + " and " + std::to_string(st.timesteps) + " steps");
    Engine* e = new Engine();
    auto done = [&](tgx_status r) {
        if (r != TGX_OK) engine_destroy(e);
        return r;
    };
    e->ctx = ctx;
    e->slots = st.slots;
    e->capacity = st.capacity;
    e->feat = feat_dim;
    e->frames = patch_size;
    e->checkpoint = ck;
    e->cache.ctx = ctx;
    e->cache.budget = st.prompt_cache_bytes;
    tgx_shape b = *base, r = *residual;
    b.capacity = r.capacity = st.capacity;
    const tgx_batch batch{st.slots, st.slots, 0, 0};
    const tgx_patch_shape patch{feat_dim, patch_size, st.timesteps, st.slots};
    TGX_TRY(done(lm_side_create(ctx, &b, &r, &batch, heads, &e->side)));
    TGX_TRY(done(encoder_create(ctx, encoder, &patch, &e->encoder)));
    TGX_TRY(done(sampler_create(ctx, dit, &patch, &e->sampler)));
    TGX_TRY(done(lm_side_load_checkpoint(e->side, ck)));
    TGX_TRY(done(encoder_load_checkpoint(e->encoder, ck)));
    TGX_TRY(done(sampler_load_checkpoint(e->sampler, ck)));
    TGX_TRY(done(patch_step_create(e->encoder, e->side, e->sampler, &e->step)));
    TGX_TRY(done(prompter_create(e->step, st.max_rows, &e->prompter)));
    e->requests.resize(st.slots);
    e->last_rows.assign(st.slots, -1);
    *out = e;
    return TGX_OK;
}

// Generator::start (generator.rs:205-262): ends any request in the slot, runs the prompt (which
// ends in audio) into the slot's caches, and waits for the first step.
tgx_status engine_start(Engine* e, int slot, const PromptView& pr, const float* voice, size_t voice_len, int max_patches,
                        float temperature, float cfg, int* prefilled) {
    if (!e) return fail(TGX_E_ARG, "null engine");
    if (slot < 0 || slot >= e->slots) return fail(TGX_E_SHAPE, "slot " + std::to_string(slot) + " of " + std::to_string(e->slots));
    e->requests[slot].reset();
    const int len = pr.len;
    if (len <= 0 || max_patches <= 0 || (int64_t)len - 1 + max_patches > e->capacity)
        return fail(TGX_E_SHAPE, std::to_string(len) + " positions of prompt and " + std::to_string(max_patches) +
                                     " patches after it in a cache of " + std::to_string(e->capacity));
    if (voice_len % (size_t)e->feat)
        return fail(TGX_E_SHAPE, "a voice of " + std::to_string(voice_len) + " values in frames of " + std::to_string(e->feat));
    int ran = 0;
    TGX_TRY(prompter_run_cached(e->prompter, (uint32_t)slot, e->checkpoint, pr, voice, voice_len, &e->cache, &ran));
    auto req = std::make_unique<Request>();
    req->position = (uint32_t)(len - 1);
    req->before = transposed(pr.patches + (size_t)(len - 1) * e->frames * e->feat, e->frames, e->feat);
    req->left = max_patches;
    req->temperature = temperature;
    req->cfg = cfg;
    e->requests[slot] = std::move(req);
    e->last_rows[slot] = -1;
    if (prefilled) *prefilled = ran;
    return TGX_OK;
}

// Generator::sample_after (generator.rs:264-279): the next patch of the request sampled after
// `frames`, [patch_size][feat_dim], rather than its last (teacher forcing).
tgx_status engine_sample_after(Engine* e, int slot, const float* frames) {
    if (!e || !frames) return fail(TGX_E_ARG, "null engine or frames");
    if (slot < 0 || slot >= e->slots || !e->requests[slot]) return no_request(slot);
    e->requests[slot]->before = transposed(frames, e->frames, e->feat);
    return TGX_OK;
}

// Generator::step (generator.rs:281-334) and advance (:405-438): a patch of every request under
// way in one patch step, each from its slot's noise ([feat_dim][patch_size] standard normal, for
// every slot, read for the slots under way); an outcome for each, its patch's frames in
// `frames` [slots][patch_size][feat_dim] at its slot.
tgx_status engine_step(Engine* e, const float* noise, tgx_engine_outcome* outcomes, float* frames, int* n) {
    if (!e || !noise || !outcomes || !frames || !n) return fail(TGX_E_ARG, "null engine, noise or output");
    *n = 0;
    const int S = e->slots, P = e->feat * e->frames;
    // The requests under way, a row each in slot order; the patch step runs them on its program
    // of the fewest rows that holds them (generator.rs:286-318).
    std::vector<int> under_way;
    for (int s = 0; s < S; ++s) {
        const Request* r = e->requests[s].get();
        if (r && r->left > 0) under_way.push_back(s);
    }
    if (under_way.empty()) return TGX_OK;
    const int N = (int)under_way.size();
    std::vector<tgx_row> rows(N);
    std::vector<float> cond((size_t)N * P), noises((size_t)N * P), sampling((size_t)N * 2);
    for (int k = 0; k < N; ++k) {
        const int s = under_way[k];
        const Request* r = e->requests[s].get();
        rows[k] = tgx_row{r->position, (uint32_t)s};
        std::memcpy(&cond[(size_t)k * P], r->before.data(), (size_t)P * 4);
        std::memcpy(&noises[(size_t)k * P], noise + (size_t)s * P, (size_t)P * 4);
        sampling[2 * k] = r->temperature;
        sampling[2 * k + 1] = r->cfg;
    }
    std::vector<float> patch((size_t)N * P), stop((size_t)N * 2);
    TGX_TRY(patch_step_run(e->step, rows.data(), N, cond.data(), noises.data(), sampling.data(), patch.data(), stop.data()));
    std::fill(e->last_rows.begin(), e->last_rows.end(), -1);
    for (int k = 0; k < N; ++k) {
        const int s = under_way[k];
        Request& r = *e->requests[s];
        e->last_rows[s] = k;
        tgx_engine_outcome& o = outcomes[(*n)++];
        o.slot = s;
        o.stop_logits[0] = stop[2 * k];
        o.stop_logits[1] = stop[2 * k + 1];
        const float* p = &patch[(size_t)k * P];
        bool finite = std::isfinite(o.stop_logits[0]) && std::isfinite(o.stop_logits[1]);
        for (int i = 0; i < P && finite; ++i) finite = std::isfinite(p[i]);
        if (!finite) {
            // graph::Error::NotFinite (generator.rs:413-415): the request ends.
            o.status = TGX_E_NOT_FINITE;
            o.last = 1;
            r.left = 0;
            continue;
        }
        r.sampled += 1;
        const bool stops = o.stop_logits[1] > o.stop_logits[0];  // Sampled::stops (patch.rs:232-235)
        r.left = stops ? 0 : r.left - 1;
        r.position += 1;
        const std::vector<float> f = transposed(p, e->feat, e->frames);  // [patch_size][feat_dim]
        std::memcpy(frames + (size_t)s * P, f.data(), (size_t)P * 4);
        r.frames.insert(r.frames.end(), f.begin(), f.end());
        r.before.assign(p, p + P);
        o.status = TGX_OK;
        o.last = r.left == 0;
    }
    return TGX_OK;
}

// Generator::levels (generator.rs:336-362): the scalar quantizer's levels the last patch of the
// request in `slot` was sampled after, as integers.
tgx_status engine_levels(Engine* e, int slot, float* out) {
    if (!e || !out) return fail(TGX_E_ARG, "null engine or output");
    if (slot < 0 || slot >= e->slots || !e->requests[slot] || e->last_rows[slot] < 0) return no_request(slot);
    const int L = e->side->latent;
    std::vector<float> all((size_t)e->side->rows * L);  // the last step's program's rows
    TGX_TRY(lm_side_read(e->side, "levels", all.data(), all.size()));
    for (int i = 0; i < L; ++i) out[i] = std::nearbyint(all[(size_t)e->last_rows[slot] * L + i] * (float)e->side->levels);
    return TGX_OK;
}

// take_audio (generator.rs:364-369) for the frames: those sampled since last taken; `n` frames of
// feat_dim values, at most `max`.
tgx_status engine_take_frames(Engine* e, int slot, float* out, int max, int* n) {
    if (!e || !n) return fail(TGX_E_ARG, "null engine or count");
    *n = 0;
    if (slot < 0 || slot >= e->slots) return fail(TGX_E_SHAPE, "slot " + std::to_string(slot) + " of " + std::to_string(e->slots));
    Request* r = e->requests[slot].get();
    if (!r) return TGX_OK;
    const int have = (int)(r->frames.size() / e->feat);
    if (have > max) return fail(TGX_E_ARG, std::to_string(have) + " frames waiting, room for " + std::to_string(max));
    if (have && !out) return fail(TGX_E_ARG, "null output");
    std::memcpy(out, r->frames.data(), r->frames.size() * 4);
    r->frames.clear();
    *n = have;
    return TGX_OK;
}

// Generator::finish (generator.rs:395-403): ends the request, giving the frames not yet taken.
tgx_status engine_finish(Engine* e, int slot, float* out, int max, int* n) {
    if (!e || !n) return fail(TGX_E_ARG, "null engine or count");
    if (slot < 0 || slot >= e->slots || !e->requests[slot]) return no_request(slot);
    TGX_TRY(engine_take_frames(e, slot, out, max, n));
    e->requests[slot].reset();
    e->last_rows[slot] = -1;
    return TGX_OK;
}

}  // namespace tgx

using namespace tgx;

struct tgx_engine {
    Engine* e;
};

namespace {
PromptView engine_view(const tgx_prompt* pr) { return PromptView{pr->tokens, pr->patches, pr->audio, pr->len}; }
}  // namespace

extern "C" {

tgx_status tgx_engine_create(tgx_context* ctx, const tgx_checkpoint* ck, const tgx_shape* base, const tgx_shape* residual,
                             const tgx_heads_shape* heads, const tgx_shape* encoder, const tgx_shape* dit, int feat_dim,
                             int patch_size, const tgx_engine_settings* settings, tgx_engine** out) {
    clear_error();
    if (!ctx || !ck || !out) return fail(TGX_E_ARG, "null context, checkpoint or output");
    *out = nullptr;
    Engine* e = nullptr;
    TGX_TRY(engine_create(ctx->ctx, ck->ck, base, residual, heads, encoder, dit, feat_dim, patch_size, settings, &e));
    *out = new tgx_engine{e};
    return TGX_OK;
}

void tgx_engine_destroy(tgx_engine* e) {
    if (!e) return;
    engine_destroy(e->e);
    delete e;
}

tgx_status tgx_engine_slots(const tgx_engine* e, int* out) {
    clear_error();
    if (!e || !out) return fail(TGX_E_ARG, "null engine or output");
    *out = e->e->slots;
    return TGX_OK;
}

tgx_status tgx_engine_start(tgx_engine* e, int slot, const tgx_prompt* prompt, const float* voice, size_t voice_len,
                            int max_patches, float temperature, float cfg, int* prefilled) {
    clear_error();
    if (!e || !prompt) return fail(TGX_E_ARG, "null engine or prompt");
    return engine_start(e->e, slot, engine_view(prompt), voice, voice_len, max_patches, temperature, cfg, prefilled);
}

tgx_status tgx_engine_sample_after(tgx_engine* e, int slot, const float* frames) {
    clear_error();
    if (!e) return fail(TGX_E_ARG, "null engine");
    return engine_sample_after(e->e, slot, frames);
}

tgx_status tgx_engine_step(tgx_engine* e, const float* noise, tgx_engine_outcome* outcomes, float* frames, int* n) {
    clear_error();
    if (!e) return fail(TGX_E_ARG, "null engine");
    return engine_step(e->e, noise, outcomes, frames, n);
}

tgx_status tgx_engine_levels(tgx_engine* e, int slot, float* out) {
    clear_error();
    if (!e) return fail(TGX_E_ARG, "null engine");
    return engine_levels(e->e, slot, out);
}

tgx_status tgx_engine_take_frames(tgx_engine* e, int slot, float* out, int max, int* n) {
    clear_error();
    if (!e) return fail(TGX_E_ARG, "null engine");
    return engine_take_frames(e->e, slot, out, max, n);
}

tgx_status tgx_engine_finish(tgx_engine* e, int slot, float* out, int max, int* n) {
    clear_error();
    if (!e) return fail(TGX_E_ARG, "null engine");
    return engine_finish(e->e, slot, out, max, n);
}

tgx_status tgx_engine_prompt_cache(const tgx_engine* e, size_t* bytes, int* voices) {
    clear_error();
    if (!e) return fail(TGX_E_ARG, "null engine");
    if (bytes) *bytes = e->e->cache.bytes;
    if (voices) *voices = (int)e->e->cache.voices.size();
    return TGX_OK;
}

}  // extern "C"
