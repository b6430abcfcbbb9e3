// The prompter and the prompt cache (crates/graph/src/prompt.rs), over a patch step's encoder and
// LM side: the embeddings on the host and the encoder, the two LMs' prefills with the layers
// between them on the device, and the cache's keys and values copied block by block.
#include "prompt.hpp"

#include <algorithm>
#include <cstring>
#include <set>

#include "handles.hpp"
#include "heads_kernels.hpp"

namespace tgx {

DeviceMem::~DeviceMem() {
    if (ptr) (void)hipFree(ptr);
}

namespace {

// The base LM's embedding table in the checkpoint (prompt.rs:80).
constexpr const char* EMBED_TOKENS = "base_lm.embed_tokens.weight";

template <typename T>
tgx_status prompt_alloc(Prompter* p, T** out, size_t count) {
    void* ptr = nullptr;
    const size_t bytes = std::max<size_t>(count, 1) * sizeof(T);
    hipError_t e = hipMalloc(&ptr, bytes);
    if (e != hipSuccess) return fail(TGX_E_HIP, "hipMalloc of " + std::to_string(bytes) + " bytes: " + hipGetErrorString(e));
    p->allocations.push_back({ptr, bytes});
    *out = static_cast<T*>(ptr);
    return TGX_OK;
}

std::vector<uint32_t> bits_of(const float* v, size_t n) {
    std::vector<uint32_t> b(n);
    std::memcpy(b.data(), v, n * 4);
    return b;
}

// prompt.rs:754-768: a prompt that does not end in audio, or has no positions, is refused.
tgx_status check_prompt(const PromptView& pr) {
    if (pr.len <= 0 || !pr.tokens || !pr.patches || !pr.audio || !pr.audio[pr.len - 1])
        return fail(TGX_E_SHAPE, "a prompt of " + std::to_string(pr.len) + " positions, which must end in audio");
    return TGX_OK;
}

bool busy(const Prompter* p) { return p->step->pending || p->step->side->pending || p->step->encoder->pending; }

// A cache block of one layer: every KV head's key tile and value tile of 64 positions.
size_t block_elems(const Decoder* d) { return (size_t)d->shape.kv_heads * 2 * kv_tile(d->shape.head_dim); }
uint16_t* kv_block(Decoder* d, int layer, uint32_t block) {
    return d->kv + ((size_t)layer * d->nblocks + block) * block_elems(d);
}

int blocks_for(int positions) { return (positions + BLOCK_TOKENS - 1) / BLOCK_TOKENS; }

// cache_regions (prompt.rs:471-500) for the paged caches: the slot's first `blocks` blocks of every
// layer of the base LM, then of the residual LM, into `pre.kept` one after another.
tgx_status copy_out(Prompter* p, uint32_t slot, int held, Prefix& pre) {
    LmSide* s = p->step->side;
    const int blocks = blocks_for(held);
    size_t elems = 0;
    for (Decoder* d : {s->base, s->residual}) elems += (size_t)d->shape.layers * blocks * block_elems(d);
    const size_t bytes = elems * 2;
    hipError_t e = hipMalloc(&pre.kept.ptr, bytes);
    if (e != hipSuccess) {
        pre.kept.ptr = nullptr;
        return fail(TGX_E_HIP, "hipMalloc of " + std::to_string(bytes) + " bytes: " + hipGetErrorString(e));
    }
    pre.kept.bytes = bytes;
    pre.blocks = blocks;
    hipStream_t st = s->ctx->stream;
    uint16_t* dst = static_cast<uint16_t*>(pre.kept.ptr);
    for (Decoder* d : {s->base, s->residual}) {
        if (d->slot_blocks[slot] < blocks) return fail(TGX_E_SHAPE, "the slot holds fewer blocks than the prompt ran");
        for (int l = 0; l < d->shape.layers; ++l)
            for (int b = 0; b < blocks; ++b) {
                const uint32_t blk = d->table_host[(size_t)slot * d->max_blocks + b];
                TGX_HIP(hipMemcpyAsync(dst, kv_block(d, l, blk), block_elems(d) * 2, hipMemcpyDeviceToDevice, st));
                dst += block_elems(d);
            }
    }
    TGX_HIP(hipStreamSynchronize(st));
    return TGX_OK;
}

// The kept keys and values of the first `shared` positions back into the slot's blocks (the rest of
// the last block they touch is written again by the positions that run after them).
tgx_status copy_in(Prompter* p, uint32_t slot, int shared, const Prefix& pre) {
    LmSide* s = p->step->side;
    const int blocks = std::min(blocks_for(shared), pre.blocks);
    hipStream_t st = s->ctx->stream;
    const uint16_t* src = static_cast<const uint16_t*>(pre.kept.ptr);
    for (Decoder* d : {s->base, s->residual}) {
        TGX_TRY(hold_slot(d, slot, (uint32_t)shared));
        for (int l = 0; l < d->shape.layers; ++l)
            for (int b = 0; b < pre.blocks; ++b) {
                if (b < blocks) {
                    const uint32_t blk = d->table_host[(size_t)slot * d->max_blocks + b];
                    TGX_HIP(hipMemcpyAsync(kv_block(d, l, blk), src, block_elems(d) * 2, hipMemcpyDeviceToDevice, st));
                }
                src += block_elems(d);
            }
    }
    TGX_HIP(hipStreamSynchronize(st));
    return TGX_OK;
}

// PromptCache::take (prompt.rs:440-449).
Voice take(PromptCache* c, const std::vector<uint32_t>& key) {
    c->clock += 1;
    auto it = c->voices.find(key);
    if (it == c->voices.end()) return Voice{};
    c->bytes -= 4 * key.size() + it->second.bytes();
    Voice v = std::move(it->second);
    c->voices.erase(it);
    return v;
}

// PromptCache::put (prompt.rs:451-469): without the prefix if only that way it fits, not at all if
// it does not fit alone; the voices used longest ago dropped to make room.
void put(PromptCache* c, const std::vector<uint32_t>& key, Voice v) {
    auto bytes = [&](const Voice& voice) { return 4 * key.size() + voice.bytes(); };
    if (bytes(v) > c->budget) v.prefix.reset();
    if (bytes(v) > c->budget) return;
    while (c->bytes + bytes(v) > c->budget) {
        auto oldest = std::min_element(c->voices.begin(), c->voices.end(),
                                       [](const auto& a, const auto& b) { return a.second.used < b.second.used; });
        c->bytes -= 4 * oldest->first.size() + oldest->second.bytes();
        c->voices.erase(oldest);
    }
    v.used = c->clock;
    c->bytes += bytes(v);
    c->voices[key] = std::move(v);
}

}  // namespace

size_t Prefix::bytes() const {
    const size_t patch = len ? patches.size() / len : 0;
    return kept.bytes + (4 + 1 + 4 * patch) * (size_t)len;
}

// Prefix::shared (prompt.rs:394-409): the positions `p` begins with that this holds.
int Prefix::shared(const PromptView& p, int patch) const {
    const int n = std::min(len, p.len);
    int at = 0;
    for (; at < n; ++at) {
        if ((audio[at] != 0) != (p.audio[at] != 0)) break;
        if (p.audio[at]) {
            if (std::memcmp(&patches[(size_t)at * patch], p.patches + (size_t)at * patch, (size_t)patch * 4) != 0) break;
        } else if (tokens[at] != p.tokens[at]) {
            break;
        }
    }
    return at;
}

size_t Voice::bytes() const {
    size_t b = 0;
    for (const auto& [k, v] : embeddings) b += 4 * k.size() + 4 * v.size();
    return b + (prefix ? prefix->bytes() : 0);
}

tgx_status prompter_create(PatchStep* step, int max_rows, Prompter** out) {
    if (!step || !out) return fail(TGX_E_ARG, "null patch step or output");
    *out = nullptr;
    LmSide* s = step->side;
    Encoder* e = step->encoder;
    if (max_rows < 1 || max_rows > s->base->shape.capacity)
        return fail(TGX_E_SHAPE, "runs of " + std::to_string(max_rows) + " positions, a cache of " + std::to_string(s->base->shape.capacity));
    if (e->shape.hidden != s->encoder)
        return fail(TGX_E_SHAPE, "an encoder " + std::to_string(e->shape.hidden) + " wide for enc_to_lm_proj of " + std::to_string(s->encoder));
    Prompter* p = new Prompter();
    p->step = step;
    p->max_rows = max_rows;
    p->hidden = s->hidden;
    p->latent = s->latent;
    p->feat = e->feat;
    p->frames = e->frames;
    const size_t R = (size_t)max_rows, h = (size_t)s->hidden;
    tgx_status r = TGX_OK;
    auto A = [&](auto** ptr, size_t n) {
        if (r == TGX_OK) r = prompt_alloc(p, ptr, n);
    };
    A(&p->levels, R * s->latent);
    A(&p->quantized, R * h);
    A(&p->lm_hidden, R * h);
    A(&p->residual_in, R * h);
    A(&p->audio_x, R * h);
    A(&p->flags, R);
    A(&p->enc_out, (size_t)e->max_rows * s->encoder);
    A(&p->embedded, (size_t)e->max_rows * h);
    if (r != TGX_OK) {
        prompter_destroy(p);
        return r;
    }
    *out = p;
    return TGX_OK;
}

void prompter_destroy(Prompter* p) {
    if (!p) return;
    for (auto& b : p->allocations) (void)hipFree(b.ptr);
    delete p;
}

// Prompter::embed (prompt.rs:559-566), the encoder's rows at a time: each patch [patch_size][feat_dim]
// laid out as the patch step's cond, [feat_dim][patch_size], then enc_to_lm_proj of its embedding.
// A row's embedding is the same whatever the other rows of the encoder hold.
tgx_status prompter_embed(Prompter* p, const float* patches, int n, float* out) {
    if (!p || (n > 0 && (!patches || !out))) return fail(TGX_E_ARG, "null prompter, patches or output");
    if (busy(p)) return fail(TGX_E_BUSY, "a step is under way");
    Encoder* e = p->step->encoder;
    LmSide* s = p->step->side;
    TGX_TRY(encoder_use_rows(e, e->max_rows));  // all its rows at a time
    const int R = e->rows, C = e->feat, F = e->frames, h = p->hidden;
    hipStream_t st = s->ctx->stream;
    std::vector<float> cond((size_t)R * C * F);
    for (int first = 0; first < n; first += R) {
        const int rows = std::min(R, n - first);
        std::fill(cond.begin(), cond.end(), 0.f);
        for (int r = 0; r < rows; ++r)
            for (int f = 0; f < F; ++f)
                for (int c = 0; c < C; ++c) cond[((size_t)r * C + c) * F + f] = patches[(((size_t)first + r) * F + f) * C + c];
        TGX_HIP(hipMemcpyAsync(e->patch, cond.data(), cond.size() * 4, hipMemcpyHostToDevice, st));
        TGX_HIP(encoder_enqueue(e, e->patch, p->enc_out, nullptr));
        const LinearArgs la{s->enc_to_lm.w, s->enc_to_lm.b, p->enc_out, nullptr, p->embedded, s->enc_to_lm.K, 0,
                            s->enc_to_lm.N, rows, 0, h, ACT_NONE, (float)s->levels};
        TGX_HIP(launch_linear("enc_to_lm_proj", la, st, nullptr));
        TGX_HIP(hipMemcpyAsync(out + (size_t)first * h, p->embedded, (size_t)rows * h * 4, hipMemcpyDeviceToHost, st));
        TGX_HIP(hipStreamSynchronize(st));
    }
    return TGX_OK;
}

// Prompter::embeddings_from (prompt.rs:650-690): the tokens' rows read from the checkpoint, each
// distinct patch's embedding from `known` or else from the encoder, and kept there.
tgx_status prompter_embeddings(Prompter* p, const Checkpoint* ck, const PromptView& pr, int from,
                               std::map<std::vector<uint32_t>, std::vector<float>>& known, std::vector<float>& x,
                               std::vector<float>& audio_x) {
    if (!p || !ck) return fail(TGX_E_ARG, "null prompter or checkpoint");
    TGX_TRY(check_prompt(pr));
    const int len = pr.len, h = p->hidden, patch = p->frames * p->feat;
    if (from < 0 || from > len - 1) return fail(TGX_E_SHAPE, "positions from " + std::to_string(from) + " of " + std::to_string(len));
    const int n = len - 1 - from;
    x.assign((size_t)n * h, 0.f);
    audio_x.assign((size_t)n * h, 0.f);
    std::vector<int64_t> tokens;
    std::vector<int> text_at;
    for (int q = from; q < len - 1; ++q)
        if (!pr.audio[q]) {
            tokens.push_back(pr.tokens[q]);
            text_at.push_back(q);
        }
    if (!tokens.empty()) {
        auto it = ck->entries.find(EMBED_TOKENS);
        if (it == ck->entries.end()) return fail(TGX_E_WEIGHTS, ck->path + ": " + EMBED_TOKENS + ": no such tensor");
        if (it->second.shape.size() != 2 || it->second.shape[1] != h)
            return fail(TGX_E_WEIGHTS, ck->path + ": " + EMBED_TOKENS + ": not [vocab][" + std::to_string(h) + "]");
        std::vector<float> rows(tokens.size() * (size_t)h);
        int64_t columns = 0;
        TGX_TRY(checkpoint_gather(ck, EMBED_TOKENS, tokens.data(), (int)tokens.size(), rows.data(), &columns));
        for (size_t i = 0; i < text_at.size(); ++i)
            std::memcpy(&x[(size_t)(text_at[i] - from) * h], &rows[i * h], (size_t)h * 4);
    }
    std::vector<std::vector<uint32_t>> missing;
    std::vector<float> missing_patches;
    std::set<std::vector<uint32_t>> asked;
    for (int q = from; q < len - 1; ++q) {
        if (!pr.audio[q]) continue;
        std::vector<uint32_t> key = bits_of(pr.patches + (size_t)q * patch, patch);
        if (known.count(key) || asked.count(key)) continue;
        asked.insert(key);
        missing.push_back(key);
        missing_patches.insert(missing_patches.end(), pr.patches + (size_t)q * patch, pr.patches + (size_t)(q + 1) * patch);
    }
    if (!missing.empty()) {
        std::vector<float> emb(missing.size() * (size_t)h);
        TGX_TRY(prompter_embed(p, missing_patches.data(), (int)missing.size(), emb.data()));
        for (size_t i = 0; i < missing.size(); ++i) known[missing[i]] = std::vector<float>(emb.begin() + i * h, emb.begin() + (i + 1) * h);
    }
    for (int q = from; q < len - 1; ++q) {
        if (!pr.audio[q]) continue;
        const std::vector<float>& v = known.at(bits_of(pr.patches + (size_t)q * patch, patch));
        std::memcpy(&x[(size_t)(q - from) * h], v.data(), (size_t)h * 4);
        std::memcpy(&audio_x[(size_t)(q - from) * h], v.data(), (size_t)h * 4);
    }
    return TGX_OK;
}

// Prompter::run_rows (prompt.rs:692-752): the positions from `start` whose embeddings are x
// ([len][hidden]) through both LMs into slot `slot` of the LM side's caches, max_rows at a time.
tgx_status prompter_run_rows(Prompter* p, uint32_t start, uint32_t slot, const float* x, const float* audio_x,
                             const uint8_t* audio, int len) {
    if (!p || (len > 0 && (!x || !audio_x || !audio))) return fail(TGX_E_ARG, "null prompter, embeddings or flags");
    if (busy(p)) return fail(TGX_E_BUSY, "a step is under way");
    LmSide* s = p->step->side;
    Decoder *base = s->base, *res = s->residual;
    if (len < 0 || (uint64_t)start + (uint64_t)len > (uint64_t)base->shape.capacity || slot >= (uint32_t)base->slots)
        return fail(TGX_E_SHAPE, std::to_string(len) + " positions from " + std::to_string(start) + " in slot " +
                                     std::to_string(slot) + " of " + std::to_string(base->slots) + " of " +
                                     std::to_string(base->shape.capacity));
    const int h = p->hidden;
    hipStream_t st = s->ctx->stream;
    std::vector<uint32_t> flags(p->max_rows);
    for (int first = 0; first < len; first += p->max_rows) {
        const int rows = std::min(p->max_rows, len - first);
        const tgx_run run{slot, start + (uint32_t)first, (uint32_t)rows};
        TGX_TRY(prefill_device(base, &run, 1, x + (size_t)first * h, false));
        for (int r = 0; r < rows; ++r) flags[r] = audio[first + r] ? 1u : 0u;
        TGX_HIP(hipMemcpyAsync(p->flags, flags.data(), (size_t)rows * 4, hipMemcpyHostToDevice, st));
        TGX_HIP(hipMemcpyAsync(p->audio_x, audio_x + (size_t)first * h, (size_t)rows * h * 4, hipMemcpyHostToDevice, st));
        const float lv = (float)s->levels;
        const LinearArgs fin{s->fsq_in.w, s->fsq_in.b, base->pf.out, nullptr, p->levels, s->fsq_in.K, 0, s->fsq_in.N, rows, 0,
                             s->fsq_in.N, ACT_LEVELS, lv};
        TGX_HIP(launch_linear("fsq_layer.in_proj", fin, st, nullptr));
        const LinearArgs fout{s->fsq_out.w, s->fsq_out.b, p->levels, nullptr, p->quantized, s->fsq_out.K, 0, s->fsq_out.N, rows, 0,
                              s->fsq_out.N, ACT_NONE, lv};
        TGX_HIP(launch_linear("fsq_layer.out_proj", fout, st, nullptr));
        TGX_HIP(launch_select_rows(p->flags, p->quantized, base->pf.out, p->lm_hidden, rows, h, st, nullptr));
        const LinearArgs fus{s->fusion.w, s->fusion.b, p->lm_hidden, p->audio_x, p->residual_in, h, h, s->fusion.N, rows, 0,
                             s->fusion.N, ACT_NONE, lv};
        TGX_HIP(launch_linear("fusion_concat_proj", fus, st, nullptr));
        TGX_TRY(prefill_device(res, &run, 1, p->residual_in, true));
        TGX_HIP(hipStreamSynchronize(st));
        p->last_rows = rows;
    }
    return TGX_OK;
}

// Prompter::run (prompt.rs:568-583): every position but the last, from position 0.
tgx_status prompter_run(Prompter* p, uint32_t slot, const Checkpoint* ck, const PromptView& pr) {
    std::map<std::vector<uint32_t>, std::vector<float>> known;
    std::vector<float> x, audio_x;
    TGX_TRY(prompter_embeddings(p, ck, pr, 0, known, x, audio_x));
    return prompter_run_rows(p, 0, slot, x.data(), audio_x.data(), pr.audio, pr.len - 1);
}

// Prompter::run_cached (prompt.rs:585-641).
tgx_status prompter_run_cached(Prompter* p, uint32_t slot, const Checkpoint* ck, const PromptView& pr, const float* voice,
                               size_t voice_len, PromptCache* cache, int* ran) {
    if (!p || !ck || !cache || (voice_len && !voice)) return fail(TGX_E_ARG, "null prompter, checkpoint, cache or voice");
    TGX_TRY(check_prompt(pr));
    const int len = pr.len, patch = p->frames * p->feat;
    const std::vector<uint32_t> key = bits_of(voice, voice_len);
    Voice kept = take(cache, key);
    const int shared = kept.prefix ? std::min(kept.prefix->shared(pr, patch), len - 1) : 0;
    std::vector<float> x, audio_x;
    tgx_status r = prompter_embeddings(p, ck, pr, shared, kept.embeddings, x, audio_x);
    if (r == TGX_OK && slot >= (uint32_t)p->step->side->base->slots)
        r = fail(TGX_E_SHAPE, "slot " + std::to_string(slot) + " of " + std::to_string(p->step->side->base->slots));
    if (r == TGX_OK && kept.prefix && shared > 0) r = copy_in(p, slot, shared, *kept.prefix);
    if (r == TGX_OK) r = prompter_run_rows(p, (uint32_t)shared, slot, x.data(), audio_x.data(), pr.audio + shared, len - 1 - shared);
    if (r == TGX_OK && !kept.prefix) {
        int held = 0;
        for (int q = len - 1; q >= 0; --q)
            if (!pr.audio[q]) {
                held = q + 1;
                break;
            }
        if (held > 0) {
            size_t kv = 0;
            for (Decoder* d : {p->step->side->base, p->step->side->residual})
                kv += (size_t)d->shape.layers * blocks_for(held) * block_elems(d) * 2;
            const size_t prefix = kv + (4 + 1 + 4 * (size_t)patch) * held;
            if (4 * key.size() + kept.bytes() + prefix <= cache->budget) {
                auto pre = std::make_unique<Prefix>();
                r = copy_out(p, slot, held, *pre);
                if (r == TGX_OK) {
                    pre->len = held;
                    pre->tokens.assign(pr.tokens, pr.tokens + held);
                    pre->patches = bits_of(pr.patches, (size_t)held * patch);
                    pre->audio.assign(pr.audio, pr.audio + held);
                    kept.prefix = std::move(pre);
                }
            }
        }
    }
    put(cache, key, std::move(kept));
    if (r == TGX_OK && ran) *ran = len - shared;
    return r;
}

tgx_status prompter_read(Prompter* p, const char* tensor, float* out, size_t count) {
    if (!p || !tensor || !out) return fail(TGX_E_ARG, "null prompter, tensor or output");
    if (!p->last_rows) return fail(TGX_E_SHAPE, "no run to read");
    LmSide* s = p->step->side;
    const std::string t = tensor;
    const float* src = nullptr;
    size_t width = (size_t)p->hidden;
    if (t == "base_out") src = s->base->pf.out;
    else if (t == "levels") src = p->levels, width = (size_t)p->latent;
    else if (t == "quantized") src = p->quantized;
    else if (t == "lm_hidden") src = p->lm_hidden;
    else if (t == "residual_in") src = p->residual_in;
    else if (t == "residual_out") src = s->residual->pf.out;
    else return fail(TGX_E_ARG, t + ": no such tensor of the prompt");
    const size_t n = (size_t)p->last_rows * width;
    if (count != n) return fail(TGX_E_ARG, t + ": " + std::to_string(n) + " values, not " + std::to_string(count));
    TGX_HIP(hipMemcpy(out, src, n * 4, hipMemcpyDeviceToHost));
    return TGX_OK;
}

}  // namespace tgx

using namespace tgx;

struct tgx_prompter {
    Prompter* p;
};
struct tgx_prompt_cache {
    PromptCache* c;
};

namespace {
PromptView view(const tgx_prompt* pr) { return PromptView{pr->tokens, pr->patches, pr->audio, pr->len}; }
}  // namespace

extern "C" {

tgx_status tgx_prompter_create(tgx_patch_step* step, int max_rows, tgx_prompter** out) {
    clear_error();
    if (!step || !out) return fail(TGX_E_ARG, "null patch step or output");
    *out = nullptr;
    Prompter* p = nullptr;
    TGX_TRY(prompter_create(step->p, max_rows, &p));
    *out = new tgx_prompter{p};
    return TGX_OK;
}

void tgx_prompter_destroy(tgx_prompter* p) {
    if (!p) return;
    prompter_destroy(p->p);
    delete p;
}

tgx_status tgx_prompter_max_rows(const tgx_prompter* p, int* out) {
    clear_error();
    if (!p || !out) return fail(TGX_E_ARG, "null prompter or output");
    *out = p->p->max_rows;
    return TGX_OK;
}

tgx_status tgx_prompter_embed(tgx_prompter* p, const float* patch, float* out) {
    clear_error();
    if (!p) return fail(TGX_E_ARG, "null prompter");
    return prompter_embed(p->p, patch, 1, out);
}

tgx_status tgx_prompter_embeddings(tgx_prompter* p, const tgx_checkpoint* ck, const tgx_prompt* prompt, float* x, float* audio_x) {
    clear_error();
    if (!p || !ck || !prompt || !x || !audio_x) return fail(TGX_E_ARG, "null prompter, checkpoint, prompt or output");
    std::map<std::vector<uint32_t>, std::vector<float>> known;
    std::vector<float> xv, av;
    TGX_TRY(prompter_embeddings(p->p, ck->ck, view(prompt), 0, known, xv, av));
    std::memcpy(x, xv.data(), xv.size() * 4);
    std::memcpy(audio_x, av.data(), av.size() * 4);
    return TGX_OK;
}

tgx_status tgx_prompter_run_rows(tgx_prompter* p, tgx_row at, const float* x, const float* audio_x, const uint8_t* audio, int len) {
    clear_error();
    if (!p) return fail(TGX_E_ARG, "null prompter");
    return prompter_run_rows(p->p, at.position, at.slot, x, audio_x, audio, len);
}

tgx_status tgx_prompter_run(tgx_prompter* p, uint32_t slot, const tgx_checkpoint* ck, const tgx_prompt* prompt) {
    clear_error();
    if (!p || !ck || !prompt) return fail(TGX_E_ARG, "null prompter, checkpoint or prompt");
    return prompter_run(p->p, slot, ck->ck, view(prompt));
}

tgx_status tgx_prompter_run_cached(tgx_prompter* p, uint32_t slot, const tgx_checkpoint* ck, const tgx_prompt* prompt,
                                   const float* voice, size_t voice_len, tgx_prompt_cache* cache, int* ran) {
    clear_error();
    if (!p || !ck || !prompt || !cache) return fail(TGX_E_ARG, "null prompter, checkpoint, prompt or cache");
    return prompter_run_cached(p->p, slot, ck->ck, view(prompt), voice, voice_len, cache->c, ran);
}

tgx_status tgx_prompter_read(tgx_prompter* p, const char* tensor, float* out, size_t count) {
    clear_error();
    if (!p) return fail(TGX_E_ARG, "null prompter");
    return prompter_read(p->p, tensor, out, count);
}

tgx_status tgx_prompt_cache_create(tgx_context* ctx, size_t budget, tgx_prompt_cache** out) {
    clear_error();
    if (!ctx || !out) return fail(TGX_E_ARG, "null context or output");
    PromptCache* c = new PromptCache();
    c->ctx = ctx->ctx;
    c->budget = budget;
    *out = new tgx_prompt_cache{c};
    return TGX_OK;
}

void tgx_prompt_cache_destroy(tgx_prompt_cache* c) {
    if (!c) return;
    delete c->c;
    delete c;
}

tgx_status tgx_prompt_cache_bytes(const tgx_prompt_cache* c, size_t* out) {
    clear_error();
    if (!c || !out) return fail(TGX_E_ARG, "null cache or output");
    *out = c->c->bytes;
    return TGX_OK;
}

tgx_status tgx_prompt_cache_voices(const tgx_prompt_cache* c, int* out) {
    clear_error();
    if (!c || !out) return fail(TGX_E_ARG, "null cache or output");
    *out = (int)c->c->voices.size();
    return TGX_OK;
}

}  // extern "C"
