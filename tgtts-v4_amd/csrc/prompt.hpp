// A prompt run into a slot of the patch step's caches (crates/graph/src/prompt.rs): every position
// but the last, which the step of the first patch after it runs as the patch before. A text
// position's embedding is its row of the base LM's embedding table, read from the checkpoint; an
// audio position's is the local encoder's and enc_to_lm_proj's of its patch. Then, a run of up to
// max_rows positions at a time: the base LM's prefill over the embeddings, the scalar quantizer
// over its outputs at the audio positions (the base LM's outputs at text), fusion_concat_proj of
// those beside the audio embeddings (zero at text), and the residual LM's prefill over that, both
// LMs writing their keys and values into the LM side's caches.
//
// A PromptCache keeps, for each voice, its patches' embeddings and the LMs' keys and values over
// the positions its first prompt began with, which a later prompt beginning with them copies back
// into the caches rather than run.
#pragma once
#include <stdint.h>

#include <map>
#include <memory>
#include <vector>

#include "checkpoint.hpp"
#include "patch.hpp"

namespace tgx {

// prompt::Prompt (prompt.rs:322-332): each position's token (read where it is text), patch
// ([patch_size][feat_dim], read where it is audio) and whether it is audio.
struct PromptView {
    const uint32_t* tokens;
    const float* patches;
    const uint8_t* audio;
    int len;
};

// Device memory freed with its holder.
struct DeviceMem {
    void* ptr = nullptr;
    size_t bytes = 0;
    DeviceMem() = default;
    DeviceMem(const DeviceMem&) = delete;
    DeviceMem& operator=(const DeviceMem&) = delete;
    ~DeviceMem();
};

// The positions a prompt began with and the LMs' keys and values over them (prompt.rs:367-380):
// for the base LM's layers then the residual LM's, the slot's first `blocks` cache blocks.
struct Prefix {
    std::vector<uint32_t> tokens, patches;  // patches: each position's patch's bits
    std::vector<uint8_t> audio;
    int len = 0, blocks = 0;
    DeviceMem kept;
    size_t bytes() const;
    int shared(const PromptView& p, int patch) const;
};

struct Voice {
    std::map<std::vector<uint32_t>, std::vector<float>> embeddings;  // a patch's bits -> [hidden]
    std::unique_ptr<Prefix> prefix;
    uint64_t used = 0;
    size_t bytes() const;
};

struct PromptCache {
    Context* ctx = nullptr;
    size_t budget = 0, bytes = 0;
    uint64_t clock = 0;
    std::map<std::vector<uint32_t>, Voice> voices;
};

struct Prompter {
    PatchStep* step = nullptr;
    int max_rows = 0, hidden = 0, latent = 0, feat = 0, frames = 0;
    std::vector<DeviceBuffer> allocations;
    float *levels = nullptr, *quantized = nullptr, *lm_hidden = nullptr, *residual_in = nullptr, *audio_x = nullptr;
    float *enc_out = nullptr, *embedded = nullptr;
    uint32_t* flags = nullptr;
    int last_rows = 0;  // the rows of the last run's last piece, which read() gives
};

tgx_status prompter_create(PatchStep* step, int max_rows, Prompter** out);
void prompter_destroy(Prompter* p);
// The embeddings of n patches, [n][patch_size][feat_dim] -> [n][hidden], as the base LM takes
// them: the encoder's rows at a time.
tgx_status prompter_embed(Prompter* p, const float* patches, int n, float* out);
// The embeddings of the prompt's positions from `from` to its last (not included), and those of
// its audio positions, zero at text: [len - 1 - from][hidden] each.
tgx_status prompter_embeddings(Prompter* p, const Checkpoint* ck, const PromptView& prompt, int from,
                               std::map<std::vector<uint32_t>, std::vector<float>>& known, std::vector<float>& x,
                               std::vector<float>& audio_x);
tgx_status prompter_run_rows(Prompter* p, uint32_t start, uint32_t slot, const float* x, const float* audio_x,
                             const uint8_t* audio, int len);
tgx_status prompter_run(Prompter* p, uint32_t slot, const Checkpoint* ck, const PromptView& prompt);
tgx_status prompter_run_cached(Prompter* p, uint32_t slot, const Checkpoint* ck, const PromptView& prompt, const float* voice,
                               size_t voice_len, PromptCache* cache, int* ran);
// The last piece's tensors: "base_out", "levels", "quantized", "lm_hidden", "residual_in",
// "residual_out", [rows][width] f32.
tgx_status prompter_read(Prompter* p, const char* tensor, float* out, size_t count);

}  // namespace tgx
