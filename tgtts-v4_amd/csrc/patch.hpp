// The host side of what runs around the LMs for each patch: the patch sampler over the local
// DiT (crates/graph/src/local/dit.rs) and the LM side (crates/graph/src/lm_side.rs).
#pragma once
#include <hip/hip_runtime.h>

#include <map>
#include <vector>

#include "heads_kernels.hpp"
#include "local_kernels.hpp"
#include "runtime.hpp"

namespace tgx {

// The condition tokens leading the DiT's sequence (dit.rs:36), and where the time token and the
// patch before start (dit.rs:40-41).
constexpr int MU_TOKENS = 2;
constexpr int TIME_AT = MU_TOKENS;
constexpr int COND_AT = TIME_AT + 1;

// A component's recorded graphs for one row count (a program, patch.rs:98-166 keeps one per row
// count): the step and, where it has one, the step that moves the rows on a position.
struct RowProgram {
    hipGraphExec_t exec = nullptr, advance = nullptr;
    int dispatches = 0;
};
void destroy_programs(std::map<int, RowProgram>& programs);

// schedule and euler_steps (dit.rs:44-79) in f32: the (t, dt) of each DiT evaluation.
std::vector<float> euler_schedule(int timesteps);
void euler_steps(int timesteps, std::vector<float>& t, std::vector<float>& dt);

// A timestep embedding's MLP, linear_2(SiLU(linear_1(x))), in f64 on the host (dit.rs:390-422).
struct TimeMlp {
    std::vector<double> w1, b1, w2, b2;
    int loaded = 0;  // a bit per tensor
    std::vector<double> forward(const std::vector<double>& x, int hidden) const;
};

struct Sampler {
    Context* ctx = nullptr;
    Shape shape{};  // the DiT's stack; capacity = T
    // rows: the current program's rows (1..max_rows), M and M_pad its tokens; max_rows: the
    // rows the tensors hold.
    int feat = 0, frames = 0, timesteps = 0, rows = 0, max_rows = 0;
    int T = 0, M = 0, M_pad = 0, o_parts = LOCAL_O_PARTS, down_parts = LOCAL_DOWN_PARTS;
    std::vector<float> step_t, step_dt;
    std::vector<DeviceBuffer> allocations;
    size_t device_bytes = 0;
    std::vector<Layer> layers;
    float* final_norm = nullptr;
    float *in_w = nullptr, *in_b = nullptr, *cond_w = nullptr, *cond_b = nullptr, *out_b = nullptr;
    uint16_t* out_w = nullptr;  // bf16 16-row tiles
    float* time_tokens = nullptr;  // [steps][hidden]
    bool times_dirty = true;
    TimeMlp time_mlp, delta_mlp;
    float *cos = nullptr, *sin = nullptr;
    float *x0 = nullptr, *x = nullptr, *h = nullptr, *partial = nullptr, *out = nullptr, *row_sq = nullptr, *row_sq0 = nullptr;
    uint16_t *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attended = nullptr, *mlp = nullptr, *normed0 = nullptr;
    float *mu = nullptr, *cond = nullptr, *noise = nullptr, *state = nullptr, *sampling = nullptr;
    std::map<int, RowProgram> programs;  // recorded on first launch; dropped when the times change
    hipGraphExec_t exec = nullptr;  // the current program's
    bool exec_dirty = true;
    int dispatches = 0;
    hipEvent_t ev_start = nullptr, ev_end = nullptr;
    bool pending = false, timed = false, use_graph = true;
    DispatchTimer timer;
    std::vector<hipEvent_t> timer_start, timer_stop;
    std::vector<const char*> timer_labels;

    LocalArgs args() const;
};

tgx_status sampler_create(Context* ctx, const tgx_shape* stack, const tgx_patch_shape* patch, Sampler** out);
void sampler_destroy(Sampler* s);
tgx_status sampler_load(Sampler* s, const char* name, const void* data, tgx_dtype dtype, size_t count);
// Copies the inputs in (mu [rows][MU_TOKENS][hidden], cond / noise [rows][feat][frames],
// sampling [rows][2]); any may be null to keep what the device holds.
tgx_status sampler_set_inputs(Sampler* s, const float* mu, const float* cond, const float* noise, const float* sampling);
// The program of `rows` rows (1 to the rows it was created for).
tgx_status sampler_use_rows(Sampler* s, int rows);
tgx_status sampler_launch(Sampler* s, int times);
tgx_status sampler_wait(Sampler* s);
tgx_status sampler_read(Sampler* s, float* patch);
// The sample's dispatches on the context's stream (timed when `timer`), mu read from `mu`.
hipError_t sampler_enqueue(Sampler* s, const float* mu, DispatchTimer* timer, int* dispatches);
tgx_status sampler_prepare(Sampler* s);
// Records the sample as the sampler's graph.
tgx_status sampler_record(Sampler* s);

// The local encoder (crates/graph/src/local/encoder.rs:42-128): each row's patch before, its
// frames through in_proj after a learned token, through a bidirectional local stack (a sequence
// of 1 + frames tokens to a row); the learned token's output after the final norm is the row's
// embedding.
struct Encoder {
    Context* ctx = nullptr;
    Shape shape{};  // the stack; capacity = T
    int feat = 0, frames = 0, rows = 0, max_rows = 0;  // as the sampler's
    int T = 0, M = 0, M_pad = 0, o_parts = LOCAL_O_PARTS, down_parts = LOCAL_DOWN_PARTS;
    std::vector<DeviceBuffer> allocations;
    size_t device_bytes = 0;
    std::vector<Layer> layers;
    float* final_norm = nullptr;
    float *in_w = nullptr, *in_b = nullptr, *special = nullptr;  // f32 [hidden][feat], [hidden], [hidden]
    float *cos = nullptr, *sin = nullptr;
    float *x0 = nullptr, *x = nullptr, *h = nullptr, *partial = nullptr, *out = nullptr, *row_sq = nullptr, *row_sq0 = nullptr;
    uint16_t *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attended = nullptr, *mlp = nullptr, *normed0 = nullptr;
    float *patch = nullptr, *embedding = nullptr;  // [rows][feat][frames], [rows][hidden]
    std::map<int, RowProgram> programs;  // patch -> embedding, by rows
    hipGraphExec_t exec = nullptr;       // the current program's
    int dispatches = 0;
    hipEvent_t ev_start = nullptr, ev_end = nullptr;
    bool pending = false;

    LocalArgs args() const;
};

tgx_status encoder_create(Context* ctx, const tgx_shape* stack, const tgx_patch_shape* patch, Encoder** out);
void encoder_destroy(Encoder* e);
tgx_status encoder_load(Encoder* e, const char* name, const void* data, tgx_dtype dtype, size_t count);
// The encoding's dispatches on the context's stream: the patches read from `patch`
// ([rows][feat][frames]), the embeddings written to `dst` ([rows][hidden]).
hipError_t encoder_enqueue(Encoder* e, const float* patch, float* dst, int* dispatches);
// Embeds the rows' patches (host arrays) and waits: Encoder::encode (encoder.rs:194-198).
tgx_status encoder_encode(Encoder* e, const float* patch, float* out);
// The program of `rows` rows (1 to the rows it was created for).
tgx_status encoder_use_rows(Encoder* e, int rows);

// The LM side: both LMs' decoders, the heads, and the tensors between them.
struct Linear {
    uint16_t* w = nullptr;  // 16-row tiles of [N_pad][K]
    float* b = nullptr;     // [N]
    int N = 0, K = 0;
};

struct LmSide {
    Context* ctx = nullptr;
    Decoder* base = nullptr;
    Decoder* residual = nullptr;
    // rows: the current program's rows (1..max_rows); max_rows: the rows the tensors hold.
    int rows = 0, max_rows = 0, hidden = 0, encoder = 0, dit = 0, latent = 0, levels = 0;
    std::vector<DeviceBuffer> allocations;
    Linear enc_to_lm, fsq_in, fsq_out, fusion, lm_to_dit, res_to_dit, stop_proj, stop_head;
    float *enc = nullptr, *levels_out = nullptr, *lm_hidden = nullptr, *stop_hidden = nullptr;
    float *mu = nullptr, *stop_logits = nullptr;
    std::map<int, RowProgram> programs;
    hipGraphExec_t exec = nullptr, advance_exec = nullptr;  // the current program's
    int dispatches = 0;
    hipEvent_t ev_start = nullptr, ev_end = nullptr;
    bool pending = false, use_graph = true;
};

tgx_status lm_side_create(Context* ctx, const tgx_shape* base, const tgx_shape* residual, const tgx_batch* batch,
                          const tgx_heads_shape* heads, LmSide** out);
void lm_side_destroy(LmSide* s);
tgx_status lm_side_load(LmSide* s, const char* name, const void* data, tgx_dtype dtype, size_t count);
// The layers between the LMs by name (Heads::named, lm_side.rs:127-140), and whether each has a bias.
struct LmHead {
    const char* name;
    bool bias;
};
std::vector<LmHead> lm_side_heads();
tgx_status lm_side_set_rows(LmSide* s, const tgx_row* rows, int nrows, const float* enc);
// The program of `rows` rows for both LMs and the heads (decoder_use_rows).
tgx_status lm_side_use_rows(LmSide* s, int rows);
tgx_status lm_side_launch(LmSide* s, int times, int advance);
tgx_status lm_side_wait(LmSide* s);
tgx_status lm_side_read(LmSide* s, const char* tensor, float* out, size_t count);
hipError_t lm_side_enqueue(LmSide* s, int advance, DispatchTimer* timer, int* dispatches);

// A patch step (crates/graph/src/patch.rs:98-166, 356-415): the encoder embeds each row's patch
// before, the LM side steps on the embeddings, the sampler samples on the LM side's mu and the
// same patch before. The three share a context and a row count; nothing leaves the device
// between them.
struct PatchStep {
    Encoder* encoder = nullptr;
    LmSide* side = nullptr;
    Sampler* sampler = nullptr;
    std::map<int, RowProgram> encodes;  // the sampler's cond -> the LM side's enc, by rows
    hipGraphExec_t encode = nullptr;    // the current program's
    hipEvent_t ev_start = nullptr, ev_end = nullptr;
    bool pending = false;
};

tgx_status patch_step_create(Encoder* e, LmSide* side, Sampler* s, PatchStep** out);
void patch_step_destroy(PatchStep* p);
// The row counts of a patch step's programs (generator.rs:115-123): each power of two below
// `rows`, then `rows`; and the fewest of them that holds `n` rows.
std::vector<int> program_rows(int rows);
int program_for(int rows, int n);
// The program of `rows` rows for the encoder, the LM side and the sampler.
tgx_status patch_step_use_rows(PatchStep* p, int rows);
// PatchStep::run_rows (patch.rs:356-415): on the program of the fewest rows that holds the
// `nrows` rows (the rest spare), places the rows, copies the patches before, the noise and the
// sampling in ([nrows][...]), runs the step and waits; the rows' patches and stop logits out.
tgx_status patch_step_run(PatchStep* p, const tgx_row* rows, int nrows, const float* cond, const float* noise,
                          const float* sampling, float* patch, float* stop_logits);
// `times` steps back to back over what the device holds (with `advance` every placed row moves
// on a position each step).
tgx_status patch_step_launch(PatchStep* p, int times, int advance);
tgx_status patch_step_wait(PatchStep* p);

}  // namespace tgx
