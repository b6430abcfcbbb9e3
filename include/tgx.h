/*
 * tgx — the MI355X (gfx950) runtime for tgtts-v4's MiniCPM-4 hot path, as a C ABI.
 *
 * It replaces the reference's Vulkan runtime crate (crates/vulkan) and the graph crate's GPU
 * programs for the decode step and the prefill (crates/graph/src/{decode,prefill,step}.rs) with
 * hand-written HIP kernels for gfx950, recorded once into a HIP graph and launched every step.
 * Every entry point takes plain pointers and sizes; the library owns all device memory, the
 * caller owns the host arrays it passes in and out.
 *
 * Threading: a context and everything made from it belong to one thread at a time (as the
 * reference's single GPU thread owns its Engine, crates/tgtts/src/rt.rs:1-7). Nothing here is
 * safe to call from two threads at once on the same context.
 *
 * Errors: every function returns a tgx_status; on failure tgx_last_error() holds a message for
 * the calling thread. Shapes and placements are checked on the host before anything is
 * launched (decode.rs:440-449, :198-227).
 */
#ifndef TGX_H
#define TGX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the classes of vulkan::Error (crates/vulkan/src/error.rs:5-43) and graph::Error
 * (crates/graph/src/lib.rs:41-59) a caller can act on. */
typedef enum {
    TGX_OK = 0,
    TGX_E_SHAPE = 1,      /* graph::Error::Shape: shapes or placements the kernels cannot run */
    TGX_E_HIP = 2,        /* vulkan::Error::Vk: a HIP call failed */
    TGX_E_KERNELS = 3,    /* graph::Error::Kernels: the code object lacks a kernel or target */
    TGX_E_WEIGHTS = 4,    /* graph::Error::Checkpoint: a weight of the wrong name or size */
    TGX_E_NOT_FINITE = 5, /* graph::Error::NotFinite: an output came out NaN or infinite */
    TGX_E_TIMEOUT = 6,    /* the fence wait's 60 s timeout (crates/vulkan/src/context.rs:24) */
    TGX_E_BUSY = 7,       /* a run is under way: the host may not touch its buffers */
    TGX_E_ARG = 8,        /* a null handle or pointer */
    TGX_E_NO_DEVICE = 9   /* vulkan::Error::NoDevice */
} tgx_status;

/* The last error message of the calling thread ("" when none). */
const char* tgx_last_error(void);

/* Element types of host arrays handed to tgx_decoder_load, and of a kernel's bindings
 * (ElementType, crates/vulkan/src/element.rs; u32 only for bindings). */
typedef enum { TGX_F32 = 0, TGX_BF16 = 1, TGX_F16 = 2, TGX_U32 = 3 } tgx_dtype;

/* ---- context: replaces vulkan::Context (crates/vulkan/src/context.rs:237-540) ---- */

typedef struct tgx_context tgx_context;

typedef struct {
    char name[64];         /* e.g. "AMD Instinct MI355X" */
    char arch[32];         /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int compute_units;
    int clock_khz;         /* peak engine clock */
    int memory_clock_khz;
    size_t memory_bytes;
    int wavefront;         /* 64 */
} tgx_device_report;

/* Context::new: opens `device` and the stream every program of the context runs on. */
tgx_status tgx_context_create(int device, tgx_context** out);
void tgx_context_destroy(tgx_context* ctx);
/* Context::report. */
tgx_status tgx_context_report(const tgx_context* ctx, tgx_device_report* out);
/* Context::set_fence_spin (crates/vulkan/src/context.rs:467-474, its wait Inner::wait_for,
 * :116-133): every wait for the context's work (tgx_decoder_wait, tgx_program_wait and the
 * sampler's, LM side's, encoder's and patch step's) polls for up to `ns` nanoseconds before it
 * sleeps between polls, 20 µs apart, 60 s at most in all; 0, the default, sleeps at once. */
tgx_status tgx_context_set_fence_spin(tgx_context* ctx, uint64_t ns);
/* Calibration (context.rs:73-88): the GPU's clock read `ticks` while the host's CLOCK_MONOTONIC
 * read `monotonic_ns`, give or take `deviation_ns`; `period_ns` nanoseconds a tick. */
typedef struct {
    uint64_t ticks;
    uint64_t monotonic_ns;
    uint64_t deviation_ns;
    float period_ns;
} tgx_calibration;
/* Context::calibrate (context.rs:445-465): the GPU's constant-rate wall clock
 * (hipDeviceAttributeWallClockRate) read by a one-wave kernel between two readings of the host's
 * clock, once the context's stream is idle: monotonic_ns their midpoint, deviation_ns half their
 * distance (a launch and a wait, tens of µs). */
tgx_status tgx_context_calibrate(tgx_context* ctx, tgx_calibration* out);

/* The stream-read floor (kernels/glsl/stream_read.comp:1-23, as decode_timing.rs:430-441 reports
 * it): a buffer of `bytes` (rounded down to 32 KiB) read once a launch, 16 bytes a load, `times`
 * launches each timed by events; the best and the mean milliseconds. The bandwidth the decode
 * kernels are held to. Allocates the buffer for the call. */
tgx_status tgx_stream_read(tgx_context* ctx, size_t bytes, int times, float* best_ms, float* mean_ms);

/* ---- the decode step: crates/graph/src/decode.rs ---- */

/* decode::Shape (decode.rs:65-82). `capacity` is the most positions one request (slot) may
 * reach. rope_factors: LongRoPE's short_factor (head_dim / 2 values), or NULL for all 1. */
typedef struct {
    int hidden, inner, heads, kv_heads, head_dim, layers, capacity;
    float eps, rope_theta;
    int rope;
    const double* rope_factors;
} tgx_shape;

/* decode::Batch (decode.rs:171-178) and the paged cache that replaces the reference's
 * [slots][kv_heads][capacity][head_dim] caches: `rows` run per step, `slots` requests are kept,
 * the cache is a pool of `blocks` blocks of `block_tokens` positions (0: enough for every slot at
 * full capacity) handed out to slots as their positions grow. */
typedef struct {
    int rows;
    int slots;
    int block_tokens; /* 64 is the only size the kernels take; 0 means 64 */
    int blocks;
} tgx_batch;

/* decode::Row (decode.rs:230-235): a row's position in its slot. A row whose position is
 * TGX_SPARE is spare: it writes no cache and attends to nothing (batch.glsl:9-14). */
typedef struct {
    uint32_t position;
    uint32_t slot;
} tgx_row;
#define TGX_SPARE 0xFFFFFFFFu

typedef struct tgx_decoder tgx_decoder;

/* The shape checks tgx_decoder_create makes, on the host alone (Shape::new's refusals and
 * decode_batch_graph's, decode.rs:87-126, :468-491): TGX_OK or TGX_E_SHAPE with the reason. */
tgx_status tgx_shape_check(const tgx_shape* shape, const tgx_batch* batch);

/* Batch::placement (decode.rs:198-227), on the host alone: writes 2 * nrows words, each row's
 * position then each row's slot, TGX_SPARE for a spare row; refuses two rows in one slot, a slot
 * past `slots` and a position past `capacity`. */
tgx_status tgx_batch_placement(int slots, int capacity, const tgx_row* rows, int nrows,
                               uint32_t* words);

/* Decoder::with_batch (decode.rs:799-813): allocates weights (zero until loaded), the paged
 * cache and the step's buffers, writes the RoPE tables and records the step as a HIP graph. */
tgx_status tgx_decoder_create(tgx_context* ctx, const tgx_shape* shape, const tgx_batch* batch,
                              tgx_decoder** out);
void tgx_decoder_destroy(tgx_decoder* dec);

/* load_stack's write of one tensor (decode.rs:740-776), under the names the step's graph gives
 * them (decode.rs:632-650, 716): "layers.{l}.input_layernorm", "layers.{l}.qkv_proj" (q_proj;
 * k_proj; v_proj joined along their outputs, [(heads + 2 kv_heads) head_dim][hidden]),
 * "layers.{l}.o_proj" ([hidden][heads head_dim]), "layers.{l}.post_attention_layernorm",
 * "layers.{l}.gate_up_proj" (gate_proj; up_proj, [2 inner][hidden]), "layers.{l}.down_proj"
 * ([hidden][inner]) and "norm". `count` elements of `dtype`, row-major; converted to bf16
 * (round to nearest even) and laid out in the kernels' tiles. */
tgx_status tgx_decoder_load(tgx_decoder* dec, const char* name, const void* data, tgx_dtype dtype,
                            size_t count);

/* Decoder::set_rows (decode.rs:857-862): `x` is [rows][hidden] f32, `rows` one per row of the
 * batch (nrows == batch.rows). Refuses two rows in one slot and positions past the capacity
 * (Batch::placement, decode.rs:198-227). Hands out cache blocks to slots as needed. */
tgx_status tgx_decoder_set_rows(tgx_decoder* dec, const tgx_row* rows, int nrows, const float* x);
/* Decoder::start (decode.rs:865-867): launches the step over the input last written. */
tgx_status tgx_decoder_start(tgx_decoder* dec);
/* Submission::wait (crates/vulkan/src/recording.rs:747-753): waits for it, 60 s at most. */
tgx_status tgx_decoder_wait(tgx_decoder* dec);
/* Decoder::output (decode.rs:870-872): [rows][hidden] f32 after the final norm; a spare row's
 * values are meaningless. */
tgx_status tgx_decoder_output(tgx_decoder* dec, float* out);
/* Decoder::step_rows (decode.rs:849-853): set_rows, start, wait, output. */
tgx_status tgx_decoder_step_rows(tgx_decoder* dec, const tgx_row* rows, int nrows, const float* x,
                                 float* out);
/* Decoder::step (decode.rs:833-837): batch 1, slot 0. */
tgx_status tgx_decoder_step(tgx_decoder* dec, uint32_t position, const float* x, float* out);

/* Releases the cache blocks of `slot`, which a new request may then take (the paged cache's
 * counterpart of starting a request over in a slot). */
tgx_status tgx_decoder_release_slot(tgx_decoder* dec, uint32_t slot);
/* Hands `slot` the blocks for positions 0..positions-1 now, so that steps running ahead on the
 * device (tgx_decoder_launch with advance) find them. */
tgx_status tgx_decoder_reserve(tgx_decoder* dec, uint32_t slot, uint32_t positions);
/* The blocks free in the pool. */
tgx_status tgx_decoder_free_blocks(const tgx_decoder* dec, int* out);

/* Launches the recorded step `times` times back to back on the context's stream over the
 * device-resident input, without copying anything in or out: what a caller whose inputs are
 * already in HBM runs. With `advance`, each step moves every placed row on by one position
 * after it (teacher-forced continuation); the slots must hold the blocks (tgx_decoder_reserve).
 * Returns when launched; tgx_decoder_wait waits. */
tgx_status tgx_decoder_launch(tgx_decoder* dec, int times, int advance);

/* The GPU time of the last tgx_decoder_launch or step, in milliseconds, from HIP events on the
 * context's stream around it (Step::elapsed, step.rs:381-384). */
tgx_status tgx_decoder_elapsed_ms(const tgx_decoder* dec, float* out);

/* Decoder::new's `timed` (decode.rs:788-796, recording.rs:15-17): when on, steps are launched
 * dispatch by dispatch instead of as the recorded graph, each dispatch timed by events its own
 * dispatch records, so that its time is the kernel's alone. */
tgx_status tgx_decoder_set_timed(tgx_decoder* dec, int timed);

/* Whether steps launch the recorded HIP graph (the default) or their dispatches one by one,
 * as a profiler that follows single dispatches needs. The same kernels either way. */
tgx_status tgx_decoder_set_graph(tgx_decoder* dec, int use_graph);

/* Decoder::timings (decode.rs:891-893): each dispatch's label and GPU time in the last timed step,
 * in order; *n is the number of dispatches (0 when not timed), of which `max` are written. */
typedef struct {
    char label[32];
    float ms;
} tgx_timing;
tgx_status tgx_decoder_timings(tgx_decoder* dec, int max, tgx_timing* out, int* n);

/* The step's dispatches and device bytes (Step::dispatches / arena_bytes, step.rs:398-411). */
tgx_status tgx_decoder_dispatches(const tgx_decoder* dec, int* out);
tgx_status tgx_decoder_device_bytes(const tgx_decoder* dec, size_t* out);

/* Reads the cache of `slot` back, for tests: keys and values of positions 0..positions-1 as
 * [layers][kv_heads][positions][head_dim] f32 each. */
tgx_status tgx_decoder_read_cache(tgx_decoder* dec, uint32_t slot, uint32_t positions, float* k,
                                  float* v);

/* ---- the prefill: crates/graph/src/prefill.rs ---- */

/* Prefill::run (prefill.rs:473-503): runs `len` positions from `start` of `slot` at once, their
 * hidden states x [len][hidden] f32, writing their keys and values into the decoder's cache for
 * its steps to go on from, each position attending over the slot up to itself. Returns the
 * outputs after the final norm, [len][hidden] f32. The reference runs slot 0 only and at most
 * 1024 positions a program; any slot and any length within the capacity are taken here. */
tgx_status tgx_prefill_run(tgx_decoder* dec, uint32_t slot, uint32_t start, uint32_t len,
                           const float* x, float* out);

/* Several runs at once, each in its own slot, as one prefill: x holds their hidden states one run
 * after another ([sum of len][hidden]), and out their outputs in the same order. */
typedef struct {
    uint32_t slot, start, len;
} tgx_run;
tgx_status tgx_prefill_runs(tgx_decoder* dec, const tgx_run* runs, int nruns, const float* x,
                            float* out);

/* Launches the last prefill again `times` times over its input still on the device, copying
 * nothing in or out (what a caller whose inputs are already in HBM runs; it writes the same
 * keys and values again). Returns when launched; tgx_decoder_wait waits, and
 * tgx_decoder_elapsed_ms times it. */
tgx_status tgx_prefill_launch(tgx_decoder* dec, int times);

/* tgx_prefill_runs without allocating: no counterpart in the reference. It is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc), where tgx_prefill_runs grows its tensors on a call longer than any before it.
 * The same runs, outputs and cache writes, bit for bit; the tensors live in a fixed array of
 * 32 MiB on each GPU (held until the process ends), which at the backbone's shape (hidden 1024,
 * inner 4096, 16 heads) holds 1024 positions a call: runs past it are refused with TGX_E_SHAPE
 * before anything runs. Every call on a GPU shares that GPU's array, so calls that overlap on one
 * GPU (from several threads, or decoders on one device) race; the call returns when its output is
 * copied out. */
tgx_status tgx_prefill_runs_noalloc(tgx_decoder* dec, const tgx_run* runs, int nruns, const float* x,
                                    float* out);

/* ---- the patch sampler: crates/graph/src/local/dit.rs ---- */

/* What sampler_graph takes besides the DiT's stack (dit.rs:114-131): a patch of `feat_dim`
 * channels by `patch_size` frames, sampled in `timesteps` Euler steps, for `rows` rows at once.
 * The DiT's sequences are MU_TOKENS (2) condition tokens, the time, the patch before and the
 * noisy patch: 3 + 2 patch_size tokens. */
typedef struct {
    int feat_dim, patch_size, timesteps, rows;
} tgx_patch_shape;

typedef struct tgx_sampler tgx_sampler;

/* euler_steps (dit.rs:61-79), in f32: the time and step length of each step the DiT runs at in
 * `timesteps` steps (the first 4 %, at least one, run nothing); *n of them, `max` written. */
tgx_status tgx_euler_steps(int timesteps, int max, float* t, float* dt, int* n);

/* Sampler::new (dit.rs:270-282): the DiT's stack as a tgx_shape (head_dim 64; capacity is
 * ignored, the sequence is the capacity), weights zero until loaded; records the sample, every
 * Euler step with its DiT run, as one HIP graph. */
tgx_status tgx_sampler_create(tgx_context* ctx, const tgx_shape* stack, const tgx_patch_shape* patch,
                              tgx_sampler** out);
void tgx_sampler_destroy(tgx_sampler* s);

/* load_sampler (dit.rs:329-365), one tensor: the stack's as tgx_decoder_load names them
 * ("layers.{l}.qkv_proj", ..., "norm"); "in_proj.weight" and "cond_proj.weight"
 * ([hidden][feat_dim]), "out_proj.weight" ([feat_dim][hidden]) and their ".bias"; and the time
 * MLPs "time_mlp.linear_1.weight", "time_mlp.linear_1.bias", "time_mlp.linear_2.weight",
 * "time_mlp.linear_2.bias" and the same under "delta_time_mlp." ([hidden][hidden], [hidden]),
 * from which each step's time token is computed in f64 on the host. */
tgx_status tgx_sampler_load(tgx_sampler* s, const char* name, const void* data, tgx_dtype dtype,
                            size_t count);

/* Sampler::sample (dit.rs:294-309): each row's patch [feat_dim][patch_size] f32 from its
 * conditions mu [MU_TOKENS][hidden] (lm_to_dit_proj's output, then res_to_dit_proj's), its patch
 * before `cond` and its `noise` (both [feat_dim][patch_size]), at its temperature and guidance
 * scale (`sampling` [rows][2]); every array a row after a row, f32. */
tgx_status tgx_sampler_sample(tgx_sampler* s, const float* mu, const float* cond, const float* noise,
                              const float* sampling, float* patch);
/* Launches the sample `times` times over the inputs on the device, copying nothing (each from
 * the same noise); tgx_sampler_wait waits, tgx_sampler_elapsed_ms times it. */
tgx_status tgx_sampler_launch(tgx_sampler* s, int times);
tgx_status tgx_sampler_wait(tgx_sampler* s);
tgx_status tgx_sampler_elapsed_ms(const tgx_sampler* s, float* out);
/* Sampler::timings (dit.rs:311-313): as tgx_decoder_set_timed / tgx_decoder_timings. */
tgx_status tgx_sampler_set_timed(tgx_sampler* s, int timed);
tgx_status tgx_sampler_timings(tgx_sampler* s, int max, tgx_timing* out, int* n);
tgx_status tgx_sampler_dispatches(const tgx_sampler* s, int* out);

/* ---- the LM side: crates/graph/src/lm_side.rs ---- */

/* LmSideShape's widths besides the LMs' (lm_side.rs:59-72): the local encoder's (the step's
 * input), the DiT's (mu is [rows][2 dit]), the scalar quantizer's bottleneck and its levels to a
 * unit (scalar_quantization_scale). */
typedef struct {
    int encoder, dit, latent, levels;
} tgx_heads_shape;

typedef struct tgx_lm_side tgx_lm_side;

/* lm_side_batch_graph (lm_side.rs:337-491): the base LM and the residual LM (a tgx_shape each;
 * the residual's rope = 0, decode.rs:47-50) as decoders over one batch, and the layers between
 * them; records the step as one HIP graph. */
tgx_status tgx_lm_side_create(tgx_context* ctx, const tgx_shape* base, const tgx_shape* residual,
                              const tgx_batch* batch, const tgx_heads_shape* heads, tgx_lm_side** out);
void tgx_lm_side_destroy(tgx_lm_side* s);

/* load_lm_side (lm_side.rs:496-533), one tensor: "base_lm.<name>" and "residual_lm.<name>" as
 * tgx_decoder_load names them; "enc_to_lm_proj", "fsq_layer.in_proj", "fsq_layer.out_proj",
 * "fusion_concat_proj", "lm_to_dit_proj", "res_to_dit_proj", "stop_proj" each ".weight"
 * ([out][in]) and ".bias"; "stop_head.weight" (no bias, Heads::named, lm_side.rs:131-142). */
tgx_status tgx_lm_side_load(tgx_lm_side* s, const char* name, const void* data, tgx_dtype dtype,
                            size_t count);
/* The decoder of the base LM (which = 0) or the residual LM (1), to prefill its cache or release
 * its slots; owned by the LM side. */
tgx_status tgx_lm_side_decoder(tgx_lm_side* s, int which, tgx_decoder** out);

/* LmSide::step_rows (lm_side.rs:599-625): `enc` [rows][encoder] f32 at the rows' places
 * (both LMs' caches written there); returns mu [rows][2 dit] and the stop logits [rows][2]. */
tgx_status tgx_lm_side_step(tgx_lm_side* s, const tgx_row* rows, int nrows, const float* enc,
                            float* mu, float* stop_logits);
/* Places the rows and copies `enc` in without launching. */
tgx_status tgx_lm_side_set_rows(tgx_lm_side* s, const tgx_row* rows, int nrows, const float* enc);
/* Launches the step `times` times over what the device holds; with `advance` each moves every
 * placed row on by a position (the slots must hold the blocks: tgx_decoder_reserve on both). */
tgx_status tgx_lm_side_launch(tgx_lm_side* s, int times, int advance);
tgx_status tgx_lm_side_wait(tgx_lm_side* s);
tgx_status tgx_lm_side_elapsed_ms(const tgx_lm_side* s, float* out);
/* One of the step's tensors after the last step, f32, `count` values: "embed" [rows][hidden],
 * "base_out", "levels" [rows][latent], "lm_hidden", "residual_in", "residual_out",
 * "stop_hidden" ([rows][hidden]), "mu" [rows][2 dit], "stop_logits" [rows][2]. */
tgx_status tgx_lm_side_read(tgx_lm_side* s, const char* tensor, float* out, size_t count);
tgx_status tgx_lm_side_dispatches(const tgx_lm_side* s, int* out);

/* ---- a patch step: the LM side, then the sampler on its mu (crates/graph/src/patch.rs) ---- */

/* Launches `times` patch steps back to back on the context's stream over what the devices hold:
 * each runs the LM side with advance (every placed row moves on a position) and the sampler on
 * the LM side's mu, copied on the device (PatchStep's order, patch.rs:356-415, without the local
 * encoder: each step's `enc` stays as last set). The two must share a context and a row count,
 * and the sampler's width must be the LM side's DiT width. tgx_lm_side_wait waits; the time is
 * tgx_patch_elapsed_ms's. */
tgx_status tgx_patch_launch(tgx_lm_side* side, tgx_sampler* sampler, int times);
tgx_status tgx_patch_elapsed_ms(const tgx_lm_side* side, float* out);

/* ---- the local encoder: crates/graph/src/local/encoder.rs ---- */

typedef struct tgx_encoder tgx_encoder;

/* Encoder::new (encoder.rs:171-183): the encoder's stack as a tgx_shape (head_dim 64; capacity
 * is ignored, a row's sequence is its learned token and the patch's frames, 1 + patch_size
 * tokens), for patches of patch->feat_dim channels by patch->patch_size frames, patch->rows rows
 * at once (patch->timesteps is ignored); weights zero until loaded. */
tgx_status tgx_encoder_create(tgx_context* ctx, const tgx_shape* stack, const tgx_patch_shape* patch,
                              tgx_encoder** out);
void tgx_encoder_destroy(tgx_encoder* e);
/* load_encoder (encoder.rs:133-162), one tensor: the stack's as tgx_decoder_load names them,
 * "special_token" [hidden], "in_proj.weight" [hidden][feat_dim] and "in_proj.bias" [hidden]. */
tgx_status tgx_encoder_load(tgx_encoder* e, const char* name, const void* data, tgx_dtype dtype,
                            size_t count);
/* Encoder::encode (encoder.rs:194-198): each row's embedding [rows][hidden] f32 from its patch
 * [feat_dim][patch_size] f32, a row after a row; waits. */
tgx_status tgx_encoder_encode(tgx_encoder* e, const float* patch, float* out);
tgx_status tgx_encoder_dispatches(const tgx_encoder* e, int* out);

/* ---- the patch step with its encoder: crates/graph/src/patch.rs ---- */

typedef struct tgx_patch_step tgx_patch_step;

/* patch_batch_graph (patch.rs:98-166) over an encoder, an LM side and a sampler made alike (one
 * context, one row count, the encoder as wide as the LM side's encoder width, the sampler as wide
 * as its DiT width, one patch shape): each step embeds the patches before, steps the LM side on
 * the embeddings and samples on its mu, nothing leaving the device between them. The three stay
 * owned by the caller and must outlive the step. */
tgx_status tgx_patch_step_create(tgx_encoder* e, tgx_lm_side* side, tgx_sampler* sampler, tgx_patch_step** out);
void tgx_patch_step_destroy(tgx_patch_step* p);
/* PatchStep::run_rows (patch.rs:356-415): the rows' places (spare ones TGX_SPARE), each row's
 * patch before `cond` and `noise` ([rows][feat_dim][patch_size]) and `sampling` ([rows][2]:
 * temperature, guidance scale); returns each row's patch and stop logits [rows][2]. Waits.
 * `nrows` may be fewer than the step's rows: the step runs on its program of the fewest rows that
 * holds them (each power of two below its rows, then its rows: generator.rs:115-123), the rest
 * spare, each row's results as on any other program. The encoder's, LM side's and sampler's own
 * entry points take their whole batch again. */
tgx_status tgx_patch_step_run(tgx_patch_step* p, const tgx_row* rows, int nrows, const float* cond,
                              const float* noise, const float* sampling, float* patch, float* stop_logits);
/* Launches `times` steps back to back over what the device holds (with `advance` every placed row
 * moves on a position each step; the slots must hold the blocks); tgx_patch_step_wait waits and
 * tgx_patch_step_elapsed_ms times them. */
tgx_status tgx_patch_step_launch(tgx_patch_step* p, int times, int advance);
tgx_status tgx_patch_step_wait(tgx_patch_step* p);
tgx_status tgx_patch_step_elapsed_ms(const tgx_patch_step* p, float* out);

/* ---- weights from a safetensors checkpoint: crates/graph/src/checkpoint.rs ---- */

typedef struct tgx_checkpoint tgx_checkpoint;

/* Checkpoint::open (checkpoint.rs:36-71): parses the header (at most 100 MiB) and checks every
 * entry (BF16, F16 or F32; bytes equal to its shape's) against the file; tensors are read from
 * their offsets when asked for. TGX_E_WEIGHTS (graph::Error::Checkpoint) with the reason. */
tgx_status tgx_checkpoint_open(const char* path, tgx_checkpoint** out);
void tgx_checkpoint_close(tgx_checkpoint* ck);
/* The tensors' names in order (the header is a BTreeMap, checkpoint.rs:31): count, then name i. */
tgx_status tgx_checkpoint_count(const tgx_checkpoint* ck, int* out);
tgx_status tgx_checkpoint_name(const tgx_checkpoint* ck, int index, char* out, size_t capacity);
/* Checkpoint::shape (checkpoint.rs:74-76): the dims (up to `max`), their number and the dtype. */
tgx_status tgx_checkpoint_shape(const tgx_checkpoint* ck, const char* name, int64_t* dims, int max, int* ndims,
                                tgx_dtype* dtype);
/* Checkpoint::f16 (checkpoint.rs:106-125), in f32: exact from BF16 and F16. `count` must be the
 * tensor's. */
tgx_status tgx_checkpoint_read(const tgx_checkpoint* ck, const char* name, float* out, size_t count);
/* Checkpoint::gather_f16 (checkpoint.rs:127-139), in f32: rows `rows` of a 2-D tensor one after
 * another (an embedding lookup reading those rows alone); a row past the tensor is refused. */
tgx_status tgx_checkpoint_gather(const tgx_checkpoint* ck, const char* name, const int64_t* rows, int n, float* out);

/* load_stack (decode.rs:738-776): the decoder's layers from `prefix` ("base_lm.", "residual_lm."
 * or ""): q/k/v and gate/up joined along their rows, the norms, then norm.weight. */
tgx_status tgx_decoder_load_checkpoint(tgx_decoder* dec, const tgx_checkpoint* ck, const char* prefix);
/* load_lm_side (lm_side.rs:496-533): both stacks and the layers between them. */
tgx_status tgx_lm_side_load_checkpoint(tgx_lm_side* s, const tgx_checkpoint* ck);
/* load_sampler (local/dit.rs:329-365): feat_decoder.estimator.{decoder.*, in_proj, cond_proj,
 * out_proj, time_mlp, delta_time_mlp}. */
tgx_status tgx_sampler_load_checkpoint(tgx_sampler* s, const tgx_checkpoint* ck);
/* load_encoder (local/encoder.rs:129-162): feat_encoder.{encoder.*, special_token, in_proj}. */
tgx_status tgx_encoder_load_checkpoint(tgx_encoder* e, const tgx_checkpoint* ck);

/* ---- a prompt into the patch step's caches: crates/graph/src/prompt.rs ---- */

typedef struct tgx_prompter tgx_prompter;
typedef struct tgx_prompt_cache tgx_prompt_cache;

/* prompt::Prompt (prompt.rs:322-332): each position's token (read where it is text), patch
 * ([patch_size][feat_dim] f32, read where it is audio) and whether it is audio (0 or 1). */
typedef struct {
    const uint32_t* tokens;
    const float* patches;
    const uint8_t* audio;
    int len;
} tgx_prompt;

/* Prompter::new (prompt.rs:527-552) over a patch step's encoder and LM side: runs of up to
 * `max_rows` positions at a time. */
tgx_status tgx_prompter_create(tgx_patch_step* step, int max_rows, tgx_prompter** out);
void tgx_prompter_destroy(tgx_prompter* p);
tgx_status tgx_prompter_max_rows(const tgx_prompter* p, int* out);
/* Prompter::embed (prompt.rs:559-566): a patch [patch_size][feat_dim] -> [hidden] as the base LM
 * takes it (the encoder, then enc_to_lm_proj). */
tgx_status tgx_prompter_embed(tgx_prompter* p, const float* patch, float* out);
/* Prompter::embeddings (prompt.rs:636-648): the prompt's positions but its last, [len - 1][hidden],
 * and those of its audio positions (zero at text): a token's row of base_lm.embed_tokens.weight
 * read from `ck`, a patch's embedding once for each distinct patch. */
tgx_status tgx_prompter_embeddings(tgx_prompter* p, const tgx_checkpoint* ck, const tgx_prompt* prompt, float* x,
                                   float* audio_x);
/* Prompter::run_rows (prompt.rs:692-752): `len` positions from `at` through the base LM, the
 * quantizer at the audio positions, fusion_concat_proj beside the audio embeddings and the
 * residual LM, both LMs' keys and values into the slot's caches; max_rows at a time. */
tgx_status tgx_prompter_run_rows(tgx_prompter* p, tgx_row at, const float* x, const float* audio_x, const uint8_t* audio,
                                 int len);
/* Prompter::run (prompt.rs:568-583): every position of a prompt that ends in audio but the last,
 * from position 0 of `slot`; the first patch step after it runs the last as the patch before. */
tgx_status tgx_prompter_run(tgx_prompter* p, uint32_t slot, const tgx_checkpoint* ck, const tgx_prompt* prompt);
/* Prompter::run_cached (prompt.rs:585-641): as tgx_prompter_run in the voice whose latent frames
 * are `voice`: from the positions it begins with that `cache` keeps of the voice (their keys and
 * values copied back into the slot), with the patches' embeddings it keeps; keeps there what the
 * next prompts in the voice can use. `ran`: the positions that ran through the LMs, the last
 * among them. */
tgx_status tgx_prompter_run_cached(tgx_prompter* p, uint32_t slot, const tgx_checkpoint* ck, const tgx_prompt* prompt,
                                   const float* voice, size_t voice_len, tgx_prompt_cache* cache, int* ran);
/* The last run's last piece: "base_out", "levels", "quantized", "lm_hidden", "residual_in" or
 * "residual_out", [rows][width] f32 (the stage-by-stage view the tests compare). */
tgx_status tgx_prompter_read(tgx_prompter* p, const char* tensor, float* out, size_t count);
/* PromptCache::new (prompt.rs:414-424): keeps at most `budget` bytes, host and device together;
 * the voices used longest ago make room for others. */
tgx_status tgx_prompt_cache_create(tgx_context* ctx, size_t budget, tgx_prompt_cache** out);
void tgx_prompt_cache_destroy(tgx_prompt_cache* c);
tgx_status tgx_prompt_cache_bytes(const tgx_prompt_cache* c, size_t* out);
tgx_status tgx_prompt_cache_voices(const tgx_prompt_cache* c, int* out);

/* ---- the engine the service's GPU thread drives: crates/tgtts/src/rt.rs, crates/graph/src/generator.rs ---- */

typedef struct tgx_engine tgx_engine;

/* generator::Settings (generator.rs:35-56): the requests at once (the patch step's rows, a row to
 * a slot), the positions a slot's caches hold, a prompt's positions one run takes, the Euler
 * steps, and the prompt cache's bytes. */
typedef struct {
    int slots, capacity, max_rows, timesteps;
    size_t prompt_cache_bytes;
} tgx_engine_settings;

/* What a step gave the request in `slot` (generator::Outcome, generator.rs:76): TGX_OK and its
 * patch (in the step's frames), or TGX_E_NOT_FINITE, after which it has ended; `last` when it was
 * the request's last (the stop head's argmax, or its most patches sampled). */
typedef struct {
    int slot;
    tgx_status status;
    int last;
    float stop_logits[2];
} tgx_engine_outcome;

/* Generator::new (generator.rs:130-193) over the shapes config.json gives (the base LM, the
 * residual LM, the layers between them, the local encoder's and the DiT's stacks, the latent
 * frames of a patch) and the weights in `ck`, which the engine reads token embeddings from and
 * which must outlive it. The audio VAE is not part of the engine: it hands back latent frames. */
tgx_status tgx_engine_create(tgx_context* ctx, const tgx_checkpoint* ck, const tgx_shape* base, const tgx_shape* residual,
                             const tgx_heads_shape* heads, const tgx_shape* encoder, const tgx_shape* dit, int feat_dim,
                             int patch_size, const tgx_engine_settings* settings, tgx_engine** out);
/* Engine::close (rt.rs:108-110). */
void tgx_engine_destroy(tgx_engine* e);
/* Engine::slots (rt.rs:96). */
tgx_status tgx_engine_slots(const tgx_engine* e, int* out);
/* Engine::start (rt.rs:98-100; Generator::start, generator.rs:205-262): ends any request in the
 * slot and runs `prompt` into it from what the prompt cache keeps of the voice (its latent frames,
 * feat_dim values each), to sample up to `max_patches` patches at `temperature` and guidance
 * `cfg`; `prefilled`: the prompt's positions that ran through the LMs. */
tgx_status tgx_engine_start(tgx_engine* e, int slot, const tgx_prompt* prompt, const float* voice, size_t voice_len,
                            int max_patches, float temperature, float cfg, int* prefilled);
/* Generator::sample_after (generator.rs:264-279): the slot's next patch sampled after `frames`,
 * [patch_size][feat_dim], rather than its last (teacher forcing). */
tgx_status tgx_engine_sample_after(tgx_engine* e, int slot, const float* frames);
/* Engine::step (rt.rs:102-104; Generator::step, generator.rs:281-334): a patch of every request
 * under way in one patch step, each from its slot's noise (`noise` [slots][feat_dim][patch_size],
 * read for the slots under way); `n` outcomes, each request's patch in `frames`
 * [slots][patch_size][feat_dim] at its slot. A request whose last patch was sampled waits in its
 * slot to be finished. */
tgx_status tgx_engine_step(tgx_engine* e, const float* noise, tgx_engine_outcome* outcomes, float* frames, int* n);
/* Generator::levels (generator.rs:336-362): the quantizer's levels (integers) the slot's last
 * patch was sampled after, [latent]. */
tgx_status tgx_engine_levels(tgx_engine* e, int slot, float* out);
/* Generator::take_audio (generator.rs:364-369) for the latent frames: those sampled since last
 * taken, `n` frames of feat_dim values (at most `max`). */
tgx_status tgx_engine_take_frames(tgx_engine* e, int slot, float* out, int max, int* n);
/* Engine::finish (rt.rs:106-107; Generator::finish, generator.rs:395-403): ends the request,
 * giving the frames not yet taken. */
tgx_status tgx_engine_finish(tgx_engine* e, int slot, float* out, int max, int* n);
/* What the prompt cache keeps (Generator::prompt_cache, generator.rs:364-367). */
tgx_status tgx_engine_prompt_cache(const tgx_engine* e, size_t* bytes, int* voices);

/* ---- the runtime beneath the models: crates/vulkan's Memory, Kernel and Recording ----
 *
 * What the graph crate asks of crates/vulkan (lib.rs:50-60), for callers that compose programs of
 * their own from the library's kernels: memory in a residence, read and written by the host
 * between runs; the kernels by name, each with its bindings in order (crates/graph/src/kernels.rs:
 * 27-63,104-161); and programs, chains of dispatches recorded once (here a HIP graph) and run as
 * often as needed (crates/vulkan/src/recording.rs:116-760). */

/* Residence (crates/vulkan/src/memory.rs:61-72): HBM for TGX_DEVICE; pinned host memory the
 * GPU reaches over PCIe for TGX_UPLOAD (the host writes, kernels read) and TGX_READBACK (kernels
 * write, the host reads). */
typedef enum { TGX_DEVICE = 0, TGX_UPLOAD = 1, TGX_READBACK = 2 } tgx_residence;

typedef struct tgx_memory tgx_memory;

/* Context::memory_in (context.rs:495-498): `bytes` (> 0) of zeroed memory in `residence`. */
tgx_status tgx_alloc(tgx_context* ctx, uint64_t bytes, tgx_residence residence, tgx_memory** out);
/* Frees `mem`; TGX_E_BUSY while a program that binds it exists (a recording owns its buffers,
 * recording.rs:6-13), and then nothing is freed. */
tgx_status tgx_free(tgx_memory* mem);
tgx_status tgx_memory_info(const tgx_memory* mem, uint64_t* bytes, tgx_residence* residence);
/* Buffer::write_at / read_at: `bytes` at `offset`, copied before the call returns; refuses a
 * range past the end (TGX_E_SHAPE) and, while a program that binds `mem` runs, TGX_E_BUSY. */
tgx_status tgx_write(tgx_memory* mem, uint64_t offset, const void* src, uint64_t bytes);
tgx_status tgx_read(tgx_memory* mem, uint64_t offset, void* dst, uint64_t bytes);

/* How the kernels keep a weight matrix: bf16 MFMA tiles of strips of 16 rows (with q/k/v's rows
 * ordered so that a strip holds 8 RoPE pairs of one head, each pair's two rows side by side: heads
 * of 64 dimensions, TGX_TILES_QKV, or of 128, TGX_TILES_QKV128), or of 4 rows (o_proj and
 * down_proj at batches of up to 16 rows). */
typedef enum { TGX_TILES_16 = 0, TGX_TILES_4 = 1, TGX_TILES_QKV = 2, TGX_TILES_QKV128 = 3 } tgx_tiles;
/* The bytes a [rows][cols] matrix takes as `tiles` (0 for a shape the tiles cannot hold). */
uint64_t tgx_tiles_bytes(tgx_tiles tiles, int rows, int cols);
/* The most positions an attention_rows tile may hold for heads over kv_heads of head_dim (0 for a
 * shape the kernels do not take): 32, 40 at 3 heads a KV head, 24 at 5, 16 at 6 to 16, 8 at 9 to
 * 16 of 128 dimensions. The kernel skips a tile of more (it cannot refuse what device memory
 * holds), so a caller sizes its tiles by this. No counterpart in the reference, whose attention
 * kernel takes a fixed number of positions a workgroup (attention_rows.comp). */
int tgx_attention_tile(int heads, int kv_heads, int head_dim);
/* Writes a row-major [rows][cols] matrix of `dtype` at `offset` as `tiles`, rounded to bf16 to
 * nearest even, as tgx_decoder_load lays out its weights (load_stack's write, decode.rs:740-776). */
tgx_status tgx_write_tiles(tgx_memory* mem, uint64_t offset, const void* src, tgx_dtype dtype, tgx_tiles tiles,
                           int rows, int cols);
/* Shape::rope_tables (decode.rs:143-168): cos and sin [capacity][head_dim / 2] f32. */
tgx_status tgx_rope_tables(const tgx_shape* shape, float* cos, float* sin);

/* The kernels (kernels.rs KernelInfo): each has a name, bindings in order and constants in order.
 * The decode step's kernels keep the reference's names but for "attention_decode", which does
 * attention_split's and attention_combine's work in one; every decode kernel takes the constants
 * hidden, inner, heads, kv_heads, rows, capacity, slots, max_blocks, blocks, eps (its f32 bits),
 * rope, head_dim (64 or 128), then its own. The prefill's (prefill.rs:32-116: norm_rows,
 * final_norm_rows, and the GEMMs with the reference's row kernels as epilogues, gemm_rope_rows,
 * gemm_add_norm_rows, gemm_silu_mul_rows, beside attention_rows) take rows, hidden, inner, heads,
 * kv_heads, head_dim, capacity, slots, max_blocks, blocks, eps, rope first; the local stacks' and
 * the sampler's (local/mod.rs:28-113: local_norm, local_qkv_rope, local_attention, local_partial,
 * local_add_norm, local_final_norm, local_gemm_add_norm, local_gate_up, local_embed, dit_euler)
 * take tokens, seq_tokens, hidden, inner, heads, kv_heads, eps, rope first; cfm_noise, gemv_linear
 * (lm_side.rs:28-38, and prompt.rs's linear_rows) and select_rows take their own only. An optional
 * binding may be left out (memory NULL). */
typedef enum { TGX_READ = 0, TGX_WRITE = 1 } tgx_access;
typedef struct {
    char name[24];
    tgx_access access;
    tgx_dtype element;
    int optional;
} tgx_binding_info;
int tgx_kernel_count(void);
/* The kernel called `name` (TGX_E_KERNELS when none is). */
tgx_status tgx_kernel_find(const char* name, int* kernel);
tgx_status tgx_kernel_info(int kernel, const char** name, int* bindings, int* constants);
tgx_status tgx_kernel_binding(int kernel, int i, tgx_binding_info* out);
tgx_status tgx_kernel_constant(int kernel, int i, const char** name);

/* recording.rs Binding (:31-61): `size` bytes of `memory` from `offset`; size 0 for the rest. */
typedef struct {
    tgx_memory* memory;
    uint64_t offset;
    uint64_t size;
} tgx_binding;

/* recording.rs Dispatch (:74-86): a kernel, one binding per binding it declares in order, its
 * constants in order (f32 ones as their bits), the grid (all 0: the grid the kernel takes for the
 * constants; otherwise it must be that grid, as check_groups holds, context.rs:46-57), and whether
 * it waits for every earlier dispatch of the program (`barrier`; without it, it waits only for
 * those before the last barrier and may run beside the dispatches since). Every binding must hold
 * the bytes the kernel reaches for the constants (Kernels::check, kernels.rs), else TGX_E_SHAPE. */
typedef struct {
    int kernel;
    const tgx_binding* bindings;
    int nbindings;
    const uint32_t* constants;
    int nconstants;
    uint32_t groups[3];
    int barrier;
} tgx_dispatch;

typedef struct tgx_program tgx_program;

/* Context::dispatch (context.rs:517-540): one dispatch run alone and waited for, its bindings
 * checked as a program's are; *ms (when not NULL) its GPU time between events on either side. */
tgx_status tgx_context_dispatch(tgx_context* ctx, const tgx_dispatch* d, float* ms);

/* Context::record (context.rs:507-518): a program, its dispatches added by
 * tgx_program_launch, recorded as a HIP graph by tgx_program_end; `timed` as Recording's (each
 * dispatch launched alone between events of its own, so that tgx_program_timings gives its time). */
tgx_status tgx_program_begin(tgx_context* ctx, int timed, tgx_program** out);
/* Adds a dispatch, checked against its kernel's bindings, constants and grid. */
tgx_status tgx_program_launch(tgx_program* p, const tgx_dispatch* d);
/* Ends the recording: the program may run from now on and takes no more dispatches. */
tgx_status tgx_program_end(tgx_program* p);
/* Recording::start_program / Submission::wait (recording.rs:616-660, 747-753; 60 s at most) /
 * submit_program (:610-614: both). */
tgx_status tgx_program_start(tgx_program* p);
tgx_status tgx_program_wait(tgx_program* p);
tgx_status tgx_program_run(tgx_program* p);
/* Recording::timings (recording.rs:663-674): each dispatch's kernel name and GPU time in the last
 * run of a timed program; *n the dispatches (0 when not timed), of which `max` are written. */
tgx_status tgx_program_timings(tgx_program* p, int max, tgx_timing* out, int* n);
/* Recording::elapsed (recording.rs:676-681): the last run's GPU time, from events around it. */
tgx_status tgx_program_elapsed_ms(tgx_program* p, float* ms);
/* Recording::ends (recording.rs:681-686): the GPU clock's ticks (tgx_calibration's clock) when
 * the last run started and when it ended, which a calibration places on the host's clock:
 * the run's events taken from an anchor the start re-takes at most once a second (the clock read
 * by a one-wave kernel, an event after it), so within that kernel's few µs. TGX_E_BUSY before a
 * run has finished. */
tgx_status tgx_program_ends(tgx_program* p, uint64_t ends[2]);
/* Recording::replace_program (recording.rs:219-244): waits for the program, then drops its
 * dispatches and the memories they bound; it takes dispatches again (tgx_program_launch, then
 * tgx_program_end), timed or not, in their place. */
tgx_status tgx_program_reset(tgx_program* p, int timed);
tgx_status tgx_program_destroy(tgx_program* p);

/* Recording::copy_in / copy_out (recording.rs:522-597): regions copied from `src` to `dst` on the
 * context's stream, in order, before the call returns; TGX_E_SHAPE for a region past either end. */
typedef struct {
    uint64_t src_offset;
    uint64_t dst_offset;
    uint64_t bytes;
} tgx_region;
tgx_status tgx_copy_regions(tgx_context* ctx, tgx_memory* dst, tgx_memory* src, const tgx_region* regions, int n);

#ifdef __cplusplus
}
#endif
#endif
