// The host side of the runtime: the context, the decoder's device memory and paged cache, and the
// step recorded as a HIP graph. The C ABI (api.cpp) is a thin layer over these.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <functional>
#include <string>
#include <map>
#include <vector>

#include "../../include/tgx.h"
#include "decode_kernels.hpp"
#include "prefill_kernels.hpp"

namespace tgx {

// The thread's last error message (tgx_last_error).
tgx_status fail(tgx_status status, const std::string& message);
void clear_error();
const char* last_error();
#define TGX_HIP(call)                                                                        \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess)                                                                \
            return ::tgx::fail(TGX_E_HIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)
#define TGX_TRY(expr)                        \
    do {                                     \
        tgx_status s_ = (expr);              \
        if (s_ != TGX_OK) return s_;         \
    } while (0)

struct Context {
    int device = 0;
    hipStream_t stream = nullptr;
    hipDeviceProp_t prop{};
    size_t lds_bytes = 0;  // LDS a workgroup may take
    void* scratch = nullptr;  // the device's prefill scratch (PREFILL_SCRATCH_BYTES), its device address
    // How long a wait for the context's work polls before it sleeps between polls, in ns
    // (tgx_context_set_fence_spin; 0 sleeps at once).
    std::atomic<uint64_t> fence_spin_ns{0};
    double tick_ns = 10.0;            // a tick of the GPU's wall clock (read_clock), in ns
    uint64_t* clock_host = nullptr;   // pinned host word read_clock writes for tgx_context_calibrate
};

// Waits for `ev`, recorded on the context's stream: polls it without pause for the context's
// fence spin, then every 20 µs, for 60 s at most (Inner::wait_for, crates/vulkan/src/context.rs:
// 116-133, and its FENCE_TIMEOUT_NS). TGX_E_HIP for an error the event reports, TGX_E_TIMEOUT
// past 60 s, each naming `what`.
tgx_status wait_event(const Context* ctx, hipEvent_t ev, const char* what);

// decode::Shape, checked against what the kernels cover.
struct Shape {
    int hidden, inner, heads, kv_heads, head_dim, layers, capacity;
    float eps, rope_theta;
    bool rope;
    std::vector<double> factors;
};

// One allocation of device memory, freed with the decoder.
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
};

struct Layer {
    uint16_t *qkv = nullptr, *o = nullptr, *gate_up = nullptr, *down = nullptr;
    float *input_norm = nullptr, *post_norm = nullptr;
};

// The prefill's tensors, kept between runs and grown to the longest seen.
struct PrefillState {
    std::vector<DeviceBuffer> allocations;
    int rows_held = 0, tiles_held = 0;
    int M = 0, M_pad = 0, ntiles = 0;  // the last prefill
    float *x = nullptr, *h = nullptr, *mid = nullptr, *out = nullptr;
    uint16_t *normed = nullptr, *q = nullptr, *attended = nullptr, *mlp = nullptr;
    float* row_sq = nullptr;
    uint32_t *tok_pos = nullptr, *tok_slot = nullptr;
    PrefillTile* tiles = nullptr;
};

struct Decoder {
    Context* ctx = nullptr;
    Shape shape{};
    // rows: the batch the step runs (its program, 1..max_rows); max_rows: the rows the tensors
    // hold, the batch it was created for.
    int rows = 0, max_rows = 0, slots = 0, block_tokens = 64, nblocks = 0, max_blocks = 0;
    std::vector<DeviceBuffer> allocations;
    size_t device_bytes = 0;
    std::vector<Layer> layers;
    float* final_norm = nullptr;
    // step tensors
    float *x_in = nullptr, *h_a = nullptr, *h_b = nullptr, *out = nullptr;
    // h_a, h_b times the next norm's gain in bf16, and their sums of squares [rows][hidden / 4]
    uint16_t *xn_a = nullptr, *xn_b = nullptr;
    float *sq_a = nullptr, *sq_b = nullptr;
    int od_rows = 4;  // strip height of o_proj and down_proj (decode_residual_rows)
    uint16_t *q = nullptr, *attended = nullptr, *mlp = nullptr, *kv = nullptr;
    uint32_t *positions = nullptr, *slot_of_row = nullptr, *table = nullptr;
    uint32_t* row_table = nullptr;  // [rows][max_blocks]: each row's slot's table row
    float *cos = nullptr, *sin = nullptr;
    // host mirrors of the placement ([positions..., slots...]) and of the slots' block tables
    std::vector<uint32_t> placement_host, table_host;
    // Pinned staging (coherent: the device reads it past its caches) that copies to the device
    // read from, through each buffer's device address (*_mapped): each is filled just before its
    // copy is staged in `copies`, once the copies queued from the staging before have run
    // (staging_wait); staging_queued launches them, one kernel, and the event follows it on the
    // stream. out_host takes the step's output, which a kernel stores through out_mapped.
    float *x_host = nullptr, *out_host = nullptr, *x_mapped = nullptr, *out_mapped = nullptr;
    uint32_t *placement_stage = nullptr, *table_stage = nullptr, *row_table_host = nullptr;
    uint32_t *placement_mapped = nullptr, *table_mapped = nullptr, *row_table_mapped = nullptr;
    CopySegments copies{};
    hipEvent_t ev_staged = nullptr;
    bool staged = false;
    bool table_dirty = true, rows_dirty = true;
    std::vector<int> slot_blocks;     // blocks each slot holds
    std::vector<uint32_t> free_list;  // blocks nobody holds
    // the recorded step, a program per row count run (step_exec, advance_exec: the current one's)
    struct Program {
        hipGraphExec_t step = nullptr, advance = nullptr;
        int dispatches = 0;
    };
    std::map<int, Program> programs;
    hipGraphExec_t step_exec = nullptr, advance_exec = nullptr;
    int dispatches = 0;
    hipEvent_t ev_start = nullptr, ev_end = nullptr, ev_done = nullptr;
    bool pending = false;
    bool timed = false;  // launch dispatch by dispatch, each timed (Decoder::new's `timed`)
    bool use_graph = true;  // launch the recorded graph (else dispatch by dispatch)
    DispatchTimer timer;
    std::vector<hipEvent_t> timer_start, timer_stop;
    std::vector<const char*> timer_labels;
    PrefillState pf;

    DecodeArgs args() const;
    // Layer l's tensors: its input is x_in at layer 0, else h_a (with xn_a, sq_a); o_proj writes
    // mid to h_b (with xn_b, sq_b), down_proj the next input to h_a.
    LayerArgs layer_args(int l) const;
    ResidualArgs o_args(int l) const;
    ResidualArgs down_args(int l) const;
};

// A graph just instantiated: its resources uploaded on `stream` (hipGraphUpload) and the stream
// drained before its first launch, so that no first launch of a graph overlaps its setup.
tgx_status upload_graph(hipGraphExec_t exec, hipStream_t stream);

tgx_status context_create(int device, Context** out);
void context_destroy(Context* ctx);

tgx_status check_shape(const tgx_shape* in, Shape* out);
tgx_status check_batch(const Shape& s, const tgx_batch* batch);
tgx_status placement(int slots, int capacity, const tgx_row* rows, int nrows, uint32_t* words);
tgx_status decoder_create(Context* ctx, const tgx_shape* shape, const tgx_batch* batch, Decoder** out);
void decoder_destroy(Decoder* dec);
tgx_status decoder_load(Decoder* dec, const char* name, const void* data, tgx_dtype dtype, size_t count);
tgx_status decoder_set_rows(Decoder* dec, const tgx_row* rows, int nrows, const float* x);
// Runs the next steps at `rows` rows (1 to the rows it was created for): the program of that many
// rows, recorded on its first use; every row spare until placed again. A row's results are the
// same whatever the program (the kernels' batch invariance).
tgx_status decoder_use_rows(Decoder* dec, int rows);
// set_rows without the input: places the rows (positions, slots, blocks) alone.
tgx_status decoder_place(Decoder* dec, const tgx_row* rows, int nrows);
// The step's dispatches on the context's stream, reading x_in and writing out.
hipError_t decoder_enqueue(Decoder* d, int advance, DispatchTimer* timer, int* dispatches);
tgx_status decoder_start(Decoder* dec);
tgx_status decoder_wait(Decoder* dec);
tgx_status decoder_output(Decoder* dec, float* out);
tgx_status decoder_release_slot(Decoder* dec, uint32_t slot);
tgx_status decoder_reserve(Decoder* dec, uint32_t slot, uint32_t positions);
tgx_status decoder_launch(Decoder* dec, int times, int advance);
// Hands `slot` the blocks for positions 0..positions-1 (in the host's table); sync_slots queues
// copies of the block table, and of the rows' copies of their slots' rows of it, to the device
// on the context's stream when they changed, without waiting for them.
tgx_status hold_slot(Decoder* d, uint32_t slot, uint32_t positions);
tgx_status sync_slots(Decoder* d);
// Before `times` steps (each placed row moved on a position a step with `advance`): holds every
// placed row's blocks up to the last position the steps write, refusing (TGX_E_SHAPE) a row the
// steps would take past the capacity, or a pool that runs out.
tgx_status hold_ahead(Decoder* d, int times, int advance);
// The host's copy of the placement moved on as an advancing step moves the rows on the device.
void moved_on(Decoder* d, int times);
tgx_status prefill_runs(Decoder* d, const tgx_run* runs, int nruns, const float* x, float* out);
// The same, enqueued on the context's stream without waiting: x from the host, or from the device
// when x_on_device; the output, [rows of the runs in order][hidden] f32, left in d->pf.out.
tgx_status prefill_device(Decoder* d, const tgx_run* runs, int nruns, const float* x, bool x_on_device);
tgx_status prefill_launch(Decoder* d, int times);
// prefill_runs with the tensors in the context's scratch: allocates no device memory; refuses
// (TGX_E_SHAPE) runs whose tensors pass PREFILL_SCRATCH_BYTES. Calls that overlap on one GPU race.
tgx_status prefill_runs_noalloc(Decoder* d, const tgx_run* runs, int nruns, const float* x, float* out);
// Device bytes the prefill's own tensors hold (grown by the longest prefill_runs so far).
size_t prefill_bytes(const Decoder* d);
void prefill_release(Decoder* d);
tgx_status decoder_timings(Decoder* d, int max, tgx_timing* out, int* n);
tgx_status decoder_read_cache(Decoder* dec, uint32_t slot, uint32_t positions, float* k, float* v);

// A weight's values as f32; W [n][k] in MFMA tiles of R-row strips, rows through `row_of`
// (strip, r) -> source row; and one layer's tensor `what` of a stack ("qkv_proj", "o_proj",
// "gate_up_proj", "down_proj", "input_layernorm", "post_attention_layernorm"), q/k/v and gate/up
// in 16-row strips, o_proj in `o_rows` and down_proj in `down_rows`.
std::vector<float> as_f32(const void* data, tgx_dtype dtype, size_t count);
std::vector<uint16_t> tile_rows(const std::vector<float>& w, int n, int k, int R,
                                const std::function<int(int, int)>& row_of);
tgx_status load_layer_tensor(Layer& L, const Shape& s, const std::string& name, const std::string& what,
                             const void* data, tgx_dtype dtype, size_t count, int o_rows, int down_rows);

// f32 <- bf16 / f16 bits; f32 -> bf16 bits, rounding to nearest even.
float bf16_to_f32(uint16_t h);
float f16_to_f32(uint16_t h);
uint16_t f32_to_bf16(float f);

// The RoPE tables in f32 as decode.rs:146-168 computes them.
void rope_tables(const Shape& s, std::vector<float>& cos, std::vector<float>& sin);

}  // namespace tgx
