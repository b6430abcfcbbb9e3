// Arguments and launchers of the decode step's kernels (decode_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.hpp"

namespace tgx {

// What every kernel of a step reads: the shape, and where each row runs (Batch::placement,
// decode.rs:198-227, plus the paged cache's block table).
struct DecodeArgs {
    int hidden, inner, heads, kv_heads;
    int head_dim;    // 64 or 128
    int rows;        // rows of the batch
    int capacity;    // positions a slot may reach
    int nslots;
    int max_blocks;  // blocks per slot in the table
    int nblocks;     // blocks in the pool
    float eps, scale;
    int rope;
    const uint32_t* positions;  // [rows]
    const uint32_t* slots;      // [rows]
    const uint32_t* table;      // [nslots][max_blocks], UINT32_MAX where none
    const uint32_t* row_table;  // [rows][max_blocks]: each row's slot's table row (UINT32_MAX for a spare row)
    const float* cos;           // [capacity][head_dim / 2]
    const float* sin;
};

// One layer's tensors. A norm's input comes as the f32 rows and, past layer 0, also as the rows
// times the norm's gain in bf16 with their sums of squares over each 4 columns (each 16 where the
// projection that wrote the rows took 16-row strips), which that projection left
// (ResidualArgs::next_norm): the consumer then reads 2 bytes a column and adds the row's sums in a
// fixed order, the same whichever width they span.
struct LayerArgs {
    const float* x;           // layer input [rows][hidden] f32
    // The projections' bf16 operands (xn, attended, mid_n, mlp) are kept in operand order: k-block
    // by k-block, [K / 32][rows][32].
    const uint16_t* xn;       // x input_norm in bf16 [rows][hidden], or null: taken from x
    const float* x_sq;        // [rows][hidden / 4], or [rows][hidden / 16] (wide)
    const float* input_norm;  // [hidden] f32
    const uint16_t* qkv;      // tiled bf16, rows permuted (qkv_row_of)
    uint16_t* q;              // [rows][heads][head_dim] bf16
    uint16_t* kv;             // the layer's cache pool: [blocks][kv_heads][key tile, value tile]
    uint16_t* attended;       // [rows][heads head_dim] bf16
    const uint16_t* mid_n;    // o_proj's output times post_norm in bf16 [rows][hidden]
    const float* mid_sq;      // [rows][hidden / 4], or [rows][hidden / 16] (wide)
    const uint16_t* gate_up;  // tiled bf16 [2 inner][hidden]
    uint16_t* mlp;            // [rows][inner] bf16
};

// out = residual + W x, W in R-row tiles of [N][K]; with next_norm set, also out next_norm in
// bf16 and out's sums of squares over each R columns (a workgroup's strip), for the norm that
// reads out next.
struct ResidualArgs {
    const uint16_t* w;
    const uint16_t* x;  // [rows][K] bf16 in operand order
    int K, N;
    int R;                  // strip height of w: 4 or 16
    const float* residual;  // [rows][N]
    float* out;             // [rows][N]
    const float* next_norm; // [N], or null
    uint16_t* out_n;        // [rows][N] in operand order
    float* out_sq;          // [rows][N / R]
};

// The strip height of o_proj and down_proj for a batch of `rows`: 4 while the batch is one
// 16-row tile (spreading their few output rows over every CU), 16 past it (each workgroup's
// vectors then serve 16 rows).
int decode_residual_rows(int rows);

// Per-dispatch timing of a step launched without its graph: each dispatch takes the next pair of
// events, recorded by the kernel's own dispatch (hipExtLaunchKernelGGL), so that the time between
// them is the kernel's alone, as a profiler reports it.
struct DispatchTimer {
    hipEvent_t* start = nullptr;
    hipEvent_t* stop = nullptr;
    const char** labels = nullptr;
    int used = 0, capacity = 0;
};

// Tiles of 16 rows a batch of `rows` takes, the longest K the projections take (the norms' and
// q/k/v's K, hidden, at most decode_max_hidden()), and the LDS the attention takes.
int decode_tiles(int rows);
int decode_max_k();
int decode_max_hidden();
// The longest capacity the attention takes at a head width: a lane to each turn a wave takes.
int decode_max_capacity(int head_dim);
size_t decode_attention_lds(int heads, int kv_heads, int head_dim);
// Lets the attention take up to `device_lds` bytes of LDS per workgroup.
hipError_t decode_prepare(size_t device_lds);
// A dispatch of one of the step's kernels: the kernel instance chosen for the shape, with its grid,
// block and LDS. The step's launchers and the program API both launch these, so that a kernel
// dispatched either way is the same code. Each takes (DecodeArgs, LayerArgs) but for
// gemv_residual (DecodeArgs, ResidualArgs), final_rmsnorm (DecodeArgs, x, gain, out, positions,
// advance) and stream_read (data, out).
struct KernelLaunch {
    const void* func = nullptr;
    dim3 grid, block;
    uint32_t lds = 0;
};
// wide: x_sq holds a sum of squares for each 16 columns (written by 16-row strips), else each 4.
KernelLaunch qkv_launch(const DecodeArgs& a, bool prenormed, bool wide);
KernelLaunch attention_launch(const DecodeArgs& a);
KernelLaunch residual_launch(const DecodeArgs& a, const ResidualArgs& r);  // func null unless r.R is 4 or 16
KernelLaunch gate_up_launch(const DecodeArgs& a, bool wide);
KernelLaunch final_norm_launch(const DecodeArgs& a);
KernelLaunch stream_read_launch(size_t bytes);

hipError_t launch_decode_layer(const DecodeArgs& a, const LayerArgs& l, const ResidualArgs& o, const ResidualArgs& down,
                               hipStream_t stream, DispatchTimer* timer = nullptr);
hipError_t launch_final_norm(const DecodeArgs& a, const float* x, const float* gain, float* out, uint32_t* positions,
                             int advance, hipStream_t stream, DispatchTimer* timer = nullptr);

// The stream-read floor's kernel (kernels/glsl/stream_read.comp): `bytes` (a multiple of
// stream_read_unit()) read once, one word a wave of their XOR into out (bytes / 4096 words).
size_t stream_read_unit();
hipError_t launch_stream_read(const void* data, size_t bytes, uint32_t* out, hipStream_t stream);
// One wave reads the GPU's constant-rate wall clock (hipDeviceAttributeWallClockRate ticks a
// second) into *out, on `stream`.
hipError_t launch_read_clock(uint64_t* out, hipStream_t stream);

}  // namespace tgx
