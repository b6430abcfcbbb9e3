// Arguments and launchers of the prefill's kernels (prefill_kernels.hip): the causal run of many
// positions at once (crates/graph/src/prefill.rs:218-413).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "decode_kernels.hpp"

namespace tgx {

// A tile of up to 32 positions of one run for the attention: rows row0 .. row0 + count - 1 of
// the prefill's tensors are positions pos0 .. pos0 + count - 1 of `slot`.
struct PrefillTile {
    uint32_t row0, pos0, count, slot;
};

// What every prefill kernel reads.
struct PrefillArgs {
    int M;        // rows (positions over every run)
    int M_pad;    // rows the tensors hold, a multiple of 256
    int hidden, inner, heads, kv_heads;
    int head_dim;  // 64 or 128
    int capacity, nslots, max_blocks, nblocks;
    float eps, scale;
    int rope;
    const uint32_t* tok_pos;   // [M_pad], TGX_SPARE past M
    const uint32_t* tok_slot;  // [M_pad]
    const uint32_t* table;     // [nslots][max_blocks]
    const float* cos;
    const float* sin;
};

// One layer's tensors of a prefill.
struct PrefillLayer {
    const uint16_t* qkv;      // 16-row tiles, rows permuted (qkv_row_of)
    const uint16_t* o;
    const uint16_t* gate_up;
    const uint16_t* down;
    const float* input_norm;
    const float* post_norm;
    uint16_t* kv;  // the layer's cache pool
    int od_rows;   // strip height of o and down: 4 or 16 (qkv and gate_up: 16)
};

// The prefill's tensors, [M_pad] rows each.
struct PrefillBuffers {
    const float* x;     // the run's hidden states, f32 [M_pad][hidden], as written
    float* h;           // residual stream, f32 [M_pad][hidden]
    float* mid;         // after the attention, f32
    uint16_t* normed;   // RMSNorm of the stream, bf16 [M_pad][hidden] in fragment order (act_index)
    uint16_t* q;        // bf16 [M_pad][heads][head_dim], times scale log2(e) (the attention softmax's units)
    uint16_t* attended; // bf16 [M_pad][heads head_dim] in fragment order
    uint16_t* mlp;      // bf16 [M_pad][inner] in fragment order
    float* row_sq;      // a norm's input's sums of squares over each 128 columns, [M_pad][hidden / 128]
    float* out;         // after the final norm, f32 [M_pad][hidden]
    const PrefillTile* tiles;
    int ntiles;
};

// The epilogue fused into a prefill GEMM (prefill_gemm in prefill_kernels.hip): q/k/v's RoPE and
// cache write (rope_rows.comp), the residual add and the next norm's input (add_norm_rows.comp;
// EPI_RESIDUAL adds the residual rows to the products in the epilogue, EPI_RESIDUAL_IN starts the
// accumulators at them: for o_proj, whose short K leaves that wait exposed, not for down_proj, whose
// long K hides it), or SiLU(gate) up (silu_mul_rows.comp).
enum PrefillEpilogue { EPI_QKV = 0, EPI_RESIDUAL = 1, EPI_SILU = 2, EPI_RESIDUAL_IN = 3 };
__host__ __device__ constexpr bool residual_epilogue(int epi) { return epi == EPI_RESIDUAL || epi == EPI_RESIDUAL_IN; }

// A prefill GEMM's operands and its epilogue's tensors.
struct GemmArgs {
    const uint16_t* w;  // tiles of [N][K] in strips of 16 rows (o_proj and down_proj: 4 or 16)
    const uint16_t* x;  // bf16 [M_pad][K] in fragment order (act_index)
    int K, N;
    // epilogues
    const float* residual;  // EPI_RESIDUAL(_IN): f32 [M_pad][N]
    float* out;             // EPI_RESIDUAL(_IN): f32 [M_pad][N]
    uint16_t* mlp;          // EPI_SILU: bf16 [M_pad][N / 2] in fragment order
    uint16_t* q;            // EPI_QKV
    uint16_t* kv;           // EPI_QKV: the layer's cache pool
    // X as an RMSNorm's input times its gain, the rows' scales still to apply (EPI_QKV,
    // EPI_SILU): row m's sums of squares over each 128 columns, [M_pad][K / 128]; null when X is
    // normed already.
    const float* row_sq;
    // EPI_RESIDUAL(_IN), when set: out next_gain in bf16 in fragment order into out_n, and out's
    // sums of squares over each 128 columns into out_sq, for the norm that reads out next.
    const float* next_gain;
    uint16_t* out_n;
    float* out_sq;
};

// The prefill's kernels one at a time, as launch_prefill launches them (the instance, grid and LDS
// the shape picks): a GEMM with its epilogue (strip_rows: W's strip height, 4 or 16 for o_proj and
// down_proj, 16 otherwise), the causal attention over `ntiles` tiles of a run, and a norm of rows
// (layer 0's input norm into bf16 in fragment order, or the final norm into f32).
hipError_t launch_prefill_gemm(const PrefillArgs& a, int epi, int strip_rows, const GemmArgs& g, hipStream_t stream,
                               DispatchTimer* timer);
hipError_t launch_prefill_attention(const PrefillArgs& a, const uint16_t* q, const uint16_t* kv, uint16_t* attended,
                                    const PrefillTile* tiles, int ntiles, hipStream_t stream, DispatchTimer* timer);
hipError_t launch_prefill_norm(const PrefillArgs& a, bool final, const float* x, const float* gain, uint16_t* out_bf16,
                               float* out_f32, hipStream_t stream, DispatchTimer* timer);
// The LDS the attention takes for a slot table of `max_blocks` blocks.
size_t prefill_attention_lds(int max_blocks);

// Launches the whole prefill of the M rows of b.x (f32) through every layer into b.out.
hipError_t launch_prefill(const PrefillArgs& a, const PrefillLayer* layers, int nlayers, const float* final_norm,
                          const PrefillBuffers& b, hipStream_t stream, DispatchTimer* timer = nullptr);
hipError_t prefill_prepare(size_t device_lds);
// The positions of a run the attention takes to a workgroup (its PrefillTiles' most) for `group`
// query heads to a KV head and heads of `head_dim`.
int prefill_attention_tile(int group, int head_dim);

// The size of each GPU's prefill scratch (tgx_prefill_runs_noalloc's tensors): 32 MiB, which at
// the backbone's shape (hidden 1024, inner 4096, 16 heads) holds 1024 positions a call.
constexpr size_t PREFILL_SCRATCH_BYTES = (size_t)32 << 20;
// The device address of `device`'s scratch, looked up (hipGetSymbolAddress) on the first call for
// the device, which must be current then, and kept for the process.
hipError_t prefill_scratch_address(int device, void** out);
// Zeroes `bytes` (a multiple of 16, 16-byte aligned) at p with a kernel on `stream`.
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream);
// `bytes` (a multiple of 16) from device memory at src to host memory the device maps at dst (a
// pinned allocation's device address), by a kernel on `stream`.
hipError_t launch_copy_words(const void* src, void* dst, size_t bytes, hipStream_t stream);
// Up to COPY_SEGMENTS copies of 4-byte words in one kernel: segment k copies words
// end[k - 1] .. end[k] - 1 of the whole (end[-1] = 0) from src[k] (memory the device reads: a
// pinned host allocation's device address, or device memory) to dst[k].
constexpr int COPY_SEGMENTS = 8;
struct CopySegments {
    const uint32_t* src[COPY_SEGMENTS];
    uint32_t* dst[COPY_SEGMENTS];
    uint32_t end[COPY_SEGMENTS];
    int n;
};
hipError_t launch_copy_segments(const CopySegments& c, hipStream_t stream);

}  // namespace tgx
