// The local stack's and the patch sampler's kernels (crates/graph/src/local/mod.rs,
// crates/graph/src/local/dit.rs): a bidirectional MiniCPM-4 stack over sequences of a few tokens,
// the embeddings of a patch's frames, and the Euler step with CFG-Zero* guidance.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "decode_kernels.hpp"
#include "device.hpp"

namespace tgx {

// The tokens a local stack runs over: `seqs` sequences of T tokens, token m at place m % T.
struct LocalArgs {
    int M;      // tokens
    int M_pad;  // rows of the token tensors, local_rows_padded(M); rows past M hold zeros
    int T;      // tokens to a sequence
    int hidden, inner, heads, kv_heads;
    float eps, scale;
    int rope;
    const float* cos;  // [T][HEAD_DIM / 2]
    const float* sin;
};

constexpr int LOCAL_MAX_T = 16;        // the longest sequence: local_attention takes one as an MFMA tile
constexpr int LOCAL_MAX_PARTS = 4;
constexpr int LOCAL_O_PARTS = 2;     // o_proj's columns summed in 2 parts, down_proj's in 4, in part order
constexpr int LOCAL_DOWN_PARTS = 4;
constexpr int LOCAL_SQ_COLS = 64;    // the columns of a row that one of its sums of squares spans

struct LocalLayer {
    const uint16_t *qkv, *o, *gate_up, *down;  // 16-row MFMA tiles, q/k/v rows RoPE-paired
    const float *input_norm, *post_norm;
};

// The stack's tensors, [M_pad][...] each.
struct LocalBuffers {
    const float* x0;     // the embedded tokens, the first layer's residual
    float *x, *h;        // the residual stream after each layer / after each attention
    // The GEMMs' inputs are in MFMA fragment order (act_index: each 16 tokens by 32 columns a
    // contiguous KiB), so that a wave's load of one is one contiguous KiB.
    uint16_t* normed;    // bf16 [M_pad][hidden], fragment order: an RMSNorm's input times its gain, the rows' scales
                         // still to apply (the GEMM that reads it applies them)
    float* row_sq;       // f32 [M_pad][hidden / LOCAL_SQ_COLS]: normed's rows' sums of squares, each
                         // over LOCAL_SQ_COLS columns
    // The first layer's normed input and its sums of squares, as the embedding wrote them
    // (EmbedArgs::gain); null for the stack to norm x0 itself.
    const uint16_t* normed0;
    const float* row_sq0;
    uint16_t *q, *k, *v; // bf16 [M_pad][heads | kv_heads][64]
    uint16_t* attended;  // bf16 [M_pad][heads 64], fragment order
    uint16_t* mlp;       // bf16 [M_pad][inner], fragment order
    float* partial;      // f32 [LOCAL_MAX_PARTS][M_pad][hidden]
    // f32 [M_pad][hidden]: the last layer's output after the final norm; null to leave the norm
    // to the stack's reader (x and row_sq then hold its input and sums of squares)
    float* out;
    int o_parts, down_parts;
};

// A linear layer over a patch's frames, `src` [rows][channels][frames] (channel-major, as the
// sampler keeps a patch): W f32 [hidden][channels] and bias [hidden]; the FRAMES results are
// written as tokens `first` .. of each of the row's `seqs` sequences (2 for the sampler's
// conditional and unconditional ones, 1 for the encoder), and `copies` tokens of `copy_src` at
// `copy_at` (per row unless `shared`; zero in the second sequence when `guided`).
// With a gain, each token written is also written as the first layer's norm input: x0 gain in
// bf16 into `normed` (fragment order) and its sums of squares into `row_sq`.
struct EmbedArgs {
    const float* src;
    const float* w;
    const float* bias;
    const float* copy_src;
    float* x0;
    int channels, frames, first, copy_at, copies, guided, shared;
    int seqs;
    const float* gain;  // the first layer's input norm gain, or null
    uint16_t* normed;
    float* row_sq;
};

// One Euler step: velocities out_proj(norm(x[tokens first..])) + b of the conditional and the
// unconditional sequence, guided as CFG-Zero* guides them, and state -= dt * guided. The stack's
// final norm is taken here, for the tokens read.
struct EulerArgs {
    const float* x;       // f32 [M_pad][hidden], the stack's last residual (before its final norm)
    const float* row_sq;  // x's sums of squares, [M_pad][hidden / LOCAL_SQ_COLS]
    const float* gain;    // the final norm's gain [hidden]
    const uint16_t* w;  // bf16 [channels][hidden] in 16-row MFMA tiles
    const float* bias;  // [channels]
    const float* sampling;  // [rows][2]: temperature, guidance scale
    float* state;       // [rows][channels][frames]
    int channels, frames, first;
    float dt;
};

// What a local stack's projection writes beside its products (local_gemm_direct, local_gemm_ring):
// q/k/v with RoPE, the parts of a sum (o_proj and down_proj up to 64 tokens), SiLU(gate) up, or
// the parts added with the residual and the next norm's input (o_proj and down_proj past 64).
enum LocalEpilogue { LEPI_QKV = 0, LEPI_PARTIAL = 1, LEPI_SILU = 2, LEPI_ADD = 3 };

// A local projection's operands and its epilogue's tensors.
struct LocalGemm {
    const uint16_t* w;  // 16-row tiles of [N][K]
    const uint16_t* x;  // bf16 [M_pad][K] in fragment order
    int K, N;
    float* partial;     // LEPI_PARTIAL: f32 [parts][M_pad][N]
    uint16_t* mlp;      // LEPI_SILU: bf16 [M_pad][N / 2]
    uint16_t *q, *k, *v;
    // LEPI_QKV, LEPI_SILU: X is an RMSNorm's input times its gain; row m's sums of squares
    // [M_pad][K / LOCAL_SQ_COLS] give the row's scale, applied to its sums.
    const float* row_sq;
    // LEPI_ADD (local_gemm_ring): sum = residual + the parts' sums, and with next_gain, the next
    // norm's input: normed = sum next_gain in bf16 and sum's sums of squares into sum_sq.
    const float* residual;
    float* sum;
    const float* next_gain;
    uint16_t* normed;
    float* sum_sq;
};

// The local stack's kernels one at a time, as launch_local_stack launches them: q/k/v with RoPE
// (its N the q/k/v rows), the attention within each sequence, o_proj's or down_proj's parts
// (up to 64 tokens) and their sum with the residual and the next norm's input (or the final norm
// into `out`), the same fused (past 64 tokens; 2 or 4 parts), and gate/up with SiLU.
hipError_t launch_local_qkv(const LocalArgs& a, const LocalGemm& g, hipStream_t stream, DispatchTimer* timer);
hipError_t launch_local_attention(const LocalArgs& a, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* attended,
                                  hipStream_t stream, DispatchTimer* timer);
hipError_t launch_local_partial(const LocalArgs& a, const LocalGemm& g, int parts, hipStream_t stream, DispatchTimer* timer);
hipError_t launch_local_add_norm(const LocalArgs& a, bool final, const float* partial, int parts, const float* residual, float* sum,
                                 const float* gain, uint16_t* normed, float* row_sq, float* out, hipStream_t stream,
                                 DispatchTimer* timer);
hipError_t launch_local_add(const LocalArgs& a, const LocalGemm& g, int parts, hipStream_t stream, DispatchTimer* timer);
hipError_t launch_local_gate_up(const LocalArgs& a, const LocalGemm& g, hipStream_t stream, DispatchTimer* timer);

// Lets the ring GEMM take its rings of token tiles (up to 66 KiB) in LDS; once per process.
hipError_t local_prepare();
// The stacks the kernels take: hidden 1024, query heads a multiple of 4, and o_proj's and
// down_proj's columns in 2 or 4 parts of 16 or 32 k-blocks of 32 columns each.
bool local_supported(int hidden, int inner, int heads, int kv_heads, int o_parts, int down_parts);
// The rows the token tensors of M tokens take: a multiple of 16 up to 64 tokens, else of 64.
int local_rows_padded(int M);
hipError_t launch_local_stack(const LocalArgs& a, const LocalLayer* layers, int nlayers, const float* final_norm,
                              const LocalBuffers& b, hipStream_t stream, DispatchTimer* timer);
// The dispatches launch_local_stack makes.
int local_stack_dispatches(const LocalArgs& a, const LocalBuffers& b, int nlayers);
hipError_t launch_local_embed(const LocalArgs& a, const EmbedArgs& e, int rows, hipStream_t stream, DispatchTimer* timer);
hipError_t launch_dit_euler(const LocalArgs& a, const EulerArgs& e, int rows, hipStream_t stream, DispatchTimer* timer);
hipError_t launch_cfm_noise(const float* noise, const float* sampling, float* state, int rows, int len,
                            hipStream_t stream, DispatchTimer* timer);

}  // namespace tgx
