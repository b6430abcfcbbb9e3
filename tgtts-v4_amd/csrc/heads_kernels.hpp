// The linear layers between VoxCPM2's LMs (gemv_linear.comp; crates/graph/src/lm_side.rs:246-297).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "decode_kernels.hpp"

namespace tgx {

enum LinearAct { ACT_NONE = 0, ACT_SILU = 1, ACT_LEVELS = 2 };

// out[b][offset + n] = act(sum_k W[n][k] [x0; x1][b][k] + bias[n]) for rows b < rows: W in 16-row
// MFMA tiles of [N_pad][K0 + K1] (rows past N zero), x0 [rows][K0] and x1 [rows][K1] in f32,
// out rows `stride` apart.
struct LinearArgs {
    const uint16_t* w;
    const float* bias;  // [N]
    const float* x0;
    const float* x1;
    float* out;
    int K0, K1, N, rows, offset, stride, act;
    float levels;
};

// The inputs' columns a linear layer takes (its x0 and x1 together): VoxCPM2's fusion_concat_proj
// joins two 2048-wide rows. The inputs are staged in LDS, 32 KiB a 1024 columns.
constexpr int LINEAR_MAX_K = 4096;

hipError_t launch_linear(const char* label, const LinearArgs& a, hipStream_t stream, DispatchTimer* timer);
// Lets gemv_linear take the LDS of LINEAR_MAX_K columns (of the device's `device_lds` a workgroup).
hipError_t heads_prepare(size_t device_lds);
// out[r] = flags[r] ? a[r] : b[r], rows of K f32 values (K a multiple of 4): the quantizer's output at
// a prompt's audio positions and the base LM's at its text (select_rows.comp).
hipError_t launch_select_rows(const uint32_t* flags, const float* a, const float* b, float* out, int rows, int K,
                              hipStream_t stream, DispatchTimer* timer);

}  // namespace tgx
