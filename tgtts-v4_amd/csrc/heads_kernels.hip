// gemv_linear.comp on gfx950 (and select_rows.comp beside it): a workgroup of four waves to a strip of 16 rows of W and a tile of
// 16 batch rows. The batch rows' inputs are staged in LDS in bf16 in the MFMA's B-operand order;
// wave w sums the k-blocks w, w + 4, ... and the four waves' sums are added in wave order, so a
// row's result does not depend on the batch around it.
#include "heads_kernels.hpp"

#include <math.h>

#include "dispatch.hpp"

namespace tgx {

namespace {

__global__ void __launch_bounds__(256) gemv_linear(LinearArgs a) {
    extern __shared__ uint4 xs[];  // [k-block][lane]: 32 KiB a 1024 columns (128 KiB at K 4096)
    __shared__ f32x4 red[4][WAVE];
    const int strip = blockIdx.x, tile = blockIdx.y;
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int K = a.K0 + a.K1, kblocks = K / 32;
    // Fragment (kb, lane): batch row 16 tile + lane % 16, k = 32 kb + 8 (lane / 16) .. + 7.
#pragma unroll 8
    for (int i = threadIdx.x; i < kblocks * 64; i += 256) {
        const int kb = i / 64, l = i % 64;
        const int b = tile * 16 + l % 16;
        const int k = kb * 32 + (l / 16) * 8;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (b < a.rows) {
            const float* src = k < a.K0 ? a.x0 + (size_t)b * a.K0 + k : a.x1 + (size_t)b * a.K1 + (k - a.K0);
            const float4 lo = *reinterpret_cast<const float4*>(src);
            const float4 hi = *reinterpret_cast<const float4*>(src + 4);
            v = make_uint4(pack_bf16x2(lo.x, lo.y), pack_bf16x2(lo.z, lo.w), pack_bf16x2(hi.x, hi.y), pack_bf16x2(hi.z, hi.w));
        }
        xs[i] = v;
    }
    __syncthreads();
    // Wave w's chain over k-blocks w, w + 4, ... in order, eight k-blocks' weights loaded at once.
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    constexpr int AHEAD = 8;
    for (int kb0 = w; kb0 < kblocks; kb0 += 4 * AHEAD) {
        uint4 af[AHEAD];
#pragma unroll
        for (int j = 0; j < AHEAD; ++j) {
            const int kb = min(kb0 + 4 * j, kblocks - 1);  // past the last, the last again (not used)
            af[j] = *reinterpret_cast<const uint4*>(a.w + weight_tile_index(strip, kb, kblocks, 16) + lane * 8);
        }
#pragma unroll
        for (int j = 0; j < AHEAD; ++j)
            if (kb0 + 4 * j < kblocks) acc = mfma16(af[j], xs[(kb0 + 4 * j) * 64 + lane], acc);
    }
    red[w][lane] = acc;
    __syncthreads();
    if (w != 0) return;
    f32x4 sum = red[0][lane];
#pragma unroll
    for (int v = 1; v < 4; ++v) sum += red[v][lane];
    const int b = tile * 16 + lane % 16;
    if (b >= a.rows) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = strip * 16 + (lane / 16) * 4 + i;
        if (n >= a.N) continue;
        float v = sum[i] + a.bias[n];
        if (a.act == ACT_SILU) {
            v = silu(v);
        } else if (a.act == ACT_LEVELS) {
            // The scalar quantizer (gemv_linear.comp:54-59): tanh rounded to a multiple of 1 / L,
            // ties to even.
            v = rintf(copysignf(tanhf(fabsf(v)), v) * a.levels) / a.levels;
        }
        a.out[(size_t)b * a.stride + a.offset + n] = v;
    }
}

// select_rows.comp: out[r] = flags[r] ? a[r] : b[r] over rows of K f32 values, a thread to 4.
__global__ void __launch_bounds__(256) select_rows(const uint32_t* __restrict__ flags, const float* __restrict__ a,
                                                   const float* __restrict__ b, float* __restrict__ out, int rows, int K) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= (size_t)rows * K) return;
    const int r = (int)(i / K);
    const float* src = flags[r] ? a : b;
    *reinterpret_cast<float4*>(out + i) = *reinterpret_cast<const float4*>(src + i);
}

}  // namespace

hipError_t launch_select_rows(const uint32_t* flags, const float* a, const float* b, float* out, int rows, int K,
                              hipStream_t stream, DispatchTimer* timer) {
    if (K % 4) return hipErrorInvalidValue;
    const size_t threads = (size_t)rows * K / 4;
    dispatch("select_rows", select_rows, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, timer, flags, a, b, out, rows, K);
    return hipGetLastError();
}

hipError_t launch_linear(const char* label, const LinearArgs& a, hipStream_t stream, DispatchTimer* timer) {
    const int K = a.K0 + a.K1;
    if (K <= 0 || K % 32 || K > LINEAR_MAX_K) return hipErrorInvalidValue;
    dispatch(label, gemv_linear, dim3((a.N + 15) / 16, (a.rows + 15) / 16), dim3(256), (size_t)K / 32 * 64 * sizeof(uint4), stream,
             timer, a);
    return hipGetLastError();
}

hipError_t heads_prepare(size_t device_lds) {
    hipFuncAttributes attr{};
    hipError_t e = hipFuncGetAttributes(&attr, (const void*)gemv_linear);
    if (e != hipSuccess) return e;
    if ((size_t)LINEAR_MAX_K / 32 * 64 * sizeof(uint4) + attr.sharedSizeBytes > device_lds) return hipErrorInvalidValue;
    return hipFuncSetAttribute((const void*)gemv_linear, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)(device_lds - attr.sharedSizeBytes));
}

}  // namespace tgx
