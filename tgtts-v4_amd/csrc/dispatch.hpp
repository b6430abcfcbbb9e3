// Kernel launch shared by the launchers: a plain launch, or, when a step is timed, a launch that
// records the timer's next pair of events around the kernel alone (hipExtLaunchKernelGGL), as a
// profiler would time it.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "decode_kernels.hpp"

namespace tgx {

template <typename... KernelArgs, typename... Args>
inline void dispatch(const char* label, void (*kernel)(KernelArgs...), dim3 grid, dim3 block, size_t lds,
                     hipStream_t stream, DispatchTimer* timer, Args... args) {
    if (timer && timer->used < timer->capacity) {
        const int i = timer->used++;
        timer->labels[i] = label;
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, timer->start[i], timer->stop[i], 0, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
}

}  // namespace tgx
