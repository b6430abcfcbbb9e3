// Kernel launch shared by the launchers: a plain launch, or, when a step is timed, a launch that
// records the timer's next pair of events around the kernel alone (hipExtLaunchKernelGGL), as a
// profiler would time it; or, while a capture is set on the calling thread, no launch at all but a
// record of it (the kernel, its grid, block and LDS, and each argument's bytes as the kernel takes
// it), from which a program recorded through the runtime API launches the same kernel the models do.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

#include "decode_kernels.hpp"

namespace tgx {

struct CapturedLaunch {
    const void* func = nullptr;
    dim3 grid, block;
    uint32_t lds = 0;
    std::vector<std::vector<unsigned char>> args;  // each argument's bytes, in order
};

// Where dispatch() records launches instead of making them, on this thread; null to launch.
inline thread_local std::vector<CapturedLaunch>* dispatch_capture = nullptr;

template <typename T>
std::vector<unsigned char> argument_bytes(const T& v) {
    std::vector<unsigned char> b(sizeof(T));
    std::memcpy(b.data(), &v, sizeof(T));
    return b;
}

template <typename... KernelArgs, typename... Args>
inline void dispatch(const char* label, void (*kernel)(KernelArgs...), dim3 grid, dim3 block, size_t lds,
                     hipStream_t stream, DispatchTimer* timer, Args... args) {
    static_assert(sizeof...(KernelArgs) == sizeof...(Args), "an argument for every parameter");
    if (dispatch_capture) {
        CapturedLaunch c;
        c.func = (const void*)kernel;
        c.grid = grid;
        c.block = block;
        c.lds = (uint32_t)lds;
        (c.args.push_back(argument_bytes<KernelArgs>(static_cast<KernelArgs>(args))), ...);
        dispatch_capture->push_back(std::move(c));
        return;
    }
    if (timer && timer->used < timer->capacity) {
        const int i = timer->used++;
        timer->labels[i] = label;
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, timer->start[i], timer->stop[i], 0, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
}

// The launches `f` makes, captured on this thread instead of made.
template <typename F>
std::vector<CapturedLaunch> capture_launches(F&& f) {
    std::vector<CapturedLaunch> out;
    std::vector<CapturedLaunch>* before = dispatch_capture;
    dispatch_capture = &out;
    f();
    dispatch_capture = before;
    return out;
}

}  // namespace tgx
