// Optional per-launch timing of the hot kernels: while enabled (gpeed_prof_*
// in the C ABI), launches go through hipExtLaunchKernelGGL with a start/stop
// event pair stamped by the dispatch itself, so durations are the kernel's
// own execution time, not the host's view of the stream.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace gpeed {

enum ProfKind { kProfGemv = 0, kProfGrouped = 1, kProfGemm = 2, kProfKinds = 3 };

// Next free event pair for a launch of `kind`, or false when timing is off
// or the pool is full (the launch then goes untimed).
bool prof_slot(int kind, hipEvent_t* start, hipEvent_t* stop);

template <typename F, typename... Args>
inline hipError_t launch_timed(int kind, F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                               Args... args) {
    hipEvent_t a = nullptr, b = nullptr;
    if (prof_slot(kind, &a, &b))
        hipExtLaunchKernelGGL(kernel, grid, block, lds, s, a, b, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
    return hipGetLastError();
}

}  // namespace gpeed
