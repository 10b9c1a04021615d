// Host-side launch helper shared by the fused entry points.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace ss {

// Launches `kernel`; with a (start, end) event pair, the events are recorded by the dispatch
// itself (hipExtLaunchKernelGGL), so they time exactly this kernel and add no packets to the
// stream between it and its neighbours.
template <class Kernel, class... Args>
inline void launch_timed(Kernel kernel, dim3 grid, dim3 block, size_t shared, hipStream_t stream,
                         void *start, void *end, Args... args) {
    if (start && end)
        hipExtLaunchKernelGGL(kernel, grid, block, shared, stream, (hipEvent_t)start, (hipEvent_t)end, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, shared, stream, args...);
}

}  // namespace ss
