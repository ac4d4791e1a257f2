// Kernel launch helper shared by the HIP translation units.  When the caller
// armed rwkv_time_next_launch(), the launch records its own start / stop
// timestamps (hipExtLaunchKernelGGL), so an event pair measures the kernel
// alone, without the dispatch overhead a stream-recorded event pair adds.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "common.h"

namespace rwkv {

// `lds` bytes of dynamic shared memory.
template <typename Kernel, typename... Args>
inline void launch_lds(Kernel kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
    const TimingEvents ev = take_timing();
    if (ev.start && ev.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, reinterpret_cast<hipEvent_t>(ev.start),
                              reinterpret_cast<hipEvent_t>(ev.stop), 0, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
}

template <typename Kernel, typename... Args>
inline void launch(Kernel kernel, dim3 grid, dim3 block, hipStream_t stream, Args... args) {
    launch_lds(kernel, grid, block, 0, stream, args...);
}

}  // namespace rwkv
