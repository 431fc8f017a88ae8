// Status codes and small host helpers shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <cstdint>
#include "fp8kv_amd.h"

namespace fp8kv {

// Last status of the void-returning h4mv_launch on this host thread (h4mv_launch keeps the
// reference's void signature, so callers that want the error ask for it afterwards).
extern thread_local int g_last_status;

// HIP error code behind the last FP8KV_ERR_LAUNCH on this host thread.
extern thread_local int g_last_hip_error;

// Clear an error left by earlier, unrelated HIP calls so that finish_launch() reports only the
// launch that follows.
inline void begin_launch() { (void)hipGetLastError(); }

inline int finish_launch() {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) return FP8KV_OK;
    g_last_hip_error = (int)e;
    return FP8KV_ERR_LAUNCH;
}

// Events armed by fp8kv_time_next_launch() for the next kernel this host thread launches.
extern thread_local hipEvent_t g_time_start;
extern thread_local hipEvent_t g_time_stop;

// Every kernel of the library is launched through here: an ordinary launch, or, when events are
// armed, hipExtLaunchKernel, which stamps them with the dispatch's own start and end, so a timed
// launch reports the kernel's execution time (what a kernel trace reports), not the time between
// two markers queued around it.
template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds_bytes,
                          hipStream_t stream, Args... args) {
    hipEvent_t a = g_time_start, b = g_time_stop;
    if (a == nullptr && b == nullptr) {
        hipLaunchKernelGGL(kernel, grid, block, lds_bytes, stream, static_cast<KArgs>(args)...);
        return;
    }
    g_time_start = g_time_stop = nullptr;
    hipExtLaunchKernelGGL(kernel, grid, block, lds_bytes, stream, a, b, 0, static_cast<KArgs>(args)...);
}

__host__ __device__ inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace fp8kv
