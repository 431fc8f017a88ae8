// Status codes and small host helpers shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>
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

__host__ __device__ inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace fp8kv
