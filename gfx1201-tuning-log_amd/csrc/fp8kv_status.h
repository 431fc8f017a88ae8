// Status codes and small host helpers shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include "fp8kv_amd.h"

namespace fp8kv {

// Last status of the void-returning h4mv_launch on this host thread (h4mv_launch keeps the
// reference's void signature, so callers that want the error ask for it afterwards).
extern thread_local int g_last_status;

inline int finish_launch() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? FP8KV_OK : FP8KV_ERR_LAUNCH;
}

__host__ __device__ inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace fp8kv
