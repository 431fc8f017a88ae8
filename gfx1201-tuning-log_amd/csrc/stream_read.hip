// Measurement helper (not part of the drop-in ABI, and built into its own library,
// libfp8kv_measure.so, which only the benchmark loads): one launch that reads a buffer once.
//
// The benchmark times it beside the HBM-bound kernels at their own byte counts, so their roofline
// fractions can be read against what a single read-only launch of the same size reaches on the
// box (launch, ramp-up and drain included), not only against the 8 TB/s peak.  Every thread
// issues all its 16-byte non-temporal loads (up to 16) before folding them, at least 1024
// workgroups of 256 threads (in a probe of 256..2048 workgroups of 256..1024 threads reading 32
// and 64 MB, 512-2048 workgroups were fastest, 1024 x 256 within 1%).
#include "fp8kv_common.h"
#include "fp8kv_status.h"

namespace fp8kv {
namespace stream_detail {

constexpr int kThreads = 256;
constexpr int kMaxPer = 16;                  // loads per thread, all issued before any is used
constexpr int kMaxBlocks = 4096;

// Workgroup b reads the contiguous vectors [b * 256 per, (b + 1) * 256 per), thread t those at
// t + 256 u, u < per <= kMaxPer (predicated past the end): every load of the launch is in flight
// at once, with no loop-carried wait.  (Contiguous per-workgroup ranges measured faster than a
// grid-wide stride: 10.3 against 11.9 us for 62 MB.)
__global__ void __launch_bounds__(kThreads) stream_read_kernel(const u32x4_t* __restrict__ src, size_t n16,
                                                               int per, uint32_t* __restrict__ sink)
{
    const size_t i = blockIdx.x * (size_t)kThreads * per + threadIdx.x;
    u32x4_t v[kMaxPer];
#pragma unroll
    for (int u = 0; u < kMaxPer; ++u) {
        const size_t j = i + (size_t)u * kThreads;
        v[u] = (u < per && j < n16) ? load_nt_16(src + j) : (u32x4_t){0u, 0u, 0u, 0u};
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < kMaxPer; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    // one value per workgroup, so the loads are not dead
    acc = __reduce_xor_sync(~0ull, acc);
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

}  // namespace stream_detail
}  // namespace fp8kv

extern "C" int fp8kv_stream_read(const void* src, size_t bytes, void* sink, void* stream, void* start_event,
                                 void* stop_event)
{
    using namespace fp8kv::stream_detail;
    if (!src || !sink || bytes < 16 || (bytes & 15) || !fp8kv::aligned(src, 16) || !fp8kv::aligned(sink, 4))
        return FP8KV_ERR_ARG;
    // 1024 workgroups while that keeps 16 or fewer loads per thread (the probe's best shape for 32
    // and 64 MB), more beyond; sizes past kMaxBlocks * 256 * 16 vectors (16 GiB) are refused.
    const size_t n16 = bytes / 16;
    size_t blocks = (n16 + (size_t)kThreads * kMaxPer - 1) / ((size_t)kThreads * kMaxPer);
    if (blocks < 1024) blocks = 1024;
    if (blocks > kMaxBlocks) return FP8KV_ERR_SHAPE;
    const int per = (int)((n16 + blocks * kThreads - 1) / (blocks * kThreads));
    (void)hipGetLastError();
    if (!start_event && !stop_event) {               // a plain launch (also inside a graph capture)
        hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                           reinterpret_cast<hipStream_t>(stream), static_cast<const u32x4_t*>(src), n16, per,
                           static_cast<uint32_t*>(sink));
    } else {
        // hipExtLaunchKernel stamps the events (either may be NULL) at the dispatch's own start and end
        hipExtLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                              reinterpret_cast<hipStream_t>(stream), static_cast<hipEvent_t>(start_event),
                              static_cast<hipEvent_t>(stop_event), 0, static_cast<const u32x4_t*>(src), n16,
                              per, static_cast<uint32_t*>(sink));
    }
    return hipGetLastError() == hipSuccess ? FP8KV_OK : FP8KV_ERR_LAUNCH;
}
