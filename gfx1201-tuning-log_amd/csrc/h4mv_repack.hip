// Load-time repack of MXFP4 block scales for the matvec: the checkpoint's weight_scale
// [K/32, N] (one e8m0 byte per 32 k of every output row, output rows contiguous) becomes the
// matvec's [N, K/32] (the scales of one output row contiguous, streamed with that row's codes).
//
// Reference: h4mv/fp8kv_hipw4.py:32-43 (_st_for: weight_scale.t().contiguous(), cached per
// weight and never run during graph capture).
//
// gfx950 design: a 64 x 64 byte tile per workgroup, read along N and written along K/32 through
// LDS (row pitch 68 bytes to spread the column reads of the write phase over the banks); each
// thread moves 4 bytes per step.  It runs once per weight (3.7 MB at configs[1]), so it is written for
// plain coalescing rather than peak bandwidth.
#include "fp8kv_common.h"
#include "fp8kv_status.h"

namespace fp8kv {
namespace repack_detail {

constexpr int kTile = 64;
constexpr int kPitch = 68;

__global__ void __launch_bounds__(256)
repack_scales_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out, int N, int G)
{
    __shared__ uint8_t tile[kTile * kPitch];
    const int n0 = blockIdx.x * kTile, g0 = blockIdx.y * kTile;
    const int t = threadIdx.x;
    // read: 64 rows g x 64 columns n, thread t moves 4 consecutive n of row t / 16 + 16 i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = t / 16 + 16 * i;
        const int c = 4 * (t % 16);
        const int g = g0 + r;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int n = n0 + c + b;
            tile[r * kPitch + c + b] = (g < G && n < N) ? in[(int64_t)g * N + n] : 0;
        }
    }
    __syncthreads();
    // write: 64 rows n x 64 columns g
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = t / 16 + 16 * i;
        const int c = 4 * (t % 16);
        const int n = n0 + r;
        if (n >= N) continue;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int g = g0 + c + b;
            if (g < G) out[(int64_t)n * G + g] = tile[(c + b) * kPitch + r];
        }
    }
}

}  // namespace repack_detail
}  // namespace fp8kv

using namespace fp8kv;

extern "C" int h4mv_repack_scales(const void* scale_kn, void* scale_nk, int N, int K, void* stream)
{
    if (!scale_kn || !scale_nk || N < 1 || K < 1) return FP8KV_ERR_ARG;
    if (K % 32 != 0) return FP8KV_ERR_SHAPE;
    const int G = K / 32;
    const dim3 grid((unsigned)((N + repack_detail::kTile - 1) / repack_detail::kTile),
                    (unsigned)((G + repack_detail::kTile - 1) / repack_detail::kTile));
    if (grid.y > 65535) return FP8KV_ERR_SHAPE;
    begin_launch();
    launch_kernel(repack_detail::repack_scales_kernel, grid, dim3(256), 0,
                  reinterpret_cast<hipStream_t>(stream), static_cast<const uint8_t*>(scale_kn),
                  static_cast<uint8_t*>(scale_nk), N, G);
    return finish_launch();
}
