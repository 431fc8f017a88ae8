// Layer epilogues around the MXFP4 matvec for gfx950: fused residual add + RMSNorm, SiLU-and-mul,
// and the load-time gate/up row interleave that lets the matvec apply SiLU-and-mul itself
// (h4mv_silu_mul in h4mv.hip).
//
// Reference: the reference engine runs these as compiler-fused kernels of its vLLM model code,
// listed in its profiles (profiling/prof_engine.txt:13,15 "fused_add_rms_norm", :17 "mul ... silu
// slice"; profiling/prof_h4mv.txt:11,13,15), around every MXFP4 linear.  vLLM itself is absent
// here; the arithmetic follows vLLM's RMSNorm and SiluAndMul in their two forms:
//   mode 0 - the compiled native path (what the reference's profiles show):
//       z = f32(x) + f32(residual);  residual <- bf16(z);  r = rsqrt(mean(z^2) + eps)   (z in f32)
//       out = bf16( f32(bf16(z * r)) * f32(weight) )
//       silu_mul: out = bf16( silu(f32(g)) * f32(u) )            (one rounding, fused)
//   mode 1 - vLLM's custom ops (_C.fused_add_rms_norm / _C.silu_and_mul):
//       z = bf16(f32(x) + f32(residual)), residual <- z, the mean and the product use that bf16 z
//       silu_mul: out = bf16( f32(bf16(silu(f32(g)))) * f32(u) ) (two roundings)
//
// gfx950 design: every kernel here is a pure HBM stream of bf16 rows (16-byte loads and stores,
// f32 math in registers).  RMSNorm runs one 256-thread workgroup per row with the row held in
// registers between the sum of squares and the scaling (so the residual can be updated in place
// and x may alias out); the interleave is a row gather with 16-byte copies.
#include "fp8kv_common.h"
#include "fp8kv_status.h"

namespace fp8kv {
namespace epi_detail {

constexpr int kNormThreads = 256;
constexpr int kNormMaxChunks = 8;                  // 16-byte chunks per thread: H <= 16384

struct NormParams {
    const uint16_t* x;
    uint16_t* res;
    const uint16_t* w;
    uint16_t* out;
    int64_t x_stride, res_stride, out_stride;      // elements
    int H;
    float eps;
    int mode;
};

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

template <int C>
__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_kernel(NormParams P)
{
    __shared__ float wsum[kNormThreads / 64];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const uint16_t* xr = P.x + (int64_t)row * P.x_stride;
    uint16_t* rr = P.res + (int64_t)row * P.res_stride;
    uint16_t* orow = P.out + (int64_t)row * P.out_stride;

    // Every load is issued unconditionally (chunks past H re-read the row's last 16 bytes and are
    // masked to zero): a load under a divergent branch would wait for its data at the join, one
    // HBM round trip per chunk.  The weight chunks are fetched here too, so all 3*C loads of a
    // thread are in flight together.
    float z[C][8];
    u32x4_t wv[C];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int e0 = (tid + c * kNormThreads) * 8;
        const int el = min(e0, P.H - 8);
        const bool in = e0 < P.H;
        u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xr + el);
        u32x4_t rv = *reinterpret_cast<const u32x4_t*>(rr + el);
        wv[c] = *reinterpret_cast<const u32x4_t*>(P.w + el);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            xv[k] = in ? xv[k] : 0u;
            rv[k] = in ? rv[k] : 0u;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float a = bf_lo(xv[k]) + bf_lo(rv[k]);
            float b = bf_hi(xv[k]) + bf_hi(rv[k]);
            if (P.mode == 1) {
                a = round_to_bf16(a);
                b = round_to_bf16(b);
            }
            z[c][2 * k] = a;
            z[c][2 * k + 1] = b;
            ss += a * a;
            ss += b * b;
        }
    }
    // sum of squares over the workgroup: xor-shuffles in each wave, then the four wave sums
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((tid & 63) == 0) wsum[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kNormThreads / 64; ++w) tot += wsum[w];
    const float r = rsqrtf(tot / (float)P.H + P.eps);

#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int e0 = (tid + c * kNormThreads) * 8;
        if (e0 < P.H) {
            u32x4_t rs, os;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float a = z[c][2 * k], b = z[c][2 * k + 1];
                rs[k] = pack_bf16x2(a, b);
                const float ya = round_to_bf16(a * r), yb = round_to_bf16(b * r);
                os[k] = pack_bf16x2(ya * bf_lo(wv[c][k]), yb * bf_hi(wv[c][k]));
            }
            *reinterpret_cast<u32x4_t*>(rr + e0) = rs;
            *reinterpret_cast<u32x4_t*>(orow + e0) = os;
        }
    }
}

struct SiluParams {
    const uint16_t* in;
    uint16_t* out;
    int64_t in_stride, out_stride;                 // elements
    int rows, d, chunks;                           // chunks: 8-element pieces per row
    int mode;
};

__global__ void __launch_bounds__(256)
silu_mul_kernel(SiluParams P)
{
    const int64_t items = (int64_t)P.rows * P.chunks;
    for (int64_t it = blockIdx.x * 256 + threadIdx.x; it < items; it += (int64_t)gridDim.x * 256) {
        const int row = (int)(it / P.chunks);
        const int j = (int)(it - (int64_t)row * P.chunks) * 8;
        const uint16_t* g = P.in + (int64_t)row * P.in_stride + j;
        const u32x4_t gv = *reinterpret_cast<const u32x4_t*>(g);
        const u32x4_t uv = *reinterpret_cast<const u32x4_t*>(g + P.d);
        u32x4_t ov;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float sa = silu_f32(bf_lo(gv[k])), sb = silu_f32(bf_hi(gv[k]));
            if (P.mode == 1) {
                sa = round_to_bf16(sa);
                sb = round_to_bf16(sb);
            }
            ov[k] = pack_bf16x2(sa * bf_lo(uv[k]), sb * bf_hi(uv[k]));
        }
        *reinterpret_cast<u32x4_t*>(P.out + (int64_t)row * P.out_stride + j) = ov;
    }
}

// Interleaved row R = 16 T + i of the gate/up weight: gate row 8 T + i for i < 8, up row
// I + 8 T + (i - 8) otherwise (I = N / 2), so each 16-row matvec tile holds 8 gate rows and the
// up rows of the same 8 features.
__host__ __device__ inline int interleave_src_row(int R, int N)
{
    const int T = R >> 4, i = R & 15;
    return i < 8 ? 8 * T + i : (N >> 1) + 8 * T + (i - 8);
}

__global__ void __launch_bounds__(256)
interleave_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ St, uint8_t* __restrict__ Wo,
                  uint8_t* __restrict__ So, int N, int K)
{
    const int R = blockIdx.x;
    const int src = interleave_src_row(R, N);
    const int wb = K >> 1, sb = K >> 5;            // bytes per row: codes (multiple of 16), scales
    const uint8_t* ws = W + (int64_t)src * wb;
    uint8_t* wd = Wo + (int64_t)R * wb;
    for (int i = threadIdx.x; i < wb / 16; i += 256)
        reinterpret_cast<u32x4_t*>(wd)[i] = reinterpret_cast<const u32x4_t*>(ws)[i];
    const uint8_t* ss = St + (int64_t)src * sb;
    uint8_t* sd = So + (int64_t)R * sb;
    for (int i = threadIdx.x; i < sb; i += 256) sd[i] = ss[i];
}

}  // namespace epi_detail
}  // namespace fp8kv

using namespace fp8kv;
using namespace fp8kv::epi_detail;

extern "C" int fp8kv_fused_add_rmsnorm(const void* x, int64_t x_row_stride, void* residual,
                                       int64_t residual_row_stride, const void* weight, void* out,
                                       int64_t out_row_stride, int num_tokens, int hidden_size,
                                       float eps, int mode, void* stream)
{
    if (!x || !residual || !weight || !out) return FP8KV_ERR_ARG;
    if (num_tokens < 0 || hidden_size < 1 || (mode != 0 && mode != 1) || !(eps >= 0.f)) return FP8KV_ERR_ARG;
    if (num_tokens == 0) return FP8KV_OK;
    if (hidden_size % 8 != 0 || hidden_size > kNormThreads * 8 * kNormMaxChunks) return FP8KV_ERR_SHAPE;
    if (x_row_stride < hidden_size || residual_row_stride < hidden_size || out_row_stride < hidden_size)
        return FP8KV_ERR_ARG;
    if (!aligned(x, 16) || !aligned(residual, 16) || !aligned(weight, 16) || !aligned(out, 16) ||
        (x_row_stride | residual_row_stride | out_row_stride) & 7)
        return FP8KV_ERR_ALIGN;
    NormParams P;
    P.x = static_cast<const uint16_t*>(x);
    P.res = static_cast<uint16_t*>(residual);
    P.w = static_cast<const uint16_t*>(weight);
    P.out = static_cast<uint16_t*>(out);
    P.x_stride = x_row_stride;
    P.res_stride = residual_row_stride;
    P.out_stride = out_row_stride;
    P.H = hidden_size;
    P.eps = eps;
    P.mode = mode;
    const int chunks = (hidden_size / 8 + kNormThreads - 1) / kNormThreads;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)num_tokens), block(kNormThreads);
    begin_launch();
    if (chunks <= 1) launch_kernel(add_rmsnorm_kernel<1>, grid, block, 0, st, P);
    else if (chunks <= 2) launch_kernel(add_rmsnorm_kernel<2>, grid, block, 0, st, P);
    else if (chunks <= 4) launch_kernel(add_rmsnorm_kernel<4>, grid, block, 0, st, P);
    else launch_kernel(add_rmsnorm_kernel<8>, grid, block, 0, st, P);
    return finish_launch();
}

extern "C" int fp8kv_silu_mul(const void* gate_up, int64_t in_row_stride, void* out,
                              int64_t out_row_stride, int num_tokens, int d, int mode, void* stream)
{
    if (!gate_up || !out) return FP8KV_ERR_ARG;
    if (num_tokens < 0 || d < 1 || (mode != 0 && mode != 1)) return FP8KV_ERR_ARG;
    if (num_tokens == 0) return FP8KV_OK;
    if (d % 8 != 0) return FP8KV_ERR_SHAPE;
    if (in_row_stride < 2 * (int64_t)d || out_row_stride < d) return FP8KV_ERR_ARG;
    if (!aligned(gate_up, 16) || !aligned(out, 16) || ((in_row_stride | out_row_stride) & 7))
        return FP8KV_ERR_ALIGN;
    SiluParams P;
    P.in = static_cast<const uint16_t*>(gate_up);
    P.out = static_cast<uint16_t*>(out);
    P.in_stride = in_row_stride;
    P.out_stride = out_row_stride;
    P.rows = num_tokens;
    P.d = d;
    P.chunks = d / 8;
    P.mode = mode;
    const int64_t items = (int64_t)num_tokens * P.chunks;
    int64_t blocks = (items + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    begin_launch();
    launch_kernel(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), P);
    return finish_launch();
}

extern "C" int h4mv_interleave_gate_up(const void* W, const void* St, void* W_out, void* St_out,
                                       int N, int K, void* stream)
{
    if (!W || !St || !W_out || !St_out || N < 1 || K < 32) return FP8KV_ERR_ARG;
    if (N % 16 != 0 || K % 32 != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(W, 16) || !aligned(W_out, 16)) return FP8KV_ERR_ALIGN;
    begin_launch();
    launch_kernel(interleave_kernel, dim3((unsigned)N), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                  static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St),
                  static_cast<uint8_t*>(W_out), static_cast<uint8_t*>(St_out), N, K);
    return finish_launch();
}
