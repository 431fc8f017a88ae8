// MXFP4 W4A16 matvec for gfx950: Out[M,N] = X[M,K] . dequant(W[N,K/2], St[N,K/32])^T.
//
// Reference semantics: h4mv/h4mv.cu:43-104 (layout, e2m1 table, per-32 e8m0 scale,
// fp32 accumulation, bf16 output) and its C ABI h4mv/h4mv.cu:106-122.
//
// gfx950 design (not a translation of the wave-per-row dot2 kernel):
//   * A workgroup owns a 16-row tile of W and runs one v_mfma_f32_16x16x32_bf16 chain per wave;
//     the four waves split K and meet in LDS once at the end (split-K inside the workgroup, so
//     N/16 workgroups of equal size fill the 256 CUs evenly).
//   * Lane (r, q) = (lane % 16, lane / 16) streams whole 16-byte scale groups of row r: one
//     global_load_dwordx4 = 32 codes = exactly one e8m0 group, so each load needs one scale.
//     The 16 bytes become four MFMA A fragments via v_cvt_scalef32_pk_bf16_fp4, which applies
//     the group scale during the conversion (e2m1 * 2^k is exact in bf16).
//   * K is a reduction index, so the kernel may visit it in any order as long as the A (weights)
//     and B (activations) fragments agree: quad q of the wave handles group g = g0 + 4u + q and
//     fragment j covers k = 32 g + 8 j + (0..7) on both sides.
//   * X is the B operand: lane (m, q) loads X[m, 32 g + 8 j .. +8] for m < M and holds zeros for the
//     padded columns m >= M, so one kernel serves 1 <= M <= 16.  X is small and stays in L2.
//   * Output tile: lane (m, q) register i holds row n0 + 4 q + i of column m, so each lane of the
//     first wave writes 4 consecutive bf16 of Out[m, :].
#include "fp8kv_common.h"
#include "fp8kv_status.h"

namespace fp8kv {

thread_local int g_last_status = FP8KV_OK;

namespace {

constexpr int kRowsPerWG = 16;
constexpr int kWavesPerWG = 4;

template <int U>
__global__ void __launch_bounds__(256)
h4mv_mfma_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ St,
                 const __bf16* __restrict__ X, __bf16* __restrict__ Out,
                 int N, int K, int M, int groups_per_wave)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;        // weight row within the tile / activation column m
    const int q = lane >> 4;        // which of 4 consecutive scale groups this lane streams
    const int G = K >> 5;           // scale groups per row
    const int n0 = blockIdx.x * kRowsPerWG;
    const int row = n0 + r;
    const bool row_ok = row < N;
    const bool col_ok = r < M;

    const int g_begin = wave * groups_per_wave;
    const int g_end = min(G, g_begin + groups_per_wave);

    const uint8_t* wrow = W + (size_t)(row_ok ? row : 0) * (size_t)(K >> 1);
    const uint8_t* srow = St + (size_t)(row_ok ? row : 0) * (size_t)G;
    const __bf16* xrow = X + (size_t)(col_ok ? r : 0) * (size_t)K;

    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};

    for (int g0 = g_begin; g0 < g_end; g0 += 4 * U) {
        u32x4_t wv[U];
        uint32_t sb[U];
        u32x4_t xv[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int g = g0 + 4 * u + q;
            const bool g_ok = g < g_end;
            const u32x4_t zero = {0u, 0u, 0u, 0u};
            wv[u] = (g_ok && row_ok) ? load_nt_16(wrow + (size_t)g * 16) : zero;
            sb[u] = (g_ok && row_ok) ? (uint32_t)srow[g] : 127u;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xv[u][j] = (g_ok && col_ok) ? load_16(xrow + (size_t)g * 32 + 8 * j) : zero;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float sc = e8m0_to_f32(sb[u]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bf16x8_t a = fp4x8_to_bf16x8(wv[u][j], sc);
                acc = mfma16x16x32_bf16(a, as_bf16x8(xv[u][j]), acc);
            }
        }
    }

    __shared__ f32x4_t red[kWavesPerWG - 1][64];
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < kWavesPerWG - 1; ++w) acc += red[w][lane];

    const int m = r;
    if (m >= M) return;
    const int n = n0 + 4 * q;
    __bf16* orow = Out + (size_t)m * (size_t)N;
    if (n + 3 < N && ((N & 3) == 0) && aligned(Out, 8)) {
        u32x2_t v = {pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
        *reinterpret_cast<u32x2_t*>(orow + n) = v;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (n + i < N) orow[n + i] = (__bf16)acc[i];
    }
}

}  // namespace
}  // namespace fp8kv

extern "C" int h4mv_launch_status(const void* W, const void* St, const void* Xb, void* Out,
                                  int N, int K, int M, void* stream)
{
    using namespace fp8kv;
    if (!W || !St || !Xb || !Out) return FP8KV_ERR_ARG;
    if (N < 1 || K < 32 || M < 1) return FP8KV_ERR_ARG;
    if (M > 16 || (K & 31) != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(W, 16) || !aligned(Xb, 16) || !aligned(Out, 2)) return FP8KV_ERR_ALIGN;
    const int G = K >> 5;
    int per_wave = (G + kWavesPerWG - 1) / kWavesPerWG;
    per_wave = (per_wave + 3) & ~3;
    const dim3 grid((unsigned)((N + kRowsPerWG - 1) / kRowsPerWG));
    const dim3 block(64 * kWavesPerWG);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(h4mv_mfma_kernel<4>, grid, block, 0, s,
                       static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St),
                       static_cast<const __bf16*>(Xb), static_cast<__bf16*>(Out), N, K, M, per_wave);
    return finish_launch();
}

extern "C" void h4mv_launch(const void* W, const void* St, const void* Xb, void* Out,
                            int N, int K, int M, void* stream)
{
    fp8kv::g_last_status = h4mv_launch_status(W, St, Xb, Out, N, K, M, stream);
}

extern "C" int fp8kv_last_status(void) { return fp8kv::g_last_status; }

extern "C" const char* fp8kv_status_string(int status)
{
    switch (status) {
        case FP8KV_OK: return "ok";
        case FP8KV_ERR_ARG: return "invalid argument";
        case FP8KV_ERR_SHAPE: return "unsupported shape";
        case FP8KV_ERR_ALIGN: return "misaligned pointer or stride";
        case FP8KV_ERR_LAUNCH: return "kernel launch failed";
        case FP8KV_ERR_SCRATCH: return "scratch buffer missing or too small";
        default: return "unknown status";
    }
}
