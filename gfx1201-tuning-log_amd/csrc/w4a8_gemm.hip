// MXFP4 x MXFP8 GEMM for M >= 16 (prefill-sized linears) on gfx950's block-scaled MFMA, and the
// MXFP8 activation quantiser that feeds it.
//
//   Out[m, n] = bf16( sum_k  xq[m, k] * 2^(sx[m, k/32] - 127)  *  w[n, k] * 2^(sw[n, k/32] - 127) )
//
// w: e2m1 codes [N, K/2] (low nibble = even k) with e8m0 scales St [N, K/32] - the matvec's layout
// (h4mv/h4mv.cu:1-3 with the scale repack of h4mv/fp8kv_hipw4.py:32-43); xq: e4m3fn [M, K] with
// e8m0 scales Sx [M, K/32] from h4a8_quant_act (OCP MX v1.0: per 32 consecutive k, shared
// exponent floor(log2(max |x|)) - 8, elements x / 2^e rounded to nearest even and saturated to
// +-448).
//
// Reference: the reference engine's prefill runs its vLLM fork's radiance_mxfp4_fp8_gemm (W4A8,
// per-token fp8 activations from dynamic_per_token_scaled_fp8_quant): profiling/prof_engine.txt:3-4,
// profiling/prof_prefill.txt:8, docs/06-w4gemm-hip-roadmap.md:140.  That library is closed and
// absent, so the activation format here is gfx950's native one (MXFP8, whose block scales the
// MFMA applies itself) and parity is against this file's own definition (oracle/w4a8.py).
//
// gfx950 design:
//   * v_mfma_scale_f32_16x16x128_f8f6f4 with A = 16 weight rows (fp4, cbsz 4) and B = 16 token
//     rows (fp8, blgp 0): D[n][m] += sum over 128 k, the e8m0 scales applied by the MFMA.  Lane
//     (r, j) = (lane % 16, lane / 16) supplies A row r, k 32j .. 32j+31 (16 bytes) and B row r,
//     k 16j .. 16j+15 and 64+16j .. 64+16j+15 (two 16-byte pieces); the scale of (row r, k block j)
//     comes from lane (r, j), four tiles' scales packed in one VGPR and picked with op_sel.
//   * A workgroup of 4 waves computes a 128 (n) x 128 (m) tile, each wave 64 x 64 (4 x 4 MFMA
//     tiles, 16 MFMAs per 128-k step).  Fragments are loaded straight from global memory into
//     registers (the weight tile and the activation tile stay in L2 across the workgroups that
//     share them), two k steps in flight: every load is issued unconditionally (row and k indices
//     clamped into the operands) so the compiler's waits are exact.
//   * Tiles are numbered so that each XCD (workgroups w, w + 8, ...) takes a contiguous range of
//     weight-row blocks with all token blocks of each, keeping a weight tile in one L2.
#include "fp8kv_common.h"
#include "fp8kv_status.h"

namespace fp8kv {
namespace w4a8_detail {

constexpr int kBN = 128, kBM = 128, kBK = 128;
constexpr int kXcds = 8;

typedef int v8i __attribute__((ext_vector_type(8)));

struct Frags {
    u32x4_t a[4];        // weight n-tile i: 16 bytes (32 e2m1 codes)
    u32x4_t b[4][2];     // token m-tile i: 16 bytes at k 16j and at 64 + 16j
    uint32_t sa[4];      // scale dword of (row, k step) per n-tile: 4 blocks, this lane's is byte j
    uint32_t sb[4];
};

struct Params {
    const uint8_t* W;
    const uint8_t* St;
    const uint8_t* Xq;
    const uint8_t* Sx;
    __bf16* Out;
    int N, K, M;
    int nblk, mblk;
};

__device__ __forceinline__ uint32_t load_u32(const void* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Fragments of the k step starting at k0 (clamped to the last step) for the wave's rows.
__device__ __forceinline__ void load_frags(Frags& f, const Params& P, const uint8_t* const (&wrow)[4],
                                           const uint8_t* const (&srow)[4], const uint8_t* const (&xrow)[4],
                                           const uint8_t* const (&sxrow)[4], int k0, int j)
{
    const int kk = k0 < P.K ? k0 : P.K - kBK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f.a[i] = load_nt_16(wrow[i] + ((kk + 32 * j) >> 1));
        f.b[i][0] = load_16(xrow[i] + kk + 16 * j);
        f.b[i][1] = load_16(xrow[i] + kk + 64 + 16 * j);
        f.sa[i] = load_u32(srow[i] + (kk >> 5));
        f.sb[i] = load_u32(sxrow[i] + (kk >> 5));
    }
}

template <int I, int J>
__device__ __forceinline__ f32x4_t mfma_tile(const Frags& f, uint32_t sa, uint32_t sb, f32x4_t acc)
{
    const v8i a = {(int)f.a[I][0], (int)f.a[I][1], (int)f.a[I][2], (int)f.a[I][3], 0, 0, 0, 0};
    const v8i b = {(int)f.b[J][0][0], (int)f.b[J][0][1], (int)f.b[J][0][2], (int)f.b[J][0][3],
                   (int)f.b[J][1][0], (int)f.b[J][1][1], (int)f.b[J][1][2], (int)f.b[J][1][3]};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 4, 0, I, (int)sa, J, (int)sb);
}

__device__ __forceinline__ void compute(const Frags& f, f32x4_t (&acc)[4][4], int j)
{
    // this lane's scale byte (k block j) of each tile, packed: tile i in byte i (op_sel picks it)
    uint32_t sa = 0, sb = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sa |= ((f.sa[i] >> (8 * j)) & 0xFFu) << (8 * i);
        sb |= ((f.sb[i] >> (8 * j)) & 0xFFu) << (8 * i);
    }
    acc[0][0] = mfma_tile<0, 0>(f, sa, sb, acc[0][0]);
    acc[0][1] = mfma_tile<0, 1>(f, sa, sb, acc[0][1]);
    acc[0][2] = mfma_tile<0, 2>(f, sa, sb, acc[0][2]);
    acc[0][3] = mfma_tile<0, 3>(f, sa, sb, acc[0][3]);
    acc[1][0] = mfma_tile<1, 0>(f, sa, sb, acc[1][0]);
    acc[1][1] = mfma_tile<1, 1>(f, sa, sb, acc[1][1]);
    acc[1][2] = mfma_tile<1, 2>(f, sa, sb, acc[1][2]);
    acc[1][3] = mfma_tile<1, 3>(f, sa, sb, acc[1][3]);
    acc[2][0] = mfma_tile<2, 0>(f, sa, sb, acc[2][0]);
    acc[2][1] = mfma_tile<2, 1>(f, sa, sb, acc[2][1]);
    acc[2][2] = mfma_tile<2, 2>(f, sa, sb, acc[2][2]);
    acc[2][3] = mfma_tile<2, 3>(f, sa, sb, acc[2][3]);
    acc[3][0] = mfma_tile<3, 0>(f, sa, sb, acc[3][0]);
    acc[3][1] = mfma_tile<3, 1>(f, sa, sb, acc[3][1]);
    acc[3][2] = mfma_tile<3, 2>(f, sa, sb, acc[3][2]);
    acc[3][3] = mfma_tile<3, 3>(f, sa, sb, acc[3][3]);
}

__global__ void __launch_bounds__(256)
gemm_kernel(Params P)
{
    // XCD-aware tile order: workgroup id L runs on XCD L % 8; XCD x takes tiles
    // [x * per, (x + 1) * per) of the n-major order (all token blocks of a weight block together).
    const int L = blockIdx.x;
    const int total = P.nblk * P.mblk;
    const int per = (total + kXcds - 1) / kXcds;
    const int t = (L % kXcds) * per + L / kXcds;
    if (t >= total) return;
    const int nb = t / P.mblk, mb = t - nb * P.mblk;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, j = lane >> 4;
    const int n0 = nb * kBN + (wave & 1) * 64;
    const int m0 = mb * kBM + (wave >> 1) * 64;
    const int kh = P.K >> 1, ks = P.K >> 5;

    const uint8_t* wrow[4];
    const uint8_t* srow[4];
    const uint8_t* xrow[4];
    const uint8_t* sxrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int n = n0 + 16 * i + r;
        n = n < P.N ? n : P.N - 1;
        int m = m0 + 16 * i + r;
        m = m < P.M ? m : P.M - 1;
        wrow[i] = P.W + (int64_t)n * kh;
        srow[i] = P.St + (int64_t)n * ks;
        xrow[i] = P.Xq + (int64_t)m * P.K;
        sxrow[i] = P.Sx + (int64_t)m * ks;
    }

    f32x4_t acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

    Frags f0, f1;
    load_frags(f0, P, wrow, srow, xrow, sxrow, 0, j);
    load_frags(f1, P, wrow, srow, xrow, sxrow, kBK, j);
    for (int k0 = 0; k0 < P.K; k0 += 2 * kBK) {
        compute(f0, acc, j);
        load_frags(f0, P, wrow, srow, xrow, sxrow, k0 + 2 * kBK, j);
        if (k0 + kBK < P.K) compute(f1, acc, j);
        load_frags(f1, P, wrow, srow, xrow, sxrow, k0 + 3 * kBK, j);
    }

    // D[n][m]: lane (m = r, q = j) holds rows n = 4j .. 4j + 3 of each 16 x 16 tile
#pragma unroll
    for (int im = 0; im < 4; ++im) {
        const int m = m0 + 16 * im + r;
        if (m >= P.M) continue;
        __bf16* orow = P.Out + (int64_t)m * P.N;
#pragma unroll
        for (int in = 0; in < 4; ++in) {
            const int n = n0 + 16 * in + 4 * j;
            if (n >= P.N) continue;
            const f32x4_t v = acc[in][im];
            *reinterpret_cast<u32x2_t*>(orow + n) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
    }
}

// ---- activation quantiser: bf16 [M, K] -> e4m3fn [M, K] + e8m0 [M, K/32] ---------------------
// One thread per 32-element block: four 16-byte loads, the block maximum, two 16-byte stores.
__global__ void __launch_bounds__(256)
quant_kernel(const uint16_t* __restrict__ X, int64_t x_stride, uint8_t* __restrict__ Xq,
             uint8_t* __restrict__ Sx, int M, int K)
{
    const int nb = K >> 5;
    const int64_t items = (int64_t)M * nb;
    for (int64_t it = blockIdx.x * 256 + threadIdx.x; it < items; it += (int64_t)gridDim.x * 256) {
        const int m = (int)(it / nb), b = (int)(it - (int64_t)m * nb);
        const uint16_t* src = X + (int64_t)m * x_stride + 32 * b;
        u32x4_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = load_16(src + 8 * i);
        float amax = 0.f;
        bool bad = false;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float lo = __uint_as_float(v[i][k] << 16), hi = __uint_as_float(v[i][k] & 0xFFFF0000u);
                bad |= !(__builtin_fabsf(lo) <= 3.4e38f) || !(__builtin_fabsf(hi) <= 3.4e38f);
                amax = __builtin_fmaxf(amax, __builtin_fmaxf(__builtin_fabsf(lo), __builtin_fabsf(hi)));
            }
        // shared exponent floor(log2(amax)) - 8 (e4m3's largest exponent), as an e8m0 byte
        // clamped to [0, 254]; 255 (NaN) when the block holds a NaN or an infinity
        int e = 0;
        if (amax > 0.f) {
            const uint32_t bits = __float_as_uint(amax);
            const int be = (int)(bits >> 23);
            e = be > 0 ? be - 127 : -118 - (int)__builtin_clz(bits & 0x7FFFFFu);   // subnormal amax
        }
        int sbyte = e - 8 + 127;
        sbyte = sbyte < 0 ? 0 : (sbyte > 254 ? 254 : sbyte);
        if (amax == 0.f) sbyte = 0;
        if (bad) sbyte = 255;
        // 2^-(sbyte - 127); finite inputs give sbyte <= 246, so this is a normal float
        const float inv = bad ? 1.f : __uint_as_float((uint32_t)(254 - sbyte) << 23);
        u32x4_t q[2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t d0 = v[i][2 * h], d1 = v[i][2 * h + 1];
                float a0 = __uint_as_float(d0 << 16) * inv, a1 = __uint_as_float(d0 & 0xFFFF0000u) * inv;
                float a2 = __uint_as_float(d1 << 16) * inv, a3 = __uint_as_float(d1 & 0xFFFF0000u) * inv;
                a0 = __builtin_fminf(__builtin_fmaxf(a0, -448.f), 448.f);
                a1 = __builtin_fminf(__builtin_fmaxf(a1, -448.f), 448.f);
                a2 = __builtin_fminf(__builtin_fmaxf(a2, -448.f), 448.f);
                a3 = __builtin_fminf(__builtin_fmaxf(a3, -448.f), 448.f);
                const uint32_t p0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a0, a1, 0, false) & 0xFFFFu;
                const uint32_t p1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a2, a3, 0, false) & 0xFFFFu;
                const int o = 2 * i + h;                      // output dword: elements 4 o .. 4 o + 3
                q[o >> 2][o & 3] = p0 | (p1 << 16);
            }
        uint8_t* dst = Xq + (int64_t)m * K + 32 * b;
        *reinterpret_cast<u32x4_t*>(dst) = q[0];
        *reinterpret_cast<u32x4_t*>(dst + 16) = q[1];
        Sx[(int64_t)m * nb + b] = (uint8_t)sbyte;
    }
}

}  // namespace w4a8_detail
}  // namespace fp8kv

using namespace fp8kv;
using namespace fp8kv::w4a8_detail;

extern "C" int h4a8_quant_act(const void* X, int64_t x_row_stride, void* Xq, void* Sx, int M, int K,
                              void* stream)
{
    if (!X || !Xq || !Sx || M < 0 || K < 32) return FP8KV_ERR_ARG;
    if (M == 0) return FP8KV_OK;
    if (K % 32 != 0) return FP8KV_ERR_SHAPE;
    if (x_row_stride < K) return FP8KV_ERR_ARG;
    if (!aligned(X, 16) || !aligned(Xq, 16) || (x_row_stride & 7)) return FP8KV_ERR_ALIGN;
    const int64_t items = (int64_t)M * (K / 32);
    int64_t blocks = (items + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    begin_launch();
    launch_kernel(quant_kernel, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                  static_cast<const uint16_t*>(X), x_row_stride, static_cast<uint8_t*>(Xq),
                  static_cast<uint8_t*>(Sx), M, K);
    return finish_launch();
}

extern "C" int h4a8_gemm(const void* W, const void* St, const void* Xq, const void* Sx, void* Out,
                         int N, int K, int M, void* stream)
{
    if (!W || !St || !Xq || !Sx || !Out || N < 1 || K < 1 || M < 0) return FP8KV_ERR_ARG;
    if (M == 0) return FP8KV_OK;
    if (K % kBK != 0 || N % 4 != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(W, 16) || !aligned(Xq, 16) || !aligned(St, 4) || !aligned(Sx, 4) || !aligned(Out, 8))
        return FP8KV_ERR_ALIGN;
    Params P;
    P.W = static_cast<const uint8_t*>(W);
    P.St = static_cast<const uint8_t*>(St);
    P.Xq = static_cast<const uint8_t*>(Xq);
    P.Sx = static_cast<const uint8_t*>(Sx);
    P.Out = static_cast<__bf16*>(Out);
    P.N = N;
    P.K = K;
    P.M = M;
    P.nblk = (N + kBN - 1) / kBN;
    P.mblk = (M + kBM - 1) / kBM;
    const int64_t total = (int64_t)P.nblk * P.mblk;
    if (total > 0x7FFFFFFF - kXcds) return FP8KV_ERR_SHAPE;
    const int64_t grid = ((total + kXcds - 1) / kXcds) * kXcds;
    begin_launch();
    launch_kernel(gemm_kernel, dim3((unsigned)grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), P);
    return finish_launch();
}
