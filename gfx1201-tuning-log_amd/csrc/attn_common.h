// Device helpers shared by the paged fp8 attention kernels (decode and prefill) for gfx950.
#pragma once
#include "fp8kv_common.h"

namespace fp8kv {

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// Reductions over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the k-parts of one MFMA column) with
// the gfx950 lane swaps: v_permlane16_swap_b32 on (x, x) hands every lane the values of lanes
// l & ~16 and l | 16, v_permlane32_swap_b32 those of lanes l & ~32 and l | 32.  Pure VALU, no LDS
// round trip; every lane gets the bitwise-identical result.
__device__ __forceinline__ float max_xor16_32(float v)
{
    const uint32_t b = __float_as_uint(v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const float m = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const uint32_t c = __float_as_uint(m);
    const auto r32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}
__device__ __forceinline__ float sum_xor16_32(float v)
{
    const uint32_t b = __float_as_uint(v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const float m = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const uint32_t c = __float_as_uint(m);
    const auto r32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

__device__ __forceinline__ uint32_t bf16x2_bits(bf16x2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Device-coherent (agent-scope) accesses for the cross-workgroup partial records: they bypass the
// per-XCD L2 state that ordinary accesses may hit, so no cache-wide write-back or invalidate is
// needed to hand records from one workgroup to another.
__device__ __forceinline__ float load_coherent(const float* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Two adjacent floats (8-byte aligned) in one device-coherent 8-byte store.
__device__ __forceinline__ void store_coherent2(float* p, float a, float b)
{
    const uint64_t v = __builtin_bit_cast(uint64_t, (f32x2_t){a, b});
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Four adjacent floats (16-byte aligned) in one device-coherent 16-byte store (global_store_dwordx4
// with the agent-scope sc1 bit; HIP's atomic stores stop at 8 bytes).  The caller waits for it
// with s_waitcnt vmcnt like any other store.
__device__ __forceinline__ void store_coherent4(float* p, f32x4_t v)
{
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
// Two adjacent floats (8-byte aligned) in one device-coherent 8-byte load.
__device__ __forceinline__ f32x2_t load_coherent2(const float* p)
{
    const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_bit_cast(f32x2_t, v);
}

// MFMA A fragments of O^T = V^T . P^T for one 32-token group from lane (c, p)'s V bytes:
// vr[j] = bytes d = 8c .. 8c+7 of the group's k-slot j token (two e4m3 dwords).  The 8 x 8 byte
// block is transposed in registers: each output dword pairs two tokens at one d (v_perm_b32), then
// v_cvt_scalef32_pk_bf16_fp8 widens the byte pairs.  Fragment n (d row 8c + n) dword k is the bf16
// pair (k-slot 2k, k-slot 2k + 1).
__device__ __forceinline__ void v_fragments(const u32x2_t (&vr)[8], u32x4_t (&bf)[8])
{
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t a = vr[2 * k][w], b = vr[2 * k + 1][w];
            const uint32_t x = __builtin_amdgcn_perm(b, a, 0x05010400u);   // a0 b0 a1 b1
            const uint32_t y = __builtin_amdgcn_perm(b, a, 0x07030602u);   // a2 b2 a3 b3
            bf[4 * w + 0][k] = bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, false));
            bf[4 * w + 1][k] = bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, true));
            bf[4 * w + 2][k] = bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(y, 1.0f, false));
            bf[4 * w + 3][k] = bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(y, 1.0f, true));
        }
    }
}

// The same fragments from bf16 V (no widening): vr[j] = d = 8c .. 8c+7 of k-slot j's token (four
// dwords, d pair (2w, 2w + 1) in dword w).  v_perm_b32 pairs the two tokens' halves: fragment
// 2w + h (d row 8c + 2w + h) dword k is (k-slot 2k, k-slot 2k + 1) at that d.
__device__ __forceinline__ void v_fragments_b16(const u32x4_t (&vr)[8], u32x4_t (&bf)[8])
{
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t a = vr[2 * k][w], b = vr[2 * k + 1][w];
            bf[2 * w + 0][k] = __builtin_amdgcn_perm(b, a, 0x05040100u);   // a.lo b.lo
            bf[2 * w + 1][k] = __builtin_amdgcn_perm(b, a, 0x07060302u);   // a.hi b.hi
        }
    }
}

typedef int v8i __attribute__((ext_vector_type(8)));

// D += A . B^T over 128 k on the block-scaled MFMA with e4m3 A and B (both block scales 1.0):
// lane (r, p) supplies row r's k 16p .. 16p+15 in bytes 0..15 and 64+16p .. +15 in bytes 16..31
// of each operand; the products are exact and accumulate in fp32.
__device__ __forceinline__ f32x4_t mfma_fp8_16x16x128(const v8i& a, const v8i& b, f32x4_t c)
{
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// One query row's 32 bf16 values held by this lane (the 128-value row is spread over the four
// lanes n, n + 16, n + 32, n + 48) -> e4m3 hi and lo parts with q * 2^e = hi + lo, where 2^e is
// the row's scale: the largest |q| of the row times 2^e lies in [128, 256).  Returns 2^-e.
// hi is q * 2^e rounded to 4 significant bits; the remainder lo is a multiple of the bf16 value's
// last place below 2^-4 of it, exact in e4m3 whenever |q| >= 2^-9 of the row's largest |q| (the
// subnormal range covers smaller values to 2^-10 of their place).  The products of the two MFMAs
// with exact e4m3 K then sum to the bf16 path's S up to fp32 accumulation order.  sign_mask
// (0x80808080 or 0) negates the row in e4m3 (exact).
__device__ __forceinline__ float q_fp8_split(const u32x4_t (&qf)[4], uint32_t sign_mask, v8i& hi, v8i& lo)
{
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            amax = fmaxf(amax, fabsf(__uint_as_float(qf[c][d] << 16)));
            amax = fmaxf(amax, fabsf(__uint_as_float(qf[c][d] & 0xFFFF0000u)));
        }
    amax = max_xor16_32(amax);
    // biased exponent of the scale 2^e = 2^(7 - floor(log2 amax)), kept where 2^-e is normal too
    int be = 261 - (int)((__float_as_uint(amax) >> 23) & 0xFFu);
    be = be < 1 ? 1 : (be > 253 ? 253 : be);
    const float scale = __uint_as_float((uint32_t)be << 23);
    const float inv = __uint_as_float((uint32_t)(254 - be) << 23);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) {               // dword pair (2h, 2h + 1) of chunk c -> 4 values
            float x[4];
            x[0] = __uint_as_float(qf[c][2 * h] << 16) * scale;
            x[1] = __uint_as_float(qf[c][2 * h] & 0xFFFF0000u) * scale;
            x[2] = __uint_as_float(qf[c][2 * h + 1] << 16) * scale;
            x[3] = __uint_as_float(qf[c][2 * h + 1] & 0xFFFF0000u) * scale;
            uint32_t hw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
            hw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], (int)hw, true);
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hw, false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hw, true);
            uint32_t lw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[0] - h01[0], x[1] - h01[1], 0, false);
            lw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[2] - h23[0], x[3] - h23[1], (int)lw, true);
            // chunk c holds d 16p + 8 (c & 1) + 4 h .. of the low half (c < 2) or the high half
            const int slot = 4 * (c >> 1) + 2 * (c & 1) + h;
            hw ^= sign_mask;
            lw ^= sign_mask;
            // opaque to the compiler, which would otherwise re-derive the parts inside the key loop
            asm volatile("" : "+v"(hw), "+v"(lw));
            hi[slot] = (int)hw;
            lo[slot] = (int)lw;
        }
    return inv;
}

}  // namespace fp8kv
