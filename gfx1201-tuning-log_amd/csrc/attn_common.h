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
__device__ __forceinline__ void store_coherent(float* p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

}  // namespace fp8kv
