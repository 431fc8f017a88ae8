// Device helpers shared by the paged fp8 attention kernels (decode and prefill) for gfx950.
#pragma once
#include "fp8kv_common.h"

namespace fp8kv {

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

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
