// Shared device helpers for the gfx950 (CDNA4, wave64) kernels of this library.
//
// Formats handled here:
//   * e2m1 (MXFP4 element): sign | 2-bit exponent (bias 1) | 1-bit mantissa; two codes per byte,
//     LOW nibble = even k (the Quark checkpoint layout read by h4mv/h4mv.cu:2-3).
//   * e8m0 (MX block scale): 2^(b-127) for b in [0,254], b = 255 is NaN (OCP MX v1.0).
//   * e4m3fn (KV cache): bias 7, no infinities, 0x7F/0xFF are NaN, max 448.
// All conversions use the gfx950 scaled-convert instructions, which take the packed codes
// straight from a VGPR and return bf16 pairs; e2m1 * 2^k and e4m3 values are exact in bf16.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define FP8KV_WAVE 64

// e8m0 byte -> f32 scale.  Byte 0 is 2^-127 (an f32 subnormal), byte 255 is NaN.
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
    uint32_t bits = b << 23;
    bits = (b == 0u) ? 0x00400000u : bits;
    bits = (b == 255u) ? 0x7fc00000u : bits;
    return __uint_as_float(bits);
}

// Two e2m1 codes held in byte `sel` (0..3) of `w` -> (lo nibble, hi nibble) as bf16, times `scale`.
template <int SEL>
__device__ __forceinline__ bf16x2_t fp4x2_to_bf16x2(uint32_t w, float scale) {
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, SEL);
}

// Four e2m1 bytes (8 codes) of one dword -> 8 bf16 (an MFMA A/B fragment), times `scale`.
__device__ __forceinline__ bf16x8_t fp4x8_to_bf16x8(uint32_t w, float scale) {
    bf16x2_t p0 = fp4x2_to_bf16x2<0>(w, scale);
    bf16x2_t p1 = fp4x2_to_bf16x2<1>(w, scale);
    bf16x2_t p2 = fp4x2_to_bf16x2<2>(w, scale);
    bf16x2_t p3 = fp4x2_to_bf16x2<3>(w, scale);
    bf16x8_t r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// Two e4m3fn bytes held in the low (HI=false) or high (HI=true) 16 bits of `w` -> bf16 pair.
template <bool HI>
__device__ __forceinline__ bf16x2_t fp8x2_to_bf16x2(uint32_t w) {
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
}

// Eight e4m3fn bytes (two dwords, byte order = element order) -> bf16x8, assembled from whole
// dwords (element-wise 16-bit inserts would cost a register move per element).
__device__ __forceinline__ bf16x8_t fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
    u32x4_t r;
    r[0] = __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<false>(lo));
    r[1] = __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<true>(lo));
    r[2] = __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<false>(hi));
    r[3] = __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<true>(hi));
    return __builtin_bit_cast(bf16x8_t, r);
}

// f32 -> bf16 bits, round to nearest even (NaN stays NaN): v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// bf16 round trip of an f32 (round to nearest even): the value a bf16 store would hold.
__device__ __forceinline__ float round_to_bf16(float f) { return (float)(__bf16)f; }

// SiLU in f32, x / (1 + e^-x): one definition for the stand-alone activation kernel and the
// matvec epilogue, so both give the same bits.
__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ f32x4_t mfma16x16x32_bf16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// LDS pointer type for the direct global->LDS loads (global_load_lds_dword{,x4}).
typedef __attribute__((address_space(3))) void lds_void_t;

// Copy 16 bytes per lane from global memory straight into LDS: lane i lands at lds_base + 16 i.
// lds_base must be wave-uniform.  Completion is tracked by vmcnt only: the compiler does NOT
// order later LDS reads after it, so callers wait with wait_vmcnt<> before reading.
__device__ __forceinline__ void dma16_to_lds(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4_to_lds(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_base, 4, 0, 0);
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | expcnt 7 | lgkmcnt 15 | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// s_waitcnt vmcnt(n) for a wave-uniform n known only at run time (n in [LO, HI), by bisection;
// n >= 63 waits for 63).
template <int LO, int HI>
__device__ __forceinline__ void wait_vmcnt_range(int n) {
    if constexpr (HI - LO <= 1) {
        wait_vmcnt<LO>();
    } else {
        constexpr int MID = (LO + HI) / 2;
        if (n >= MID) wait_vmcnt_range<MID, HI>(n);
        else wait_vmcnt_range<LO, MID>(n);
    }
}
__device__ __forceinline__ void wait_vmcnt_dyn(int n) { wait_vmcnt_range<0, 64>(n < 63 ? n : 63); }

// Non-temporal 16-byte global load: weight and KV streams are read exactly once per launch.
__device__ __forceinline__ u32x4_t load_nt_16(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ u32x4_t load_16(const void* p) {
    return *reinterpret_cast<const u32x4_t*>(p);
}
