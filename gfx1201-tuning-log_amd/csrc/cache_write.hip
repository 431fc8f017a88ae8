// fp8-e4m3 KV-cache write for gfx950: quantise new K and V rows and scatter them into the paged
// cache that the decode and prefill attention kernels read.
//
// Semantics (vLLM's reshape_and_cache_flash with an fp8 per-tensor cache, the kernel
// reshape_and_cache_kernel_flash the reference's engine runs before every attention call:
// profiling/prof_h4mv.txt:9, profiling/prof_prefill.txt:23):
//   for token i with s = slot_mapping[i] >= 0 (negative slots are padding and write nothing),
//   block = s / block_size, slot = s % block_size, and every (head, d):
//     cache[block, slot, head, d] = e4m3fn( float(x[i, head, d]) / scale )
//   with the division in fp32 (correctly rounded), round to nearest even, finite values and
//   +-inf saturated to +-448, NaN kept as NaN with its sign.
//
// gfx950 design: pure streaming (2 bytes read and 1 byte written per element).  One thread
// handles 16 consecutive elements of one head of K or V: two 16-byte loads, 16 fp32 divisions by
// the device-side scale, v_cvt_pk_fp8_f32 on the clamped quotients (round to nearest even), one
// 16-byte store (two 8-byte stores for a V cache only 8-byte aligned).  A grid-stride loop over
// (token, tensor, 16-element chunk) items keeps every lane busy for any head count.
#include "fp8kv_common.h"
#include "fp8kv_status.h"

namespace fp8kv {
namespace cache_write_detail {

struct Params {
    const uint16_t* key;        // bf16 bits
    const uint16_t* value;
    uint8_t* kc;
    uint8_t* vc;
    int64_t key_stride, value_stride;           // elements per token row
    int64_t sk0, sk1, sk2, sv0, sv1, sv2;       // bytes
    const int64_t* slots;
    const float* k_scale;
    const float* v_scale;
    int num_tokens, head_size, chunks, pblk, pshift;   // chunks: 16-element chunks per token and tensor
};

// e4m3fn code of a finite-or-not fp32 value: NaN -> 0x7F with the sign bit; everything else is
// clamped to +-448 (exact) and converted with round to nearest even.
__device__ __forceinline__ uint32_t e4m3_pair(float a, float b)
{
    const float ca = __builtin_fminf(__builtin_fmaxf(a, -448.f), 448.f);
    const float cb = __builtin_fminf(__builtin_fmaxf(b, -448.f), 448.f);
    uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false) & 0xFFFFu;
    if (a != a) r = (r & 0xFF00u) | 0x7Fu | ((__float_as_uint(a) >> 24) & 0x80u);
    if (b != b) r = (r & 0x00FFu) | 0x7F00u | ((__float_as_uint(b) >> 16) & 0x8000u);
    return r;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) { return __uint_as_float(bits << 16); }

template <bool V16>
__global__ void __launch_bounds__(256)
cache_write_kernel(Params P)
{
    const int per_tok = 2 * P.chunks;
    const int n_items = P.num_tokens * per_tok;
    for (int it = blockIdx.x * 256 + threadIdx.x; it < n_items; it += gridDim.x * 256) {
        const int tok = it / per_tok;
        const int r = it - tok * per_tok;
        const bool isv = r >= P.chunks;
        const int e = (isv ? r - P.chunks : r) * 16;
        const int64_t s = P.slots[tok];
        if (s < 0) continue;
        const int head = e / P.head_size;
        const int d0 = e - head * P.head_size;
        const uint16_t* src = isv ? P.value + (int64_t)tok * P.value_stride + e
                                  : P.key + (int64_t)tok * P.key_stride + e;
        const u32x4_t x0 = load_16(src);
        const u32x4_t x1 = load_16(src + 8);
        const float scale = isv ? P.v_scale[0] : P.k_scale[0];
        u32x4_t w;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4_t& x = k < 2 ? x0 : x1;
            const uint32_t lo = x[2 * (k & 1)], hi = x[2 * (k & 1) + 1];
            const float f0 = bf16_bits_to_f32(lo & 0xFFFFu) / scale;
            const float f1 = bf16_bits_to_f32(lo >> 16) / scale;
            const float f2 = bf16_bits_to_f32(hi & 0xFFFFu) / scale;
            const float f3 = bf16_bits_to_f32(hi >> 16) / scale;
            w[k] = e4m3_pair(f0, f1) | (e4m3_pair(f2, f3) << 16);
        }
        const int64_t blk = s >> P.pshift;
        const int64_t slot = s & (P.pblk - 1);
        uint8_t* dst = isv ? P.vc + blk * P.sv0 + slot * P.sv1 + (int64_t)head * P.sv2 + d0
                           : P.kc + blk * P.sk0 + slot * P.sk1 + (int64_t)head * P.sk2 + d0;
        if (V16 || !isv) {
            *reinterpret_cast<u32x4_t*>(dst) = w;
        } else {
            *reinterpret_cast<u32x2_t*>(dst) = (u32x2_t){w[0], w[1]};
            *reinterpret_cast<u32x2_t*>(dst + 8) = (u32x2_t){w[2], w[3]};
        }
    }
}

}  // namespace cache_write_detail
}  // namespace fp8kv

using namespace fp8kv;
using namespace fp8kv::cache_write_detail;

extern "C" int fp8kv_cache_write(const void* key, int64_t key_row_stride,
                                 const void* value, int64_t value_row_stride,
                                 void* k_cache, void* v_cache,
                                 int64_t sk0, int64_t sk1, int64_t sk2,
                                 int64_t sv0, int64_t sv1, int64_t sv2,
                                 const int64_t* slot_mapping,
                                 const float* k_scale, const float* v_scale,
                                 int num_tokens, int num_kv_heads, int head_size, int block_size,
                                 void* stream)
{
    if (!key || !value || !k_cache || !v_cache || !slot_mapping || !k_scale || !v_scale)
        return FP8KV_ERR_ARG;
    if (num_tokens < 0 || num_kv_heads < 1 || head_size < 1 || block_size < 1) return FP8KV_ERR_ARG;
    if (num_tokens == 0) return FP8KV_OK;
    if (head_size % 16 != 0 || (block_size & (block_size - 1)) != 0) return FP8KV_ERR_SHAPE;
    const int64_t chunks = (int64_t)num_kv_heads * head_size / 16;
    if ((int64_t)num_tokens * 2 * chunks >= ((int64_t)1 << 31)) return FP8KV_ERR_SHAPE;
    if (!aligned(key, 16) || !aligned(value, 16) || (key_row_stride & 7) || (value_row_stride & 7))
        return FP8KV_ERR_ALIGN;
    if (key_row_stride < chunks * 16 || value_row_stride < chunks * 16) return FP8KV_ERR_ARG;
    if (!aligned(k_cache, 16) || ((sk0 | sk1 | sk2) & 15)) return FP8KV_ERR_ALIGN;
    if (!aligned(v_cache, 8) || ((sv0 | sv1 | sv2) & 7)) return FP8KV_ERR_ALIGN;
    const bool v16 = aligned(v_cache, 16) && ((sv0 | sv1 | sv2) & 15) == 0;

    Params P;
    P.key = static_cast<const uint16_t*>(key);
    P.value = static_cast<const uint16_t*>(value);
    P.kc = static_cast<uint8_t*>(k_cache);
    P.vc = static_cast<uint8_t*>(v_cache);
    P.key_stride = key_row_stride;
    P.value_stride = value_row_stride;
    P.sk0 = sk0; P.sk1 = sk1; P.sk2 = sk2;
    P.sv0 = sv0; P.sv1 = sv1; P.sv2 = sv2;
    P.slots = slot_mapping;
    P.k_scale = k_scale;
    P.v_scale = v_scale;
    P.num_tokens = num_tokens;
    P.head_size = head_size;
    P.chunks = (int)chunks;
    P.pblk = block_size;
    P.pshift = __builtin_ctz((unsigned)block_size);

    const int64_t items = (int64_t)num_tokens * 2 * chunks;
    int64_t blocks = (items + 255) / 256;
    if (blocks > 4096) blocks = 4096;                 // grid-stride beyond: 16 waves per CU
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    begin_launch();
    if (v16)
        launch_kernel(cache_write_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, st, P);
    else
        launch_kernel(cache_write_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st, P);
    return finish_launch();
}
