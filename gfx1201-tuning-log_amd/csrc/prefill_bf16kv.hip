// Paged causal prefill attention over bf16 K/V caches for gfx950: the reference's K_FP8 = False
// branch of its prefill (vllm-fp8kv/fp8kv_prefill.py:57-60,77-82,117, dispatched by cache dtype at
// :143).  For bf16 caches the reference ignores k_scale and v_scale: S = (q . k) * sm_scale and
// out = softmax(S) . V, with the probabilities rounded to bf16 before P.V (:88,114).
//
// gfx950 design (the engine's caches are fp8, so this path serves callers of the reference's
// run() with bf16 caches; it uses the decode kernel's register-direct chunk loads rather than the
// fp8 prefill kernels' LDS tile rings):
//   * one workgroup per (16-token block, kv head, group of up to 16 query heads, sequence); each
//     wave owns two query heads of its block (one for MHA), i.e. two row-sets of 16 queries that
//     share every K/V load, and streams every key the block sees (q0 + 16 b + 16, capped at the
//     context) through kv_chunk: 32-key chunks straight into MFMA fragments, the next chunk's
//     block ids a round trip ahead;
//   * S^T = K . Q^T and O^T = V^T . P^T on v_mfma_f32_16x16x32_bf16 with the query token in
//     lane % 16 (the rescale is lane-local); the causal mask applies only to chunks that reach
//     past the block's first query position;
//   * the waves of a workgroup read the same K/V rows (L2 hits after the first), and no wave
//     waits for another: there is no LDS and no barrier.
#include "fp8kv_common.h"
#include "fp8kv_status.h"
#include "fp8kv_diag.h"
#include "attn_common.h"
#include "kv_chunk.h"

namespace fp8kv {
namespace prefill_b16_detail {

using namespace kv_chunk;

constexpr int kD = 128;
constexpr int kMaxGqa = 16;
constexpr int kWavesPerWG = 8;
constexpr int kNG = 2;                         // 16-token groups per chunk
constexpr float kLog2e = 1.4426950408889634f;

struct Params {
    const __bf16* q;
    const uint8_t* k;           // caches as bytes; strides below in bytes
    const uint8_t* v;
    __bf16* out;
    const int32_t* cu_q;        // [NS + 1] or null (single sequence: q0_host / qlen_host)
    const int32_t* seq_lens;    // [NS] total context of each sequence (new tokens included)
    const int32_t* bt;
    int64_t q_stride, o_stride, bt_stride;
    int64_t sk0, sk1, sk2, sv0, sv1, sv2;
    float sm_scale;
    int hkv, gqa, pblk, pshift;
    int n16_grid;               // token blocks per (sequence, kv head) the grid covers
    int q0_host, qlen_host;
};

template <int RS>
__global__ void __launch_bounds__(kWavesPerWG * 64)
prefill_bf16kv_kernel(Params P)
{
    constexpr int CH = 16 * kNG;
    const int lin = blockIdx.x, seq = blockIdx.z;
    const int kh = lin % P.hkv;
    const int rank = lin / P.hkv;                                  // longest causal rows first
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15;
    const int lp = lane >> 4;
    // query heads (within the kv head) g0 .. g0 + RS - 1 of this wave; past gqa: head g0 again,
    // computed and not stored
    const int g0 = (blockIdx.y * kWavesPerWG + wave) * RS;
    if (g0 >= P.gqa) return;                                       // no barriers: waves are independent

    int q_begin, qlen, q0;
    if (P.cu_q) {
        q_begin = P.cu_q[seq];
        qlen = P.cu_q[seq + 1] - q_begin;
        q0 = P.seq_lens[seq] - qlen;
    } else {
        q_begin = 0;
        qlen = P.qlen_host;
        q0 = P.q0_host;
    }
    const int n16 = (qlen + 15) >> 4;
    const int b = P.n16_grid - 1 - rank;
    if (b < 0 || b >= n16 || q0 < 0) return;
    const int qpos0 = q0 + 16 * b;                                 // the block's first query position
    const int k_hi = q0 + min(16 * b + 16, qlen);                  // keys [0, k_hi)
    const int tok = 16 * b + lr;
    const bool tok_ok = tok < qlen;
    const int qpos = q0 + tok;                                     // this lane's query sees keys <= qpos

    // Q^T fragments of this lane's query row (rows past qlen read the last row again; their
    // results are not stored): d = 16 lp + 0..15 and 64 + 16 lp + 0..15.
    u32x4_t qf[RS][4];
    WaveState st[RS];
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        const int g = g0 + j < P.gqa ? g0 + j : g0;
        const __bf16* qrow = P.q + (int64_t)(q_begin + (tok_ok ? tok : qlen - 1)) * P.q_stride +
                             (int64_t)(kh * P.gqa + g) * kD;
        qf[j][0] = load_16(qrow + 16 * lp);
        qf[j][1] = load_16(qrow + 16 * lp + 8);
        qf[j][2] = load_16(qrow + 64 + 16 * lp);
        qf[j][3] = load_16(qrow + 64 + 16 * lp + 8);
        st[j].m_run = neg_inf();
        st[j].l_run = 0.f;
#pragma unroll
        for (int n = 0; n < 8; ++n) st[j].o[n] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }
    const float qk_scale = P.sm_scale * kLog2e;

    const int32_t* btrow = P.bt + (int64_t)seq * P.bt_stride;
    const int last = (k_hi - 1) & ~15;
    const LaneOffsets lofs = lane_offsets<true>(P, lr, lp);
    // One chunk in flight; the next chunk's block ids go out before this chunk is consumed.  (Two
    // chunks in flight measured slower: 408 against 377 us at configs[3] with one head per wave,
    // and two heads per wave then spill.)
    ChunkIds<kNG> ia = load_chunk_ids<kNG>(P, btrow, 0, last);
    ChunkIds<kNG> ib = load_chunk_ids<kNG>(P, btrow, CH, last);
    ChunkRegs<kNG, true> ca;
    int c0 = 0;
    do {
        ids_ready(ia, ib);
        issue_chunk<kNG, true, true>(ca, P, lofs, ia, kh, c0, k_hi, last);
        ia = ib;
        if (c0 + 2 * CH < k_hi) ib = load_chunk_ids<kNG>(P, btrow, c0 + 2 * CH, last);
#pragma unroll
        for (int j = 0; j < RS; ++j)
            consume_chunk<kNG, true>(ca, st[j], qf[j], qk_scale, c0, qpos, c0 + CH - 1 > qpos0, k_hi, lp);
        c0 += CH;
    } while (c0 < k_hi);

    // o[n][i] is this lane's query at d = 32 lp + 8 i + n: one 16-byte store per i.
    float l[RS];
#pragma unroll
    for (int j = 0; j < RS; ++j) l[j] = sum_xor16_32(st[j].l_run);
    if (!tok_ok) return;
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        if (g0 + j >= P.gqa) break;
        const float f = l[j] > 0.f ? 1.f / l[j] : 0.f;
        __bf16* orow = P.out + (int64_t)(q_begin + tok) * P.o_stride + (int64_t)(kh * P.gqa + g0 + j) * kD + 32 * lp;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u32x4_t w;
            w[0] = pack_bf16x2(st[j].o[0][i] * f, st[j].o[1][i] * f);
            w[1] = pack_bf16x2(st[j].o[2][i] * f, st[j].o[3][i] * f);
            w[2] = pack_bf16x2(st[j].o[4][i] * f, st[j].o[5][i] * f);
            w[3] = pack_bf16x2(st[j].o[6][i] * f, st[j].o[7][i] * f);
            *reinterpret_cast<u32x4_t*>(orow + 8 * i) = w;
        }
    }
}

// Argument checks shared by both entry points; cache strides are converted to bytes in P.
int setup(Params& P, const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
          int64_t sk0, int64_t sk1, int64_t sk2, int64_t sv0, int64_t sv1, int64_t sv2, void* out,
          int64_t out_row_stride, const int32_t* block_table, int64_t bt_stride, float sm_scale,
          int num_q_heads, int num_kv_heads, int head_size, int block_size)
{
    if (!q || !k_cache || !v_cache || !out || !block_table) return FP8KV_ERR_ARG;
    if (num_kv_heads < 1 || num_q_heads < 1 || block_size < 1 || bt_stride < 0) return FP8KV_ERR_ARG;
    if (num_kv_heads > 65535) return FP8KV_ERR_SHAPE;
    if (head_size != kD || num_q_heads % num_kv_heads != 0) return FP8KV_ERR_SHAPE;
    if (num_q_heads / num_kv_heads > kMaxGqa) return FP8KV_ERR_SHAPE;
    if (block_size < 16 || (block_size & (block_size - 1)) != 0) return FP8KV_ERR_SHAPE;
    // K and V rows are read with 16-byte loads (8 bf16), q with 16-byte loads, out with 16-byte stores.
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(q, 16) || !aligned(out, 16))
        return FP8KV_ERR_ALIGN;
    if ((sk0 | sk1 | sk2 | sv0 | sv1 | sv2) & 7) return FP8KV_ERR_ALIGN;
    if ((q_row_stride & 7) || (out_row_stride & 7)) return FP8KV_ERR_ALIGN;
    // Per-lane offsets within a 16-token group are 32-bit.
    if (sk1 < 0 || sv1 < 0 || sk1 > ((int64_t)1 << 25) || sv1 > ((int64_t)1 << 25)) return FP8KV_ERR_SHAPE;
    P.q = static_cast<const __bf16*>(q);
    P.k = static_cast<const uint8_t*>(k_cache);
    P.v = static_cast<const uint8_t*>(v_cache);
    P.out = static_cast<__bf16*>(out);
    P.cu_q = nullptr;
    P.seq_lens = nullptr;
    P.bt = block_table;
    P.q_stride = q_row_stride;
    P.o_stride = out_row_stride;
    P.bt_stride = bt_stride;
    P.sk0 = 2 * sk0; P.sk1 = 2 * sk1; P.sk2 = 2 * sk2;
    P.sv0 = 2 * sv0; P.sv1 = 2 * sv1; P.sv2 = 2 * sv2;
    P.sm_scale = sm_scale;
    P.hkv = num_kv_heads;
    P.gqa = num_q_heads / num_kv_heads;
    P.pblk = block_size;
    P.pshift = __builtin_ctz((unsigned)block_size);
    P.n16_grid = 0;
    P.q0_host = 0;
    P.qlen_host = 0;
    return FP8KV_OK;
}

// Heads per wave: two wherever GQA > 1, so both row-sets use one set of K/V loads (configs[3]:
// 222 against 377 us with one head per wave; 1024 over 1024: 98.7 against 122.6 us); one for MHA.
thread_local int g_rs_override = 0;

int launch(Params& P, int num_seqs, int max_query_len, hipStream_t stream)
{
    P.n16_grid = (max_query_len + 15) / 16;
    const int rs = g_rs_override ? g_rs_override : (P.gqa > 1 ? 2 : 1);
    const int wave_heads = kWavesPerWG * rs;
    const int groups = (P.gqa + wave_heads - 1) / wave_heads;
    const int waves_needed = (P.gqa + rs - 1) / rs;
    const int waves = waves_needed < kWavesPerWG ? waves_needed : kWavesPerWG;
    const dim3 grid((unsigned)(P.n16_grid * P.hkv), (unsigned)groups, (unsigned)num_seqs);
    begin_launch();
    if (rs == 2)
        launch_kernel(prefill_bf16kv_kernel<2>, grid, dim3(64 * waves), 0, stream, P);
    else
        launch_kernel(prefill_bf16kv_kernel<1>, grid, dim3(64 * waves), 0, stream, P);
    return finish_launch();
}

}  // namespace prefill_b16_detail
}  // namespace fp8kv

using namespace fp8kv;
using namespace fp8kv::prefill_b16_detail;

extern "C" int fp8kv_prefill_attn_bf16(const void* q, int64_t q_row_stride,
                                       const void* k_cache, const void* v_cache,
                                       int64_t sk0, int64_t sk1, int64_t sk2,
                                       int64_t sv0, int64_t sv1, int64_t sv2,
                                       void* out, int64_t out_row_stride,
                                       const int32_t* block_table, int64_t bt_stride,
                                       const float* k_scale, const float* v_scale, float sm_scale,
                                       int num_q_heads, int num_kv_heads, int head_size, int block_size,
                                       int q0, int qlen, void* stream)
{
    (void)k_scale;
    (void)v_scale;
    Params P;
    const int st = setup(P, q, q_row_stride, k_cache, v_cache, sk0, sk1, sk2, sv0, sv1, sv2, out,
                         out_row_stride, block_table, bt_stride, sm_scale, num_q_heads, num_kv_heads,
                         head_size, block_size);
    if (st != FP8KV_OK) return st;
    if (q0 < 0 || qlen < 0) return FP8KV_ERR_ARG;
    if (qlen == 0) return FP8KV_OK;
    if ((int64_t)(qlen + 15) / 16 * num_kv_heads > 0x7fffffff) return FP8KV_ERR_SHAPE;
    P.q0_host = q0;
    P.qlen_host = qlen;
    return launch(P, 1, qlen, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int fp8kv_prefill_attn_varlen_bf16(const void* q, int64_t q_row_stride,
                                              const void* k_cache, const void* v_cache,
                                              int64_t sk0, int64_t sk1, int64_t sk2,
                                              int64_t sv0, int64_t sv1, int64_t sv2,
                                              void* out, int64_t out_row_stride,
                                              const int32_t* cu_seqlens_q, const int32_t* seq_lens,
                                              const int32_t* block_table, int64_t bt_stride,
                                              const float* k_scale, const float* v_scale, float sm_scale,
                                              int num_seqs, int num_q_heads, int num_kv_heads,
                                              int head_size, int block_size, int max_query_len,
                                              void* stream)
{
    (void)k_scale;
    (void)v_scale;
    Params P;
    const int st = setup(P, q, q_row_stride, k_cache, v_cache, sk0, sk1, sk2, sv0, sv1, sv2, out,
                         out_row_stride, block_table, bt_stride, sm_scale, num_q_heads, num_kv_heads,
                         head_size, block_size);
    if (st != FP8KV_OK) return st;
    if (!cu_seqlens_q || !seq_lens || num_seqs < 1 || max_query_len < 0) return FP8KV_ERR_ARG;
    if (num_seqs > 65535) return FP8KV_ERR_SHAPE;
    if (max_query_len == 0) return FP8KV_OK;
    if ((int64_t)(max_query_len + 15) / 16 * num_kv_heads > 0x7fffffff) return FP8KV_ERR_SHAPE;
    P.cu_q = cu_seqlens_q;
    P.seq_lens = seq_lens;
    return launch(P, num_seqs, max_query_len, reinterpret_cast<hipStream_t>(stream));
}

// Sweeps and tests: query heads per wave (1 or 2); any other value restores the default.
extern "C" void fp8kv_prefill_bf16_tune(int heads_per_wave)
{
    g_rs_override = (heads_per_wave == 1 || heads_per_wave == 2) ? heads_per_wave : 0;
}
