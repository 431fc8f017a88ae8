// Paged fp8-e4m3 KV causal prefill attention for gfx950 (bf16 MFMA), single-sequence and varlen.
//
// Reference semantics: vllm-fp8kv/fp8kv_prefill.py:31-121 (kernel) and :124-144 (launch):
//   * query i of a sequence is token q0 + i and sees keys t <= q0 + i (fp8kv_prefill.py:108),
//     where the sequence's context is q0 + qlen tokens held in the paged fp8 cache;
//   * S = (q . k) * sm_scale * k_scale in the exp2 domain (fp8kv_prefill.py:57-60), fp32 softmax,
//     probabilities rounded to bf16 before P.V (:88, :114), out = acc * v_scale / l in bf16 (:117-121);
//   * the reference handles one sequence and reads block-table row 0 only (:68); here each
//     sequence of a varlen batch reads its own row, and a single-sequence call takes q0 / qlen from
//     the host exactly like fp8kv_prefill.run(q0, qlen).
//   * rows are (token, head) pairs packed per KV head; the reference kernel's row packing breaks
//     when GQA does not divide its BM (its rows 60-63 alias the next tile at GQA 6), so this kernel
//     gives every 16-row MFMA set a single head and 16 consecutive tokens instead.
//
// gfx950 design:
//   * grid (token blocks, HKV, sequences), token blocks in reverse order so the longest causal rows
//     start first; a workgroup (4 waves) owns 16 * nb query tokens of all GQA heads of one KV
//     head: nb * GQA row-sets of 16 rows, row-set r = (head r % GQA, token block r / GQA), wave w
//     taking r = w, w + 4, ... (RS row-sets at most).
//   * keys are walked in 32-key tiles; each tile is loaded once per workgroup from the paged fp8
//     cache (global -> registers one tile ahead), converted to bf16 and written to LDS in the
//     layouts the MFMA fragments are read in:
//       K  [32 keys][128 d] bf16, 16-byte chunk c of key r stored at chunk c ^ (r & 15), so the 16
//          keys of one fragment read hit distinct banks;
//       V^T [128 d][32 keys] bf16 (rows padded to 80 bytes), keys permuted into the k-slot order of
//          the P^T fragments, transposed in registers during the conversion.
//     LDS is double-buffered: one barrier per tile.
//   * S^T = K . Q^T and O^T = V^T . P^T on v_mfma_f32_16x16x32_bf16 (the decode kernel's
//     formulation): the query token stays in lane % 16 in S and O, so the online-softmax rescale is
//     lane-local; K and V fragments are read once per tile and shared by the wave's row-sets.
//   * the causal mask is applied only on diagonal tiles; tiles entirely above a row-set's diagonal
//     are skipped for that row-set.
#include "fp8kv_common.h"
#include "fp8kv_status.h"
#include "attn_common.h"

namespace fp8kv {
namespace prefill_detail {

constexpr int kD = 128;
constexpr int kBN = 32;                       // keys per tile
constexpr int kWaves = 4;
constexpr int kT = kWaves * 64;
constexpr int kMaxGqa = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kKRow = 256;                    // bytes per bf16 K row
constexpr int kKTile = kBN * kKRow;           // 8 KB
constexpr int kVRow = 80;                     // bytes per V^T row: 32 bf16 keys + 16 bytes of pad
constexpr int kVTile = kD * kVRow;            // 10 KB
constexpr int kBuf = kKTile + kVTile;

struct Params {
    const __bf16* q;
    const uint8_t* k;
    const uint8_t* v;
    __bf16* out;
    const int32_t* cu_q;        // [NS + 1] or null (single sequence: q0_host / qlen_host)
    const int32_t* seq_lens;    // [NS] total context of each sequence (new tokens included)
    const int32_t* bt;
    const float* k_scale;
    const float* v_scale;
    int64_t q_stride, o_stride, bt_stride;
    int64_t sk0, sk1, sk2, sv0, sv1, sv2;
    float sm_scale;
    int hkv, gqa, pblk, nb;
    int q0_host, qlen_host;
};

// Fragment chunk (16 bytes = 8 d) read by k-part p for QK step s: d = 16p + 8s (s < 2) and
// 64 + 16p + 8(s - 2) (s >= 2), the same d order the Q^T fragments use.
__device__ __forceinline__ int k_chunk(int s, int p) { return (s < 2 ? 0 : 8) + 2 * p + (s & 1); }

// Staging registers of one tile: thread tid converts K bytes 16 (tid & 7) .. +15 of key tid >> 3;
// threads of wave 0 also handle V for lane (c, p) = (lane % 16, lane / 16): 8 bytes d = 8c .. 8c+7
// of the tile's k-slot tokens T_p[j] = 4p + j (j < 4), 16 + 4p + (j - 4) (j >= 4).
struct Stage {
    u32x4_t kr;
    u32x2_t vr[8];
};

// Issue the global loads of tile k0 (keys >= k_hi zero-filled).  b0 / b1: cache blocks of the
// tile's two 16-key groups.
__device__ __forceinline__ void stage_load(Stage& sg, const Params& P, int kh, int k0, int k_hi,
                                           int64_t b0, int64_t b1, int tid)
{
    const int kr = tid >> 3, j8 = tid & 7;
    {
        const int tok = k0 + kr;
        const int64_t blk = (kr >> 4) ? b1 : b0;
        const int slot = tok % P.pblk;
        const uint8_t* src = P.k + blk * P.sk0 + (int64_t)slot * P.sk1 + (int64_t)kh * P.sk2 + 16 * j8;
        const u32x4_t z4 = {0u, 0u, 0u, 0u};
        sg.kr = tok < k_hi ? load_nt_16(src) : z4;
    }
    if (tid < 64) {
        const int c = tid & 15, p = tid >> 4;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int kk = (j < 4 ? 0 : 16) + 4 * p + (j & 3);
            const int tok = k0 + kk;
            const int64_t blk = j < 4 ? b0 : b1;
            const int slot = tok % P.pblk;
            const uint8_t* src = P.v + blk * P.sv0 + (int64_t)slot * P.sv1 + (int64_t)kh * P.sv2 + 8 * c;
            const u32x2_t z2 = {0u, 0u};
            sg.vr[j] = tok < k_hi ? __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(src)) : z2;
        }
    }
}

// Convert the staged tile to bf16 and write it to LDS buffer `buf` (layouts above).
__device__ __forceinline__ void stage_store(const Stage& sg, unsigned char* buf, int tid)
{
    const int kr = tid >> 3, j8 = tid & 7;
    const int sw = kr & 15;
    unsigned char* krow = buf + kr * kKRow;
    *reinterpret_cast<bf16x8_t*>(krow + 16 * ((2 * j8) ^ sw)) = fp8x8_to_bf16x8(sg.kr[0], sg.kr[1]);
    *reinterpret_cast<bf16x8_t*>(krow + 16 * ((2 * j8 + 1) ^ sw)) = fp8x8_to_bf16x8(sg.kr[2], sg.kr[3]);
    if (tid < 64) {
        const int c = tid & 15, p = tid >> 4;
        u32x4_t va[8];
        v_fragments(sg.vr, va);
        unsigned char* vt = buf + kKTile;
#pragma unroll
        for (int n = 0; n < 8; ++n)
            *reinterpret_cast<u32x4_t*>(vt + (16 * n + c) * kVRow + 16 * p) = va[n];
    }
}

// Block ids of the two 16-key groups of tile k0, one vector load (lanes alternate groups); the
// caller reads lanes 0 and 1 with readlane.
__device__ __forceinline__ int load_tile_blocks(const Params& P, const int32_t* btrow, int k0, int k_hi, int lane)
{
    const int t = k0 + 16 * (lane & 1);
    return t < k_hi ? btrow[t / P.pblk] : 0;
}

template <int RS>
__global__ void __launch_bounds__(kT)
prefill_kernel(Params P)
{
    __shared__ __align__(16) unsigned char lds[2 * kBuf];

    const int kh = blockIdx.y, seq = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;
    const int lp = lane >> 4;
    const int gqa = P.gqa;

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
    const int BT = 16 * P.nb;
    const int ntb = (qlen + BT - 1) / BT;
    const int tb = (int)gridDim.x - 1 - (int)blockIdx.x;      // longest causal rows first
    if (tb >= ntb || q0 < 0) return;                          // whole workgroup, before any barrier
    const int t0 = tb * BT;
    const int k_hi = q0 + min(t0 + BT, qlen);                 // keys [0, k_hi)
    const int32_t* btrow = P.bt + (int64_t)seq * P.bt_stride;
    const int nrs = P.nb * gqa;

    // ---- Q^T fragments of the wave's row-sets ---------------------------------------------------
    u32x4_t qf[RS][4];
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        const int r = wave + kWaves * j;
        const int g = r % gqa, b = r / gqa;
        const int tok = t0 + 16 * b + lr;
        const bool ok = r < nrs && tok < qlen;
        const u32x4_t zero = {0u, 0u, 0u, 0u};
        const __bf16* qrow = P.q + (int64_t)(q_begin + (ok ? tok : 0)) * P.q_stride +
                             (int64_t)(kh * gqa + (ok ? g : 0)) * kD;
        qf[j][0] = ok ? load_16(qrow + 16 * lp) : zero;
        qf[j][1] = ok ? load_16(qrow + 16 * lp + 8) : zero;
        qf[j][2] = ok ? load_16(qrow + 64 + 16 * lp) : zero;
        qf[j][3] = ok ? load_16(qrow + 64 + 16 * lp + 8) : zero;
    }
    const float qk_scale = P.sm_scale * P.k_scale[0] * kLog2e;
    const float vs = P.v_scale[0];

    float m_run[RS], l_run[RS];
    f32x4_t o[RS][8];
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        m_run[j] = neg_inf();
        l_run[j] = 0.f;
#pragma unroll
        for (int n = 0; n < 8; ++n) o[j][n] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }

    // ---- tile pipeline: block ids two tiles ahead, K/V bytes one tile ahead ---------------------
    const int ntiles = (k_hi + kBN - 1) / kBN;
    Stage sg;
    {
        const int bt0 = load_tile_blocks(P, btrow, 0, k_hi, lane);
        stage_load(sg, P, kh, 0, k_hi, __builtin_amdgcn_readlane(bt0, 0), __builtin_amdgcn_readlane(bt0, 1), tid);
    }
    int bt_next = load_tile_blocks(P, btrow, kBN, k_hi, lane);

    for (int it = 0; it < ntiles; ++it) {
        const int k0 = it * kBN;
        unsigned char* buf = lds + (it & 1) * kBuf;
        stage_store(sg, buf, tid);
        __syncthreads();
        if (it + 1 < ntiles) {
            const int64_t b0 = __builtin_amdgcn_readlane(bt_next, 0);
            const int64_t b1 = __builtin_amdgcn_readlane(bt_next, 1);
            bt_next = load_tile_blocks(P, btrow, k0 + 2 * kBN, k_hi, lane);
            stage_load(sg, P, kh, k0 + kBN, k_hi, b0, b1, tid);
        }

        // K fragments (2 key groups x 4 d steps) and V^T fragments (8 d blocks), shared by the
        // wave's row-sets.
        u32x4_t kf[2][4];
#pragma unroll
        for (int kg = 0; kg < 2; ++kg)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                kf[kg][s] = *reinterpret_cast<const u32x4_t*>(buf + (16 * kg + lr) * kKRow +
                                                              16 * (k_chunk(s, lp) ^ lr));
        u32x4_t vf[8];
#pragma unroll
        for (int n = 0; n < 8; ++n)
            vf[n] = *reinterpret_cast<const u32x4_t*>(buf + kKTile + (16 * n + lr) * kVRow + 16 * lp);

#pragma unroll
        for (int j = 0; j < RS; ++j) {
            const int r = wave + kWaves * j;
            if (r >= nrs) continue;
            const int qpos0 = q0 + t0 + 16 * (r / gqa);           // position of the row-set's first query
            if (k0 > qpos0 + 15) continue;                         // tile above the diagonal
            f32x4_t s[2];
#pragma unroll
            for (int kg = 0; kg < 2; ++kg) {
                f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    acc = mfma16x16x32_bf16(as_bf16x8(kf[kg][st]), as_bf16x8(qf[j][st]), acc);
                s[kg] = acc;
            }
            float mc = neg_inf();
            if (k0 + kBN - 1 <= qpos0) {
#pragma unroll
                for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        s[kg][i] *= qk_scale;
                        mc = fmaxf(mc, s[kg][i]);
                    }
            } else {
                const int qpos = qpos0 + lr;
#pragma unroll
                for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int key = k0 + 16 * kg + 4 * lp + i;
                        const float x = key <= qpos ? s[kg][i] * qk_scale : neg_inf();
                        s[kg][i] = x;
                        mc = fmaxf(mc, x);
                    }
            }
            mc = fmaxf(mc, __shfl_xor(mc, 16));
            mc = fmaxf(mc, __shfl_xor(mc, 32));
            const float m_new = fmaxf(m_run[j], mc);
            const float m_use = m_new == neg_inf() ? 0.f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run[j] - m_use);
            float psum = 0.f;
#pragma unroll
            for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pv = __builtin_amdgcn_exp2f(s[kg][i] - m_use);
                    s[kg][i] = pv;
                    psum += pv;
                }
            l_run[j] = l_run[j] * alpha + psum;
            m_run[j] = m_new;
            u32x4_t pb;
            pb[0] = pack_bf16x2(s[0][0], s[0][1]);
            pb[1] = pack_bf16x2(s[0][2], s[0][3]);
            pb[2] = pack_bf16x2(s[1][0], s[1][1]);
            pb[3] = pack_bf16x2(s[1][2], s[1][3]);
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                o[j][n] *= alpha;
                o[j][n] = mfma16x16x32_bf16(as_bf16x8(vf[n]), as_bf16x8(pb), o[j][n]);
            }
        }
    }

    // ---- normalise and store: lane (q, p) holds d = 32p + 8i + n of query row q ------------------
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        const int r = wave + kWaves * j;
        float l = l_run[j];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        if (r >= nrs) continue;
        const int g = r % gqa, b = r / gqa;
        const int tok = t0 + 16 * b + lr;
        if (tok >= qlen) continue;
        const float f = l > 0.f ? vs / l : 0.f;
        __bf16* orow = P.out + (int64_t)(q_begin + tok) * P.o_stride + (int64_t)(kh * gqa + g) * kD + 32 * lp;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u32x4_t w;
            w[0] = pack_bf16x2(o[j][0][i] * f, o[j][1][i] * f);
            w[1] = pack_bf16x2(o[j][2][i] * f, o[j][3][i] * f);
            w[2] = pack_bf16x2(o[j][4][i] * f, o[j][5][i] * f);
            w[3] = pack_bf16x2(o[j][6][i] * f, o[j][7][i] * f);
            *reinterpret_cast<u32x4_t*>(orow + 8 * i) = w;
        }
    }
}

// Token blocks of 16 per workgroup and row-sets per wave for a GQA: nb * gqa row-sets over 4 waves.
inline void plan(int gqa, int& nb, int& rs)
{
    nb = 12 / gqa;
    if (nb < 1) nb = 1;
    if (nb > 4) nb = 4;
    rs = (nb * gqa + kWaves - 1) / kWaves;
}

int launch(const Params& P0, int num_seqs, int max_query_len, hipStream_t stream)
{
    Params P = P0;
    int nb, rs;
    plan(P.gqa, nb, rs);
    P.nb = nb;
    const int bt = 16 * nb;
    const unsigned gx = (unsigned)((max_query_len + bt - 1) / bt);
    if (gx == 0) return FP8KV_OK;
    const dim3 grid(gx, (unsigned)P.hkv, (unsigned)num_seqs);
    switch (rs) {
        case 1: hipLaunchKernelGGL(prefill_kernel<1>, grid, dim3(kT), 0, stream, P); break;
        case 2: hipLaunchKernelGGL(prefill_kernel<2>, grid, dim3(kT), 0, stream, P); break;
        case 3: hipLaunchKernelGGL(prefill_kernel<3>, grid, dim3(kT), 0, stream, P); break;
        default: hipLaunchKernelGGL(prefill_kernel<4>, grid, dim3(kT), 0, stream, P); break;
    }
    return finish_launch();
}

int check_common(const void* q, const void* k_cache, const void* v_cache, void* out,
                 int64_t q_row_stride, int64_t sk0, int64_t sk1, int64_t sk2, int64_t sv0,
                 int64_t sv1, int64_t sv2, const int32_t* block_table, int64_t bt_stride,
                 const float* k_scale, const float* v_scale, int num_q_heads, int num_kv_heads,
                 int head_size, int block_size, int64_t out_row_stride)
{
    if (!q || !k_cache || !v_cache || !out || !block_table || !k_scale || !v_scale) return FP8KV_ERR_ARG;
    if (num_kv_heads < 1 || num_q_heads < 1 || block_size < 1 || bt_stride < 0) return FP8KV_ERR_ARG;
    if (num_kv_heads > 65535) return FP8KV_ERR_SHAPE;
    if (head_size != kD || num_q_heads % num_kv_heads != 0) return FP8KV_ERR_SHAPE;
    if (num_q_heads / num_kv_heads > kMaxGqa || (block_size % 16) != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(k_cache, 16) || !aligned(v_cache, 8) || !aligned(q, 16) || !aligned(out, 16))
        return FP8KV_ERR_ALIGN;
    if ((sk0 | sk1 | sk2) & 15) return FP8KV_ERR_ALIGN;
    if ((sv0 | sv1 | sv2) & 7) return FP8KV_ERR_ALIGN;
    if ((q_row_stride & 7) || (out_row_stride & 7)) return FP8KV_ERR_ALIGN;
    return FP8KV_OK;
}

Params make_params(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                   int64_t sk0, int64_t sk1, int64_t sk2, int64_t sv0, int64_t sv1, int64_t sv2,
                   void* out, int64_t out_row_stride, const int32_t* block_table, int64_t bt_stride,
                   const float* k_scale, const float* v_scale, float sm_scale, int num_q_heads,
                   int num_kv_heads, int block_size)
{
    Params P;
    P.q = static_cast<const __bf16*>(q);
    P.k = static_cast<const uint8_t*>(k_cache);
    P.v = static_cast<const uint8_t*>(v_cache);
    P.out = static_cast<__bf16*>(out);
    P.cu_q = nullptr;
    P.seq_lens = nullptr;
    P.bt = block_table;
    P.k_scale = k_scale;
    P.v_scale = v_scale;
    P.q_stride = q_row_stride;
    P.o_stride = out_row_stride;
    P.bt_stride = bt_stride;
    P.sk0 = sk0; P.sk1 = sk1; P.sk2 = sk2;
    P.sv0 = sv0; P.sv1 = sv1; P.sv2 = sv2;
    P.sm_scale = sm_scale;
    P.hkv = num_kv_heads;
    P.gqa = num_q_heads / num_kv_heads;
    P.pblk = block_size;
    P.nb = 1;
    P.q0_host = 0;
    P.qlen_host = 0;
    return P;
}

}  // namespace prefill_detail
}  // namespace fp8kv

using namespace fp8kv;
using namespace fp8kv::prefill_detail;

extern "C" int fp8kv_prefill_attn(const void* q, int64_t q_row_stride,
                                  const void* k_cache, const void* v_cache,
                                  int64_t sk0, int64_t sk1, int64_t sk2,
                                  int64_t sv0, int64_t sv1, int64_t sv2,
                                  void* out, int64_t out_row_stride,
                                  const int32_t* block_table, int64_t bt_stride,
                                  const float* k_scale, const float* v_scale, float sm_scale,
                                  int num_q_heads, int num_kv_heads, int head_size, int block_size,
                                  int q0, int qlen, void* stream)
{
    const int st = check_common(q, k_cache, v_cache, out, q_row_stride, sk0, sk1, sk2, sv0, sv1, sv2,
                                block_table, bt_stride, k_scale, v_scale, num_q_heads, num_kv_heads,
                                head_size, block_size, out_row_stride);
    if (st != FP8KV_OK) return st;
    if (q0 < 0 || qlen < 0) return FP8KV_ERR_ARG;
    if (qlen == 0) return FP8KV_OK;
    Params P = make_params(q, q_row_stride, k_cache, v_cache, sk0, sk1, sk2, sv0, sv1, sv2, out,
                           out_row_stride, block_table, bt_stride, k_scale, v_scale, sm_scale,
                           num_q_heads, num_kv_heads, block_size);
    P.q0_host = q0;
    P.qlen_host = qlen;
    return launch(P, 1, qlen, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int fp8kv_prefill_attn_varlen(const void* q, int64_t q_row_stride,
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
    const int st = check_common(q, k_cache, v_cache, out, q_row_stride, sk0, sk1, sk2, sv0, sv1, sv2,
                                block_table, bt_stride, k_scale, v_scale, num_q_heads, num_kv_heads,
                                head_size, block_size, out_row_stride);
    if (st != FP8KV_OK) return st;
    if (!cu_seqlens_q || !seq_lens || num_seqs < 1 || max_query_len < 0) return FP8KV_ERR_ARG;
    if (num_seqs > 65535) return FP8KV_ERR_SHAPE;
    if (max_query_len == 0) return FP8KV_OK;
    Params P = make_params(q, q_row_stride, k_cache, v_cache, sk0, sk1, sk2, sv0, sv1, sv2, out,
                           out_row_stride, block_table, bt_stride, k_scale, v_scale, sm_scale,
                           num_q_heads, num_kv_heads, block_size);
    P.cu_q = cu_seqlens_q;
    P.seq_lens = seq_lens;
    return launch(P, num_seqs, max_query_len, reinterpret_cast<hipStream_t>(stream));
}
