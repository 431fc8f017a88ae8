// Paged fp8-e4m3 KV decode attention for gfx950 (split-context flash decoding, one launch).
//
// Reference semantics: vllm-fp8kv/fp8kv_v3.py:3-113 (split kernel + merge kernel) and its launch
// wrapper fp8kv_v3.py:116-139:
//   * one query token per sequence, at row query_start_loc[s]; it attends to tokens [0, seq_len);
//   * token t lives in block block_table[s, t / block_size], slot t % block_size; K and V are read
//     through independent (block, slot, head) strides, so both the standalone [NB, PBLK, HKV, D]
//     cache and the engine's K|V-interleaved view work;
//   * fp8 -> bf16 is exact; S = (q . k) * sm_scale * k_scale (k_scale read on the device);
//     the probabilities are rounded to bf16 before P.V, the row sums use the fp32 values
//     (fp8kv_v3.py:67-74); the output is (sum_t p_t v_t) * v_scale / l in bf16 (fp8kv_v3.py:110-113).
//   * a sequence with no context writes zeros (the reference kernel writes NaN there).
//
// gfx950 design:
//   * grid (num_splits, HKV, NS); a workgroup of W waves owns a 16-aligned token span of its
//     (sequence, kv head); wave w takes chunks w, w + W, ... of the span, a chunk being NG
//     16-token groups.  Q and the scales are requested first; then, per chunk (DEPTH 1) or pair
//     of chunks (DEPTH 2), the block ids with scalar loads and every K and V byte with loads
//     issued back to back, the second chunk of a pair arriving while the first is computed.
//     The wave index is uniform and no load sits under a branch, so the compiler's vmcnt waits
//     are exact (each use waits for its own bytes only).
//   * S^T = K . Q^T on v_mfma_f32_16x16x32_bf16: A = 16 tokens x 32 d of K, B = Q^T with the GQA
//     query heads of the kv head in columns 0..GQA-1 (zero beyond).  Lane (r, p) = (lane % 16,
//     lane / 16) loads 16 bytes of token r at d = 16 p and at d = 64 + 16 p; the d order is
//     arbitrary for a reduction as long as the Q fragments use the same one.
//   * O^T = V^T . P^T on the same MFMA: A = V^T (16 d x 32 tokens), B = P^T (32 tokens x heads),
//     so S and O both keep the head in lane % 16 and the softmax rescale is lane-local.  The A
//     operand needs 8 tokens of one d per lane while V is d-contiguous, so lane (c, p) loads
//     8 bytes (d = 8c .. 8c+7) of each of its 8 tokens - four full 128-byte rows per load
//     instruction - and transposes the 8 x 8 byte block in its own registers (v_perm_b32) while
//     converting (v_cvt_scalef32_pk_bf16_fp8 turns byte pairs into bf16 pairs).
//   * online softmax in the exp2 domain; the W waves merge in LDS, the splits merge through a
//     per-(sequence, kv head) ticket: the workgroup that finishes last merges every split's
//     partial record and resets the ticket to zero, so no memset is needed between calls.
//     Records are written and read with device-coherent (agent-scope) accesses, which need no
//     cache-wide write-back or invalidate.  The tickets of different pairs lie 256 bytes apart.
#include "fp8kv_common.h"
#include "fp8kv_status.h"
#include "fp8kv_diag.h"
#include "attn_common.h"

#include <mutex>

namespace fp8kv {
namespace decode_detail {

constexpr int kD = 128;
constexpr int kMaxGqa = 16;
constexpr int kMergeBatch = 8;           // split records requested at once by the final merge
constexpr float kLog2e = 1.4426950408889634f;
// Ticket counters occupy a fixed region at the start of the scratch buffer, independent of the
// launch geometry, so a buffer shared by calls of different shapes never has one call's partial
// records where another call expects zeroed counters.
constexpr int kMaxPairs = 65536;
constexpr int kMaxSplits = 256;

// Ticket counter of a (sequence, kv head) pair.  Bijective on [0, kMaxPairs); the counters of
// pairs 0..1023 lie 256 bytes apart.  With adjacent counters the tickets of all pairs were
// atomics on one cache line, served one after another (measured at b8@4k, one process: 11.67 ->
// 11.36 us; a stand-alone probe with the same tail: 0.5 us at 8 splits, 2.4 us at 16).
__host__ __device__ inline int ticket_slot(int64_t pair) { return (int)((pair & 1023) * 64 + (pair >> 10)); }

struct Params {
    const __bf16* q;
    const uint8_t* k;
    const uint8_t* v;
    __bf16* out;
    const int32_t* qsl;
    const int32_t* seq_lens;
    const int32_t* bt;
    const float* k_scale;
    const float* v_scale;
    float* part;            // [records][gqa * (D + 2)]: o (gqa x D), m (gqa), l (gqa)
    uint32_t* counters;     // [kMaxPairs] tickets, indexed by ticket_slot(pair)
    int64_t q_stride, o_stride, bt_stride;
    int64_t sk0, sk1, sk2, sv0, sv1, sv2;
    float sm_scale;
    int hkv, gqa, pblk, pshift, nsplit;
};

__host__ __device__ inline int record_floats(int gqa) { return gqa * (kD + 2); }

// Token span [lo, hi) of split `sp`: cdiv(seq_len, nsplit) rounded up to 16 tokens, so every
// 16-token group of a span lies in one cache block when block_size % 16 == 0.
__host__ __device__ inline void split_span(int seqlen, int nsplit, int sp, int& lo, int& hi)
{
    int span = (seqlen + nsplit - 1) / nsplit;
    span = (span + 15) & ~15;
    lo = sp * span;
    hi = seqlen < lo + span ? seqlen : lo + span;
}

// K and V registers of one chunk of NG 16-token groups (lane (r, p) = (lane % 16, lane / 16)):
//   kr[g][j]: 16 bytes of token c0 + 16 g + r at d = 64 j + 16 p;
//   vr[G][j]: 8 bytes (d = 8 r .. 8 r + 7) of token c0 + 32 G + 4 p + j (j < 4) or
//             c0 + 32 G + 16 + 4 p + (j - 4) (j >= 4): the k-slot order of the P^T fragments.
template <int NG>
struct ChunkRegs {
    u32x4_t kr[NG][2];
    u32x2_t vr[NG / 2][8];
};

// Per-lane softmax state of one wave: running max and this lane's share of the running sum of
// head lr (log2 domain), and o[n][i] = head lr at d = 32 lp + 8 i + n.
struct WaveState {
    float m_run;
    float l_run;
    f32x4_t o[8];
};

// Block ids of one chunk, one per 16-token group, read with scalar loads (their waits count
// lgkmcnt and never hold back the K and V loads in flight).  A group that starts at or past hi
// takes the id of the span's last group (`last`: the start of the 16-token group holding token
// hi - 1), so every address formed from the ids lies in a block the sequence owns.
template <int NG>
struct ChunkIds {
    int blk[NG];
};

typedef __attribute__((address_space(4))) const int32_t const_i32_t;   // read-only for the launch
typedef __attribute__((address_space(4))) const float const_f32_t;

template <int NG>
__device__ __forceinline__ ChunkIds<NG> load_chunk_ids(const Params& P, const int32_t* btrow, int c0, int last)
{
    // The constant address space makes the compiler use scalar loads for these uniform reads,
    // whatever stores or fences come before them in the kernel.
    const_i32_t* row = (const_i32_t*)btrow;
    ChunkIds<NG> ids;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int t0 = c0 + 16 * g;
        ids.blk[g] = row[(t0 < last ? t0 : last) >> P.pshift];
    }
    return ids;
}

// Both chunks' block ids are in registers here: their scalar loads are issued together and
// waited for once, instead of one round trip per id.
// (The ids pass through the asm as in/out operands, so every use of them is ordered after it.)
template <int NG>
__device__ __forceinline__ void ids_ready(ChunkIds<NG>& a, ChunkIds<NG>& b)
{
    static_assert(NG == 2 || NG == 4, "two or four groups per chunk");
    if constexpr (NG == 2) {
        asm volatile("" : "+s"(a.blk[0]), "+s"(a.blk[1]), "+s"(b.blk[0]), "+s"(b.blk[1]));
    } else {
        asm volatile("" : "+s"(a.blk[0]), "+s"(a.blk[1]), "+s"(a.blk[2]), "+s"(a.blk[3]),
                          "+s"(b.blk[0]), "+s"(b.blk[1]), "+s"(b.blk[2]), "+s"(b.blk[3]));
    }
}

// Keeps the compiler from moving loads issued before it past it (into the branch that uses
// them), which would undo the software pipeline.
__device__ __forceinline__ void issue_fence() { asm volatile("" ::: "memory"); }

// Per-lane byte offsets of the chunk loads within one 16-token group (32-bit: the host rejects
// slot strides that could overflow them).
struct LaneOffsets {
    uint32_t k;          // token lr, d = 16 lp
    uint32_t v[4];       // token 4 lp + i, d = 8 lr
};

__device__ __forceinline__ LaneOffsets lane_offsets(const Params& P, int lr, int lp)
{
    LaneOffsets o;
    o.k = (uint32_t)lr * (uint32_t)P.sk1 + 16u * (uint32_t)lp;
#pragma unroll
    for (int i = 0; i < 4; ++i) o.v[i] = (uint32_t)(4 * lp + i) * (uint32_t)P.sv1 + 8u * (uint32_t)lr;
    return o;
}

// Request every K and V byte of the chunk starting at token c0 with the same instruction
// sequence wherever the chunk lies, so the compiler's wait counts stay exact: the group holding hi
// reads all 16 of its slots (inside its block; tokens >= hi are masked where used), and a group
// past hi reads one line of the span's last group with every lane (no new traffic).  Group g's
// base address is scalar (block id from `ids`), the per-lane part a 32-bit offset.  KF requests
// the K bytes of every group before any V byte, so the S^T MFMAs and the softmax of a chunk can
// start while its V bytes are still arriving; otherwise K and V alternate per group.
template <int NG, bool KF>
__device__ __forceinline__ void issue_chunk(ChunkRegs<NG>& c, const Params& P, const LaneOffsets& lo_,
                                            const ChunkIds<NG>& ids, int kh, int c0, int hi, int last)
{
    auto slot_of = [&](int g) -> int64_t {
        const int t0 = c0 + 16 * g;
        return (int64_t)((t0 < last ? t0 : last) & (P.pblk - 1));
    };
    auto issue_k = [&](int g) {
        const uint32_t m = c0 + 16 * g < hi ? ~0u : 0u;
        const uint8_t* kb = P.k + (int64_t)ids.blk[g] * P.sk0 + slot_of(g) * P.sk1 + (int64_t)kh * P.sk2;
        c.kr[g][0] = load_nt_16(kb + (lo_.k & m));
        c.kr[g][1] = load_nt_16(kb + (lo_.k & m) + 64);
    };
    auto issue_v = [&](int g) {
        const uint32_t m = c0 + 16 * g < hi ? ~0u : 0u;
        const uint8_t* vb = P.v + (int64_t)ids.blk[g] * P.sv0 + slot_of(g) * P.sv1 + (int64_t)kh * P.sv2;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            c.vr[g >> 1][4 * (g & 1) + i] =
                __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(vb + (lo_.v[i] & m)));
    };
    if constexpr (KF) {
#pragma unroll
        for (int g = 0; g < NG; ++g) issue_k(g);
#pragma unroll
        for (int g = 0; g < NG; ++g) issue_v(g);
    } else {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            issue_k(g);
            issue_v(g);
        }
    }
    issue_fence();
}

// S^T = K . Q^T, online softmax update, O^T += V^T . P^T for one chunk.
template <int NG>
__device__ __forceinline__ void consume_chunk(const ChunkRegs<NG>& c, WaveState& st, const u32x4_t (&qf)[4],
                                              float qk_scale, int c0, int hi, int lp)
{
    // lane (h, p) gets S[token c0 + 16 g + 4 p + i][head h]
    f32x4_t s[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        acc = mfma16x16x32_bf16(fp8x8_to_bf16x8(c.kr[g][0][0], c.kr[g][0][1]), as_bf16x8(qf[0]), acc);
        acc = mfma16x16x32_bf16(fp8x8_to_bf16x8(c.kr[g][0][2], c.kr[g][0][3]), as_bf16x8(qf[1]), acc);
        acc = mfma16x16x32_bf16(fp8x8_to_bf16x8(c.kr[g][1][0], c.kr[g][1][1]), as_bf16x8(qf[2]), acc);
        acc = mfma16x16x32_bf16(fp8x8_to_bf16x8(c.kr[g][1][2], c.kr[g][1][3]), as_bf16x8(qf[3]), acc);
        s[g] = acc;
    }
    float mc = neg_inf();
    if (c0 + 16 * NG <= hi) {
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[g][i] *= qk_scale;
                mc = fmaxf(mc, s[g][i]);
            }
    } else {
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = c0 + 16 * g + 4 * lp + i;
                const float x = tok < hi ? s[g][i] * qk_scale : neg_inf();
                s[g][i] = x;
                mc = fmaxf(mc, x);
            }
    }
    mc = max_xor16_32(mc);
    const float m_new = fmaxf(st.m_run, mc);
    const float m_use = m_new == neg_inf() ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(st.m_run - m_use);
    float psum = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pv = __builtin_amdgcn_exp2f(s[g][i] - m_use);
            s[g][i] = pv;
            psum += pv;
        }
    st.l_run = st.l_run * alpha + psum;
    st.m_run = m_new;
#pragma unroll
    for (int n = 0; n < 8; ++n) st.o[n] *= alpha;
#pragma unroll
    for (int G = 0; G < NG / 2; ++G) {
        u32x4_t pb;
        pb[0] = pack_bf16x2(s[2 * G][0], s[2 * G][1]);
        pb[1] = pack_bf16x2(s[2 * G][2], s[2 * G][3]);
        pb[2] = pack_bf16x2(s[2 * G + 1][0], s[2 * G + 1][1]);
        pb[3] = pack_bf16x2(s[2 * G + 1][2], s[2 * G + 1][3]);
        // V bytes of tokens >= hi are stale cache slots (possibly NaN codes): zero them so that
        // P = 0 contributes nothing.
        u32x2_t vv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) vv[j] = c.vr[G][j];
        if (c0 + 16 * NG > hi) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int tok = c0 + 32 * G + (j < 4 ? 4 * lp + j : 16 + 4 * lp + (j - 4));
                if (tok >= hi) vv[j] = (u32x2_t){0u, 0u};
            }
        }
        u32x4_t va[8];
        v_fragments(vv, va);
#pragma unroll
        for (int n = 0; n < 8; ++n) st.o[n] = mfma16x16x32_bf16(as_bf16x8(va[n]), as_bf16x8(pb), st.o[n]);
    }
}

// Final merge of up to SMAX split records in one round trip: every o value a thread needs (its
// elements tid + T j of every split) and every split's m and l (to LDS) are requested together
// with straight-line loads (split indices past nsplit repeat the last split and are not used), so
// the only wait is the barrier's.  Each element then weighs split s by exp2(m_s - max_s m_s).
// wm / wl: LDS for [nsplit][gqa] m and l.
template <int SMAX, int T>
__device__ __forceinline__ void merge_all(const Params& P, const float* recs, int rf, int E, int gqa,
                                          float* wm, float* wl, int tid, float vs, int64_t out_row)
{
    const int ns = P.nsplit;
    const int NSG = ns * gqa;
    for (int e0 = 0; e0 < E; e0 += 2 * T) {
        float ov[2][SMAX];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            int e = e0 + tid + T * j;
            e = e < E ? e : E - 1;
#pragma unroll
            for (int s = 0; s < SMAX; ++s)
                ov[j][s] = load_coherent(recs + (int64_t)(s < ns ? s : ns - 1) * rf + e);
        }
        if (e0 == 0) {
            // Every m and l value goes into registers first (unconditional loads, index clamped),
            // then to LDS: one wait covers them and the o values above.  Storing each value as it
            // arrives put a vmcnt(0) between the m and the l loads, a second round trip.
            constexpr int NI = (SMAX * kMaxGqa + T - 1) / T;
            float mv[NI], lv[NI];
#pragma unroll
            for (int k = 0; k < NI; ++k) {
                const int i = tid + k * T;
                const int ic = i < NSG ? i : NSG - 1;
                const int s = ic / gqa, h = ic - s * gqa;
                mv[k] = load_coherent(recs + (int64_t)s * rf + E + h);
                lv[k] = load_coherent(recs + (int64_t)s * rf + E + gqa + h);
            }
#pragma unroll
            for (int k = 0; k < NI; ++k) {
                const int i = tid + k * T;
                if (i < NSG) {
                    wm[i] = mv[k];
                    wl[i] = lv[k];
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int e = e0 + tid + T * j;
            if (e >= E) continue;
            const int h = e / kD;
            float m = neg_inf();
            for (int s = 0; s < ns; ++s) m = fmaxf(m, wm[s * gqa + h]);
            const float mu = m == neg_inf() ? 0.f : m;
            float acc = 0.f, l = 0.f;
#pragma unroll
            for (int s = 0; s < SMAX; ++s) {
                if (s < ns) {
                    const float f = __builtin_amdgcn_exp2f(wm[s * gqa + h] - mu);
                    acc += f * ov[j][s];
                    l += f * wl[s * gqa + h];
                }
            }
            const float r = l > 0.f ? acc * vs / l : 0.f;
            P.out[out_row + e] = (__bf16)r;
        }
    }
}

// seq_lens and qsl (also in P) lead the argument list: the library is built with kernel-argument
// preloading, so the hardware places them in SGPRs before the first instruction, and the sequence
// length (the head of the dependent chain seq_lens -> block ids -> K/V) and the query row are
// requested together with the rest of P instead of after it.
template <int W, int NG, int DEPTH, bool KF>
__global__ void __launch_bounds__(W * 64)
decode_kernel(const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl, Params P)
{
    // The two loads go out together with the loads of every argument the block-id, Q and K/V
    // requests need (the asm takes all of them, so one wait covers them all) rather than after
    // them; later reads of these fields reuse the loaded values.
    int seqlen = seq_lens[blockIdx.z];
    int qtok = qsl[blockIdx.z];
    int nsplit = P.nsplit;
    const int32_t* bt = P.bt;
    int64_t bt_stride = P.bt_stride;
    {
        const __bf16* qp = P.q;
        const uint8_t* kp = P.k;
        const uint8_t* vp = P.v;
        int64_t q_stride = P.q_stride, sk0 = P.sk0, sk1 = P.sk1, sk2 = P.sk2;
        int64_t sv0 = P.sv0, sv1 = P.sv1, sv2 = P.sv2;
        asm volatile("" : "+s"(seqlen), "+s"(qtok), "+s"(nsplit), "+s"(bt), "+s"(bt_stride),
                          "+s"(qp), "+s"(kp), "+s"(vp), "+s"(q_stride), "+s"(sk0), "+s"(sk1),
                          "+s"(sk2), "+s"(sv0), "+s"(sv1), "+s"(sv2));
    }
    constexpr int CH = 16 * NG;                 // tokens per chunk
    constexpr int T = W * 64;
    constexpr int EPT = (kMaxGqa * kD + T - 1) / T;   // merge elements per thread (upper bound)
    __shared__ float lds_ml[W][kMaxGqa][2];
    __shared__ __align__(16) float lds_o[W][kMaxGqa][kD];
    __shared__ int lds_last;
    static_assert(W * kMaxGqa * kD >= 2 * kMaxSplits * kMaxGqa, "merge statistics must fit in lds_o");

    const int sp = blockIdx.x, kh = blockIdx.y, seq = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15;
    const int lp = lane >> 4;
    const int gqa = P.gqa;

    int lo, hi;
    split_span(seqlen, nsplit, sp, lo, hi);
    const int32_t* btrow = bt + (int64_t)seq * bt_stride;

    // The wave's chunks start at c_first and step by `stride`.
    const int stride = CH * W;
    const int c_first = lo + CH * wave;
    const int last = (hi - 1) & ~15;
    // The first pair's block ids go out right behind the span (they head the dependent chain to
    // the K/V bytes); everything below is issued while they are in flight.
    [[maybe_unused]] ChunkIds<NG> ia, ib;
    if constexpr (DEPTH != 1) {
        if (c_first < hi) {
            ia = load_chunk_ids<NG>(P, btrow, c_first, last);
            ib = load_chunk_ids<NG>(P, btrow, c_first + stride, last);
        }
    }

    // Q^T fragments: lane (h, p) holds head h at d = 16p + (0..15) and 64 + 16p + (0..15).  Lanes
    // h >= gqa load head 0 again: their columns of S and O are never stored, and unconditional
    // loads leave no exec-masked write to a load's destination (which would make the compiler
    // wait for every load in flight).  The scales are scalar loads (lgkmcnt, not vmcnt).
    u32x4_t qf[4];
    {
        const __bf16* qrow = P.q + (int64_t)qtok * P.q_stride + (int64_t)(kh * gqa + (lr < gqa ? lr : 0)) * kD;
        qf[0] = load_16(qrow + 16 * lp);
        qf[1] = load_16(qrow + 16 * lp + 8);
        qf[2] = load_16(qrow + 64 + 16 * lp);
        qf[3] = load_16(qrow + 64 + 16 * lp + 8);
    }
    const float qk_scale = P.sm_scale * *(const_f32_t*)P.k_scale * kLog2e;
    const float vs = *(const_f32_t*)P.v_scale;

    WaveState st;
    st.m_run = neg_inf();
    st.l_run = 0.f;
#pragma unroll
    for (int n = 0; n < 8; ++n) st.o[n] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

    if (c_first < hi) {
        const LaneOffsets lofs = lane_offsets(P, lr, lp);
        ChunkRegs<NG> ca;
        [[maybe_unused]] ChunkRegs<NG> cb;
        int c0 = c_first;
        if constexpr (DEPTH == 1) {
            do {
                const ChunkIds<NG> ia = load_chunk_ids<NG>(P, btrow, c0, last);
                issue_chunk<NG, KF>(ca, P, lofs, ia, kh, c0, hi, last);
                consume_chunk<NG>(ca, st, qf, qk_scale, c0, hi, lp);
                c0 += stride;
            } while (c0 < hi);
        } else {
            // Chunks in pairs: both block-id sets in one scalar round trip, both chunks' loads
            // back to back, then chunk A is used while chunk B is still arriving.  Straight-line
            // code up to the use of B keeps the compiler's wait counts exact.  A chunk B past hi
            // reads one broadcast line per instruction and is not used.
            do {
                ids_ready(ia, ib);
                issue_chunk<NG, KF>(ca, P, lofs, ia, kh, c0, hi, last);
                issue_chunk<NG, KF>(cb, P, lofs, ib, kh, c0 + stride, hi, last);
                if (c0 + 2 * stride < hi) {            // the next pair's ids, a round trip ahead
                    ia = load_chunk_ids<NG>(P, btrow, c0 + 2 * stride, last);
                    ib = load_chunk_ids<NG>(P, btrow, c0 + 3 * stride, last);
                }
                consume_chunk<NG>(ca, st, qf, qk_scale, c0, hi, lp);
                if (c0 + stride >= hi) break;
                consume_chunk<NG>(cb, st, qf, qk_scale, c0 + stride, hi, lp);
                c0 += 2 * stride;
            } while (c0 < hi);
        }
    }

    // ---- merge the W waves in LDS ---------------------------------------------------------------
    float l_run = st.l_run;
    l_run = sum_xor16_32(l_run);
    if (lp == 0 && lr < gqa) {
        lds_ml[wave][lr][0] = st.m_run;
        lds_ml[wave][lr][1] = l_run;
    }
    if (lr < gqa) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f32x4_t a = {st.o[0][i], st.o[1][i], st.o[2][i], st.o[3][i]};
            f32x4_t b = {st.o[4][i], st.o[5][i], st.o[6][i], st.o[7][i]};
            *reinterpret_cast<f32x4_t*>(&lds_o[wave][lr][32 * lp + 8 * i]) = a;
            *reinterpret_cast<f32x4_t*>(&lds_o[wave][lr][32 * lp + 8 * i + 4]) = b;
        }
    }
    __syncthreads();

    const int E = gqa * kD;
    const int64_t pair = (int64_t)seq * P.hkv + kh;
    if (P.nsplit == 1) {
        for (int e = tid; e < E; e += T) {
            const int h = e / kD, d = e % kD;
            float m = neg_inf();
#pragma unroll
            for (int w = 0; w < W; ++w) m = fmaxf(m, lds_ml[w][h][0]);
            const float mu = m == neg_inf() ? 0.f : m;
            float acc = 0.f, l = 0.f;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float f = __builtin_amdgcn_exp2f(lds_ml[w][h][0] - mu);
                acc += f * lds_o[w][h][d];
                l += f * lds_ml[w][h][1];
            }
            const float r = l > 0.f ? acc * vs / l : 0.f;
            P.out[(int64_t)qtok * P.o_stride + (int64_t)(kh * gqa + h) * kD + d] = (__bf16)r;
        }
        return;
    }

    // ---- this split's partial record -------------------------------------------------------------
    const int rf = record_floats(gqa);
    float* rec = P.part + (pair * P.nsplit + sp) * rf;
    for (int e = tid; e < E; e += T) {
        const int h = e / kD, d = e % kD;
        float m = neg_inf();
#pragma unroll
        for (int w = 0; w < W; ++w) m = fmaxf(m, lds_ml[w][h][0]);
        const float mu = m == neg_inf() ? 0.f : m;
        float acc = 0.f, l = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float f = __builtin_amdgcn_exp2f(lds_ml[w][h][0] - mu);
            acc += f * lds_o[w][h][d];
            l += f * lds_ml[w][h][1];
        }
        store_coherent(rec + e, acc);
        if (d == 0) {
            store_coherent(rec + E + h, m);
            store_coherent(rec + E + gqa + h, l);
        }
    }

    // ---- ticket: the last split of this (sequence, kv head) merges --------------------------------
    // The records were written with device-coherent stores; once they have completed
    // (vmcnt(0)) the ticket increment may be observed.  The merging workgroup reads them with
    // device-coherent loads issued after it has seen the final ticket value.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const uint32_t t = __hip_atomic_fetch_add(P.counters + ticket_slot(pair), 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        lds_last = (t == (uint32_t)(P.nsplit - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!lds_last) return;

    const float* recs_all = P.part + pair * P.nsplit * rf;
    const int64_t out_row = (int64_t)qtok * P.o_stride + (int64_t)(kh * gqa) * kD;
    if (P.nsplit <= 32) {
        float* wm_all = &lds_o[0][0][0];
        float* wl_all = wm_all + 32 * kMaxGqa;
        if (P.nsplit <= 8)
            merge_all<8, T>(P, recs_all, rf, E, gqa, wm_all, wl_all, tid, vs, out_row);
        else if (P.nsplit <= 16)
            merge_all<16, T>(P, recs_all, rf, E, gqa, wm_all, wl_all, tid, vs, out_row);
        else
            merge_all<32, T>(P, recs_all, rf, E, gqa, wm_all, wl_all, tid, vs, out_row);
        if (tid == 0)
            __hip_atomic_store(P.counters + ticket_slot(pair), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // More than 32 splits (only when the caller asks for them): one round trip per kMergeBatch
    // splits: m and l of every split go to LDS once
    // (one load per split and head), each thread loads the o values of its own elements
    // tid + T j, and both are in flight together before the barrier.
    const float* recs = P.part + pair * P.nsplit * rf;
    const int NSG = P.nsplit * gqa;
    float* wm = &lds_o[0][0][0];            // [nsplit][gqa] m, then [nsplit][gqa] l
    float m[EPT], acc[EPT], l[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) { m[j] = neg_inf(); acc[j] = 0.f; l[j] = 0.f; }
    for (int s0 = 0; s0 < P.nsplit; s0 += kMergeBatch) {
        float ov[EPT][kMergeBatch];
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int e = tid + T * j;
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) {
                const int s2 = s0 + b < P.nsplit ? s0 + b : P.nsplit - 1;
                ov[j][b] = e < E ? load_coherent(recs + (int64_t)s2 * rf + e) : 0.f;
            }
        }
        if (s0 == 0) {
            for (int i = tid; i < NSG; i += T) {
                const int s2 = i / gqa, h = i % gqa;
                wm[i] = load_coherent(recs + (int64_t)s2 * rf + E + h);
                wm[NSG + i] = load_coherent(recs + (int64_t)s2 * rf + E + gqa + h);
            }
            __syncthreads();
        }
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int h = (tid + T * j) / kD;
            if (h >= gqa) continue;
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) {
                if (s0 + b >= P.nsplit) break;
                const float ms = wm[(s0 + b) * gqa + h];
                const float mn = fmaxf(m[j], ms);
                const float mu = mn == neg_inf() ? 0.f : mn;
                const float a = __builtin_amdgcn_exp2f(m[j] - mu);
                const float f = __builtin_amdgcn_exp2f(ms - mu);
                acc[j] = acc[j] * a + f * ov[j][b];
                l[j] = l[j] * a + f * wm[NSG + (s0 + b) * gqa + h];
                m[j] = mn;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int e = tid + T * j;
        if (e < E) {
            const float r = l[j] > 0.f ? acc[j] * vs / l[j] : 0.f;
            P.out[(int64_t)qtok * P.o_stride + (int64_t)(kh * gqa) * kD + e] = (__bf16)r;
        }
    }
    if (tid == 0)
        __hip_atomic_store(P.counters + ticket_slot(pair), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

inline size_t counters_bytes() { return (size_t)kMaxPairs * sizeof(uint32_t); }

inline size_t scratch_bytes(int ns, int hq, int hkv, int nsplit)
{
    if (nsplit <= 1) return 0;
    const int gqa = hq / hkv;
    return counters_bytes() +
           (size_t)ns * (size_t)hkv * (size_t)nsplit * (size_t)record_floats(gqa) * sizeof(float);
}

// Launch variants (waves per workgroup, 16-token groups per chunk, chunks in flight per wave,
// K bytes of a chunk requested before its V bytes).
struct Variant {
    int waves, ng, depth;
    bool kfirst;
};
constexpr Variant kVariants[] = {{8, 4, 1, false}, {8, 2, 1, false}, {4, 4, 1, false}, {4, 4, 2, false},
                                 {8, 2, 2, true},  {8, 2, 2, false}, {8, 2, 1, true}};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);

// Launch tunables (host state; fp8kv_decode_tune changes them for sweeps).
constexpr int kDefaultVariant = 4;
int g_variant = kDefaultVariant;
int g_target_wgs = 256;

// Splits per (sequence, kv head): enough workgroups to reach g_target_wgs (one per CU: at the
// kernel's register use only one 8-wave workgroup fits on a CU, so a larger grid runs in two
// rounds), never fewer than one chunk per workgroup, and at most kMaxPlannedSplits, since the
// merging workgroup reads the split records kMergeBatch at a time.  A wave loops over as many
// chunk pairs as its span holds.
constexpr int kMaxPlannedSplits = 32;

inline int plan_splits(int ns, int hkv, int max_seq_len)
{
    if (max_seq_len <= 0) return 1;
    const Variant v = kVariants[g_variant];
    const int chunk = 16 * v.ng;
    const int pairs = ns * hkv;
    const int by_fill = (g_target_wgs + pairs - 1) / pairs;                  // fill the GPU
    const int by_chunks = (max_seq_len + chunk - 1) / chunk;                 // >= 1 chunk per WG
    int n = by_fill < by_chunks ? by_fill : by_chunks;
    if (n > kMaxPlannedSplits) n = kMaxPlannedSplits;
    if (n < 1) n = 1;
    return n;
}

// Zero-fill of a decode scratch region (ticket counters and records), a kernel rather than a
// memset so that it can sit in a captured graph.
// n4 dwords from p (16-byte aligned): 16-byte stores, then the last n4 % 4 dwords.
__global__ void __launch_bounds__(256) scratch_zero_kernel(uint32_t* p, size_t n4)
{
    const size_t n16 = n4 / 4;
    uint4* p16 = reinterpret_cast<uint4*>(p);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
        p16[i] = make_uint4(0u, 0u, 0u, 0u);
    if (blockIdx.x == 0 && threadIdx.x < n4 % 4) p[4 * n16 + threadIdx.x] = 0u;
}

int launch_scratch_zero(void* p, size_t bytes, hipStream_t st)
{
    const size_t n4 = bytes / 4;
    if (n4 == 0) return FP8KV_OK;
    const size_t want = (n4 / 4 + 255) / 256;
    const unsigned grid = (unsigned)(want < 1 ? 1 : (want < 1024 ? want : 1024));
    begin_launch();
    launch_kernel(scratch_zero_kernel, dim3(grid), dim3(256), 0, st, static_cast<uint32_t*>(p), n4);
    return finish_launch();
}

// Checks the arguments and fills P (scratch pointers excluded); returns the scratch bytes the
// call needs through `need`.
int decode_setup(Params& P, const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                 int64_t sk0, int64_t sk1, int64_t sk2, int64_t sv0, int64_t sv1, int64_t sv2, void* out,
                 int64_t out_row_stride, const int32_t* query_start_loc, const int32_t* seq_lens,
                 const int32_t* block_table, int64_t bt_stride, const float* k_scale, const float* v_scale,
                 float sm_scale, int num_seqs, int num_q_heads, int num_kv_heads, int head_size, int block_size,
                 int num_splits, size_t& need)
{
    if (!q || !k_cache || !v_cache || !out || !query_start_loc || !seq_lens || !block_table ||
        !k_scale || !v_scale)
        return FP8KV_ERR_ARG;
    if (num_seqs < 1 || num_kv_heads < 1 || num_q_heads < 1 || block_size < 1 || num_splits < 1 ||
        num_splits > kMaxSplits || bt_stride < 0)
        return FP8KV_ERR_ARG;
    if (num_seqs > 65535 || num_kv_heads > 65535 || (int64_t)num_seqs * num_kv_heads > kMaxPairs)
        return FP8KV_ERR_SHAPE;
    if (head_size != kD || num_q_heads % num_kv_heads != 0) return FP8KV_ERR_SHAPE;
    const int gqa = num_q_heads / num_kv_heads;
    if (gqa > kMaxGqa) return FP8KV_ERR_SHAPE;
    if (block_size < 16 || (block_size & (block_size - 1)) != 0) return FP8KV_ERR_SHAPE;
    // K rows are read with 16-byte loads and V rows with 8-byte loads; q with 16-byte loads.
    if (!aligned(k_cache, 16) || !aligned(v_cache, 8) || !aligned(q, 16) || !aligned(out, 2))
        return FP8KV_ERR_ALIGN;
    if ((sk0 | sk1 | sk2) & 15) return FP8KV_ERR_ALIGN;
    if ((sv0 | sv1 | sv2) & 7) return FP8KV_ERR_ALIGN;
    if (q_row_stride & 7) return FP8KV_ERR_ALIGN;
    // Per-lane offsets within a 16-token group are 32-bit.
    if (sk1 < 0 || sv1 < 0 || sk1 > ((int64_t)1 << 26) || sv1 > ((int64_t)1 << 26)) return FP8KV_ERR_SHAPE;
    need = scratch_bytes(num_seqs, num_q_heads, num_kv_heads, num_splits);

    P.q = static_cast<const __bf16*>(q);
    P.k = static_cast<const uint8_t*>(k_cache);
    P.v = static_cast<const uint8_t*>(v_cache);
    P.out = static_cast<__bf16*>(out);
    P.qsl = query_start_loc;
    P.seq_lens = seq_lens;
    P.bt = block_table;
    P.k_scale = k_scale;
    P.v_scale = v_scale;
    P.counters = nullptr;
    P.part = nullptr;
    P.q_stride = q_row_stride;
    P.o_stride = out_row_stride;
    P.bt_stride = bt_stride;
    P.sk0 = sk0; P.sk1 = sk1; P.sk2 = sk2;
    P.sv0 = sv0; P.sv1 = sv1; P.sv2 = sv2;
    P.sm_scale = sm_scale;
    P.hkv = num_kv_heads;
    P.gqa = gqa;
    P.pblk = block_size;
    P.pshift = __builtin_ctz((unsigned)block_size);
    P.nsplit = num_splits;
    return FP8KV_OK;
}

void use_scratch(Params& P, void* buf, size_t need)
{
    if (need == 0) return;
    P.counters = static_cast<uint32_t*>(buf);
    P.part = reinterpret_cast<float*>(static_cast<unsigned char*>(buf) + counters_bytes());
}

int decode_launch(const Params& P, int num_seqs, hipStream_t st)
{
    const dim3 grid((unsigned)P.nsplit, (unsigned)P.hkv, (unsigned)num_seqs);
    begin_launch();
    switch (g_variant) {
        case 0: launch_kernel(decode_kernel<8, 4, 1, false>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P); break;
        case 1: launch_kernel(decode_kernel<8, 2, 1, false>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P); break;
        case 2: launch_kernel(decode_kernel<4, 4, 1, false>, grid, dim3(4 * 64), 0, st, P.seq_lens, P.qsl, P); break;
        case 3: launch_kernel(decode_kernel<4, 4, 2, false>, grid, dim3(4 * 64), 0, st, P.seq_lens, P.qsl, P); break;
        case 5: launch_kernel(decode_kernel<8, 2, 2, false>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P); break;
        case 6: launch_kernel(decode_kernel<8, 2, 1, true>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P); break;
        default: launch_kernel(decode_kernel<8, 2, 2, true>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P); break;
    }
    return finish_launch();
}

}  // namespace decode_detail
}  // namespace fp8kv

// Scratch of fp8kv_decode_attn_noalloc: tickets then split records, one copy per GPU the library
// runs on, held until the process ends.  In host code this name is a host-side stand-in, not a
// device address: the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace fp8kv {
namespace decode_detail {

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device.  The first call on a device resolves it
// and zeroes its ticket region with a kernel on `st` (the records need no initial state).
int noalloc_scratch(hipStream_t st, void** out)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        g_last_hip_error = (int)e;
        return FP8KV_ERR_LAUNCH;
    }
    if (dev < 0 || dev >= kMaxDevices) return FP8KV_ERR_ARG;
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (g_noalloc_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr) {
            g_last_hip_error = (int)e;
            return FP8KV_ERR_LAUNCH;
        }
        const int rc = launch_scratch_zero(ptr, counters_bytes(), st);
        if (rc != FP8KV_OK) return rc;
        g_noalloc_ptr[dev] = ptr;
    }
    *out = g_noalloc_ptr[dev];
    return FP8KV_OK;
}

}  // namespace decode_detail
}  // namespace fp8kv

using namespace fp8kv;
using namespace fp8kv::decode_detail;

extern "C" int fp8kv_decode_num_splits(int num_seqs, int num_kv_heads, int max_seq_len)
{
    if (num_seqs < 1 || num_kv_heads < 1) return 1;
    return plan_splits(num_seqs, num_kv_heads, max_seq_len);
}

extern "C" size_t fp8kv_decode_scratch_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                             int head_size, int num_splits)
{
    if (num_seqs < 1 || num_kv_heads < 1 || num_q_heads < num_kv_heads || head_size != kD)
        return 0;
    return scratch_bytes(num_seqs, num_q_heads, num_kv_heads, num_splits);
}

extern "C" int fp8kv_decode_scratch_reset(void* scratch_buf, size_t scratch_bytes_given, void* stream)
{
    if (!scratch_buf || !aligned(scratch_buf, 256)) return FP8KV_ERR_ARG;
    return launch_scratch_zero(scratch_buf, scratch_bytes_given, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int fp8kv_decode_attn(const void* q, int64_t q_row_stride,
                                 const void* k_cache, const void* v_cache,
                                 int64_t sk0, int64_t sk1, int64_t sk2,
                                 int64_t sv0, int64_t sv1, int64_t sv2,
                                 void* out, int64_t out_row_stride,
                                 const int32_t* query_start_loc, const int32_t* seq_lens,
                                 const int32_t* block_table, int64_t bt_stride,
                                 const float* k_scale, const float* v_scale, float sm_scale,
                                 int num_seqs, int num_q_heads, int num_kv_heads, int head_size,
                                 int block_size, int num_splits, void* scratch_buf,
                                 size_t scratch_bytes_given, void* stream)
{
    Params P;
    size_t need = 0;
    const int rc = decode_setup(P, q, q_row_stride, k_cache, v_cache, sk0, sk1, sk2, sv0, sv1, sv2, out,
                                out_row_stride, query_start_loc, seq_lens, block_table, bt_stride, k_scale,
                                v_scale, sm_scale, num_seqs, num_q_heads, num_kv_heads, head_size, block_size,
                                num_splits, need);
    if (rc != FP8KV_OK) return rc;
    if (need > 0 && (!scratch_buf || scratch_bytes_given < need || !aligned(scratch_buf, 256)))
        return FP8KV_ERR_SCRATCH;
    use_scratch(P, scratch_buf, need);
    return decode_launch(P, num_seqs, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int fp8kv_decode_attn_noalloc(const void* q, int64_t q_row_stride,
                                         const void* k_cache, const void* v_cache,
                                         int64_t sk0, int64_t sk1, int64_t sk2,
                                         int64_t sv0, int64_t sv1, int64_t sv2,
                                         void* out, int64_t out_row_stride,
                                         const int32_t* query_start_loc, const int32_t* seq_lens,
                                         const int32_t* block_table, int64_t bt_stride,
                                         const float* k_scale, const float* v_scale, float sm_scale,
                                         int num_seqs, int num_q_heads, int num_kv_heads, int head_size,
                                         int block_size, int num_splits, void* stream)
{
    Params P;
    size_t need = 0;
    int rc = decode_setup(P, q, q_row_stride, k_cache, v_cache, sk0, sk1, sk2, sv0, sv1, sv2, out,
                          out_row_stride, query_start_loc, seq_lens, block_table, bt_stride, k_scale,
                          v_scale, sm_scale, num_seqs, num_q_heads, num_kv_heads, head_size, block_size,
                          num_splits, need);
    if (rc != FP8KV_OK) return rc;
    if (need > kNoAllocScratchBytes) return FP8KV_ERR_SCRATCH;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    void* ptr = nullptr;
    if (need > 0) {
        rc = noalloc_scratch(st, &ptr);
        if (rc != FP8KV_OK) return rc;
    }
    use_scratch(P, ptr, need);
    return decode_launch(P, num_seqs, st);
}

extern "C" void fp8kv_decode_tune(int variant, int target_wgs)
{
    g_variant = (variant >= 0 && variant < kNumVariants) ? variant : kDefaultVariant;
    g_target_wgs = target_wgs > 0 ? target_wgs : 256;
}
