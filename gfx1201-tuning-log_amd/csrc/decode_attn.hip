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
//     The merging workgroup loads its records straight into registers (a wave's (m, l) pairs of
//     every split in one 8-byte load per lane, read across the wave with readlane) and merges
//     with independent per-split terms: no LDS round trip and no barrier after the loads.  Both
//     merges give each thread adjacent elements of one head, so one set of exp2 factors serves them.
#include "fp8kv_common.h"
#include "fp8kv_status.h"
#include "fp8kv_diag.h"
#include "attn_common.h"
#include "kv_chunk.h"

#include <mutex>

namespace fp8kv {
namespace decode_detail {

using namespace kv_chunk;

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
    float* part;            // [records][record_floats(gqa)]: o (gqa x D), then (m, l) of each head
    uint32_t* counters;     // [kMaxPairs] tickets, indexed by ticket_slot(pair)
    int64_t q_stride, o_stride, bt_stride;
    int64_t sk0, sk1, sk2, sv0, sv1, sv2;
    float sm_scale;
    int hkv, gqa, pblk, pshift, nsplit;
};

// Floats per split record, rounded up to a multiple of four so that every record starts 16-byte
// aligned (the workgroup merge stores four adjacent values per lane at once).
__host__ __device__ inline int record_floats(int gqa) { return (gqa * (kD + 2) + 3) & ~3; }

// Token span [lo, hi) of split `sp`: cdiv(seq_len, nsplit) rounded up to 16 tokens, so every
// 16-token group of a span lies in one cache block when block_size % 16 == 0.
__host__ __device__ inline void split_span(int seqlen, int nsplit, int sp, int& lo, int& hi)
{
    int span = (seqlen + nsplit - 1) / nsplit;
    span = (span + 15) & ~15;
    lo = sp * span;
    hi = seqlen < lo + span ? seqlen : lo + span;
}

// Final merge of up to SMAX split records in one round trip, with no LDS and no barrier.  Thread t
// takes the two adjacent elements 2t, 2t + 1 (+ 2T per pass), so the 128 elements of a wave are one
// head.  Each split's two o values (one 8-byte load) and, in lane s, split s's (m, l) pair of the
// wave's head are requested together with straight-line loads (split indices past nsplit repeat
// the last split); the wave reads the pairs with readlane, computes the factors exp2(m_s - max m)
// once for both elements, and adds every split's term independently of the others.
template <int SMAX, int T>
__device__ __forceinline__ void merge_regs(const Params& P, const float* recs, int rf, int E, int tid, float vs,
                                            int64_t out_row)
{
    static_assert(SMAX <= 64, "one (m, l) pair per lane");
    const int ns = P.nsplit;
    const int lane = tid & 63;
    const int sl = lane < ns ? lane : ns - 1;
    for (int e0 = 0; e0 < E; e0 += 2 * T) {
        int e = e0 + 2 * tid;
        const bool live = e < E;                       // wave-uniform
        e = live ? e : E - 2;
        const int h = e / kD;
        f32x2_t ov[SMAX];
#pragma unroll
        for (int s = 0; s < SMAX; ++s) ov[s] = load_coherent2(recs + (int64_t)(s < ns ? s : ns - 1) * rf + e);
        const f32x2_t ml = load_coherent2(recs + (int64_t)sl * rf + E + 2 * h);
        if (!live) continue;
        float ms[SMAX], ls[SMAX];
#pragma unroll
        for (int s = 0; s < SMAX; ++s) {
            ms[s] = s < ns ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml[0]), s)) : neg_inf();
            ls[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml[1]), s));
        }
        float m = neg_inf();
#pragma unroll
        for (int s = 0; s < SMAX; ++s) m = fmaxf(m, ms[s]);
        const float mu = m == neg_inf() ? 0.f : m;
        float a0 = 0.f, a1 = 0.f, l = 0.f;
#pragma unroll
        for (int s = 0; s < SMAX; ++s) {
            if (s < ns) {
                const float f = __builtin_amdgcn_exp2f(ms[s] - mu);
                a0 += f * ov[s][0];
                a1 += f * ov[s][1];
                l += f * ls[s];
            }
        }
        const float r0 = l > 0.f ? a0 * vs / l : 0.f;
        const float r1 = l > 0.f ? a1 * vs / l : 0.f;
        P.out[out_row + e] = (__bf16)r0;
        P.out[out_row + e + 1] = (__bf16)r1;
    }
}

// seq_lens and qsl (also in P) lead the argument list: the library is built with kernel-argument
// preloading, so the hardware places them in SGPRs before the first instruction, and the sequence
// length (the head of the dependent chain seq_lens -> block ids -> K/V) and the query row are
// requested together with the rest of P instead of after it.
// The kernel body, for e4m3 (B16 = false) or bf16 K/V caches.
template <int W, int NG, int DEPTH, bool KF, bool B16>
__device__ __forceinline__ void decode_body(const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl,
                                            const Params& P)
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
    // bf16 caches carry no scales (the reference ignores k_scale and v_scale for them).
    const float qk_scale = B16 ? P.sm_scale * kLog2e : P.sm_scale * *(const_f32_t*)P.k_scale * kLog2e;
    const float vs = B16 ? 1.f : *(const_f32_t*)P.v_scale;

    WaveState st;
    st.m_run = neg_inf();
    st.l_run = 0.f;
#pragma unroll
    for (int n = 0; n < 8; ++n) st.o[n] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

    if (c_first < hi) {
        const LaneOffsets lofs = lane_offsets<B16>(P, lr, lp);
        ChunkRegs<NG, B16> ca;
        [[maybe_unused]] ChunkRegs<NG, B16> cb;
        int c0 = c_first;
        if constexpr (DEPTH == 1) {
            do {
                const ChunkIds<NG> ia = load_chunk_ids<NG>(P, btrow, c0, last);
                issue_chunk<NG, KF, B16>(ca, P, lofs, ia, kh, c0, hi, last);
                consume_chunk<NG, B16>(ca, st, qf, qk_scale, c0, hi - 1, c0 + CH > hi, hi, lp);
                c0 += stride;
            } while (c0 < hi);
        } else {
            // Chunks in pairs: both block-id sets in one scalar round trip, both chunks' loads
            // back to back, then chunk A is used while chunk B is still arriving.  Straight-line
            // code up to the use of B keeps the compiler's wait counts exact.  A chunk B past hi
            // reads one broadcast line per instruction and is not used.
            do {
                ids_ready(ia, ib);
                issue_chunk<NG, KF, B16>(ca, P, lofs, ia, kh, c0, hi, last);
                issue_chunk<NG, KF, B16>(cb, P, lofs, ib, kh, c0 + stride, hi, last);
                if (c0 + 2 * stride < hi) {            // the next pair's ids, a round trip ahead
                    ia = load_chunk_ids<NG>(P, btrow, c0 + 2 * stride, last);
                    ib = load_chunk_ids<NG>(P, btrow, c0 + 3 * stride, last);
                }
                consume_chunk<NG, B16>(ca, st, qf, qk_scale, c0, hi - 1, c0 + CH > hi, hi, lp);
                if (c0 + stride >= hi) break;
                consume_chunk<NG, B16>(cb, st, qf, qk_scale, c0 + stride, hi - 1, c0 + stride + CH > hi, hi, lp);
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
    // Each thread merges four adjacent elements of one head over the W waves' partial states: every
    // LDS read goes out before any use (the o values of each wave in one 16-byte read, the (m, l)
    // reads are broadcasts), and the W factors exp2(m_w - max m) serve all four elements.
    auto merge_waves = [&](int e, f32x4_t& acc, float& mx, float& l) {
        const int h = e / kD, d = e % kD;
        float mw[W], lw[W];
        f32x4_t ow[W];
#pragma unroll
        for (int w = 0; w < W; ++w) {
            mw[w] = lds_ml[w][h][0];
            lw[w] = lds_ml[w][h][1];
            ow[w] = *reinterpret_cast<const f32x4_t*>(&lds_o[w][h][d]);
        }
        float m = neg_inf();
#pragma unroll
        for (int w = 0; w < W; ++w) m = fmaxf(m, mw[w]);
        const float mu = m == neg_inf() ? 0.f : m;
        acc = (f32x4_t){0.f, 0.f, 0.f, 0.f};
        l = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float f = __builtin_amdgcn_exp2f(mw[w] - mu);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += f * ow[w][i];
            l += f * lw[w];
        }
        mx = m;
    };
    if (P.nsplit == 1) {
        for (int e0 = 0; e0 < E; e0 += 4 * T) {
            const int e = e0 + 4 * tid;
            if (e >= E) break;
            f32x4_t acc;
            float m, l;
            merge_waves(e, acc, m, l);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float r = l > 0.f ? acc[i] * vs / l : 0.f;
                P.out[(int64_t)qtok * P.o_stride + (int64_t)(kh * gqa) * kD + e + i] = (__bf16)r;
            }
        }
        return;
    }

    // ---- this split's partial record -------------------------------------------------------------
    const int rf = record_floats(gqa);
    float* rec = P.part + (pair * P.nsplit + sp) * rf;
    for (int e0 = 0; e0 < E; e0 += 4 * T) {
        const int e = e0 + 4 * tid;
        if (e >= E) break;
        f32x4_t acc;
        float m, l;
        merge_waves(e, acc, m, l);
        store_coherent4(rec + e, acc);
        if (e % kD == 0) store_coherent2(rec + E + 2 * (e / kD), m, l);
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
        if (P.nsplit <= 2)
            merge_regs<2, T>(P, recs_all, rf, E, tid, vs, out_row);
        else if (P.nsplit <= 4)
            merge_regs<4, T>(P, recs_all, rf, E, tid, vs, out_row);
        else if (P.nsplit <= 8)
            merge_regs<8, T>(P, recs_all, rf, E, tid, vs, out_row);
        else if (P.nsplit <= 16)
            merge_regs<16, T>(P, recs_all, rf, E, tid, vs, out_row);
        else
            merge_regs<32, T>(P, recs_all, rf, E, tid, vs, out_row);
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
                wm[i] = load_coherent(recs + (int64_t)s2 * rf + E + 2 * h);
                wm[NSG + i] = load_coherent(recs + (int64_t)s2 * rf + E + 2 * h + 1);
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

template <int W, int NG, int DEPTH, bool KF>
__global__ void __launch_bounds__(W * 64)
decode_kernel(const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl, Params P)
{
    decode_body<W, NG, DEPTH, KF, false>(seq_lens, qsl, P);
}

// bf16 K/V caches: the same kernel with twice the bytes per chunk and no widening (the reference's
// K_FP8 = False branch, vllm-fp8kv/fp8kv_v3.py:44-45,61-66,110).
template <int W, int NG, int DEPTH, bool KF>
__global__ void __launch_bounds__(W * 64)
decode_bf16kv_kernel(const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl, Params P)
{
    decode_body<W, NG, DEPTH, KF, true>(seq_lens, qsl, P);
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

// Launch tunables (host state; fp8kv_decode_tune changes them for sweeps).  The default requests
// each 16-token group's K and V bytes together: against all K of a chunk before its V (variant 4)
// it runs 0.1-0.3 us shorter per launch on both clocks from b8@1k to b8@8k, and ties at b1@512.
constexpr int kDefaultVariant = 5;
thread_local int g_variant = kDefaultVariant;
thread_local int g_target_wgs = 256;

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
// call needs through `need`.  Cache strides are in elements of elem_bytes bytes (1: e4m3, 2: bf16,
// whose calls need no scales).
int decode_setup(Params& P, const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                 int64_t sk0, int64_t sk1, int64_t sk2, int64_t sv0, int64_t sv1, int64_t sv2, void* out,
                 int64_t out_row_stride, const int32_t* query_start_loc, const int32_t* seq_lens,
                 const int32_t* block_table, int64_t bt_stride, const float* k_scale, const float* v_scale,
                 float sm_scale, int num_seqs, int num_q_heads, int num_kv_heads, int head_size, int block_size,
                 int num_splits, size_t& need, int elem_bytes = 1)
{
    if (!q || !k_cache || !v_cache || !out || !query_start_loc || !seq_lens || !block_table)
        return FP8KV_ERR_ARG;
    if (elem_bytes == 1 && (!k_scale || !v_scale)) return FP8KV_ERR_ARG;
    if (num_seqs < 1 || num_kv_heads < 1 || num_q_heads < 1 || block_size < 1 || num_splits < 1 ||
        num_splits > kMaxSplits || bt_stride < 0)
        return FP8KV_ERR_ARG;
    if (num_seqs > 65535 || num_kv_heads > 65535 || (int64_t)num_seqs * num_kv_heads > kMaxPairs)
        return FP8KV_ERR_SHAPE;
    if (head_size != kD || num_q_heads % num_kv_heads != 0) return FP8KV_ERR_SHAPE;
    const int gqa = num_q_heads / num_kv_heads;
    if (gqa > kMaxGqa) return FP8KV_ERR_SHAPE;
    if (block_size < 16 || (block_size & (block_size - 1)) != 0) return FP8KV_ERR_SHAPE;
    // Strides in bytes from here on.  K rows are read with 16-byte loads and V rows with 8-byte
    // (e4m3) or 16-byte (bf16) loads; q with 16-byte loads.
    const int64_t vbytes = 8 * elem_bytes;
    sk0 *= elem_bytes; sk1 *= elem_bytes; sk2 *= elem_bytes;
    sv0 *= elem_bytes; sv1 *= elem_bytes; sv2 *= elem_bytes;
    if (!aligned(k_cache, 16) || !aligned(v_cache, (size_t)vbytes) || !aligned(q, 16) || !aligned(out, 2))
        return FP8KV_ERR_ALIGN;
    if ((sk0 | sk1 | sk2) & 15) return FP8KV_ERR_ALIGN;
    if ((sv0 | sv1 | sv2) & (vbytes - 1)) return FP8KV_ERR_ALIGN;
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

// bf16 caches: one shape, <8 waves, 2 groups, 2 chunks in flight, K of a chunk before its V>.
int decode_launch_bf16kv(const Params& P, int num_seqs, hipStream_t st)
{
    const dim3 grid((unsigned)P.nsplit, (unsigned)P.hkv, (unsigned)num_seqs);
    begin_launch();
    launch_kernel(decode_bf16kv_kernel<8, 2, 2, true>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P);
    return finish_launch();
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
        case 4: launch_kernel(decode_kernel<8, 2, 2, true>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P); break;
        case 6: launch_kernel(decode_kernel<8, 2, 1, true>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P); break;
        default: launch_kernel(decode_kernel<8, 2, 2, false>, grid, dim3(8 * 64), 0, st, P.seq_lens, P.qsl, P); break;
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

// The device address of `scratch` on the current device, resolved by the first call on that
// device.  Nothing is launched for it: the array is zero when the code object is loaded (it has no
// initializer), and every completed decode call leaves its tickets at zero again, so a first call
// captured into a graph records no extra node (the records need no initial state).
int noalloc_scratch(void** out)
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
        rc = noalloc_scratch(&ptr);
        if (rc != FP8KV_OK) return rc;
    }
    use_scratch(P, ptr, need);
    return decode_launch(P, num_seqs, st);
}

extern "C" int fp8kv_decode_attn_bf16(const void* q, int64_t q_row_stride,
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
                                num_splits, need, 2);
    if (rc != FP8KV_OK) return rc;
    if (need > 0 && (!scratch_buf || scratch_bytes_given < need || !aligned(scratch_buf, 256)))
        return FP8KV_ERR_SCRATCH;
    use_scratch(P, scratch_buf, need);
    return decode_launch_bf16kv(P, num_seqs, reinterpret_cast<hipStream_t>(stream));
}

extern "C" void fp8kv_decode_tune(int variant, int target_wgs)
{
    g_variant = (variant >= 0 && variant < kNumVariants) ? variant : kDefaultVariant;
    g_target_wgs = target_wgs > 0 ? target_wgs : 256;
}
