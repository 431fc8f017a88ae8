// Register-direct K/V chunk loads of the paged attention kernels (decode, and prefill over bf16
// caches) for gfx950: one chunk is NG 16-token groups of one (sequence, kv head), read straight
// into the MFMA fragment layout of S^T = K . Q^T and O^T = V^T . P^T (no LDS staging).
//
// KV element type: e4m3 bytes (B16 = false) or bf16 (B16 = true).  Strides in the kernel
// parameters are in bytes either way.  Lane (r, p) = (lane % 16, lane / 16):
//   kr[g][j]: K of token c0 + 16 g + r: e4m3: 16 bytes at d = 64 j + 16 p (j < 2); bf16: 16 bytes
//             (8 values) at d = 64 (j / 2) + 16 p + 8 (j % 2) (j < 4): the same d order;
//   vr[G][j]: V of token c0 + 32 G + 4 p + j (j < 4) or c0 + 32 G + 16 + 4 p + (j - 4) (j >= 4),
//             d = 8 r .. 8 r + 7 (8 bytes e4m3, 16 bytes bf16): the k-slot order of the P^T
//             fragments, transposed into V^T fragments by v_fragments / v_fragments_b16.
// Every chunk is requested with the same instruction sequence wherever it lies, so the compiler's
// vmcnt waits stay exact (each use waits for its own bytes only): the group holding `hi` reads
// all 16 slots of its block (tokens >= hi are masked where used), and a group at or past hi reads
// one line of the span's last group with every lane.
#pragma once
#include "fp8kv_common.h"
#include "attn_common.h"

namespace fp8kv {
namespace kv_chunk {

template <bool B16> struct VRow;
template <> struct VRow<false> { typedef u32x2_t type; };
template <> struct VRow<true> { typedef u32x4_t type; };

template <int NG, bool B16>
struct ChunkRegs {
    u32x4_t kr[NG][B16 ? 4 : 2];
    typename VRow<B16>::type vr[NG / 2][8];
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

template <int NG, typename PT>
__device__ __forceinline__ ChunkIds<NG> load_chunk_ids(const PT& P, const int32_t* btrow, int c0, int last)
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

// Per-lane byte offsets of the chunk loads within one 16-token group (32-bit: the hosts reject
// slot strides that could overflow them).
struct LaneOffsets {
    uint32_t k;          // token lr, d = 16 lp
    uint32_t v[4];       // token 4 lp + i, d = 8 lr
};

template <bool B16, typename PT>
__device__ __forceinline__ LaneOffsets lane_offsets(const PT& P, int lr, int lp)
{
    constexpr uint32_t es = B16 ? 2u : 1u;       // bytes per element
    LaneOffsets o;
    o.k = (uint32_t)lr * (uint32_t)P.sk1 + 16u * es * (uint32_t)lp;
#pragma unroll
    for (int i = 0; i < 4; ++i) o.v[i] = (uint32_t)(4 * lp + i) * (uint32_t)P.sv1 + 8u * es * (uint32_t)lr;
    return o;
}

// Request every K and V byte of the chunk starting at token c0 (see the file comment).  Group g's
// base address is scalar (block id from `ids`), the per-lane part a 32-bit offset.  KF requests
// the K bytes of every group before any V byte, so the S^T MFMAs and the softmax of a chunk can
// start while its V bytes are still arriving; otherwise K and V alternate per group.
template <int NG, bool KF, bool B16, typename PT>
__device__ __forceinline__ void issue_chunk(ChunkRegs<NG, B16>& c, const PT& P, const LaneOffsets& lo_,
                                            const ChunkIds<NG>& ids, int kh, int c0, int hi, int last)
{
    auto slot_of = [&](int g) -> int64_t {
        const int t0 = c0 + 16 * g;
        return (int64_t)((t0 < last ? t0 : last) & (P.pblk - 1));
    };
    auto issue_k = [&](int g) {
        const uint32_t m = c0 + 16 * g < hi ? ~0u : 0u;
        const uint8_t* kb = P.k + (int64_t)ids.blk[g] * P.sk0 + slot_of(g) * P.sk1 + (int64_t)kh * P.sk2;
        if constexpr (B16) {
            c.kr[g][0] = load_nt_16(kb + (lo_.k & m));
            c.kr[g][1] = load_nt_16(kb + (lo_.k & m) + 16);
            c.kr[g][2] = load_nt_16(kb + (lo_.k & m) + 128);
            c.kr[g][3] = load_nt_16(kb + (lo_.k & m) + 144);
        } else {
            c.kr[g][0] = load_nt_16(kb + (lo_.k & m));
            c.kr[g][1] = load_nt_16(kb + (lo_.k & m) + 64);
        }
    };
    auto issue_v = [&](int g) {
        const uint32_t m = c0 + 16 * g < hi ? ~0u : 0u;
        const uint8_t* vb = P.v + (int64_t)ids.blk[g] * P.sv0 + slot_of(g) * P.sv1 + (int64_t)kh * P.sv2;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (B16)
                c.vr[g >> 1][4 * (g & 1) + i] = load_nt_16(vb + (lo_.v[i] & m));
            else
                c.vr[g >> 1][4 * (g & 1) + i] =
                    __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(vb + (lo_.v[i] & m)));
        }
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

// The four A fragments (8 bf16 each) of S^T = K . Q^T for group g, in the order of the Q^T
// fragments qf[0..3] (d = 16 p + 0..7, 16 p + 8..15, 64 + 16 p + 0..7, 64 + 16 p + 8..15).
template <int NG, bool B16>
__device__ __forceinline__ bf16x8_t k_fragment(const ChunkRegs<NG, B16>& c, int g, int f)
{
    if constexpr (B16) {
        return as_bf16x8(c.kr[g][f]);
    } else {
        const u32x4_t& w = c.kr[g][f >> 1];
        return (f & 1) ? fp8x8_to_bf16x8(w[2], w[3]) : fp8x8_to_bf16x8(w[0], w[1]);
    }
}

// Per-lane softmax state of one wave: running max and this lane's share of the running sum of
// column lr (log2 domain), and o[n][i] = column lr at d = 32 lp + 8 i + n.  A column is one query
// row: a GQA head of the decode token, or a token of a prefill row-set.
struct WaveState {
    float m_run;
    float l_run;
    f32x4_t o[8];
};

// S^T = K . Q^T, online softmax update, O^T += V^T . P^T for one chunk of keys c0 .. c0 + 16 NG.
// With `masked`, keys above `lim` (this lane's column: the decode span's last token, or the
// prefill query's position) get probability 0; V rows of keys >= vhi are stale cache slots
// (possibly NaN codes) and are zeroed so that P = 0 contributes nothing.  The probabilities are
// rounded to bf16 for P.V; the row sums use their fp32 values.
template <int NG, bool B16>
__device__ __forceinline__ void consume_chunk(const ChunkRegs<NG, B16>& c, WaveState& st, const u32x4_t (&qf)[4],
                                              float qk_scale, int c0, int lim, bool masked, int vhi, int lp)
{
    // lane (h, p) gets S[token c0 + 16 g + 4 p + i][column h]
    f32x4_t s[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int f = 0; f < 4; ++f) acc = mfma16x16x32_bf16(k_fragment(c, g, f), as_bf16x8(qf[f]), acc);
        s[g] = acc;
    }
    float mc = neg_inf();
    if (!masked) {
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
                const float x = tok <= lim ? s[g][i] * qk_scale : neg_inf();
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
        typename VRow<B16>::type vv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) vv[j] = c.vr[G][j];
        if (c0 + 16 * NG > vhi) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int tok = c0 + 32 * G + (j < 4 ? 4 * lp + j : 16 + 4 * lp + (j - 4));
                if (tok >= vhi) vv[j] = typename VRow<B16>::type{};
            }
        }
        u32x4_t va[8];
        if constexpr (B16)
            v_fragments_b16(vv, va);
        else
            v_fragments(vv, va);
#pragma unroll
        for (int n = 0; n < 8; ++n) st.o[n] = mfma16x16x32_bf16(as_bf16x8(va[n]), as_bf16x8(pb), st.o[n]);
    }
}

}  // namespace kv_chunk
}  // namespace fp8kv
