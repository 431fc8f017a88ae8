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
//   * 1-D grid over (token-block rank, kv head) per sequence.  A workgroup of W waves owns nb
//     16-token blocks of all GQA heads of one kv head: nb * GQA row-sets of 16 rows, row-set r =
//     (head r % GQA, block r / GQA), wave w taking r = w, w + W, ... (RS at most).  With `paired`
//     the two blocks are r and n16 - 1 - r, so every workgroup has the same causal work; otherwise
//     ranks start from the longest causal rows.  Workgroups are spread so that each XCD's L2
//     serves one kv head (dispatch is round-robin over the 8 XCDs).
//   * keys are walked in 32-key tiles.  Raw fp8 K and V rows stream from the paged cache into an
//     LDS ring R tiles deep with global_load_lds_dwordx4 (block id per copy instruction from a
//     register via readlane), placed so that the fragment reads are bank-conflict free; each
//     wave waits only for its own copies (explicit vmcnt) and one LDS-only barrier per tile
//     publishes the tile.
//   * every wave widens its fragments itself: K with v_cvt_scalef32_pk_bf16_fp8, V with the
//     in-register 8 x 8 byte transpose shared with the decode kernel.
//   * S^T = K . Q^T and O^T = V^T . P^T on v_mfma_f32_16x16x32_bf16 (the decode kernel's
//     formulation): the query token stays in lane % 16 in S and O, so the online-softmax rescale is
//     lane-local, and the row max reduces over the four k-parts with lane swaps.  The rescale is
//     lazy: accumulators move to a new reference max only when it grows by more than 2^8.
//   * the causal mask is applied only on diagonal tiles; tiles entirely above a row-set's diagonal
//     are skipped for that row-set.
#include "fp8kv_common.h"
#include "fp8kv_status.h"
#include "attn_common.h"
#include "fp8kv_diag.h"

namespace fp8kv {
namespace prefill_detail {

constexpr int kD = 128;
constexpr int kBN = 32;                       // keys per tile
constexpr int kMaxGqa = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.f;          // log2 growth of a row max tolerated before rescaling
constexpr int kTileBytes = 8192;              // raw fp8 tile: K rows 0..31 (4 KB), then V rows (4 KB)

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
    int hkv, gqa, pblk, pshift, nb;
    int paired;                 // 1: nb == 2 and the two 16-token blocks are r and n16 - 1 - r
    int ntb_grid;               // token blocks per (sequence, kv head) the grid covers
    int xcd_map;                // 1: kv head from the XCD index (8 % HKV == 0), see kernel
    int q0_host, qlen_host;
};

// ---- raw fp8 tile placement in LDS ---------------------------------------------------------------
// The tile is copied by eight 1 KB global_load_lds_dwordx4 instructions: I = 0..3 carry K rows
// 8I .. 8I+7, I = 4..7 carry V rows 8(I-4) .. +7; lane l of an instruction lands at 16 l.  Which
// (row, 16-byte chunk) a lane fetches is chosen so that the fragment reads below are free of bank
// conflicts:
//   K: row r (0..7), chunk c at slot 8 r + (c ^ (r >> 1)) - the 16 rows one fragment read touches
//      (same chunk) fall in 16 distinct 16-byte bank groups;
//   V: row r at slot 8 rho(r) + c with rho(r) = 2 (r & 3) + (r >> 2) - the rows 4p + j one
//      transposing read touches (p = 0..3) alternate between the two bank halves.
__host__ __device__ inline int k_slot(int r, int c) { return 8 * r + (c ^ (r >> 1)); }
__host__ __device__ inline int v_slot(int r, int c) { return 8 * (2 * (r & 3) + (r >> 2)) + c; }

// (row within the 8-row group, chunk) lane l of a K or V copy instruction fetches.
__device__ __forceinline__ void dma_lane_rc(bool is_v, int lane, int& r, int& c)
{
    if (!is_v) {
        r = lane >> 3;
        c = (lane & 7) ^ (r >> 1);
    } else {
        const int rho = lane >> 3;
        c = lane & 7;
        r = (rho >> 1) + 4 * (rho & 1);
    }
}

// global_load_lds_dwordx4 issued as inline assembly, in its scalar-base form: lane i's 16 bytes
// from sbase + voff (sbase a wave-uniform 64-bit address, voff this lane's 32-bit offset, so no
// 64-bit address arithmetic per lane) land at lds_dst + 16 i.  The compiler does not see this
// copy, so it inserts no wait for it: in particular no vmcnt(0) before LDS reads it cannot prove
// disjoint from the copy's destination, which would drain the whole prefetch ring each tile.
// Completion is tracked only by the kernel's explicit vmcnt waits (vmcnt counts in issue order,
// so the compiler's own waits for its loads stay correct - at worst they wait longer).  lds_dst
// must be wave-uniform.
__device__ __forceinline__ void dma16_saddr(const void* sbase, uint32_t voff, unsigned char* lds_dst)
{
    const uint32_t lds_addr = (uint32_t)(uintptr_t)(lds_void_t*)lds_dst;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(lds_addr), "v"(voff), "s"(sbase) : "memory", "m0");
}

// Block ids of 16-key groups 64 b .. 64 b + 63 (batch b), one per lane (0 past the context).
__device__ __forceinline__ int load_group_blocks(const Params& P, const int32_t* btrow, int batch,
                                                 int k_hi, int lane)
{
    const int key = 16 * (64 * batch + lane);
    return key < k_hi ? btrow[key >> P.pshift] : 0;
}

// Issue this wave's share (instructions I = wave, wave + W, ...) of tile t's copies into `dst`.
// One instruction covers 8 rows of one 16-key group, hence one cache block: its id comes from
// the batch register `bids` (batch `batch`, which holds tile t) with readlane, its base address is
// scalar and only slot and chunk vary per lane.  Keys >= k_hi fetch key k_hi - 1 (a real, finite
// row in the same or the previous group; the causal mask removes it).
template <int W>
__device__ __forceinline__ void issue_tile(const Params& P, unsigned char* dst, int bids, int batch,
                                           int kh, int t, int k_hi, int wave, int lane)
{
    const int g_last = (k_hi - 1) >> 4;
#pragma unroll
    for (int I = wave; I < 8; I += W) {
        const bool is_v = I >= 4;
        int r, c;
        dma_lane_rc(is_v, lane, r, c);
        const int grp = min(2 * t + ((I & 3) >> 1), g_last);
        const int64_t blk = __builtin_amdgcn_readlane(bids, grp - 64 * batch);
        int key = t * kBN + 8 * (I & 3) + r;
        key = key < k_hi ? key : k_hi - 1;
        const uint32_t slot = (uint32_t)key & (uint32_t)(P.pblk - 1);
        const uint8_t* base = is_v ? P.v + blk * P.sv0 + (int64_t)kh * P.sv2
                                   : P.k + blk * P.sk0 + (int64_t)kh * P.sk2;
        const uint32_t off = slot * (uint32_t)(is_v ? P.sv1 : P.sk1) + 16u * (uint32_t)c;
        dma16_saddr(base, off, dst + I * 1024);
    }
}

// Workgroup barrier that orders LDS only.  __syncthreads() carries a workgroup-scope release
// fence, which on gfx950 waits for every outstanding vector-memory operation - including the
// async tile copies still in flight for later tiles.  Here each wave has already waited for its
// own copies of the tile it is about to read (vmcnt), so the barrier only needs this wave's LDS
// reads of the previous tile to have completed (lgkmcnt) before the slot is overwritten; the
// "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int W>
constexpr int copies_per_wave(int wave) { return (8 - wave + W - 1) / W; }

// s_waitcnt vmcnt(n) for a runtime n in 0..12.
__device__ __forceinline__ void wait_vmcnt_rt(int n)
{
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<1>(); break;
        case 2: wait_vmcnt<2>(); break;
        case 3: wait_vmcnt<3>(); break;
        case 4: wait_vmcnt<4>(); break;
        case 5: wait_vmcnt<5>(); break;
        case 6: wait_vmcnt<6>(); break;
        case 7: wait_vmcnt<7>(); break;
        case 8: wait_vmcnt<8>(); break;
        case 9: wait_vmcnt<9>(); break;
        case 10: wait_vmcnt<10>(); break;
        case 11: wait_vmcnt<11>(); break;
        default: wait_vmcnt<12>(); break;
    }
}

template <int W, int RS, int R>
__global__ void __launch_bounds__(W * 64)
prefill_kernel(Params P)
{
    static_assert(R >= 2 && (R - 2) * ((8 + W - 1) / W) <= 12, "ring depth vs vmcnt range");
    __shared__ __align__(16) unsigned char ring[R * kTileBytes];

    // Work item from the 1-D grid.  Workgroups are dispatched round-robin over the 8 XCDs, so with
    // xcd_map workgroup lin (on XCD lin % 8) takes kv head (lin % 8) % HKV: every XCD's L2 then
    // holds the K/V of one kv head instead of all of them.  Ranks count from the longest causal
    // rows.  The mapping is a bijection whatever the dispatch order; only the L2 reuse depends on it.
    const int lin = blockIdx.x, seq = blockIdx.z;
    int kh, rank;
    if (P.xcd_map) {
        const int xcd = lin & 7, per = 8 / P.hkv;
        kh = xcd % P.hkv;
        rank = (lin >> 3) * per + xcd / P.hkv;
    } else {
        kh = lin % P.hkv;
        rank = lin / P.hkv;
    }
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
    // Token blocks (of 16) of this workgroup: nb consecutive ones, or with `paired` the blocks
    // r and n16 - 1 - r, whose causal spans add up to the same work for every workgroup.
    // Token blocks (of 16) of this workgroup: block b is blk_a + b (nb consecutive ones), or with
    // `paired` blk_a = r and blk_b = n16 - 1 - r, whose causal spans add up to the same work for
    // every workgroup.
    const int n16 = (qlen + 15) >> 4;
    const int tb = P.ntb_grid - 1 - rank;                     // longest causal rows first
    int blk_a, blk_b, nblocks, last16;
    if (P.paired) {
        if (tb < 0 || tb >= ((n16 + 1) >> 1) || q0 < 0) return;   // whole workgroup, before any barrier
        blk_a = tb;
        blk_b = n16 - 1 - tb;
        nblocks = blk_b > blk_a ? 2 : 1;
        last16 = blk_b;
    } else {
        if (tb < 0 || tb >= (n16 + P.nb - 1) / P.nb || q0 < 0) return;
        blk_a = tb * P.nb;
        blk_b = blk_a + 1;
        nblocks = min(P.nb, n16 - blk_a);
        last16 = blk_a + nblocks - 1;
    }
    const int paired = P.paired;
    auto block_of = [&](int b) { return paired ? (b ? blk_b : blk_a) : blk_a + b; };
    const int k_hi = q0 + min(16 * (last16 + 1), qlen);      // keys [0, k_hi)
    const int32_t* btrow = P.bt + (int64_t)seq * P.bt_stride;
    const int nrs = nblocks * gqa;
    const int ntiles = (k_hi + kBN - 1) / kBN;
    const int my_copies = copies_per_wave<W>(wave);

    // ---- block ids, Q^T fragments, first tiles in flight ------------------------------------------
    int bid_batch = 0;
    int bid_cur = load_group_blocks(P, btrow, 0, k_hi, lane);
    int bid_next = load_group_blocks(P, btrow, 1, k_hi, lane);

    u32x4_t qf[RS][4];
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        const int r = wave + W * j;
        const int g = r % gqa, b = r / gqa;
        const int tok = 16 * block_of(b) + lr;
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
    wait_vmcnt<0>();
#pragma unroll
    for (int t = 0; t < R - 1; ++t)
        if (t < ntiles) issue_tile<W>(P, ring + t * kTileBytes, bid_cur, 0, kh, t, k_hi, wave, lane);

    float m_run[RS], l_run[RS];
    f32x4_t o[RS][8];
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        m_run[j] = neg_inf();
        l_run[j] = 0.f;
#pragma unroll
        for (int n = 0; n < 8; ++n) o[j][n] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }

    for (int t = 0; t < ntiles; ++t) {
        const int k0 = t * kBN;
        // Tile t's copies (this wave's) are the oldest still counted; younger: tiles t+1 ..
        // min(t + R - 2, ntiles - 1).  The barrier then makes every wave's copies visible and
        // guarantees that tile t - 1's slot is no longer read.
        const int younger = min(R - 2, ntiles - 1 - t);
        wait_vmcnt_rt(younger * my_copies);
        lds_barrier();
        const int tn = t + R - 1;
        if (tn < ntiles) {
            if ((tn >> 5) != bid_batch) {                     // 32 tiles per block-id batch
                ++bid_batch;
                bid_cur = bid_next;
                bid_next = load_group_blocks(P, btrow, bid_batch + 1, k_hi, lane);
            }
            issue_tile<W>(P, ring + (tn % R) * kTileBytes, bid_cur, bid_batch, kh, tn, k_hi, wave, lane);
        }
        const unsigned char* buf = ring + (t % R) * kTileBytes;

        // K fragments: lane (r, p) of key group kg = key 16 kg + r; step s covers d = 16p + 8s
        // (s < 2) / 64 + 16p + 8(s - 2): chunk (s >> 1) * 4 + p, half s & 1.
        u32x4_t kf[2][4];
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) {
            const int row = 16 * kg + lr;
            const unsigned char* kb = buf + (row >> 3) * 1024;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const u32x2_t raw = *reinterpret_cast<const u32x2_t*>(
                    kb + 16 * k_slot(row & 7, (st >> 1) * 4 + lp) + 8 * (st & 1));
                kf[kg][st] = __builtin_bit_cast(u32x4_t, fp8x8_to_bf16x8(raw[0], raw[1]));
            }
        }
        // S^T for every row-set first (K fragments then die), softmax and P.V after.
        f32x4_t sc[RS][2];
        bool live[RS];
#pragma unroll
        for (int j = 0; j < RS; ++j) {
            const int r = wave + W * j;
            const int qpos0 = q0 + 16 * block_of(r / gqa);
            live[j] = r < nrs && k0 <= qpos0 + 15;                // else: tile above the diagonal
            if (!live[j]) continue;
#pragma unroll
            for (int kg = 0; kg < 2; ++kg) {
                f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    acc = mfma16x16x32_bf16(as_bf16x8(kf[kg][st]), as_bf16x8(qf[j][st]), acc);
                sc[j][kg] = acc;
            }
        }
        // V^T fragments: lane (c, p) transposes d = 8c .. 8c+7 of its k-slot tokens.
        u32x4_t vf[8];
        {
            u32x2_t vr[8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int row = (jj < 4 ? 0 : 16) + 4 * lp + (jj & 3);
                const unsigned char* vb = buf + 4096 + (row >> 3) * 1024;
                vr[jj] = *reinterpret_cast<const u32x2_t*>(vb + 16 * v_slot(row & 7, lr >> 1) + 8 * (lr & 1));
            }
            v_fragments(vr, vf);
        }
#pragma unroll
        for (int j = 0; j < RS; ++j) {
            if (!live[j]) continue;
            const int r = wave + W * j;
            const int qpos0 = q0 + 16 * block_of(r / gqa);
            float mc = neg_inf();
            if (k0 + kBN - 1 <= qpos0) {
#pragma unroll
                for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        sc[j][kg][i] *= qk_scale;
                        mc = fmaxf(mc, sc[j][kg][i]);
                    }
            } else {
                const int qpos = qpos0 + lr;
#pragma unroll
                for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int key = k0 + 16 * kg + 4 * lp + i;
                        const float x = key <= qpos ? sc[j][kg][i] * qk_scale : neg_inf();
                        sc[j][kg][i] = x;
                        mc = fmaxf(mc, x);
                    }
            }
            // Lazy rescale: the accumulators move to a new reference max only when the row max
            // grew by more than kRescaleSlack (then probabilities stay below 2^kRescaleSlack).
            // Some lane of a row has its own max above the threshold exactly when the row max
            // is, so the reduction across the row's four lane groups runs only in the branch.
            if (__any(mc > m_run[j] + kRescaleSlack)) {
                mc = max_xor16_32(mc);
                const bool need = mc > m_run[j] + kRescaleSlack;
                const float m_new = need ? mc : m_run[j];
                const float alpha = __builtin_amdgcn_exp2f(m_run[j] - (m_new == neg_inf() ? 0.f : m_new));
                l_run[j] *= alpha;
#pragma unroll
                for (int n = 0; n < 8; ++n) o[j][n] *= alpha;
                m_run[j] = m_new;
            }
            const float m_use = m_run[j] == neg_inf() ? 0.f : m_run[j];
            float psum = 0.f;
#pragma unroll
            for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pv = __builtin_amdgcn_exp2f(sc[j][kg][i] - m_use);
                    sc[j][kg][i] = pv;
                    psum += pv;
                }
            l_run[j] += psum;
            u32x4_t pb;
            pb[0] = pack_bf16x2(sc[j][0][0], sc[j][0][1]);
            pb[1] = pack_bf16x2(sc[j][0][2], sc[j][0][3]);
            pb[2] = pack_bf16x2(sc[j][1][0], sc[j][1][1]);
            pb[3] = pack_bf16x2(sc[j][1][2], sc[j][1][3]);
#pragma unroll
            for (int n = 0; n < 8; ++n) o[j][n] = mfma16x16x32_bf16(as_bf16x8(vf[n]), as_bf16x8(pb), o[j][n]);
        }
    }

    // ---- normalise and store: lane (q, p) holds d = 32p + 8i + n of query row q ------------------
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        const int r = wave + W * j;
        float l = l_run[j];
        l = sum_xor16_32(l);
        if (r >= nrs) continue;
        const int g = r % gqa, b = r / gqa;
        const int tok = 16 * block_of(b) + lr;
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

// ---- key-split kernel ---------------------------------------------------------------------------
// For a GQA that splits into NG groups of RS heads (gqa = NG * RS, RS row-sets per wave): a
// workgroup of 8 waves owns the pair of 16-token blocks (r, n16 - 1 - r) of one kv head and
// processes them one after the other, the longer first.  For one block, wave w takes head group
// w / NR and, of every window of NR x TPW key tiles (NR = 8 / NG), the TPW tiles of residue
// w % NR: every wave converts each of its tiles once for RS row-sets, and two waves share each
// SIMD.  The ring holds two windows; window i + 1 is copied (each wave issuing one 1 KB copy of
// every tile) while window i is consumed, and one barrier per window publishes it.  At the end
// of a block the NR partial (m, l, o) states of each head group merge in LDS in a fixed order:
// the common max first, then residue 0 stores its rescaled o and l, residues 1 .. NR - 2 add
// theirs in turn, and residue NR - 1 adds its own in registers, normalises and writes the output.
constexpr int kSplitWaves = 8;

constexpr int kStageFloats = 8 * 64 * 4 + 64;        // one row-set: o [n][lane][4], then l [lane]

// Running-max floor of the key-split kernel: finite, so that no -inf ever enters the softmax
// arithmetic (exp2(kMaxFloor - m) is 0 for any real row max m, and a row that has seen no key
// keeps l = 0 and o = 0).
constexpr float kMaxFloor = -1e30f;

// max without the NaN-quieting canonicalisation the compiler adds to fmaxf of values that come
// from MFMA results or lane swaps (the scores are never NaN: finite fp8 and bf16 inputs).
__device__ __forceinline__ float max_raw(float a, float b)
{
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float max3_raw(float a, float b, float c)
{
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float max_xor16_32_raw(float v)
{
    const uint32_t b = __float_as_uint(v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const float m = max_raw(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const uint32_t c = __float_as_uint(m);
    const auto r32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
    return max_raw(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// Online softmax and P.V of the RS row-sets of one 32-key tile.  sc holds raw scores S^T
// (lane (q, p): keys 16 kg + 4 p + e of query row q), -inf where masked; qkr[j] = this lane's
// query row's factor from raw score to log2 units (|sm_scale * k_scale| * log2(e) over the row's
// Q scale, positive: a negative scale is folded into Q's sign), so the row max of the raw scores
// times it is the max of the scaled ones and each probability is exp2(fma(s, qk, -m)).  m_run
// starts at kMaxFloor.  vf holds the tile's widened V^T fragments; o[j] += V^T.P^T with P in bf16.
//
// Lazy rescale: the accumulators move to a new reference max only when the row max grew by
// more than kRescaleSlack (then probabilities stay below 2^kRescaleSlack).  qk > 0, so some lane
// of a row has (its own max) * qk above m_run + kRescaleSlack exactly when the row max does: the
// common path tests each lane's own maximum, and only the rescale branch reduces across the row's
// four lane groups.  The branch covers all row-sets (rows that need no rescale get
// alpha = exp2(0) = 1, exact), so the exponentials of row-set j and the P.V MFMAs of row-set
// j - 1 sit in one basic block and interleave.
template <int RS>
__device__ __forceinline__ void softmax_pv_tile(const f32x4_t (&sc)[RS][2], float (&m_run)[RS],
                                                float (&l_run)[RS], f32x4_t (&o)[RS][8],
                                                const float (&qkr)[RS], const u32x4_t (&vf)[8])
{
    float m8[RS];
    bool any_need = false;
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        float m = max3_raw(sc[j][0][0], sc[j][0][1], sc[j][0][2]);
        m = max3_raw(m, sc[j][0][3], sc[j][1][0]);
        m = max3_raw(m, sc[j][1][1], sc[j][1][2]);
        m8[j] = max_raw(m, sc[j][1][3]);
        any_need |= m8[j] * qkr[j] > m_run[j] + kRescaleSlack;
    }
    if (__any(any_need)) {
#pragma unroll
        for (int j = 0; j < RS; ++j) {
            const float mc = max_xor16_32_raw(m8[j]) * qkr[j];    // -inf for a fully masked row
            const bool need = mc > m_run[j] + kRescaleSlack;
            const float m_new = need ? mc : m_run[j];
            const float alpha = __builtin_amdgcn_exp2f(m_run[j] - m_new);
            l_run[j] *= alpha;
#pragma unroll
            for (int n = 0; n < 8; ++n) o[j][n] *= alpha;
            m_run[j] = m_new;
        }
    }
#pragma unroll
    for (int j = 0; j < RS; ++j) {
        const float qk = qkr[j];
        const float nm = -m_run[j];
        float p[2][4];
#pragma unroll
        for (int kg = 0; kg < 2; ++kg)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                p[kg][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][kg][e], qk, nm));
        l_run[j] += ((p[0][0] + p[0][1]) + (p[0][2] + p[0][3])) + ((p[1][0] + p[1][1]) + (p[1][2] + p[1][3]));
        u32x4_t pb;
        pb[0] = pack_bf16x2(p[0][0], p[0][1]);
        pb[1] = pack_bf16x2(p[0][2], p[0][3]);
        pb[2] = pack_bf16x2(p[1][0], p[1][1]);
        pb[3] = pack_bf16x2(p[1][2], p[1][3]);
#pragma unroll
        for (int n = 0; n < 8; ++n) o[j][n] = mfma16x16x32_bf16(as_bf16x8(vf[n]), as_bf16x8(pb), o[j][n]);
    }
    // Interleave: the first row-set's exponentials alone, then each P.V MFMA with about three
    // VALU instructions of the next row-set's softmax.
    __builtin_amdgcn_sched_group_barrier(0x002, 28, 0);
#pragma unroll
    for (int g = 0; g < 8 * (RS - 1); ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
    }
}

template <int RS, int NG, int TPW>
__global__ void __launch_bounds__(kSplitWaves * 64)
prefill_split_kernel(Params P)
{
    constexpr int W = kSplitWaves;
    constexpr int RW = 2;                                  // ring windows
    constexpr int NR = W / NG;
    constexpr int NT = NR * TPW;                           // tiles per window
    static_assert(NG * NR == W && RS >= 1 && NT <= 64, "split shape");
    constexpr int kWinBytes = NT * kTileBytes;
    constexpr int kRingBytes = RW * kWinBytes;
    constexpr int kStageBytes = NR > 1 ? NG * RS * kStageFloats * 4 : 0;
    // The merge stage reuses the ring: it is written only after every wave has finished its
    // last tile, and the next block's copies start only after the stage has been read.
    __shared__ __align__(16) unsigned char ring[kRingBytes > kStageBytes ? kRingBytes : kStageBytes];
    __shared__ float stage_m[NR > 1 ? NG * NR * RS * 16 : 4];
    float* const stage = reinterpret_cast<float*>(ring);

    const int lin = blockIdx.x, seq = blockIdx.z;
    int kh, rank;
    if (P.xcd_map) {
        const int xcd = lin & 7, per = 8 / P.hkv;
        kh = xcd % P.hkv;
        rank = (lin >> 3) * per + xcd / P.hkv;
    } else {
        kh = lin % P.hkv;
        rank = lin / P.hkv;
    }
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave / NR;
    const int res = wave % NR;
    const int lr = lane & 15;
    const int lp = lane >> 4;

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
    const int tb = P.ntb_grid - 1 - rank;
    const int nwg = P.paired ? (n16 + 1) >> 1 : n16;              // workgroups this sequence needs
    if (tb < 0 || tb >= nwg || q0 < 0) return;                    // whole workgroup, before any barrier
    const int blk_a = tb, blk_b = P.paired ? n16 - 1 - tb : tb;
    const int nphase = blk_b > blk_a ? 2 : 1;
    const int32_t* btrow = P.bt + (int64_t)seq * P.bt_stride;
    const float qk_signed = P.sm_scale * P.k_scale[0] * kLog2e;
    const float qk = fmaxf(fabsf(qk_signed), 1e-30f);         // > 0: -inf * qk stays -inf
    const uint32_t qflip = qk_signed < 0.f ? 0x80808080u : 0u;   // negate Q (exact in e4m3)
    const float vs = P.v_scale[0];

    // This wave's copy instruction of every tile: K rows (waves 0-3) or V rows (waves 4-7)
    // 8 (wave & 3) .. +7, lane (row, chunk) as chosen by dma_lane_rc.
    const bool dma_v = wave >= 4;
    int dma_r, dma_c;
    dma_lane_rc(dma_v, lane, dma_r, dma_c);
    const int dma_rk = 8 * (wave & 3) + dma_r;                     // key offset within a tile
    const uint8_t* dma_base = dma_v ? P.v + (int64_t)kh * P.sv2 : P.k + (int64_t)kh * P.sk2;
    const int64_t dma_s0 = dma_v ? P.sv0 : P.sk0;
    const uint32_t dma_s1 = (uint32_t)(dma_v ? P.sv1 : P.sk1);    // < 2^32 / block size (host check)
    const uint32_t dma_chunk = 16u * (uint32_t)dma_c;
    // The wave's 8 rows start at a multiple of 8 and the block size is a power of two >= 16, so
    // the slot of key 32 t + dma_rk is (32 t + 8 (wave & 3)) mod block size (wave-uniform, folded
    // into the scalar base) plus dma_r (this lane's fixed offset).
    const int dma_row0 = 8 * __builtin_amdgcn_readfirstlane(wave & 3);
    const uint32_t voff_lane = (uint32_t)dma_r * dma_s1 + dma_chunk;

    for (int ph = 0; ph < nphase; ++ph) {
        const int blk = ph == 0 ? blk_b : blk_a;
        const int qpos0 = q0 + 16 * blk;
        const int k_hi = q0 + min(16 * blk + 16, qlen);           // keys [0, k_hi)
        const int ntiles = (k_hi + kBN - 1) / kBN;
        const int nwin = (ntiles + NT - 1) / NT;

        // Q as the fp8 B operand of S^T = K.Q^T (lane (n, p): d 16p .. 16p+15 and 64+16p .. +15
        // of query row n), split exactly into e4m3 hi + lo parts (q_fp8_split), with the row's
        // scale folded into this lane's softmax factor qkr.
        v8i qhi[RS], qlo[RS];
        float qkr[RS];
        const int tok = 16 * blk + lr;
        const bool tok_ok = tok < qlen;
#pragma unroll
        for (int j = 0; j < RS; ++j) {
            const u32x4_t zero = {0u, 0u, 0u, 0u};
            const __bf16* qrow = P.q + (int64_t)(q_begin + (tok_ok ? tok : 0)) * P.q_stride +
                                 (int64_t)(kh * P.gqa + grp * RS + j) * kD;
            u32x4_t qf[4];
            qf[0] = tok_ok ? load_16(qrow + 16 * lp) : zero;
            qf[1] = tok_ok ? load_16(qrow + 16 * lp + 8) : zero;
            qf[2] = tok_ok ? load_16(qrow + 64 + 16 * lp) : zero;
            qf[3] = tok_ok ? load_16(qrow + 64 + 16 * lp + 8) : zero;
            qkr[j] = qk * q_fp8_split(qf, qflip, qhi[j], qlo[j]);
        }

        // Block ids for this wave's copy instruction of each tile of window wi (its 8 rows lie
        // in one 16-key group, hence one cache block; index clamped to the last key): lane u
        // loads the id for tile u of the window, one window ahead of the copies.  With a ring of
        // two windows the wait for window i's copies also covers this load (issued after them).
        int bids = 0;
        auto load_bids = [&](int wi) {
            const int key0 = min((wi * NT + lane) * kBN + 8 * (wave & 3), k_hi - 1);
            bids = lane < NT ? btrow[key0 >> P.pshift] : 0;
        };
        // Copies of tiles u0 .. u1 - 1 of window wi (keys >= k_hi fetch key k_hi - 1; the causal
        // mask removes them).
        auto issue_window = [&](int wi, int u0, int u1) {
#pragma unroll
            for (int u = u0; u < u1; ++u) {
                const int t = wi * NT + u;
                if (t < ntiles) {
                    const int64_t b = __builtin_amdgcn_readlane(bids, u);
                    const uint8_t* sb = dma_base + b * dma_s0;
                    uint32_t voff = voff_lane;
                    if (t * kBN + kBN > k_hi) {             // the tile holding the end of the keys
                        const int key = min(t * kBN + dma_rk, k_hi - 1);
                        voff = (uint32_t)(key & (P.pblk - 1)) * dma_s1 + dma_chunk;
                    } else {
                        sb += (uint32_t)((t * kBN + dma_row0) & (P.pblk - 1)) * dma_s1;
                    }
                    dma16_saddr(sb, voff, ring + (wi % RW) * kWinBytes + u * kTileBytes + wave * 1024);
                }
            }
        };
#pragma unroll
        for (int wi = 0; wi < RW - 1; ++wi)
            if (wi < nwin) {
                load_bids(wi);
                issue_window(wi, 0, NT);
            }
        if (RW - 1 < nwin) load_bids(RW - 1);

        float m_run[RS], l_run[RS];
        f32x4_t o[RS][8];
#pragma unroll
        for (int j = 0; j < RS; ++j) {
            m_run[j] = kMaxFloor;
            l_run[j] = 0.f;
#pragma unroll
            for (int n = 0; n < 8; ++n) o[j][n] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
        }

        for (int i = 0; i < nwin; ++i) {
            // Everything this wave has in flight: window i's copies and the block ids of window
            // i + 1.  The barrier then publishes window i and frees window i - 1's slot.
            wait_vmcnt<0>();
            lds_barrier();
            const bool more = i + RW - 1 < nwin;

#pragma unroll
            for (int v = 0; v < TPW; ++v) {
                // The next window's copies go out in TPW parts, one before each tile, so that the
                // copy traffic of the eight waves spreads over the window instead of queueing
                // behind the barrier.
                if (more) issue_window(i + RW - 1, v * NT / TPW, (v + 1) * NT / TPW);
                const int tw = res * TPW + v;                    // tile within the window
                const int t = i * NT + tw;
                if (t >= ntiles) continue;
                const int k0 = t * kBN;
                const unsigned char* buf = ring + (i % RW) * kWinBytes + tw * kTileBytes;

                // K as the fp8 A operand, straight from the ring: lane (r, p) = key 16 kg + r,
                // d 16p .. 16p+15 (chunk p) and 64+16p .. +15 (chunk 4 + p).
                v8i kf[2];
#pragma unroll
                for (int kg = 0; kg < 2; ++kg) {
                    const int row = 16 * kg + lr;
                    const unsigned char* kb = buf + (row >> 3) * 1024;
                    const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(kb + 16 * k_slot(row & 7, lp));
                    const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(kb + 16 * k_slot(row & 7, 4 + lp));
                    kf[kg] = (v8i){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                                   (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
                }
                // V^T raw rows (lane (c, p) transposes d = 8c .. 8c+7) and their widening go ahead
                // of S^T = K.Q^T, so the VALU work can run between the MFMAs.
                u32x2_t vr[8];
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int row = (jj < 4 ? 0 : 16) + 4 * lp + (jj & 3);
                    const unsigned char* vb = buf + 4096 + (row >> 3) * 1024;
                    vr[jj] = *reinterpret_cast<const u32x2_t*>(vb + 16 * v_slot(row & 7, lr >> 1) + 8 * (lr & 1));
                }
                u32x4_t vf[8];
                v_fragments(vr, vf);
                f32x4_t sc[RS][2];
#pragma unroll
                for (int j = 0; j < RS; ++j)
#pragma unroll
                    for (int kg = 0; kg < 2; ++kg) {
                        const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
                        f32x4_t acc = mfma_fp8_16x16x128(kf[kg], qhi[j], zero);
                        sc[j][kg] = mfma_fp8_16x16x128(kf[kg], qlo[j], acc);
                    }
                // Interleave: one MFMA, then up to four VALU (the V widening, 48 instructions).
#pragma unroll
                for (int g = 0; g < 4 * RS; ++g) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                }
                if (k0 + kBN - 1 > qpos0) {                        // tile reaches past the first row
                    const int qpos = qpos0 + lr;
#pragma unroll
                    for (int j = 0; j < RS; ++j)
#pragma unroll
                        for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (k0 + 16 * kg + 4 * lp + e > qpos) sc[j][kg][e] = neg_inf();
                }
                softmax_pv_tile<RS>(sc, m_run, l_run, o, qkr, vf);
            }
            // Block ids for the next window's copies, after this iteration's LDS reads so that
            // no LDS wait in the tile work has to cover the scalar loads.
            if (i + RW < nwin) load_bids(i + RW);
        }

        // ---- merge the NR partial states of each head group, then normalise and store ----------
        if constexpr (NR > 1) {
            // m_run is the same in the four lane groups of a query row: lanes 0..15 publish it.
            if (lp == 0) {
#pragma unroll
                for (int j = 0; j < RS; ++j) stage_m[((grp * NR + res) * RS + j) * 16 + lr] = m_run[j];
            }
            lds_barrier();
#pragma unroll
            for (int j = 0; j < RS; ++j) {
                float mg = kMaxFloor;
#pragma unroll
                for (int r = 0; r < NR; ++r) mg = fmaxf(mg, stage_m[((grp * NR + r) * RS + j) * 16 + lr]);
                const float f = __builtin_amdgcn_exp2f(m_run[j] - mg);
                l_run[j] *= f;
#pragma unroll
                for (int n = 0; n < 8; ++n) o[j][n] *= f;
            }
            for (int r = 0; r < NR - 1; ++r) {
                if (res == r) {
#pragma unroll
                    for (int j = 0; j < RS; ++j) {
                        float* s = stage + (grp * RS + j) * kStageFloats;
#pragma unroll
                        for (int n = 0; n < 8; ++n) {
                            f32x4_t* p = reinterpret_cast<f32x4_t*>(s + (n * 64 + lane) * 4);
                            if (r > 0) o[j][n] += *p;
                            *p = o[j][n];
                        }
                        if (r > 0) l_run[j] += s[8 * 64 * 4 + lane];
                        s[8 * 64 * 4 + lane] = l_run[j];
                    }
                }
                lds_barrier();
            }
            if (res == NR - 1) {
#pragma unroll
                for (int j = 0; j < RS; ++j) {
                    const float* s = stage + (grp * RS + j) * kStageFloats;
#pragma unroll
                    for (int n = 0; n < 8; ++n) o[j][n] += *reinterpret_cast<const f32x4_t*>(s + (n * 64 + lane) * 4);
                    l_run[j] += s[8 * 64 * 4 + lane];
                }
            }
        }
        if (res == NR - 1) {
#pragma unroll
            for (int j = 0; j < RS; ++j) {
                const float l = sum_xor16_32(l_run[j]);
                if (!tok_ok) continue;
                const float f = l > 0.f ? vs / l : 0.f;
                __bf16* orow = P.out + (int64_t)(q_begin + tok) * P.o_stride +
                               (int64_t)(kh * P.gqa + grp * RS + j) * kD + 32 * lp;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    u32x4_t w;
                    w[0] = pack_bf16x2(o[j][0][e] * f, o[j][1][e] * f);
                    w[1] = pack_bf16x2(o[j][2][e] * f, o[j][3][e] * f);
                    w[2] = pack_bf16x2(o[j][4][e] * f, o[j][5][e] * f);
                    w[3] = pack_bf16x2(o[j][6][e] * f, o[j][7][e] * f);
                    *reinterpret_cast<u32x4_t*>(orow + 8 * e) = w;
                }
            }
        }
        // The next block's copies overwrite the ring, which holds the stage: every wave must be
        // done with its final stage reads above.
        if (ph + 1 < nphase) lds_barrier();
    }
}

// Launch shapes: (waves, row-sets per wave, ring depth).  nb token blocks of 16 per workgroup is
// the largest count whose nb * GQA row-sets fit waves * RS.
struct Shape {
    int waves, rs, ring, paired;
};
constexpr Shape kShapes[] = {{4, 3, 4, 0}, {4, 3, 6, 0}, {8, 2, 4, 0}, {4, 4, 4, 0}, {4, 2, 4, 0},
                             {4, 1, 4, 0}, {6, 2, 4, 1}, {8, 2, 4, 1}};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);

// Key-split shapes (RS row-sets per wave, NG head groups) for gqa = RS * NG.
struct SplitShape {
    int rs, ng;
};
constexpr SplitShape kSplitShapes[] = {{3, 2}, {3, 4}, {2, 2}, {2, 4}, {2, 8}};
constexpr int kNumSplitShapes = sizeof(kSplitShapes) / sizeof(kSplitShapes[0]);
// -1: choose by GQA; kNumShapes + s: key-split shape s; kNumShapes + kNumSplitShapes + s: the
// same with paired token blocks whatever the grid size.
thread_local int g_shape = -1;

inline int split_shape_for(int gqa)
{
    for (int s = 0; s < kNumSplitShapes; ++s)
        if (kSplitShapes[s].rs * kSplitShapes[s].ng == gqa) return s;
    return -1;
}

// Default shape per GQA (measured at configs[3], GQA 6: 8 waves x 2 row-sets with paired token
// blocks 184 us; 4 x 3 unpaired 251 us; 8 x 2 unpaired 190 us).
inline int choose_shape(int gqa)
{
    if (g_shape >= 0 && g_shape < kNumShapes) return g_shape;
    if (gqa <= 1) return 5;                       // 4 waves x 1 row-set, 4 token blocks
    if (gqa <= 2) return 4;                       // 4 waves x 2 row-sets, 4 token blocks
    if (gqa <= 8) return 7;                       // 8 waves x 2 row-sets (paired blocks when nb = 2)
    return 3;                                     // 4 waves x 4 row-sets
}

inline int plan_nb(int gqa, const Shape& s)
{
    int nb = (s.waves * s.rs) / gqa;
    if (nb < 1) nb = 1;
    if (nb > 4) nb = 4;
    return nb;
}

// Workgroups of the key-split kernel resident at once on a gfx950 part (256 CUs, one each).
constexpr int kSplitRoundWorkgroups = 256;

// Token-block ranks per (sequence, kv head) padded for the XCD-aware grid (8 % HKV == 0).
inline int split_xcd_per(int hkv) { return (hkv <= 8 && 8 % hkv == 0) ? 8 / hkv : 1; }

// True when one 16-token block per workgroup fits in one round of the key-split kernel.
inline bool split_single_blocks_fit(int n16, int hkv, int num_seqs)
{
    const int per = split_xcd_per(hkv);
    return (int64_t)((n16 + per - 1) / per * per) * hkv * num_seqs <= kSplitRoundWorkgroups;
}

// Contexts (in keys) from which the key-split kernel beats the per-wave kernel, measured on MI355X
// at GQA 6.  With paired blocks: 1024 (512 new tokens after 512 cached 42.8 vs 45.6 us, 512
// tokens alone 28.0 vs 24.4 us; 4 sequences of 512 32.0 vs 27.3 us).  With one block per
// workgroup (the grid fits one round): 256 (512 tokens alone 17.4 vs 23.8 us, 1000 alone 24.7 vs
// 42.5 us, 64 after 900 22.3 vs 42.3 us, 256 alone 13.6 vs 14.4 us, 128 alone 13.1 vs 9.8 us).
// Below them the split kernel's per-block fixed costs dominate.
constexpr int kSplitMinContext = 1024;
constexpr int kSplitMinContextSingle = 256;

// One launch as planned from the shape alone (no pointers): kernel, block pairing and grid.
struct Plan {
    int split;          // key-split shape index, or -1 for the per-wave kernel
    int shape;          // per-wave kernel shape index (split < 0)
    int nb, paired, xcd_map, ntb_grid;
    dim3 grid, block;
};

// Plans the launch; FP8KV_OK with ntb_grid == 0 means there is nothing to launch.
// ctx_hint: the longest context when the host knows it (single sequence), else the longest query.
int plan_launch(int gqa, int hkv, int num_seqs, int max_query_len, int ctx_hint, Plan& L)
{
    L = Plan{-1, 0, 1, 0, 0, 0, dim3(0u), dim3(0u)};
    const int n16 = (max_query_len + 15) / 16;
    if (n16 == 0) return FP8KV_OK;
    L.xcd_map = (hkv <= 8 && 8 % hkv == 0) ? 1 : 0;
    const int per = split_xcd_per(hkv);                // token-block ranks per kv head per XCD round
    auto round_up = [&](int n) { return (n + per - 1) / per * per; };

    // Key-split kernel when the GQA has a split shape and the context is long enough, unless the
    // tuning hook forces another.
    const int ss = split_shape_for(gqa);
    bool split = false, force_paired = false;
    if (g_shape >= kNumShapes) {
        split = (g_shape - kNumShapes) % kNumSplitShapes == ss;
        force_paired = g_shape >= kNumShapes + kNumSplitShapes;
    } else if (g_shape < 0 && ss >= 0) {
        split = ctx_hint >= kSplitMinContext ||
                (ctx_hint >= kSplitMinContextSingle && split_single_blocks_fit(n16, hkv, num_seqs));
    }
    if (split) {
        // Pairs of token blocks (r, n16 - 1 - r) give every workgroup the same causal work; when
        // one block per workgroup still fits in one round of workgroups (one per CU: the ring
        // takes most of the LDS), single blocks finish sooner (the longest workgroup sees about
        // q0 + qlen keys instead of 2 q0 + qlen; measured at GQA 6: 1024 new tokens after 1024
        // cached 61.3 -> 38.7 us, 512 after 1024 52.6 -> 30.0 us).
        L.split = ss;
        L.nb = 2;
        L.paired = (force_paired || !split_single_blocks_fit(n16, hkv, num_seqs)) ? 1 : 0;
        L.ntb_grid = round_up(L.paired ? (n16 + 1) / 2 : n16);
        L.block = dim3(64 * kSplitWaves);
    } else {
        L.shape = choose_shape(gqa);
        const Shape sh = kShapes[L.shape];
        if (sh.waves * sh.rs < gqa) return FP8KV_ERR_SHAPE;
        L.nb = plan_nb(gqa, sh);
        L.paired = sh.paired && L.nb == 2 ? 1 : 0;
        const int ntb = L.paired ? (n16 + 1) / 2 : (n16 + L.nb - 1) / L.nb;
        L.ntb_grid = L.xcd_map ? (ntb + per - 1) / per * per : ntb;
        L.block = dim3(64 * sh.waves);
    }
    L.grid = dim3((unsigned)(L.ntb_grid * hkv), 1u, (unsigned)num_seqs);
    return FP8KV_OK;
}

int launch(const Params& P0, int num_seqs, int max_query_len, int ctx_hint, hipStream_t stream)
{
    Plan L;
    const int st = plan_launch(P0.gqa, P0.hkv, num_seqs, max_query_len, ctx_hint, L);
    if (st != FP8KV_OK || L.ntb_grid == 0) return st;
    Params P = P0;
    P.nb = L.nb;
    P.paired = L.paired;
    P.xcd_map = L.xcd_map;
    P.ntb_grid = L.ntb_grid;
    begin_launch();
    if (L.split >= 0) {
        switch (L.split) {
            case 0: launch_kernel(prefill_split_kernel<3, 2, 2>, L.grid, L.block, 0, stream, P); break;
            case 1: launch_kernel(prefill_split_kernel<3, 4, 2>, L.grid, L.block, 0, stream, P); break;
            case 2: launch_kernel(prefill_split_kernel<2, 2, 2>, L.grid, L.block, 0, stream, P); break;
            case 3: launch_kernel(prefill_split_kernel<2, 4, 2>, L.grid, L.block, 0, stream, P); break;
            default: launch_kernel(prefill_split_kernel<2, 8, 2>, L.grid, L.block, 0, stream, P); break;
        }
        return finish_launch();
    }
    switch (L.shape) {
        case 0: launch_kernel(prefill_kernel<4, 3, 4>, L.grid, L.block, 0, stream, P); break;
        case 1: launch_kernel(prefill_kernel<4, 3, 6>, L.grid, L.block, 0, stream, P); break;
        case 2: launch_kernel(prefill_kernel<8, 2, 4>, L.grid, L.block, 0, stream, P); break;
        case 3: launch_kernel(prefill_kernel<4, 4, 4>, L.grid, L.block, 0, stream, P); break;
        case 4: launch_kernel(prefill_kernel<4, 2, 4>, L.grid, L.block, 0, stream, P); break;
        case 6: launch_kernel(prefill_kernel<6, 2, 4>, L.grid, L.block, 0, stream, P); break;
        case 7: launch_kernel(prefill_kernel<8, 2, 4>, L.grid, L.block, 0, stream, P); break;
        default: launch_kernel(prefill_kernel<4, 1, 4>, L.grid, L.block, 0, stream, P); break;
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
    if (num_q_heads / num_kv_heads > kMaxGqa) return FP8KV_ERR_SHAPE;
    if (block_size < 16 || (block_size & (block_size - 1)) != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(k_cache, 16) || !aligned(v_cache, 8) || !aligned(q, 16) || !aligned(out, 16))
        return FP8KV_ERR_ALIGN;
    if ((sk0 | sk1 | sk2) & 15) return FP8KV_ERR_ALIGN;
    if ((sv0 | sv1 | sv2) & 7) return FP8KV_ERR_ALIGN;
    if ((q_row_stride & 7) || (out_row_stride & 7)) return FP8KV_ERR_ALIGN;
    // The tile copies address a row within its cache block with a 32-bit offset.
    if (sk1 < 0 || sv1 < 0 || (int64_t)(block_size - 1) * (sk1 > sv1 ? sk1 : sv1) + 128 >= ((int64_t)1 << 32))
        return FP8KV_ERR_SHAPE;
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
    P.pshift = __builtin_ctz((unsigned)block_size);
    P.nb = 1;
    P.paired = 0;
    P.ntb_grid = 0;
    P.xcd_map = 0;
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
    return launch(P, 1, qlen, q0 + qlen, reinterpret_cast<hipStream_t>(stream));
}

extern "C" void fp8kv_prefill_tune(int shape)
{
    g_shape = (shape >= 0 && shape < kNumShapes + 2 * kNumSplitShapes) ? shape : -1;
}

extern "C" int fp8kv_prefill_plan(int num_q_heads, int num_kv_heads, int num_seqs,
                                  int max_query_len, int ctx_hint, int* out)
{
    if (!out || num_q_heads < 1 || num_kv_heads < 1 || num_seqs < 1 || max_query_len < 0)
        return FP8KV_ERR_ARG;
    if (num_q_heads % num_kv_heads != 0 || num_q_heads / num_kv_heads > kMaxGqa)
        return FP8KV_ERR_SHAPE;
    Plan L;
    const int st = plan_launch(num_q_heads / num_kv_heads, num_kv_heads, num_seqs, max_query_len,
                               ctx_hint, L);
    if (st != FP8KV_OK) return st;
    const int v[8] = {L.split >= 0 ? 1 : 0, L.split >= 0 ? L.split : L.shape, L.nb, L.paired,
                      L.ntb_grid, (int)L.grid.x, (int)L.grid.z, (int)L.block.x};
    for (int i = 0; i < 8; ++i) out[i] = v[i];
    return FP8KV_OK;
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
    return launch(P, num_seqs, max_query_len, max_query_len, reinterpret_cast<hipStream_t>(stream));
}
