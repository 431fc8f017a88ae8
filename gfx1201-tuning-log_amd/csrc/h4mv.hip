// MXFP4 W4A16 matvec for gfx950: Out[M,N] = X[M,K] . dequant(W[N,K/2], St[N,K/32])^T.
//
// Reference semantics: h4mv/h4mv.cu:43-104 (layout, e2m1 table, per-32 e8m0 scale,
// fp32 accumulation, bf16 output) and its C ABI h4mv/h4mv.cu:106-122.
//
// gfx950 design (not a translation of the wave-per-row dot2 kernel):
//   * A workgroup owns a 16-row tile of W and runs one v_mfma_f32_16x16x32_bf16 chain per wave;
//     its WAVES waves split K and meet in LDS once at the end (split-K inside the workgroup, so
//     N/16 workgroups of equal size spread evenly over the 256 CUs).
//   * Lane (r, q) = (lane % 16, lane / 16) streams whole 16-byte scale groups of row r: one
//     global_load_dwordx4 = 32 codes = exactly one e8m0 group, so each load needs one scale.
//     The 16 bytes become four MFMA A fragments via v_cvt_scalef32_pk_bf16_fp4, which applies
//     the group scale during the conversion (e2m1 * 2^k is exact in bf16).
//   * K is a reduction index, so the kernel may visit it in any order as long as the A (weights)
//     and B (activations) fragments agree: quad q of the wave handles group g = g0 + 4u + q and
//     fragment j covers k = 32 g + 8 j + (0..7) on both sides.
//   * All weight loads of a chunk of U groups-per-quad are issued before any of them is consumed,
//     and the next chunk is requested before the current one is converted (two register
//     buffers), so each wave keeps U * 1 KB of the weight stream in flight.
//   * X is the B operand: lane (m, q) supplies X[m, 32 g + 8 j .. +8] for m < M and zeros for the
//     padded columns m >= M, so one kernel serves 1 <= M <= 16.  When M*K*2 bytes fit, X is copied
//     to LDS once per workgroup (XLDS) and the fragments come from ds_read_b128; otherwise they are
//     read from global memory, where X stays L2-resident.
//   * Output tile: lane (m, q) register i holds row n0 + 4 q + i of column m, so each lane of the
//     first wave writes 4 consecutive outputs of Out[m, :].
#include "fp8kv_common.h"
#include "fp8kv_status.h"
#include "fp8kv_diag.h"
#include <algorithm>
#include <utility>
#include <vector>

namespace fp8kv {

thread_local int g_last_status = FP8KV_OK;
thread_local int g_last_hip_error = 0;
thread_local hipEvent_t g_time_start = nullptr;
thread_local hipEvent_t g_time_stop = nullptr;

namespace h4mv_detail {

constexpr int kRowsPerWG = 16;
constexpr int kXLdsMaxBytes = 64 * 1024;

template <int U>
struct Chunk {
    u32x4_t w[U];
    uint32_t s[U];
};

template <int U>
__device__ __forceinline__ void load_chunk(Chunk<U>& c, const uint8_t* wrow, const uint8_t* srow,
                                           int g0, int q, int g_end, bool row_ok)
{
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = g0 + 4 * u + q;
        const bool ok = row_ok && g < g_end;
        const u32x4_t zero = {0u, 0u, 0u, 0u};
        c.w[u] = ok ? load_nt_16(wrow + (size_t)g * 16) : zero;
        c.s[u] = ok ? (uint32_t)srow[g] : 127u;
    }
}

template <int U, bool XLDS>
__device__ __forceinline__ f32x4_t consume_chunk(const Chunk<U>& c, f32x4_t acc, const __bf16* xsrc,
                                                 int g0, int q, int g_end, bool col_ok)
{
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = g0 + 4 * u + q;
        const bool ok = col_ok && g < g_end;
        const float sc = e8m0_to_f32(c.s[u]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4_t zero = {0u, 0u, 0u, 0u};
            const u32x4_t xv = ok ? load_16(xsrc + (size_t)g * 32 + 8 * j) : zero;
            acc = mfma16x16x32_bf16(fp4x8_to_bf16x8(c.w[u][j], sc), as_bf16x8(xv), acc);
        }
    }
    return acc;
}

template <int WAVES, int U, bool XLDS, typename OutT>
__global__ void __launch_bounds__(WAVES * 64)
h4mv_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ St,
            const __bf16* __restrict__ X, OutT* __restrict__ Out,
            int N, int K, int M, int groups_per_wave)
{
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ f32x4_t red[WAVES > 1 ? WAVES - 1 : 1][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;        // weight row within the tile / activation column m
    const int q = lane >> 4;        // which of 4 consecutive scale groups this lane streams
    const int G = K >> 5;           // scale groups per row
    const int n0 = blockIdx.x * kRowsPerWG;
    const int row = n0 + r;
    const bool row_ok = row < N;
    const bool col_ok = r < M;

    const int g_begin = wave * groups_per_wave;
    const int g_end = min(G, g_begin + groups_per_wave);

    const uint8_t* wrow = W + (size_t)(row_ok ? row : 0) * (size_t)(K >> 1);
    const uint8_t* srow = St + (size_t)(row_ok ? row : 0) * (size_t)G;

    // Weight stream first: the first chunk is in flight while X is staged.
    Chunk<U> ca, cb;
    load_chunk<U>(ca, wrow, srow, g_begin, q, g_end, row_ok);

    const __bf16* xsrc;
    if constexpr (XLDS) {
        __bf16* xl = reinterpret_cast<__bf16*>(smem);
        const int n16 = (M * K) >> 3;                   // 16-byte pieces of X
        for (int i = threadIdx.x; i < n16; i += WAVES * 64)
            *reinterpret_cast<u32x4_t*>(xl + 8 * i) = load_16(X + 8 * i);
        __syncthreads();
        xsrc = xl + (size_t)(col_ok ? r : 0) * (size_t)K;
    } else {
        xsrc = X + (size_t)(col_ok ? r : 0) * (size_t)K;
    }

    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    int g0 = g_begin;
    while (g0 < g_end) {
        const int g1 = g0 + 4 * U;
        if (g1 < g_end) load_chunk<U>(cb, wrow, srow, g1, q, g_end, row_ok);
        acc = consume_chunk<U, XLDS>(ca, acc, xsrc, g0, q, g_end, col_ok);
        if (g1 >= g_end) break;
        const int g2 = g1 + 4 * U;
        if (g2 < g_end) load_chunk<U>(ca, wrow, srow, g2, q, g_end, row_ok);
        acc = consume_chunk<U, XLDS>(cb, acc, xsrc, g1, q, g_end, col_ok);
        g0 = g2;
    }

    if constexpr (WAVES > 1) {
        if (wave > 0) red[wave - 1][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int w = 0; w < WAVES - 1; ++w) acc += red[w][lane];
    }

    const int m = r;
    if (m >= M) return;
    const int n = n0 + 4 * q;
    OutT* orow = Out + (size_t)m * (size_t)N;
    const bool vec = n + 3 < N && ((N & 3) == 0) && aligned(Out, 4 * sizeof(OutT));
    if constexpr (sizeof(OutT) == 2) {
        if (vec) {
            u32x2_t v = {pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
            *reinterpret_cast<u32x2_t*>(orow + n) = v;
            return;
        }
    } else {
        if (vec) {
            *reinterpret_cast<f32x4_t*>(orow + n) = acc;
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (n + i < N) orow[n + i] = (OutT)acc[i];
}

// ---------------------------------------------------------------------------------------------
// Streaming kernel for K % 512 == 0 (every shape of the target model).
//
// The MFMA A layout pins lane (r, q) to weight row r, so direct per-lane loads would make adjacent
// lanes read rows K/2 bytes apart (measured: 4.9 TB/s read-only ceiling for that pattern, versus
// 6.1 TB/s for coalesced reads).  Instead each wave copies its share of the 16-row tile into LDS
// with coalesced global_load_lds_dwordx4 and reads MFMA fragments back with ds_read_b128.
//   * step = 16 scale groups (256 B) of each of the 16 rows = 4 KB of codes;
//   * a workgroup owns one tile and has NW waves; wave w owns the contiguous steps
//     [w * per, w * per + per) and streams their codes through a DEPTH-slot LDS ring: a slot is
//     refilled as soon as its fragments are in registers, before they are converted and multiplied;
//   * the wave's scale bytes (16 rows x per x 16 B) are copied once at the start, row by row, so
//     consecutive lanes read consecutive bytes (per-step 16-byte scale pieces from 16 rows cost a
//     measured 1 us per launch at cfg1);
//   * activations: each slot carries MMAX KB of activation rows next to its codes; alternatively
//     (XG, a tuning option, measured slower) every lane loads its activation fragments for step
//     s + 1 straight from L2 into registers at the end of step s;
//   * the waves of the workgroup meet once in LDS to add their partial tiles;
//   * LDS code layout: row r at 256 r, 16-byte piece p at slot p ^ (r & 7), so the 16 lanes that
//     read one piece index of 16 rows hit distinct bank groups;
//   * copies complete out of the compiler's sight, so every wait is an explicit s_waitcnt vmcnt
//     with the exact number of copy instructions still allowed in flight;
//   * columns m >= M of the B operand only feed output columns that are never stored, so lanes
//     r >= M do not read activations from LDS (XG: they load row M - 1 again, so every wave issues
//     the same number of loads per step and the explicit vmcnt counts stay exact).
// ---------------------------------------------------------------------------------------------
constexpr int kStepGroups = 16;
constexpr int kStepCodeBytes = 16 * 256;
constexpr int kXgLoads = 16;                 // XG: activation fragment loads per step and lane
constexpr int kDmaAux = 2;                    // streaming cache policy for the code copies
// Copies read once per launch take the streaming policy too: lines left in L2 by ordinary loads
// add to the gap between consecutive launches (measured under graph replay: the M = 1 kernel's
// 3.7 MB of scale slices, copied with the default policy, cost it 0.2-0.3 us per launch there).
// Not for the K-slice kernels' scale copies: their waves share each scale line through L2 (with
// the streaming policy cfg1 M = 4 / 8 went 12.6 -> 13.7 / 13.0 -> 14.4 us).
__device__ __forceinline__ void dma16_to_lds_stream(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_base, 16, 0, kDmaAux);
}

// LDS layout of one wave (bytes), shared by kernel, planner and audit.
struct WaveLds {
    int slot;        // bytes per ring slot
    int ring;        // DEPTH * slot
    int scales;      // 16 rt rows * per * 16
    int total;
};

__host__ __device__ inline WaveLds wave_lds(int mmax, bool xg, int depth, int per, int rt)
{
    WaveLds w;
    w.slot = rt * kStepCodeBytes + (xg ? 0 : mmax * 1024);
    w.ring = depth * w.slot;
    w.scales = 16 * rt * per * 16;
    w.total = w.ring + w.scales;
    return w;
}

// ---- index math shared by the kernel and the host-side address audit --------------------------
// Code copy instruction i (0 .. 4 rt - 1) of a step: lane -> row 4 i + lane / 16 of the
// workgroup's 16 rt rows (clamped to N - 1) and the 16-byte piece (lane % 16) ^ (row & 7); byte
// offset from the workgroup's first code byte.  Instruction i lands at 1024 i in the slot, so
// row-tile t of the workgroup occupies bytes [4096 t, 4096 t + 4096) of it.
__host__ __device__ inline uint32_t stream_w_lane_off(int n0, int N, int K, int lane, int i)
{
    const int rr = 4 * i + (lane >> 4);
    const int rowc = (n0 + rr < N ? n0 + rr : N - 1) - n0;
    return (uint32_t)rowc * (uint32_t)(K >> 1) + 16u * (uint32_t)((lane & 15) ^ (rr & 7));
}
// Scale copy: segment t (0 .. 16 rt per - 1) = row t / per, step t % per of the wave's slice;
// byte offset from St.  Segment t lands at 16 t in the wave's scale area.
__host__ __device__ inline size_t stream_s_seg_off(int n0, int N, int K, int per, int step0, int t)
{
    const int row = t / per, st = t % per;
    const int rowc = n0 + row < N ? n0 + row : N - 1;
    return (size_t)rowc * (size_t)(K >> 5) + (size_t)(step0 + st) * kStepGroups;
}
// Activation copy of row m (clamped to M - 1) for step gs (first group) and lane: offset from X.
__host__ __device__ inline size_t stream_x_off(int K, int M, int m, int gs, int lane)
{
    const int mm = m < M ? m : M - 1;
    return (size_t)mm * (size_t)K * 2 + (size_t)gs * 64 + 16u * (uint32_t)lane;
}
// LDS read offsets: codes of group q + 4u of row r within a slot; activation fragment (u, j) of
// row r within one 1 KB step block.
__host__ __device__ inline int stream_w_read_off(int r, int q, int u) { return 256 * r + 16 * ((q + 4 * u) ^ (r & 7)); }
__host__ __device__ inline int stream_x_frag_off(int q, int u, int j) { return q * 64 + u * 256 + j * 16; }

template <int MMAX, bool XG, int RT>
constexpr int copies_per_step() { return 4 * RT + (XG ? 0 : MMAX); }

// Wait until the oldest outstanding step has landed, leaving `ahead` younger steps in flight (and,
// with XG, the activation loads of the current step, issued after all of them).
template <int MMAX, bool XG, int RT, int A>
__device__ __forceinline__ void wait_ahead_ct(int ahead)
{
    constexpr int extra = XG ? kXgLoads : 0;
    if constexpr (A == 0) {
        wait_vmcnt<extra>();
    } else {
        if (ahead >= A) wait_vmcnt<A * copies_per_step<MMAX, XG, RT>() + extra>();
        else wait_ahead_ct<MMAX, XG, RT, A - 1>(ahead);
    }
}

template <int MMAX, bool XG, int RT>
__device__ __forceinline__ void issue_step(unsigned char* slot, const uint8_t* wtile,
                                           const unsigned char* xbytes, const uint32_t (&woff)[4 * RT],
                                           int gs, int K, int M, int lane)
{
#pragma unroll
    for (int i = 0; i < 4 * RT; ++i)
        __builtin_amdgcn_global_load_lds((const void*)(wtile + (size_t)gs * 16 + woff[i]),
                                         (lds_void_t*)(slot + i * 1024), 16, 0, kDmaAux);
    if constexpr (!XG) {
#pragma unroll
        for (int m = 0; m < MMAX; ++m)
            dma16_to_lds(xbytes + stream_x_off(K, M, m, gs, lane), slot + RT * kStepCodeBytes + m * 1024);
    }
}

// Several row tiles per workgroup need more registers than 16 waves per workgroup allow (128),
// so those variants are launched with at most kMaxWavesRT waves.
constexpr int kMaxWavesRT = 4;

// Output stage of one 16-row tile (index `tile`) whose partial products are complete: lane
// (m, q) holds rows 16 tile + 4 q + i of column m in acc[i].  EPI 0 writes Out[M, N]; EPI 1 and 2
// apply SiLU-and-mul to the gate/up rows interleaved 8 + 8 per tile (h4mv_interleave_gate_up) and
// write Out[M, N / 2]: gate and up are first rounded to bf16 (the values a plain matvec would
// store), then Out = bf16(silu(g) * u) (EPI 1) or bf16(bf16(silu(g)) * u) (EPI 2).  Every lane
// of the wave must call it (EPI 1/2 pair lanes l and l ^ 32).
template <typename OutT, int EPI>
__device__ __forceinline__ void store_tile(const f32x4_t& acc, OutT* __restrict__ Out, int tile,
                                           int N, int M, int r, int q)
{
    if constexpr (EPI != 0) {
        // lane (m, q < 2) holds gate rows 4q .. 4q + 3 of the tile's 8 features, lane (m, q + 2)
        // = lane + 32 the up rows of the same features
        f32x4_t up;
#pragma unroll
        for (int i = 0; i < 4; ++i) up[i] = __shfl_xor(acc[i], 32);
        if (r >= M || q >= 2 || 16 * tile >= N) return;
        __bf16* orow = reinterpret_cast<__bf16*>(Out) + (size_t)r * (size_t)(N >> 1);
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float sg = silu_f32(round_to_bf16(acc[i]));
            if constexpr (EPI == 2) sg = round_to_bf16(sg);
            o[i] = sg * round_to_bf16(up[i]);
        }
        *reinterpret_cast<u32x2_t*>(orow + 8 * tile + 4 * q) =
            (u32x2_t){pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    } else {
        const int n = 16 * tile + 4 * q;
        if (r >= M || n >= N) return;
        OutT* orow = Out + (size_t)r * (size_t)N;
        if (((N & 3) == 0) && aligned(Out, 4 * sizeof(OutT)) && n + 3 < N) {
            if constexpr (sizeof(OutT) == 2) {
                *reinterpret_cast<u32x2_t*>(orow + n) =
                    (u32x2_t){pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
            } else {
                *reinterpret_cast<f32x4_t*>(orow + n) = acc;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (n + i < N) orow[n + i] = (OutT)acc[i];
        }
    }
}

// EPI selects the output stage (store_tile).
template <int MMAX, bool XG, int DEPTH, int RT, typename OutT, int EPI = 0>
__global__ void __launch_bounds__(RT == 1 ? 1024 : 64 * kMaxWavesRT)
h4mv_stream_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ St,
                   const __bf16* __restrict__ X, OutT* __restrict__ Out,
                   int N, int K, int M, int per)
{
    static_assert((DEPTH - 1) * copies_per_step<MMAX, XG, RT>() + (XG ? kXgLoads : 0) < 64,
                  "vmcnt holds at most 63");
    extern __shared__ __align__(16) unsigned char smem[];
    const WaveLds L = wave_lds(MMAX, XG, DEPTH, per, RT);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int steps_total = K >> 9;
    const int n0 = blockIdx.x * kRowsPerWG * RT;
    const bool col_ok = r < M;

    unsigned char* base = smem + wave * L.total;
    unsigned char* ring = base;
    unsigned char* sarea = base + L.ring;
    const int step0 = wave * per;
    const int nsteps = max(0, min(per, steps_total - step0));

    const uint8_t* wtile = W + (size_t)n0 * (size_t)(K >> 1);
    const unsigned char* xbytes = reinterpret_cast<const unsigned char*>(X);
    uint32_t woff[4 * RT];
#pragma unroll
    for (int i = 0; i < 4 * RT; ++i) woff[i] = stream_w_lane_off(n0, N, K, lane, i);

    // ---- one-time copies: the wave's scale slice ------------------------------------------------
    if (nsteps > 0) {
        for (int t0 = 0; t0 < 16 * RT * per; t0 += 64) {
            const int t = t0 + lane;
            if (t < 16 * RT * per && (t % per) < nsteps)
                dma16_to_lds_stream(St + stream_s_seg_off(n0, N, K, per, step0, t), sarea + t0 * 16);
        }
    }
    // ---- fill the ring ------------------------------------------------------------------------
#pragma unroll
    for (int s = 0; s < DEPTH; ++s)
        if (s < nsteps)
            issue_step<MMAX, XG, RT>(ring + s * L.slot, wtile, xbytes, woff, (step0 + s) * kStepGroups,
                                     K, M, lane);

    int rdoff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) rdoff[u] = stream_w_read_off(r, q, u);

    f32x4_t acc0[RT], acc1[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        acc0[t] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
        acc1[t] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }
    u32x4_t xv[4][4];
    // XG: this lane's activation row (row M - 1 again for r >= M) and its loads of step s.
    const unsigned char* xg_row = xbytes + (size_t)(r < M ? r : M - 1) * (size_t)K * 2;
    auto load_x = [&](int s) {
        const unsigned char* b = xg_row + (size_t)(step0 + s) * kStepGroups * 64;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[u][j] = load_16(b + stream_x_frag_off(q, u, j));
    };
    if constexpr (XG) {
        if (nsteps > 0) load_x(0);
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) asm volatile("" : "=v"(xv[u][j]));   // columns m >= M: any value
    }

    for (int s = 0; s < nsteps; ++s) {
        const int slot = s % DEPTH;
        unsigned char* sl = ring + slot * L.slot;
        wait_ahead_ct<MMAX, XG, RT, DEPTH - 1>(min(nsteps - 1 - s, DEPTH - 1));
        u32x4_t sv[RT];
        u32x4_t wv[RT][4];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            sv[t] = *reinterpret_cast<const u32x4_t*>(sarea + ((16 * t + r) * per + s) * 16);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                wv[t][u] = *reinterpret_cast<const u32x4_t*>(sl + t * kStepCodeBytes + rdoff[u]);
        }
        if (!XG && col_ok) {
            const unsigned char* xrow = sl + RT * kStepCodeBytes + r * 1024;
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    xv[u][j] = *reinterpret_cast<const u32x4_t*>(xrow + stream_x_frag_off(q, u, j));
        }
        // All fragments of this slot are in registers: refill it before the math.
        __builtin_amdgcn_s_waitcnt(0xC07F);            // lgkmcnt(0)
        if (s + DEPTH < nsteps)
            issue_step<MMAX, XG, RT>(sl, wtile, xbytes, woff, (step0 + s + DEPTH) * kStepGroups,
                                     K, M, lane);
        // The activation fragments of this step serve every row tile of the workgroup.
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float sc = e8m0_to_f32((sv[t][u] >> (8 * q)) & 0xFFu);   // group q + 4u of row r
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bf16x8_t a = fp4x8_to_bf16x8(wv[t][u][j], sc);
                    if (u & 1) acc1[t] = mfma16x16x32_bf16(a, as_bf16x8(xv[u][j]), acc1[t]);
                    else       acc0[t] = mfma16x16x32_bf16(a, as_bf16x8(xv[u][j]), acc0[t]);
                }
            }
        if constexpr (XG) {
            if (s + 1 < nsteps) load_x(s + 1);
        }
    }
    f32x4_t acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = acc0[t] + acc1[t];

    // ---- reduce over the waves of the workgroup ------------------------------------------------
    if (nwaves > 1) {
        __syncthreads();                                   // every wave is done with its LDS
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < RT; ++t) reinterpret_cast<f32x4_t*>(base)[t * 64 + lane] = acc[t];
        }
        __syncthreads();
        if (wave != 0) return;
        for (int w = 1; w < nwaves; ++w)
#pragma unroll
            for (int t = 0; t < RT; ++t)
                acc[t] += reinterpret_cast<const f32x4_t*>(smem + w * L.total)[t * 64 + lane];
    }

#pragma unroll
    for (int t = 0; t < RT; ++t) store_tile<OutT, EPI>(acc[t], Out, (n0 >> 4) + t, N, M, r, q);
}

// ---------------------------------------------------------------------------------------------
// K-slice kernel: many 16-row tiles per workgroup, activations held in registers.
//
// At M >= 2 the streaming kernel moves M KB of activations into LDS with every 4 KB of codes (per
// 16-row tile and K step), so its L2 -> LDS traffic is up to three times the HBM stream.  When
// there are several tiles per CU (N / 16 >= 2 x kKsWorkgroups) and K / 512 <= kKsMaxWaves, the
// roles are swapped:
//   * a workgroup owns nt <= TMAX tiles (every G-th tile, G = workgroups: at any moment the
//     workgroups read neighbouring tiles) and has one wave per K step (512 k);
//   * wave w loads the activation fragments of step w into registers once (lane (m, q): the same
//     fragments the streaming kernel reads from LDS), then streams the codes of step w of tile
//     after tile through its own DEPTH-slot LDS ring, each slot one tile: 4 KB of codes (the
//     streaming kernel's four copy instructions and bank-conflict-free placement) and the tile's
//     16 rows x 16 scale bytes of the step (one 4-byte-per-lane copy, row r at 16 r);
//   * each tile accumulates in its own register tile (the tile loop is unrolled to TMAX) and is
//     stored to an LDS area after the rings one tile later, while the stream goes on; the waves
//     meet once, at the end, and wave w adds the partials of tiles w, w + nw, ... in wave order
//     (a fixed order: the result does not depend on timing) and writes them through store_tile.
// Activation traffic is then one step of X per wave and launch instead of per tile.  Measured
// (cfg1 and configs[4] gate/up, M = 1 .. 8): the marginal stream rate is the same at every M and
// higher than the streaming kernel's, but the fixed cost per launch is about 1 us higher, so the
// planner takes it from M = 3 on (gate/up M = 8: 20.9 -> 15.7 us, cfg1 M = 8: 14.8 -> 13.6 us;
// M = 2 and 1 stay faster on the streaming kernel).
// ---------------------------------------------------------------------------------------------
constexpr int kKsMaxWaves = 8;                 // K <= 4096; 2 waves per SIMD, 256 VGPRs each
constexpr int kKsWorkgroups = 256;             // one workgroup per CU of an MI355X
constexpr int kKsSlotBytes = kStepCodeBytes + 256;
constexpr int kKsTmax = 16;                    // tiles per workgroup (register tiles)
constexpr int kKsMinM = 3;                     // default: K-slice kernel from this M on

// Tiles of N rows, and the first row of tile t.  When N % 16 != 0 the last tile is moved back to
// rows N - 16 .. N - 1 (N >= 16), so its copies read whole rows of the operand with the full
// tiles' per-lane offsets; it stores only its rows from 16 t on (the others belong to the tile
// before it).
__host__ __device__ inline int ks_tiles(int N) { return (N + 15) >> 4; }
__host__ __device__ inline int ks_row0(int t, int N) { return 16 * t < N - 16 ? 16 * t : N - 16; }

// Output rows n0 + 4 q .. n0 + 4 q + 3 of lane (r, q)'s accumulator, those in [lo, N) only.
template <typename OutT>
__device__ __forceinline__ void store_rows(const f32x4_t& acc, OutT* __restrict__ Out, int n0, int lo, int N,
                                           int M, int r, int q)
{
    if (r >= M) return;
    OutT* orow = Out + (size_t)r * (size_t)N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = n0 + 4 * q + i;
        if (n >= lo && n < N) orow[n] = (OutT)acc[i];
    }
}

// Scale copy of a tile-step: lane l fetches bytes 4 (l % 4) .. +3 of row l / 4's 16 scale bytes
// of the step; offset from the tile's first scale byte of the step.
__host__ __device__ inline uint32_t ks_s_lane_off(int K, int lane)
{
    return (uint32_t)(lane >> 2) * (uint32_t)(K >> 5) + 4u * (uint32_t)(lane & 3);
}
// Tiles of workgroup b when T tiles are dealt to G workgroups: tile t0 + i * tstride for
// i < nt.  Interleaved (tstride = G): at any moment the workgroups read neighbouring tiles, one
// contiguous stretch of W; contiguous (tstride = 1): each workgroup a stretch of its own.
__host__ __device__ inline void ks_tiles_of(int b, int T, int G, bool interleaved, int& t0, int& nt,
                                            int& tstride)
{
    const int base = T / G, rem = T % G;
    nt = base + (b < rem ? 1 : 0);
    if (interleaved) {
        t0 = b;
        tstride = G;
    } else {
        t0 = b * base + (b < rem ? b : rem);
        tstride = 1;
    }
}

// s_waitcnt vmcnt(5 ahead) (five copies per tile) for 0 <= ahead <= A.
template <int A>
__device__ __forceinline__ void ks_wait(int ahead)
{
    if constexpr (A == 0) {
        wait_vmcnt<0>();
    } else {
        if (ahead >= A) wait_vmcnt<5 * A>();
        else ks_wait<A - 1>(ahead);
    }
}

template <int DEPTH, int TMAX, typename OutT, int EPI>
__global__ void __launch_bounds__(64 * kKsMaxWaves)
h4mv_kslice_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ St,
                   const __bf16* __restrict__ X, OutT* __restrict__ Out, int N, int K, int M,
                   int interleaved)
{
    static_assert(DEPTH * 5 < 64, "vmcnt holds at most 63");
    extern __shared__ __align__(16) unsigned char smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;                 // == K / 512
    const int r = lane & 15;
    const int q = lane >> 4;
    int t0, nt, tstride;
    ks_tiles_of(blockIdx.x, ks_tiles(N), gridDim.x, interleaved != 0, t0, nt, tstride);
    const int G = K >> 5;
    const int gs = wave * kStepGroups;                  // first scale group of this wave's step

    unsigned char* ring = smem + (size_t)wave * DEPTH * kKsSlotBytes;
    uint32_t woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) woff[i] = stream_w_lane_off(0, kRowsPerWG, K, lane, i);
    const uint32_t soff = ks_s_lane_off(K, lane);
    const uint8_t* wstep = W + (size_t)gs * 16;
    const uint8_t* sstep = St + gs;
    auto issue = [&](int i, unsigned char* slot) {
        const int n0 = ks_row0(t0 + i * tstride, N);
        const uint8_t* w = wstep + (size_t)n0 * (size_t)(K >> 1);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            __builtin_amdgcn_global_load_lds((const void*)(w + woff[c]), (lds_void_t*)(slot + c * 1024),
                                             16, 0, kDmaAux);
        __builtin_amdgcn_global_load_lds((const void*)(sstep + (size_t)n0 * (size_t)G + soff),
                                         (lds_void_t*)(slot + kStepCodeBytes), 4, 0, 0);
    };
    // Tile 0's copies go out first, then the activation loads, then the rest of the ring, filled
    // unconditionally (a workgroup with nt < DEPTH fetches its last tile again into slots it
    // never reads): exactly 5 (DEPTH - 1) copies are then younger than the activation loads on
    // every path, so the wait below covers them (and tile 0) without draining the ring, and the
    // compiler needs no wait of its own before the MFMAs.
    u32x4_t xv[4][4];
    auto load_xv = [&]() {
        if (r < M) {
            const unsigned char* xrow = reinterpret_cast<const unsigned char*>(X) +
                                        (size_t)r * (size_t)K * 2 + (size_t)gs * 64;
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) xv[u][j] = load_16(xrow + stream_x_frag_off(q, u, j));
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) asm volatile("" : "=v"(xv[u][j]));
        }
        asm volatile("" ::: "memory");
    };
    issue(0, ring);
    load_xv();
#pragma unroll
    for (int i = 1; i < DEPTH; ++i) issue(min(i, nt - 1), ring + i * kKsSlotBytes);
    wait_vmcnt<5 * (DEPTH - 1)>();

    int rdoff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) rdoff[u] = stream_w_read_off(r, q, u);

    f32x4_t acc[TMAX];
    // partial tiles [nt][nwaves][64] after the rings
    f32x4_t* red = reinterpret_cast<f32x4_t*>(smem + (size_t)nwaves * DEPTH * kKsSlotBytes);
#pragma unroll
    for (int i = 0; i < TMAX; ++i) {
        if (i < nt) {
            unsigned char* sl = ring + (i % DEPTH) * kKsSlotBytes;
            // tiles i + 1 .. min(nt, i + DEPTH) - 1 may stay in flight
            ks_wait<DEPTH - 1>(min(nt - 1 - i, DEPTH - 1));
            const u32x4_t sv = *reinterpret_cast<const u32x4_t*>(sl + kStepCodeBytes + 16 * r);
            u32x4_t wv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) wv[u] = *reinterpret_cast<const u32x4_t*>(sl + rdoff[u]);
            __builtin_amdgcn_s_waitcnt(0xC07F);             // lgkmcnt(0): the slot is free again
            if (i + DEPTH < nt) issue(i + DEPTH, sl);
            f32x4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float sc = e8m0_to_f32((sv[u] >> (8 * q)) & 0xFFu);   // group q + 4u of row r
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bf16x8_t a = fp4x8_to_bf16x8(wv[u][j], sc);
                    if (u & 1) c1 = mfma16x16x32_bf16(a, as_bf16x8(xv[u][j]), c1);
                    else       c0 = mfma16x16x32_bf16(a, as_bf16x8(xv[u][j]), c0);
                }
            }
            acc[i] = c0 + c1;
            // the previous tile's partial is complete by now: publish it while streaming
            if (i > 0) red[((i - 1) * nwaves + wave) * 64 + lane] = acc[i - 1];
        }
    }

    // ---- add the waves' partial tiles and store ------------------------------------------------
#pragma unroll
    for (int i = 0; i < TMAX; ++i)
        if (i == nt - 1) red[(i * nwaves + wave) * 64 + lane] = acc[i];
    __syncthreads();
    for (int i = wave; i < nt; i += nwaves) {
        f32x4_t a = red[(i * nwaves) * 64 + lane];
        for (int w = 1; w < nwaves; ++w) a += red[(i * nwaves + w) * 64 + lane];
        const int t = t0 + i * tstride;
        if constexpr (EPI == 0) {
            if (16 * t > N - 16) {                      // partial last tile: rows N - 16 .. N - 1
                store_rows(a, Out, N - 16, 16 * t, N, M, r, q);
                continue;
            }
        }
        store_tile<OutT, EPI>(a, Out, t, N, M, r, q);
    }
}

// Batched form of the K-slice kernel for shapes with more tiles than one round of workgroups
// holds at kKsTmax (plain output only).  The waves' partial tiles are added every B tiles instead
// of once at the end: after the B-th tile an LDS-only barrier (the ring's copies stay in flight),
// each wave adds the partials of some of the batch's tiles into the workgroup's output area in
// LDS (1 KB per tile), and a second barrier frees the partial area for the next batch.  The
// global stores all wait for the end, as in h4mv_kslice_kernel: a store issued between ring
// copies would enter the in-order vmcnt count and make the next waits drain the ring.  LDS:
// rings, then B x nwaves partial tiles, then nt_max output tiles.
template <int DEPTH, int B, typename OutT>
__global__ void __launch_bounds__(64 * kKsMaxWaves)
h4mv_kslice_batched_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ St,
                           const __bf16* __restrict__ X, OutT* __restrict__ Out, int N, int K, int M,
                           int interleaved)
{
    static_assert(DEPTH * 5 < 64, "vmcnt holds at most 63");
    extern __shared__ __align__(16) unsigned char smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;                 // == K / 512
    const int r = lane & 15;
    const int q = lane >> 4;
    int t0, nt, tstride;
    ks_tiles_of(blockIdx.x, ks_tiles(N), gridDim.x, interleaved != 0, t0, nt, tstride);
    const int G = K >> 5;
    const int gs = wave * kStepGroups;

    unsigned char* ring = smem + (size_t)wave * DEPTH * kKsSlotBytes;
    uint32_t woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) woff[i] = stream_w_lane_off(0, kRowsPerWG, K, lane, i);
    const uint32_t soff = ks_s_lane_off(K, lane);
    const uint8_t* wstep = W + (size_t)gs * 16;
    const uint8_t* sstep = St + gs;
    auto issue = [&](int i, unsigned char* slot) {
        const int n0 = ks_row0(t0 + i * tstride, N);
        const uint8_t* w = wstep + (size_t)n0 * (size_t)(K >> 1);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            __builtin_amdgcn_global_load_lds((const void*)(w + woff[c]), (lds_void_t*)(slot + c * 1024),
                                             16, 0, kDmaAux);
        __builtin_amdgcn_global_load_lds((const void*)(sstep + (size_t)n0 * (size_t)G + soff),
                                         (lds_void_t*)(slot + kStepCodeBytes), 4, 0, 0);
    };
    // tile 0's copies, the activation loads, then the rest of the ring (as in h4mv_kslice_kernel)
    u32x4_t xv[4][4];
    issue(0, ring);
    if (r < M) {
        const unsigned char* xrow = reinterpret_cast<const unsigned char*>(X) +
                                    (size_t)r * (size_t)K * 2 + (size_t)gs * 64;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[u][j] = load_16(xrow + stream_x_frag_off(q, u, j));
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) asm volatile("" : "=v"(xv[u][j]));
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 1; i < DEPTH; ++i) issue(min(i, nt - 1), ring + i * kKsSlotBytes);
    wait_vmcnt<5 * (DEPTH - 1)>();

    int rdoff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) rdoff[u] = stream_w_read_off(r, q, u);

    f32x4_t* red = reinterpret_cast<f32x4_t*>(smem + (size_t)nwaves * DEPTH * kKsSlotBytes);   // [B][nwaves][64]
    f32x4_t* outb = red + (size_t)B * nwaves * 64;                                             // [nt][64]
    for (int b0 = 0; b0 < nt; b0 += B) {
        f32x4_t acc[B];
#pragma unroll
        for (int ii = 0; ii < B; ++ii) {
            const int i = b0 + ii;
            if (i < nt) {
                unsigned char* sl = ring + (i % DEPTH) * kKsSlotBytes;
                ks_wait<DEPTH - 1>(min(nt - 1 - i, DEPTH - 1));
                const u32x4_t sv = *reinterpret_cast<const u32x4_t*>(sl + kStepCodeBytes + 16 * r);
                u32x4_t wv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) wv[u] = *reinterpret_cast<const u32x4_t*>(sl + rdoff[u]);
                __builtin_amdgcn_s_waitcnt(0xC07F);             // lgkmcnt(0): the slot is free again
                if (i + DEPTH < nt) issue(i + DEPTH, sl);
                f32x4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float sc = e8m0_to_f32((sv[u] >> (8 * q)) & 0xFFu);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const bf16x8_t a = fp4x8_to_bf16x8(wv[u][j], sc);
                        if (u & 1) c1 = mfma16x16x32_bf16(a, as_bf16x8(xv[u][j]), c1);
                        else       c0 = mfma16x16x32_bf16(a, as_bf16x8(xv[u][j]), c0);
                    }
                }
                acc[ii] = c0 + c1;
                if (ii > 0) red[((ii - 1) * nwaves + wave) * 64 + lane] = acc[ii - 1];
            }
        }
        const int nb = min(B, nt - b0);
#pragma unroll
        for (int ii = 0; ii < B; ++ii)
            if (ii == nb - 1) red[(ii * nwaves + wave) * 64 + lane] = acc[ii];
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        for (int ii = wave; ii < nb; ii += nwaves) {
            f32x4_t a = red[(ii * nwaves) * 64 + lane];
            for (int w = 1; w < nwaves; ++w) a += red[(ii * nwaves + w) * 64 + lane];
            outb[(b0 + ii) * 64 + lane] = a;
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }

    // every copy has landed (the last tile's wait was vmcnt(0)); the output tiles are in LDS
    for (int i = wave; i < nt; i += nwaves) {
        const f32x4_t a = outb[i * 64 + lane];
        const int t = t0 + i * tstride;
        if (16 * t > N - 16) store_rows(a, Out, N - 16, 16 * t, N, M, r, q);
        else store_tile<OutT, 0>(a, Out, t, N, M, r, q);
    }
}

// ---------------------------------------------------------------------------------------------
// M = 1 kernel: the codes go to the block-scaled MFMA as stored, the activation row as e4m3 hi + lo.
//
// At M = 1 the bf16 path widens every code to bf16 (64 v_cvt_scalef32_pk_bf16_fp4 per lane and
// 512-k step) for 16x16x32 MFMAs of which one column is used; measured with the copies alone
// (the same bytes, addresses and waits, no arithmetic), that work costs about 1.5 us of a cfg1
// launch.  Here A of v_mfma_scale_f32_16x16x128_f8f6f4 is the e2m1 codes straight from the ring
// (cbsz 4) with the rows' e8m0 group scales as the MFMA's A scales, and B is the activation row
// in two e4m3 columns: per block of 32 k, x * 2^e = hi + lo, where 2^e puts the block's largest
// |x| in [128, 256), hi is x * 2^e rounded to 4 significant bits and lo the remainder, and 2^-e
// is the block's B scale.  The remainder of a bf16 value is exact in e4m3 whenever |x| >= 2^-9
// of its block's largest (below that lo keeps what the e4m3 subnormals hold), so column 0 plus
// column 1 of the product is sum_k w_k x_k up to the accumulation order: the bf16 path's result.
//   * a workgroup of TW waves owns the tiles b + w G (wave w, G workgroups), one wave per tile
//     over all of K, each streaming 4 KB code steps through its own DEPTH-slot ring after a
//     one-time copy of its scale slice (the streaming kernel's copy addresses and LDS placement);
//   * the workgroup converts the activation row once: the row is copied into LDS first (ahead of
//     the rings and the scale slices, and as copies, not register loads, which would make the
//     compiler wait for every copy in flight before using them); once each wave has its own row
//     pieces (a wait that leaves its ring and scale copies in flight), one barrier, then thread t
//     converts 8 bf16 (a quarter of a 32-k block; a block's quarters sit in four consecutive
//     lanes, which take their common maximum with two DPP steps) and writes its 8 hi and 8 lo
//     bytes and the block's scale byte, while the first code steps are in flight; a second
//     barrier publishes them.  A wave without a tile copies its workgroup's first tile (its reads
//     meet wave 0's in L2), so every wave issues the same copies and all waits are exact; it
//     leaves after the second barrier;
//   * non-finite activations: NaN stays NaN through e4m3; a block holding an infinity gets the
//     NaN scale byte 0xFF, so every output is NaN (the reference gives +-inf or NaN there);
//   * step s: four MFMAs of 128 k.  Lane (n, j) = (lane % 16, lane / 16) supplies A row n's
//     group 4u + j (16 bytes from the ring, its scale byte shifted to the bottom), B column n's
//     k 16j .. 16j + 15 and 64 + 16j .. + 15 (hi for even n, lo for odd n: columns >= 2 repeat
//     them and are never stored) and the B scale of block j, four MFMAs' scales in one dword
//     picked with op_sel;
//   * lane (c, q) ends with rows 4q .. 4q + 3 of column c; one DPP exchange adds column 1 to
//     column 0 and store_tile writes them (with the SiLU-and-mul stage for h4mv_silu_mul).
// ---------------------------------------------------------------------------------------------
constexpr int kM1MaxWaves = 16;
constexpr int kM1Workgroups = 512;             // two workgroups per CU when their LDS allows it
constexpr int kM1MinTiles = 1024;              // default: when the tiles alone fill the GPU
constexpr int kM1RoundWaves = 4;               // waves per workgroup when one round cannot hold the tiles
constexpr int kM1MaxSteps = 64;                // K <= 32768
constexpr int kM1MaxScaleCopies = kM1MaxSteps / 4;   // 16 nsteps / 64 copies of the scale slice

// LDS bytes of the activation row: hi [K], lo [K], scale bytes [K / 32] (rounded to 16).
__host__ __device__ inline int m1_x_bytes(int K) { return 2 * K + (((K >> 5) + 15) & ~15); }
// Scale area of a wave: 16 rows x nsteps x 16 B, rounded up to whole 64-lane copies (1 KB).
__host__ __device__ inline int m1_scale_bytes(int nsteps) { return 16 * ((16 * nsteps + 63) & ~63); }
__host__ __device__ inline int m1_wave_bytes(int depth, int nsteps)
{
    return depth * kStepCodeBytes + m1_scale_bytes(nsteps);
}
// LDS byte of block b's B scale: the 16 blocks of a step are stored so that dword j holds blocks
// j, 4 + j, 8 + j, 12 + j (byte u = block 4u + j, the scale lane j supplies to MFMA u).
__host__ __device__ inline int m1_xe_pos(int b)
{
    const int c = b & 15;
    return (b & ~15) + 4 * (c & 3) + (c >> 2);
}
// s_waitcnt vmcnt(n) for 0 <= n <= A.
template <int A>
__device__ __forceinline__ void m1_wait_n(int n)
{
    if constexpr (A == 0) {
        wait_vmcnt<0>();
    } else {
        if (n >= A) wait_vmcnt<A>();
        else m1_wait_n<A - 1>(n);
    }
}

// s_waitcnt vmcnt(4 ahead) for 0 <= ahead <= A (four code copies per step).
template <int A>
__device__ __forceinline__ void m1_wait(int ahead)
{
    if constexpr (A == 0) {
        wait_vmcnt<0>();
    } else {
        if (ahead >= A) wait_vmcnt<4 * A>();
        else m1_wait<A - 1>(ahead);
    }
}

typedef int m1_v8i __attribute__((ext_vector_type(8)));

template <int U>
__device__ __forceinline__ f32x4_t m1_mfma(const u32x4_t& w, const m1_v8i& b, uint32_t sa, uint32_t sb, f32x4_t acc)
{
    const m1_v8i a = {(int)w[0], (int)w[1], (int)w[2], (int)w[3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 4, 0, 0, (int)sa, U, (int)sb);
}

__device__ __forceinline__ float m1_quad_max(float v)
{
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));   // quad_perm 1,0,3,2
    return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true))); // quad_perm 2,3,0,1
}

template <int DEPTH, typename OutT, int EPI>
__global__ void __launch_bounds__(64 * kM1MaxWaves)
h4mv_m1_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ St,
               const __bf16* __restrict__ X, OutT* __restrict__ Out, int N, int K)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int T = (N + kRowsPerWG - 1) / kRowsPerWG;
    const int nsteps = K >> 9;

    unsigned char* xh = smem;                                   // hi bytes, k order
    unsigned char* xl = smem + K;                               // lo bytes
    unsigned char* xe = smem + 2 * K;                           // B scale bytes (m1_xe_pos)
    unsigned char* xs = smem + m1_x_bytes(K);                   // the bf16 row as loaded
    unsigned char* ring = xs + 2 * K + wave * m1_wave_bytes(DEPTH, nsteps);
    unsigned char* sarea = ring + DEPTH * kStepCodeBytes;

    const int tile_w = blockIdx.x + wave * gridDim.x;
    const bool has_tile = tile_w < T;                           // wave-uniform
    const int tile = has_tile ? tile_w : blockIdx.x;
    const int n0 = tile * kRowsPerWG;

    // ---- the activation row, the scale slice, then the ring: all copies straight to LDS --------
    // (register loads of the row would make the compiler wait for every copy before using them)
    const int np = K >> 3;                                      // 16-byte pieces of the row
    for (int p0 = wave * 64; p0 < np; p0 += nwaves * 64)
        if (p0 + lane < np) dma16_to_lds(X + 8 * (p0 + lane), xs + 16 * p0);
    uint32_t woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) woff[i] = stream_w_lane_off(n0, N, K, lane, i);
    const uint8_t* wtile = W + (size_t)n0 * (size_t)(K >> 1);
    auto issue = [&](int s, unsigned char* slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(wtile + (size_t)s * (kStepGroups * 16) + woff[i]),
                                             (lds_void_t*)(slot + i * 1024), 16, 0, kDmaAux);
    };
    // step 0, the scale slice, then the rest of the ring: the first barrier waits for the row
    // only, and step 0's wait covers the scales.  Every slot is filled (a slice shorter than the
    // ring fetches its last step again into slots it never reads) and every scale copy is issued
    // by all lanes, so the copy counts are exact.
    issue(0, ring);
    const int nseg = 16 * nsteps;
    for (int t0 = 0; t0 < nseg; t0 += 64) {
        const int t = min(t0 + lane, nseg - 1);
        dma16_to_lds_stream(St + stream_s_seg_off(n0, N, K, nsteps, 0, t), sarea + t0 * 16);
    }
#pragma unroll
    for (int s = 1; s < DEPTH; ++s) issue(min(s, nsteps - 1), ring + s * kStepCodeBytes);
    m1_wait_n<4 * DEPTH + kM1MaxScaleCopies>(4 * DEPTH + (nseg + 63) / 64);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");    // every wave's row pieces landed

    // ---- activation row -> e4m3 hi / lo and block scales ----------------------------------------
    for (int g0 = 0; g0 < np; g0 += nwaves * 64) {
        const int gr = g0 + (int)threadIdx.x;
        const int g = gr < np ? gr : np - 4 + (gr & 3);         // a quad past the end redoes the last block
        const u32x4_t xw = *reinterpret_cast<const u32x4_t*>(xs + 16 * g);
        float v[8];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            v[2 * c] = __uint_as_float(xw[c] << 16);
            v[2 * c + 1] = __uint_as_float(xw[c] & 0xFFFF0000u);
        }
        float amax = 0.f;                          // fmaxf drops NaN: NaN values stay out of the max
#pragma unroll
        for (int c = 0; c < 8; ++c) amax = fmaxf(amax, fabsf(v[c]));
        amax = m1_quad_max(amax);
        const uint32_t eb = (__float_as_uint(amax) >> 23) & 0xFFu;
        int be = 261 - (int)eb;                    // biased exponent of 2^e = 2^(7 - floor(log2 amax))
        be = be < 1 ? 1 : (be > 253 ? 253 : be);
        const float scale = __uint_as_float((uint32_t)be << 23);
        uint32_t hw[2], lw[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float x[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) x[c] = v[4 * h + c] * scale;
            uint32_t a = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
            a = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], (int)a, true);
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)a, false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)a, true);
            uint32_t b = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[0] - h01[0], x[1] - h01[1], 0, false);
            b = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[2] - h23[0], x[3] - h23[1], (int)b, true);
            hw[h] = a;
            lw[h] = b;
        }
        *reinterpret_cast<u32x2_t*>(xh + 8 * g) = (u32x2_t){hw[0], hw[1]};
        *reinterpret_cast<u32x2_t*>(xl + 8 * g) = (u32x2_t){lw[0], lw[1]};
        xe[m1_xe_pos(g >> 2)] = (unsigned char)(eb == 255u ? 255 : 254 - be);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (!has_tile) {
        wait_vmcnt<0>();                           // its copies land before the wave leaves
        return;
    }

    // ---- stream ------------------------------------------------------------------------------
    int rdoff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) rdoff[u] = stream_w_read_off(r, q, u);
    const unsigned char* xcol = ((r & 1) ? xl : xh) + 16 * q;
    f32x4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < nsteps; ++s) {
        unsigned char* sl = ring + (s % DEPTH) * kStepCodeBytes;
        m1_wait<DEPTH - 1>(min(nsteps - 1 - s, DEPTH - 1));
        const u32x4_t sv = *reinterpret_cast<const u32x4_t*>(sarea + (r * nsteps + s) * 16);
        u32x4_t wv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) wv[u] = *reinterpret_cast<const u32x4_t*>(sl + rdoff[u]);
        m1_v8i b[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(xcol + 512 * s + 128 * u);
            const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(xcol + 512 * s + 128 * u + 64);
            b[u] = (m1_v8i){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
        const uint32_t sb = *reinterpret_cast<const uint32_t*>(xe + 16 * s + 4 * q);
        __builtin_amdgcn_s_waitcnt(0xC07F);                 // lgkmcnt(0): the slot is free again
        if (s + DEPTH < nsteps) issue(s + DEPTH, sl);
        c0 = m1_mfma<0>(wv[0], b[0], sv[0] >> (8 * q), sb, c0);
        c1 = m1_mfma<1>(wv[1], b[1], sv[1] >> (8 * q), sb, c1);
        c0 = m1_mfma<2>(wv[2], b[2], sv[2] >> (8 * q), sb, c0);
        c1 = m1_mfma<3>(wv[3], b[3], sv[3] >> (8 * q), sb, c1);
    }
    f32x4_t acc = c0 + c1;
#pragma unroll
    for (int i = 0; i < 4; ++i)                                 // column 0 (hi) + column 1 (lo)
        acc[i] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[i]), 0xB1, 0xF, 0xF, true));
    store_tile<OutT, EPI>(acc, Out, tile, N, 1, r, q);
}

// ---------------------------------------------------------------------------------------------
// M = 2 .. 8 on the block-scaled MFMA: the M = 1 kernel's scheme with one e4m3 hi / lo column
// pair per activation row.  B of v_mfma_scale_f32_16x16x128_f8f6f4 has 16 columns, so MM = 8 rows
// fill it (column 2m = hi of row m, 2m + 1 = lo); with MM = 2 or 4 the columns repeat the rows.
// A step is still four MFMAs per wave, so the math per byte of codes does not grow with M; what
// grows is the activation block the workgroup converts once (MM rows).  Each output column comes
// out of the MFMA independently of the others, so row m's result equals the M = 1 kernel's for
// that row alone, bit for bit.
//   * LDS: MM rows of 2K + kMxRowPad bytes, then MM rows of block scale bytes, then the waves'
//     rings and scale slices as in the M = 1 kernel.  Row m is copied in as bf16 (whole 1 KB
//     copies; rows m >= M repeat row M - 1) and converted in place (mx_convert_chunk): a thread
//     takes 16 values (32 bytes), the two threads of a 32-k block share their maximum with one
//     DPP step, and the thread writes its 16 hi bytes over the first half of its own 32 bytes and
//     its 16 lo bytes over the second.  A thread only ever rewrites bytes it alone read.
//   * The conversion runs cs steps of K at a time: chunk 0 before the stream starts, chunk
//     j + 1 while the waves stream chunk j (its VALU work fills the stream's waits), one
//     LDS-only barrier per chunk.  Waves without a tile convert and meet every barrier too.
//   * Only the M rows in use are converted; the columns of rows M .. MM - 1 read the unconverted
//     copies and are never stored (each MFMA output column depends on its own B column only).
//   * B fragment of lane (n, j) for MFMA u of step s: row m = (n / 2) mod MM, half n % 2, k =
//     512 s + 128 u + 16 j .. + 15 and + 64: 16-byte units 32 s + 8 u + j and + 4 of the row, at
//     byte 32 unit (+ 16 for lo).  Row stride = 32 mod 256, so lanes 0..15 of a read meet 16
//     distinct 16-byte bank groups.
//   * lane (n, q) ends with rows 4q .. 4q + 3 of column n; one DPP step adds column 2m + 1 to
//     column 2m, and the even lanes store row m (m < M).
// ---------------------------------------------------------------------------------------------
constexpr int kMxRowPad = 32;

__host__ __device__ inline int mx_row_bytes(int K) { return 2 * K + kMxRowPad; }
// Block scale bytes of one row (m1_xe_pos order), padded so that rows start in different banks.
__host__ __device__ inline int mx_xe_row_bytes(int K) { return (((K >> 5) + 15) & ~15) + 16; }
__host__ __device__ inline int mx_x_bytes(int mm, int K) { return mm * (mx_row_bytes(K) + mx_xe_row_bytes(K)); }
// Activation copy unit u (1 KB: 64 lanes x 16 B, one row's 512 values of one step) of an MM-row
// block, step-major: step u / MM, row u % MM; unit u is copied by wave u % nwaves.
__host__ __device__ inline size_t mx_copy_src(int K, int M, int mm, int u, int lane)
{
    const int st = u / mm, m = u % mm;
    const int mc = m < M ? m : M - 1;
    return (size_t)mc * (size_t)K * 2 + (size_t)st * 1024 + 16u * (uint32_t)lane;
}
__host__ __device__ inline int mx_copy_dst(int K, int mm, int u, int lane)
{
    const int st = u / mm, m = u % mm;
    return m * mx_row_bytes(K) + st * 1024 + 16 * lane;
}
// Units of [a, b) that wave w copies when units are dealt round-robin over nw waves.
__host__ __device__ inline int mx_units_of(int a, int b, int w, int nw)
{
    return b <= a ? 0 : (b - w + nw - 1) / nw - (a - w + nw - 1) / nw;
}
// Copies a wave has issued after its last activation copy of chunk j (steps cs j .. cs j + cs - 1)
// when it waits for that chunk: its copies of later chunks, the ring's first slots and the scale
// slice (all issued up front, after the activation copies), and, for a wave with a tile, the ring
// refills issued while streaming the steps before step cs (j - 1).  Waiting until at most that many
// are outstanding means the wave's copies of chunk j have landed (vmcnt retires in issue order).
__host__ __device__ inline int mx_after_chunk(int mm, int nsteps, int cs, int depth, int nscale, int j,
                                              int w, int nw, bool streams)
{
    const int end = mm * (cs * (j + 1) < nsteps ? cs * (j + 1) : nsteps);
    const int streamed = streams && cs * (j - 1) > 0 ? cs * (j - 1) : 0;      // steps consumed so far
    const int refills = streamed < nsteps - depth ? streamed : (nsteps - depth > 0 ? nsteps - depth : 0);
    return mx_units_of(end, mm * nsteps, w, nw) + 4 * depth + nscale + 4 * refills;
}

// s_waitcnt vmcnt(n) for a wave-uniform 0 <= n (counts above 63 wait for 63: stricter).
__device__ __forceinline__ void mx_wait(int n) { wait_vmcnt_dyn(n); }

typedef short mx_pk16_t __attribute__((ext_vector_type(2)));
typedef __bf16 mx_bf16x2_t __attribute__((ext_vector_type(2)));

// Converts chunk j of an MM-row activation block in place: steps cs j .. cs j + cs - 1 of its
// first `rows` rows (the M rows in use: the block's rows past M are never stored, so they stay
// as copied), cs a power of two (units past the row's end in the last chunk are skipped), U = 32 cs
// 32-byte units of 16 values per row.  Thread i of the workgroup takes unit U j + i % U of row
// i / U; the two units of a 32-k block sit in lanes 2i' and 2i' + 1, which share their maximum
// with one DPP step.  A thread rewrites only the 32 bytes it alone read (a lane with no unit reads
// unit 0 of row 0 and writes nothing); a wave whose lanes are all past the chunk skips the pass.
template <int MM>
__device__ __forceinline__ void mx_convert_chunk(unsigned char* xa, unsigned char* xe, int rowb, int xerow,
                                                 int upr, int cs_log2, int j, int rows, int wave, int lane,
                                                 int nthreads)
{
    const int ush = 5 + cs_log2;
    const int U = 1 << ush;
    const int total = rows * U;
    for (int i0 = 0; i0 < total; i0 += nthreads) {
        if (i0 + 64 * wave >= total) break;                    // wave-uniform
        const int i = i0 + 64 * wave + lane;
        const int m = i >> ush, p = U * j + (i & (U - 1));
        const bool live = i < total && p < upr;                // a block's two units live or die together
        unsigned char* up = xa + (live ? m * rowb + 32 * p : 0);
        const u32x4_t xw0 = *reinterpret_cast<const u32x4_t*>(up);
        const u32x4_t xw1 = *reinterpret_cast<const u32x4_t*>(up + 16);
        float v[16];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            v[2 * c] = __uint_as_float(xw0[c] << 16);
            v[2 * c + 1] = __uint_as_float(xw0[c] & 0xFFFF0000u);
            v[8 + 2 * c] = __uint_as_float(xw1[c] << 16);
            v[8 + 2 * c + 1] = __uint_as_float(xw1[c] & 0xFFFF0000u);
        }
        float amax = 0.f;                          // fmaxf drops NaN: NaN values stay out of the max
#pragma unroll
        for (int c = 0; c < 16; ++c) amax = fmaxf(amax, fabsf(v[c]));
        amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0xB1, 0xF, 0xF, true)));
        const uint32_t eb = (__float_as_uint(amax) >> 23) & 0xFFu;
        int be = 261 - (int)eb;                    // biased exponent of 2^e = 2^(7 - floor(log2 amax))
        be = be < 1 ? 1 : (be > 253 ? 253 : be);
        const float scale = __uint_as_float((uint32_t)be << 23);
        const float rscale = __uint_as_float((uint32_t)(254 - be) << 23);     // 2^-e, exact
        const uint32_t xd[8] = {xw0[0], xw0[1], xw0[2], xw0[3], xw1[0], xw1[1], xw1[2], xw1[3]};
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            // hi straight from the packed bf16 pairs: the scaled conversion rounds x / 2^-e = x 2^e
            // once, as the unscaled conversion of the (exact) product does
            mx_pk16_t t = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16((mx_pk16_t){0, 0},
                                                                    __builtin_bit_cast(mx_bf16x2_t, xd[2 * h]), rscale, false);
            t = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(t, __builtin_bit_cast(mx_bf16x2_t, xd[2 * h + 1]), rscale, true);
            const uint32_t a = __builtin_bit_cast(uint32_t, t);
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)a, false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)a, true);
            uint32_t b = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fmaf(v[4 * h], scale, -h01[0]),
                                                                   fmaf(v[4 * h + 1], scale, -h01[1]), 0, false);
            b = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fmaf(v[4 * h + 2], scale, -h23[0]),
                                                          fmaf(v[4 * h + 3], scale, -h23[1]), (int)b, true);
            hw[h] = a;
            lw[h] = b;
        }
        if (live) {
            *reinterpret_cast<u32x4_t*>(up) = (u32x4_t){hw[0], hw[1], hw[2], hw[3]};
            *reinterpret_cast<u32x4_t*>(up + 16) = (u32x4_t){lw[0], lw[1], lw[2], lw[3]};
            if ((p & 1) == 0) xe[m * xerow + m1_xe_pos(p >> 1)] = (unsigned char)(eb == 255u ? 255 : 254 - be);
        }
    }
}

template <int MM, int DEPTH, typename OutT, int EPI>
__global__ void __launch_bounds__(64 * kM1MaxWaves)
h4mv_mx_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ St,
               const __bf16* __restrict__ X, OutT* __restrict__ Out, int N, int K, int M, int cs_log2)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nwaves = blockDim.x >> 6;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int T = (N + kRowsPerWG - 1) / kRowsPerWG;
    const int nsteps = K >> 9;
    const int rowb = mx_row_bytes(K);
    const int xerow = mx_xe_row_bytes(K);

    unsigned char* xa = smem;                                   // MM rows: bf16, then hi / lo
    unsigned char* xe = smem + MM * rowb;                       // MM rows of B scale bytes
    unsigned char* ring = smem + mx_x_bytes(MM, K) + wave * m1_wave_bytes(DEPTH, nsteps);
    unsigned char* sarea = ring + DEPTH * kStepCodeBytes;

    const int tile_w = blockIdx.x + wave * gridDim.x;
    const bool has_tile = tile_w < T;                           // wave-uniform
    const int tile = has_tile ? tile_w : blockIdx.x;
    const int n0 = tile * kRowsPerWG;

    // ---- the activation rows (step-major), the scale slice, then the ring: all copies straight
    // to LDS.  Chunk j of the rows is waited for just before its conversion.
    const int cs = 1 << cs_log2;
    const int nchunks = (nsteps + cs - 1) >> cs_log2;
    const unsigned char* xbytes = reinterpret_cast<const unsigned char*>(X);
    const int nunits = MM * nsteps;
    for (int u = wave; u < nunits; u += nwaves)
        dma16_to_lds(xbytes + mx_copy_src(K, M, MM, u, 0) + 16 * lane, xa + mx_copy_dst(K, MM, u, 0));
    uint32_t woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) woff[i] = stream_w_lane_off(n0, N, K, lane, i);
    const uint8_t* wtile = W + (size_t)n0 * (size_t)(K >> 1);
    auto issue = [&](int s, unsigned char* slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(wtile + (size_t)s * (kStepGroups * 16) + woff[i]),
                                             (lds_void_t*)(slot + i * 1024), 16, 0, kDmaAux);
    };
    issue(0, ring);
    const int nseg = 16 * nsteps;
    for (int t0 = 0; t0 < nseg; t0 += 64) {
        const int t = min(t0 + lane, nseg - 1);
        dma16_to_lds_stream(St + stream_s_seg_off(n0, N, K, nsteps, 0, t), sarea + t0 * 16);
    }
#pragma unroll
    for (int s = 1; s < DEPTH; ++s) issue(min(s, nsteps - 1), ring + s * kStepCodeBytes);
    const int nscale = (nseg + 63) / 64;
    mx_wait(mx_after_chunk(MM, nsteps, cs, DEPTH, nscale, 0, wave, nwaves, has_tile));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");    // every wave's chunk-0 pieces landed

    // ---- activation rows -> e4m3 hi / lo in place, cs = 2^cs_log2 steps at a time --------------
    // Chunk 0 is converted while the later chunks' copies are still landing; chunk j + 1 is
    // converted while the waves stream chunk j, after a barrier that publishes chunk j's
    // conversion and follows every wave's wait for its own copies of chunk j + 1 (the LDS-only
    // barrier leaves the ring in flight).
    const int nthreads = 64 * nwaves;
    const int upr = K >> 4;
    mx_convert_chunk<MM>(xa, xe, rowb, xerow, upr, cs_log2, 0, M, wave, lane, nthreads);

    // ---- stream ------------------------------------------------------------------------------
    int rdoff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) rdoff[u] = stream_w_read_off(r, q, u);
    const int mrow = (r >> 1) & (MM - 1);
    const unsigned char* xcol = xa + mrow * rowb + 16 * (r & 1) + 32 * q;
    const unsigned char* xecol = xe + mrow * xerow + 4 * q;
    f32x4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < nchunks; ++j) {
        if (j + 1 < nchunks) mx_wait(mx_after_chunk(MM, nsteps, cs, DEPTH, nscale, j + 1, wave, nwaves, has_tile));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (j + 1 < nchunks) mx_convert_chunk<MM>(xa, xe, rowb, xerow, upr, cs_log2, j + 1, M, wave, lane, nthreads);
        if (has_tile) {
            const int s_end = min(nsteps, cs * (j + 1));
            for (int s = cs * j; s < s_end; ++s) {
                unsigned char* sl = ring + (s % DEPTH) * kStepCodeBytes;
                m1_wait<DEPTH - 1>(min(nsteps - 1 - s, DEPTH - 1));
                const u32x4_t sv = *reinterpret_cast<const u32x4_t*>(sarea + (r * nsteps + s) * 16);
                u32x4_t wv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) wv[u] = *reinterpret_cast<const u32x4_t*>(sl + rdoff[u]);
                m1_v8i b[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const u32x4_t k0 = *reinterpret_cast<const u32x4_t*>(xcol + 1024 * s + 256 * u);
                    const u32x4_t k1 = *reinterpret_cast<const u32x4_t*>(xcol + 1024 * s + 256 * u + 128);
                    b[u] = (m1_v8i){(int)k0[0], (int)k0[1], (int)k0[2], (int)k0[3], (int)k1[0], (int)k1[1], (int)k1[2], (int)k1[3]};
                }
                const uint32_t sb = *reinterpret_cast<const uint32_t*>(xecol + 16 * s);
                __builtin_amdgcn_s_waitcnt(0xC07F);                 // lgkmcnt(0): the slot is free again
                if (s + DEPTH < nsteps) issue(s + DEPTH, sl);
                c0 = m1_mfma<0>(wv[0], b[0], sv[0] >> (8 * q), sb, c0);
                c1 = m1_mfma<1>(wv[1], b[1], sv[1] >> (8 * q), sb, c1);
                c0 = m1_mfma<2>(wv[2], b[2], sv[2] >> (8 * q), sb, c0);
                c1 = m1_mfma<3>(wv[3], b[3], sv[3] >> (8 * q), sb, c1);
            }
        }
    }
    if (!has_tile) {
        wait_vmcnt<0>();                           // its copies land before the wave leaves
        return;
    }
    f32x4_t acc = c0 + c1;
#pragma unroll
    for (int i = 0; i < 4; ++i)                                 // column 2m (hi) + column 2m + 1 (lo)
        acc[i] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[i]), 0xB1, 0xF, 0xF, true));
    store_tile<OutT, EPI>(acc, Out, tile, N, M, (r & 1) ? kRowsPerWG : (r >> 1), q);
}

// Waves per tile: enough tiles x waves to cover the GPU, at most 16 per workgroup and at most one
// per step.
inline int stream_waves(int N, int K, int target_waves, int rt)
{
    const int tiles = (N + kRowsPerWG * rt - 1) / (kRowsPerWG * rt);
    const int steps = (K >> 5) / kStepGroups;
    int nw = (target_waves + tiles - 1) / tiles;
    nw = max(1, min(nw, min(rt == 1 ? 16 : kMaxWavesRT, steps)));
    return nw;
}

// Launch geometry shared by the production entry points and the tuning harness.
struct Plan {
    int waves;
    int groups_per_wave;
    bool xlds;
    size_t lds_bytes;
};

inline Plan make_plan(int K, int M, int waves)
{
    const int G = K >> 5;
    Plan p;
    p.waves = waves;
    int per = (G + waves - 1) / waves;
    p.groups_per_wave = (per + 3) & ~3;
    p.xlds = (size_t)M * (size_t)K * 2 <= (size_t)kXLdsMaxBytes;
    p.lds_bytes = p.xlds ? (size_t)M * (size_t)K * 2 : 0;
    return p;
}

template <int WAVES, int U, typename OutT>
void launch_with(const Plan& p, const void* W, const void* St, const void* Xb, void* Out,
                 int N, int K, int M, hipStream_t s)
{
    const dim3 grid((unsigned)((N + kRowsPerWG - 1) / kRowsPerWG));
    const dim3 block(64 * WAVES);
    if (p.xlds)
        launch_kernel(h4mv_kernel<WAVES, U, true, OutT>, grid, block, p.lds_bytes, s,
                           static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St),
                           static_cast<const __bf16*>(Xb), static_cast<OutT*>(Out), N, K, M,
                           p.groups_per_wave);
    else
        launch_kernel(h4mv_kernel<WAVES, U, false, OutT>, grid, block, 0, s,
                           static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St),
                           static_cast<const __bf16*>(Xb), static_cast<OutT*>(Out), N, K, M,
                           p.groups_per_wave);
}

constexpr size_t kLdsPerCU = 160 * 1024;

// Tunables (host state; fp8kv_h4mv_tune changes them for sweeps).  0 = the measured defaults:
// one wave per tile when there are >= 1024 tiles, otherwise a K split aiming at 4096 waves, and
// a two-slot ring (deeper rings measured slower at every cfg1/cfg4 shape).
thread_local int g_target_waves = 0;
thread_local int g_depth_override = 0;
thread_local int g_rt_override = 0;
thread_local int g_xg_override = 0;          // 1: activation copies through LDS, 2: direct activation loads

inline int stream_mmax(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

struct StreamPlan {
    int mmax, depth, nw, per, rt;
    bool xg;                    // activation fragments loaded straight from L2 (no LDS copies)
    size_t lds;
};

// Activation path: LDS copies by default.  Direct loads free the LDS the copies take, but measured
// slower at every cfg1 / cfg4 shape (cfg1 M = 8: 18.6 -> 23.4 us, gate+up 20.4 -> 28.6 us: 16
// per-lane loads per step cost more than M 1 KB copies), so they stay a tuning option.
inline bool stream_xg(int M)
{
    (void)M;
    return g_xg_override == 2;
}

// Row tiles (of 16) per workgroup: the activation copies of a step (M KB) then serve rt x 4 KB of
// codes.  Two tiles for M >= 4 when that still gives >= 256 single-wave workgroups that all fit
// on the GPU at once (LDS-limited); otherwise one (measured at cfg1: M = 8 18.9 -> 14.7 us,
// M = 4 14.5 -> 13.8 us; two rounds of workgroups or fewer than 256 lose: gate+up 20.7 -> 21.4,
// qkv 4.6 -> 5.8 us).  Four tiles measured slower at every shape (tuning hook only).
inline int stream_rt(int N, int K, int M)
{
    if (g_rt_override) return g_rt_override;
    if (M < 4) return 1;
    const int tiles2 = (N + 2 * kRowsPerWG - 1) / (2 * kRowsPerWG);
    if (tiles2 < 256) return 1;
    const WaveLds w = wave_lds(stream_mmax(M), stream_xg(M), 2, K >> 9, 2);
    const int per_cu = (int)(kLdsPerCU / (size_t)w.total);
    return tiles2 <= 256 * per_cu ? 2 : 1;
}

// Plan for the streaming kernel, or false when (K, M) needs the register-path kernel.
inline bool stream_plan(int N, int K, int M, StreamPlan& p)
{
    if ((K & 511) != 0 || M > 8) return false;
    p.mmax = stream_mmax(M);
    p.rt = stream_rt(N, K, M);
    p.xg = stream_xg(M);
    const int steps_total = K >> 9;
    const int tiles = (N + kRowsPerWG * p.rt - 1) / (kRowsPerWG * p.rt);
    // Defaults (measured at cfg1 / cfg4): one tile per wave when the tiles alone fill the GPU
    // (>= 1024 with one row tile, >= 256 with several), else a K split aiming at 4096 / rt waves.
    const int target = g_target_waves > 0 ? g_target_waves
                     : (tiles >= (p.rt == 1 ? 1024 : 256) ? tiles : 4096 / p.rt);
    int nreq = stream_waves(N, K, target, p.rt);
    for (;;) {
        p.per = (steps_total + nreq - 1) / nreq;
        p.nw = (steps_total + p.per - 1) / p.per;
        const WaveLds w2 = wave_lds(p.mmax, p.xg, 2, p.per, p.rt);
        if ((size_t)p.nw * w2.total <= kLdsPerCU || nreq == 1) break;
        nreq = std::max(1, nreq - 1);
    }
    const int copies = 4 * p.rt + (p.xg ? 0 : p.mmax);
    const int extra = p.xg ? kXgLoads : 0;
    int depth = 2;
    if (g_depth_override && p.rt == 1) depth = std::max(2, std::min(4, g_depth_override));
    while (depth > 2 && ((depth - 1) * copies + extra >= 64 ||
                         (size_t)p.nw * wave_lds(p.mmax, p.xg, depth, p.per, p.rt).total > kLdsPerCU))
        --depth;
    const WaveLds w = wave_lds(p.mmax, p.xg, depth, p.per, p.rt);
    p.depth = depth;
    p.lds = (size_t)p.nw * w.total;
    return p.lds <= kLdsPerCU;
}

template <int MMAX, bool XG, typename OutT, int EPI = 0>
void launch_stream_x(const StreamPlan& p, const void* W, const void* St, const void* Xb, void* Out,
                     int N, int K, int M, hipStream_t s)
{
    const dim3 grid((unsigned)((N + kRowsPerWG * p.rt - 1) / (kRowsPerWG * p.rt)));
    const dim3 block(64 * p.nw);
#define FP8KV_D(D, RT) \
    launch_kernel(h4mv_stream_kernel<MMAX, XG, D, RT, OutT, EPI>, grid, block, p.lds, s, \
                  static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St), \
                  static_cast<const __bf16*>(Xb), static_cast<OutT*>(Out), N, K, M, p.per)
    if (p.rt == 4) {
        FP8KV_D(2, 4);
    } else if (p.rt == 2) {
        FP8KV_D(2, 2);
    } else {
        switch (p.depth) {
            case 3: FP8KV_D(3, 1); break;
            case 4: FP8KV_D(4, 1); break;
            default: FP8KV_D(2, 1); break;
        }
    }
#undef FP8KV_D
}

template <typename OutT, int EPI = 0>
void launch_stream_m(const StreamPlan& p, const void* W, const void* St, const void* Xb, void* Out,
                     int N, int K, int M, hipStream_t s)
{
    if (p.xg) {                             // MMAX only sizes the LDS copies: one variant
        launch_stream_x<8, true, OutT, EPI>(p, W, St, Xb, Out, N, K, M, s);
        return;
    }
    switch (p.mmax) {
        case 1: launch_stream_x<1, false, OutT, EPI>(p, W, St, Xb, Out, N, K, M, s); break;
        case 2: launch_stream_x<2, false, OutT, EPI>(p, W, St, Xb, Out, N, K, M, s); break;
        case 4: launch_stream_x<4, false, OutT, EPI>(p, W, St, Xb, Out, N, K, M, s); break;
        default: launch_stream_x<8, false, OutT, EPI>(p, W, St, Xb, Out, N, K, M, s); break;
    }
}

// K-slice planner (tunables: fp8kv_h4mv_kslice_tune).  mode 0: used from M = kKsMinM on when
// every CU gets at least two tiles; 1: whenever the shape allows it; 2: never.
thread_local int g_kslice_mode = 0;
thread_local int g_kslice_depth = 0;
thread_local int g_kslice_order = 0;         // 0: default, 1: contiguous, 2: interleaved
thread_local int g_kslice_wgs = 0;           // workgroups the planner aims for (0: kKsWorkgroups)

constexpr int kKsBatch = 8;                    // tiles per partial-tile batch (batched kernel)

struct KsPlan {
    int nw, depth, grid, nt_max, interleaved;
    int batched;                                // h4mv_kslice_batched_kernel
    size_t lds;
};

// allow_batched: the caller can launch the batched kernel (plain output).
inline bool kslice_plan(int N, int K, int M, KsPlan& p, bool allow_batched = false)
{
    p.batched = 0;
    if (g_kslice_mode == 2) return false;
    if ((K & 511) != 0 || N < 16 || M > 8) return false;
    const int steps = K >> 9;
    if (steps > kKsMaxWaves) return false;
    const int T = ks_tiles(N);
    if (g_kslice_mode == 0 && (T < 2 * kKsWorkgroups || M < kKsMinM)) return false;
    p.nw = steps;
    p.depth = g_kslice_depth == 3 ? 3 : 2;
    p.interleaved = g_kslice_order == 1 ? 0 : 1;
    // tiles per workgroup: at most kKsTmax, and rings plus partial tiles within the LDS
    const size_t ring_bytes = (size_t)p.nw * p.depth * kKsSlotBytes;
    const int cap = std::min(kKsTmax, (int)((kLdsPerCU - ring_bytes) / ((size_t)p.nw * 1024)));
    if (cap < 1) return false;
    int G = std::min(T, g_kslice_wgs > 0 ? g_kslice_wgs : kKsWorkgroups);
    if ((T + G - 1) / G > cap && allow_batched && g_kslice_wgs == 0) {
        // More tiles than one round holds at cap: one round of the batched kernel when its rings,
        // one batch of partial tiles and the output tiles fit the LDS.
        const int nt = (T + G - 1) / G;
        const size_t lds = ring_bytes + (size_t)kKsBatch * p.nw * 1024 + (size_t)nt * 1024;
        if (lds <= kLdsPerCU) {
            p.batched = 1;
            p.grid = G;
            p.nt_max = nt;
            p.lds = lds;
            return true;
        }
    }
    if ((T + G - 1) / G > cap) {
        // More tiles than one round of workgroups holds.  Default: whole rounds of kKsWorkgroups,
        // the fewest that keep every workgroup within cap tiles (a short last round runs the GPU
        // part-empty: lm_head N = 128167, K = 3584, M = 8: 56.7 us at 573 workgroups, 14 tiles
        // each, against 51.4 us at 768, 10-11 tiles each).
        if (g_kslice_wgs > 0) G = (T + cap - 1) / cap;
        else G = std::min(T, kKsWorkgroups * ((T + kKsWorkgroups * cap - 1) / (kKsWorkgroups * cap)));
    }
    p.grid = G;
    p.nt_max = (T + G - 1) / G;
    const size_t ring = (size_t)p.nw * p.depth * kKsSlotBytes;
    const size_t red = (size_t)p.nt_max * p.nw * 1024;
    p.lds = ring + red;
    return p.lds <= kLdsPerCU;
}

template <typename OutT, int EPI = 0>
void launch_kslice(const KsPlan& p, const void* W, const void* St, const void* Xb, void* Out,
                   int N, int K, int M, hipStream_t s)
{
    const dim3 grid((unsigned)p.grid), block(64 * p.nw);
    if constexpr (EPI == 0) {
        if (p.batched) {
#define FP8KV_KSB(D) \
    launch_kernel(h4mv_kslice_batched_kernel<D, kKsBatch, OutT>, grid, block, (uint32_t)p.lds, s, \
                  static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St), \
                  static_cast<const __bf16*>(Xb), static_cast<OutT*>(Out), N, K, M, p.interleaved)
            if (p.depth == 3) FP8KV_KSB(3);
            else FP8KV_KSB(2);
#undef FP8KV_KSB
            return;
        }
    }
#define FP8KV_KS(D) \
    launch_kernel(h4mv_kslice_kernel<D, kKsTmax, OutT, EPI>, grid, block, (uint32_t)p.lds, s, \
                  static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St), \
                  static_cast<const __bf16*>(Xb), static_cast<OutT*>(Out), N, K, M, p.interleaved)
    if (p.depth == 3) FP8KV_KS(3);
    else FP8KV_KS(2);
#undef FP8KV_KS
}

// M = 1 planner (tunables: fp8kv_h4mv_m1_tune).  mode 0: used for M = 1 when the tiles alone fill
// the GPU (>= kM1MinTiles); 1: whenever the shape allows it; 2: never.
thread_local int g_m1_mode = 0;
thread_local int g_m1_depth = 0;
thread_local int g_m1_wgs = 0;               // workgroups the planner aims for (0: kM1Workgroups)

struct M1Plan {
    int tw, grid, depth;
    size_t lds;
};

inline bool m1_plan(int N, int K, int M, M1Plan& p)
{
    if (g_m1_mode == 2 || M != 1 || (K & 511) != 0 || (K >> 9) > kM1MaxSteps) return false;
    const int T = (N + kRowsPerWG - 1) / kRowsPerWG;
    if (g_m1_mode == 0 && T < kM1MinTiles) return false;
    const int nsteps = K >> 9;
    // Default: the fewest tiles per workgroup that still run every workgroup in one round, at two
    // workgroups per CU (one per CU when two do not fit the LDS).  Measured (one process, tiles
    // per workgroup 3..10): cfg1 4 tiles 11.30 us against 11.42 at 7 and 12.1-14.0 elsewhere,
    // gate/up 5 tiles 12.89 us against 13.40 at 10 and 13.6-17.0 elsewhere; a grid that needs a
    // second round of workgroups costs 1.5-3 us.
    auto plan_for = [&](int wgs) {
        const int G = std::min(T, wgs);
        p.tw = std::min((T + G - 1) / G, kM1MaxWaves);
        p.grid = (T + p.tw - 1) / p.tw;
        p.lds = (size_t)m1_x_bytes(K) + 2 * (size_t)K + (size_t)p.tw * m1_wave_bytes(p.depth, nsteps);
    };
    for (p.depth = g_m1_depth == 3 ? 3 : 2; p.depth >= 2; --p.depth) {
        if (g_m1_wgs > 0) {
            plan_for(g_m1_wgs);
            if (p.lds <= kLdsPerCU) return true;
            continue;
        }
        plan_for(kM1Workgroups);
        if (2 * p.lds <= kLdsPerCU) return true;
        plan_for(kM1Workgroups / 2);
        if (p.lds <= kLdsPerCU) return true;
    }
    // More tiles than one round holds at any wave count the LDS allows (the lm_head vocabulary:
    // 8011 tiles at K = 3584 would need 16 waves and 178 KB): workgroups of kM1RoundWaves waves,
    // two per CU, over several rounds.  Measured at N = 128167, K = 3584 (one process, two rounds,
    // events / graph replay): 4 waves 38.6-39.0 / 38.9-39.5 us against 39.7-40.3 / 40.5-41.7 on
    // the streaming kernel; 2 waves 38.7-38.8 / 39.0-39.5, 3 waves 38.7-39.1 / 39.3-39.6, 5 and 6
    // waves 39.2-40.1 / 40.1-40.6, 1 wave 42.0-42.8, ring depth 3 the same or slower.
    if (g_m1_wgs == 0) {
        p.depth = 2;
        p.tw = std::min(kM1RoundWaves, T);
        p.grid = (T + p.tw - 1) / p.tw;
        p.lds = (size_t)m1_x_bytes(K) + 2 * (size_t)K + (size_t)p.tw * m1_wave_bytes(p.depth, nsteps);
        if (2 * p.lds <= kLdsPerCU) return true;
    }
    return false;
}

template <typename OutT, int EPI = 0>
void launch_m1(const M1Plan& p, const void* W, const void* St, const void* Xb, void* Out, int N, int K,
               hipStream_t s)
{
    const dim3 grid((unsigned)p.grid), block(64 * p.tw);
#define FP8KV_M1(D) \
    launch_kernel(h4mv_m1_kernel<D, OutT, EPI>, grid, block, (uint32_t)p.lds, s, \
                  static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St), \
                  static_cast<const __bf16*>(Xb), static_cast<OutT*>(Out), N, K)
    if (p.depth == 3) FP8KV_M1(3);
    else FP8KV_M1(2);
#undef FP8KV_M1
}

// M = 2 .. 8 planner (tunables: fp8kv_h4mv_mx_tune), the M = 1 planner's rule with the MM-row
// activation block in LDS: mode 0 = used when the tiles alone fill the GPU (>= kM1MinTiles) and
// every workgroup runs in one round (two workgroups per CU where the LDS allows, else one);
// 1 = whenever the shape allows it; 2 = never.  Measured in one process, two rounds, against the
// bf16 kernels (events / graph replay): cfg1 M = 2 11.0-11.2 / 12.0-12.2 against 12.0 / 13.2-13.5
// us (streaming), M = 4 11.8-11.9 / 12.6-13.2 against 12.6-12.7 / 13.5-13.8 (K-slice), M = 8
// 12.9 / 13.7-14.0 against 13.1-13.2 / 14.0, gate/up M = 4 13.0-13.1 / 14.0-14.5 against 14.7 /
// 15.3-15.7, M = 8 14.5 / 15.4 against 15.4 / 15.8-16.1; M = 5 12.1 against 12.6 us.  With eight
// rows the block (66 KB at K = 4096) leaves room for one workgroup per CU, whose conversion of
// 32768 values is spread over the stream in two-step chunks (mx_chunk_log2).
thread_local int g_mx_mode = 0;
thread_local int g_mx_depth = 0;
thread_local int g_mx_wgs = 0;

thread_local int g_mx_chunk = 0;             // log2 steps per conversion chunk + 1 (0: default)

struct MxPlan {
    int mm, tw, grid, depth, cs_log2;
    size_t lds;
};

// Steps per conversion chunk (log2).  Measured over 1, 2, 4 and all steps (one process, two
// rounds): workgroups of up to four waves convert the whole block first (cfg1 M = 4: 11.9 us
// against 12.3 in 2-step chunks, M = 2: 11.2 against 11.4), larger ones two steps at a time
// while streaming (gate/up M = 4, 5 waves: 12.9 against 13.7; M = 8, 10 waves: 14.5 against
// 15.9; cfg1 M = 8, 7 waves: 13.0 against 14.2).
inline int mx_chunk_log2(int nsteps, int tw)
{
    if (g_mx_chunk > 0) return g_mx_chunk - 1;
    if (tw > 4) return 1;
    int l = 0;
    while ((1 << l) < nsteps) ++l;
    return l;
}

inline int mx_rows(int M) { return M <= 2 ? 2 : M <= 4 ? 4 : 8; }

inline bool mx_plan(int N, int K, int M, MxPlan& p)
{
    if (g_mx_mode == 2 || M < 2 || M > 8 || (K & 511) != 0 || (K >> 9) > kM1MaxSteps) return false;
    const int T = (N + kRowsPerWG - 1) / kRowsPerWG;
    if (g_mx_mode == 0 && T < kM1MinTiles) return false;
    const int nsteps = K >> 9;
    p.mm = mx_rows(M);
    auto plan_for = [&](int wgs) {
        const int G = std::min(T, wgs);
        p.tw = std::min((T + G - 1) / G, kM1MaxWaves);
        p.grid = (T + p.tw - 1) / p.tw;
        p.lds = (size_t)mx_x_bytes(p.mm, K) + (size_t)p.tw * m1_wave_bytes(p.depth, nsteps);
        p.cs_log2 = mx_chunk_log2(nsteps, p.tw);
    };
    for (p.depth = g_mx_depth == 3 ? 3 : 2; p.depth >= 2; --p.depth) {
        if (g_mx_wgs > 0) {
            plan_for(g_mx_wgs);
            if (p.lds <= kLdsPerCU) return true;
            continue;
        }
        plan_for(kM1Workgroups);
        if (2 * p.lds <= kLdsPerCU && (g_mx_mode == 1 || p.grid <= kM1Workgroups)) return true;
        plan_for(kM1Workgroups / 2);
        if (p.lds <= kLdsPerCU && (g_mx_mode == 1 || p.grid <= kM1Workgroups / 2)) return true;
    }
    // Two activation rows and more tiles than one round holds (the lm_head vocabulary): workgroups
    // of kM1RoundWaves waves over several rounds, as at M = 1.  Measured at N = 128167, K = 3584
    // (one process, two rounds, events / graph replay): M = 2 38.6-38.8 / 39.2-39.6 us against
    // 40.3-41.9 / 40.8-41.9 on the streaming kernel; at M = 4 the same form ties with the batched
    // K-slice kernel (41.7-42.6 against 41.6-42.1) and at M = 8 it is slower (67.7-68.0 against
    // 43.6-44.8: every workgroup converts all eight rows), so those keep the K-slice kernels.
    if (g_mx_wgs == 0 && p.mm == 2) {
        p.depth = 2;
        p.tw = std::min(kM1RoundWaves, T);
        p.grid = (T + p.tw - 1) / p.tw;
        p.lds = (size_t)mx_x_bytes(p.mm, K) + (size_t)p.tw * m1_wave_bytes(p.depth, nsteps);
        p.cs_log2 = mx_chunk_log2(nsteps, p.tw);
        if (2 * p.lds <= kLdsPerCU) return true;
    }
    return false;
}

template <typename OutT, int EPI = 0>
void launch_mx(const MxPlan& p, const void* W, const void* St, const void* Xb, void* Out, int N, int K,
               int M, hipStream_t s)
{
    const dim3 grid((unsigned)p.grid), block(64 * p.tw);
#define FP8KV_MX(MM, D) \
    launch_kernel(h4mv_mx_kernel<MM, D, OutT, EPI>, grid, block, (uint32_t)p.lds, s, \
                  static_cast<const uint8_t*>(W), static_cast<const uint8_t*>(St), \
                  static_cast<const __bf16*>(Xb), static_cast<OutT*>(Out), N, K, M, p.cs_log2)
    if (p.depth == 3) {
        if (p.mm == 2) FP8KV_MX(2, 3);
        else if (p.mm == 4) FP8KV_MX(4, 3);
        else FP8KV_MX(8, 3);
    } else {
        if (p.mm == 2) FP8KV_MX(2, 2);
        else if (p.mm == 4) FP8KV_MX(4, 2);
        else FP8KV_MX(8, 2);
    }
#undef FP8KV_MX
}

template <typename OutT>
int launch_h4mv(const void* W, const void* St, const void* Xb, void* Out, int N, int K, int M,
                void* stream)
{
    if (!W || !St || !Xb || !Out) return FP8KV_ERR_ARG;
    if (N < 1 || K < 32 || M < 1) return FP8KV_ERR_ARG;
    if (M > 16 || (K & 31) != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(W, 16) || !aligned(Xb, 16) || !aligned(Out, sizeof(OutT))) return FP8KV_ERR_ALIGN;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    begin_launch();
    M1Plan mp;
    MxPlan xp;
    KsPlan kp;
    StreamPlan p;
    if (aligned(St, 4) && m1_plan(N, K, M, mp)) {
        launch_m1<OutT>(mp, W, St, Xb, Out, N, K, s);
    } else if (aligned(St, 4) && mx_plan(N, K, M, xp)) {
        launch_mx<OutT>(xp, W, St, Xb, Out, N, K, M, s);
    } else if (aligned(St, 4) && kslice_plan(N, K, M, kp, true)) {
        launch_kslice<OutT>(kp, W, St, Xb, Out, N, K, M, s);
    } else if (aligned(St, 4) && stream_plan(N, K, M, p)) {
        launch_stream_m<OutT>(p, W, St, Xb, Out, N, K, M, s);
    } else {
        const Plan rp = make_plan(K, M, 4);
        launch_with<4, 8, OutT>(rp, W, St, Xb, Out, N, K, M, s);
    }
    return finish_launch();
}

}  // namespace h4mv_detail
}  // namespace fp8kv

extern "C" int h4mv_silu_mul(const void* W, const void* St, const void* Xb, void* Out, int N, int K,
                             int M, int mode, void* stream)
{
    using namespace fp8kv;
    using namespace fp8kv::h4mv_detail;
    if (!W || !St || !Xb || !Out) return FP8KV_ERR_ARG;
    if (N < 16 || K < 32 || M < 1 || (mode != 0 && mode != 1)) return FP8KV_ERR_ARG;
    if (M > 8 || (K & 511) != 0 || (N & 15) != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(W, 16) || !aligned(Xb, 16) || !aligned(Out, 8) || !aligned(St, 4)) return FP8KV_ERR_ALIGN;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    M1Plan mp;
    if (m1_plan(N, K, M, mp)) {
        begin_launch();
        if (mode == 0) launch_m1<__bf16, 1>(mp, W, St, Xb, Out, N, K, s);
        else launch_m1<__bf16, 2>(mp, W, St, Xb, Out, N, K, s);
        return finish_launch();
    }
    MxPlan xp;
    if (mx_plan(N, K, M, xp)) {
        begin_launch();
        if (mode == 0) launch_mx<__bf16, 1>(xp, W, St, Xb, Out, N, K, M, s);
        else launch_mx<__bf16, 2>(xp, W, St, Xb, Out, N, K, M, s);
        return finish_launch();
    }
    KsPlan kp;
    if (kslice_plan(N, K, M, kp)) {
        begin_launch();
        if (mode == 0) launch_kslice<__bf16, 1>(kp, W, St, Xb, Out, N, K, M, s);
        else launch_kslice<__bf16, 2>(kp, W, St, Xb, Out, N, K, M, s);
        return finish_launch();
    }
    StreamPlan p;
    if (!stream_plan(N, K, M, p)) return FP8KV_ERR_SHAPE;
    begin_launch();
    if (mode == 0) launch_stream_m<__bf16, 1>(p, W, St, Xb, Out, N, K, M, s);
    else launch_stream_m<__bf16, 2>(p, W, St, Xb, Out, N, K, M, s);
    return finish_launch();
}

// ---------------------------------------------------------------------------------------------
// Host-side address audit of the streaming kernel: enumerates, for the launch the entry points
// would make for (N, K, M), every global byte each copy instruction reads and every LDS byte each
// copy writes or each fragment read touches, and checks them against the operand sizes and the
// dynamic LDS allocation.  Returns 0 when every access is in bounds, 1 when the shape does not
// use the streaming kernel, and 2 + the index of the first violated check otherwise.
// ---------------------------------------------------------------------------------------------
namespace fp8kv { namespace h4mv_detail {

int audit_stream(int N, int K, int M, const StreamPlan& p)
{
    const int steps_total = K >> 9;
    const int per = p.per, nw = p.nw, depth = p.depth, MMAX = p.mmax, RT = p.rt;
    if (RT != 1 && RT != 2 && RT != 4) return 3;
    if (nw > (RT == 1 ? 16 : kMaxWavesRT) || nw * per < steps_total || (nw - 1) * per >= steps_total) return 2;
    if (p.lds > kLdsPerCU || depth < 2 || depth > 4 || (RT > 1 && depth != 2)) return 3;
    if ((depth - 1) * (4 * RT + (p.xg ? 0 : MMAX)) + (p.xg ? kXgLoads : 0) >= 64) return 3;
    const WaveLds L = wave_lds(MMAX, p.xg, depth, per, RT);
    if ((size_t)nw * L.total != p.lds) return 3;
    const size_t wbytes = (size_t)N * (size_t)(K >> 1), sbytes = (size_t)N * (size_t)(K >> 5);
    const size_t xbytes = (size_t)M * (size_t)K * 2;
    const int rows = kRowsPerWG * RT;
    for (int wg = 0; wg * rows < N; ++wg) {
        const int n0 = wg * rows;
        for (int w = 0; w < nw; ++w) {
            const size_t wb = (size_t)w * L.total;
            const int step0 = w * per;
            const int nsteps = std::max(0, std::min(per, steps_total - step0));
            if (nsteps > 0) {
                for (int t = 0; t < 16 * RT * per; ++t) {     // one-time scale copies
                    if ((t % per) >= nsteps) continue;
                    if (stream_s_seg_off(n0, N, K, per, step0, t) + 16 > sbytes) return 6;
                    if (wb + L.ring + 16 * (size_t)t + 16 > wb + L.ring + L.scales) return 7;
                }
            }
            for (int s = 0; s < nsteps; ++s) {
                const int gs = (step0 + s) * kStepGroups;
                const size_t slot = wb + (size_t)(s % depth) * L.slot;
                for (int lane = 0; lane < 64; ++lane) {
                    for (int i = 0; i < 4 * RT; ++i) {
                        const size_t g = (size_t)n0 * (K >> 1) + (size_t)gs * 16 + stream_w_lane_off(n0, N, K, lane, i);
                        if (g + 16 > wbytes) return 4;
                        if (slot + i * 1024 + 16 * lane + 16 > slot + RT * kStepCodeBytes) return 5;
                    }
                    if (!p.xg)
                        for (int m = 0; m < MMAX; ++m) {
                            if (stream_x_off(K, M, m, gs, lane) + 16 > xbytes) return 8;
                            if (RT * kStepCodeBytes + m * 1024 + 16 * lane + 16 > L.slot) return 9;
                        }
                    const int r = lane & 15, q = lane >> 4;
                    for (int t = 0; t < RT; ++t) {
                        if (L.ring + (size_t)((16 * t + r) * per + s) * 16 + 16 > (size_t)(L.ring + L.scales)) return 10;
                        for (int u = 0; u < 4; ++u)
                            if (t * kStepCodeBytes + stream_w_read_off(r, q, u) + 16 > RT * kStepCodeBytes) return 11;
                    }
                    for (int u = 0; u < 4; ++u)
                        for (int j = 0; j < 4; ++j) {
                            if (p.xg) {                    // direct loads, row M - 1 for r >= M
                                const size_t xo = (size_t)(r < M ? r : M - 1) * (size_t)K * 2 +
                                                  (size_t)gs * 64 + stream_x_frag_off(q, u, j);
                                if (xo + 16 > xbytes) return 14;
                                continue;
                            }
                            if (r >= M) continue;
                            const size_t xo = (size_t)(s % depth) * L.slot + RT * kStepCodeBytes + r * 1024;
                            const size_t end = (size_t)(s % depth) * L.slot + L.slot;
                            if (xo + stream_x_frag_off(q, u, j) + 16 > end) return 12;
                        }
                }
            }
            if (wb + (size_t)RT * 64 * 16 > p.lds) return 13;    // partial-tile exchange
        }
    }
    return 0;
}

// Audit of the K-slice kernel (same return convention as audit_stream): tile coverage, every
// code / scale / activation byte read, every LDS byte written or read.
int audit_kslice(int N, int K, int M, const KsPlan& p)
{
    const int T = ks_tiles(N), G = p.grid, nw = p.nw, depth = p.depth;
    if (N < 16 || (K & 511) || nw != (K >> 9) || nw > kKsMaxWaves || G < 1 || G > T) return 2;
    if (depth < 2 || depth > 3 || p.lds > kLdsPerCU) return 3;
    if (p.batched) {
        if ((size_t)nw * depth * kKsSlotBytes + (size_t)kKsBatch * nw * 1024 + (size_t)p.nt_max * 1024 > p.lds)
            return 3;
    } else if ((size_t)nw * depth * kKsSlotBytes + (size_t)p.nt_max * nw * 1024 > p.lds) {
        return 3;
    }
    const size_t wbytes = (size_t)N * (size_t)(K >> 1), sbytes = (size_t)N * (size_t)(K >> 5);
    const size_t xbytes = (size_t)M * (size_t)K * 2;
    const size_t slot = kKsSlotBytes;
    std::vector<unsigned char> seen((size_t)T, 0), stored((size_t)N, 0);
    for (int b = 0; b < G; ++b) {
        int t0, nt, tstride;
        ks_tiles_of(b, T, G, p.interleaved != 0, t0, nt, tstride);
        if (nt < 1 || (!p.batched && nt > kKsTmax) || nt > p.nt_max) return 4;
        for (int i = 0; i < nt; ++i) {                    // every tile exactly once
            const long t = (long)t0 + (long)i * tstride;
            if (t < 0 || t >= T || seen[(size_t)t]) return 4;
            seen[(size_t)t] = 1;
            // output rows the tile stores: 16 t .. min(row0 + 16, N) - 1 (store_tile / store_rows)
            const int hi = std::min(ks_row0((int)t, N) + kRowsPerWG, N);
            for (int n = 16 * (int)t; n < hi; ++n) {
                if (stored[(size_t)n]) return 15;
                stored[(size_t)n] = 1;
            }
        }
        for (int w = 0; w < nw; ++w) {
            const int gs = w * kStepGroups;
            const size_t ring = (size_t)w * depth * slot;
            if (ring + depth * slot > p.lds) return 5;
            for (int lane = 0; lane < 64; ++lane) {
                const int r = lane & 15, q = lane >> 4;
                if (r < M)
                    for (int u = 0; u < 4; ++u)
                        for (int j = 0; j < 4; ++j)
                            if ((size_t)r * K * 2 + (size_t)gs * 64 + stream_x_frag_off(q, u, j) + 16 > xbytes) return 6;
                for (int i = 0; i < nt; ++i) {
                    const size_t sl = ring + (size_t)(i % depth) * slot;
                    const int tile = t0 + i * tstride;
                    const size_t n0 = (size_t)ks_row0(tile, N);
                    if (n0 + kRowsPerWG > (size_t)N) return 7;
                    if (16 * tile < N - 16 ? n0 != (size_t)(16 * tile) : n0 + kRowsPerWG != (size_t)N) return 7;
                    const size_t wt = n0 * (K >> 1) + (size_t)gs * 16;
                    for (int c = 0; c < 4; ++c) {
                        if (wt + stream_w_lane_off(0, kRowsPerWG, K, lane, c) + 16 > wbytes) return 7;
                        if (c * 1024 + 16 * lane + 16 > kStepCodeBytes) return 8;
                    }
                    const size_t st = n0 * (K >> 5) + gs;
                    if (st + ks_s_lane_off(K, lane) + 4 > sbytes) return 9;
                    if (kStepCodeBytes + 4 * lane + 4 > (int)slot) return 10;
                    if (kStepCodeBytes + 16 * r + 16 > (int)slot) return 11;
                    for (int u = 0; u < 4; ++u)
                        if (stream_w_read_off(r, q, u) + 16 > kStepCodeBytes) return 12;
                    if (sl + slot > p.lds) return 13;
                    const size_t rings = (size_t)nw * depth * slot;
                    if (p.batched) {
                        // partial tile (i mod B, w), then output tile i (batched kernel)
                        const size_t redb = (size_t)kKsBatch * nw * 1024;
                        if ((((size_t)(i % kKsBatch) * nw + w) * 64 + lane) * 16 + 16 > redb) return 14;
                        if (rings + redb + ((size_t)i * 64 + lane) * 16 + 16 > p.lds) return 14;
                    } else if (rings + (((size_t)i * nw + w) * 64 + lane) * 16 + 16 > p.lds) {
                        return 14;
                    }
                }
            }
        }
    }
    for (int t = 0; t < T; ++t)
        if (!seen[(size_t)t]) return 4;
    for (int n = 0; n < N; ++n)
        if (!stored[(size_t)n]) return 15;
    return 0;
}

// Audit of the M = 1 kernel (same return convention as audit_stream): tile coverage, every
// activation / code / scale byte read, every LDS byte written or read, the activation groups of
// each block held by one quad of lanes.
int audit_m1(int N, int K, const M1Plan& p)
{
    const int T = (N + kRowsPerWG - 1) / kRowsPerWG, G = p.grid, tw = p.tw, depth = p.depth;
    if ((K & 511) || tw < 1 || tw > kM1MaxWaves || G < 1 || (long)G * tw < T || depth < 2 || depth > 3) return 2;
    const int nsteps = K >> 9, nthreads = 64 * tw, np = K >> 3;
    const size_t xb = (size_t)m1_x_bytes(K), xs = xb, wb = (size_t)m1_wave_bytes(depth, nsteps);
    if (xb + 2 * (size_t)K + (size_t)tw * wb != p.lds || p.lds > kLdsPerCU) return 3;
    const size_t wbytes = (size_t)N * (size_t)(K >> 1), sbytes = (size_t)N * (size_t)(K >> 5);
    const size_t xbytes = (size_t)K * 2;
    // the row's copies: every piece once, inside the operand and the staging area
    std::vector<unsigned char> pseen((size_t)np, 0);
    for (int w = 0; w < tw; ++w)
        for (int p0 = w * 64; p0 < np; p0 += tw * 64)
            for (int lane = 0; lane < 64 && p0 + lane < np; ++lane) {
                const int pc = p0 + lane;
                if (16 * (size_t)pc + 16 > xbytes || xs + 16 * (size_t)p0 + 16 * lane + 16 > xs + xbytes) return 4;
                if (pseen[(size_t)pc]) return 4;
                pseen[(size_t)pc] = 1;
            }
    for (size_t i = 0; i < pseen.size(); ++i)
        if (!pseen[i]) return 4;
    // conversion: staging reads and hi / lo / scale writes in range, the four groups of a block
    // in one quad of lanes, every group converted
    std::vector<unsigned char> gseen((size_t)np, 0);
    for (int g0 = 0; g0 < np; g0 += nthreads)
        for (int t = 0; t < nthreads; ++t) {
            const int gr = g0 + t, g = gr < np ? gr : np - 4 + (gr & 3);
            const int gq = g0 + (t & ~3), gq0 = gq < np ? gq : np - 4;
            if ((g & ~3) != gq0 || (g & 3) != (t & 3)) return 5;
            if (16 * (size_t)g + 16 > xbytes || 8 * (size_t)g + 8 > (size_t)K) return 5;
            if (2 * (size_t)K + (size_t)m1_xe_pos(g >> 2) + 1 > xb) return 5;
            gseen[(size_t)g] = 1;
        }
    for (size_t g = 0; g < gseen.size(); ++g)
        if (!gseen[g]) return 5;
    std::vector<unsigned char> seen((size_t)T, 0);
    for (int b = 0; b < G; ++b)
        for (int w = 0; w < tw; ++w) {
            const int tw_tile = b + w * G;
            const bool has = tw_tile < T;
            if (has) {
                if (seen[(size_t)tw_tile]) return 6;
                seen[(size_t)tw_tile] = 1;
            }
            const int n0 = (has ? tw_tile : b) * kRowsPerWG;
            const size_t ring = xs + 2 * (size_t)K + (size_t)w * wb, sarea = ring + (size_t)depth * kStepCodeBytes;
            if (ring + wb > p.lds) return 7;
            for (int lane = 0; lane < 64; ++lane) {
                for (int t0 = 0; t0 < 16 * nsteps; t0 += 64) {        // scale slice copies
                    const int t = std::min(t0 + lane, 16 * nsteps - 1);
                    if (stream_s_seg_off(n0, N, K, nsteps, 0, t) + 16 > sbytes) return 8;
                    if (sarea + 16 * (size_t)(t0 + lane) + 16 > ring + wb) return 8;
                }
                for (int s = 0; s < nsteps; ++s)                       // code copies
                    for (int i = 0; i < 4; ++i) {
                        const size_t g = (size_t)n0 * (K >> 1) + (size_t)s * 256 + stream_w_lane_off(n0, N, K, lane, i);
                        if (g + 16 > wbytes) return 9;
                        if ((size_t)(s % depth) * kStepCodeBytes + i * 1024 + 16 * lane + 16 > (size_t)depth * kStepCodeBytes) return 9;
                    }
                const int r = lane & 15, q = lane >> 4;
                for (int s = 0; s < nsteps; ++s) {                     // fragment reads
                    if ((size_t)((r * nsteps + s) * 16 + 16) > (size_t)m1_scale_bytes(nsteps)) return 10;
                    for (int u = 0; u < 4; ++u) {
                        if (stream_w_read_off(r, q, u) + 16 > kStepCodeBytes) return 11;
                        const size_t k = (size_t)512 * s + 128 * u + 16 * q;
                        if ((r & 1 ? (size_t)K : 0) + k + 64 + 16 > (size_t)2 * K) return 12;
                        if (k + 64 + 16 > (size_t)K) return 12;
                    }
                    if (2 * (size_t)K + 16 * (size_t)s + 4 * q + 4 > xb) return 13;
                }
            }
        }
    for (int t = 0; t < T; ++t)
        if (!seen[(size_t)t]) return 6;
    return 0;
}

// Audit of the M = 2 .. 8 kernel (same return convention): tile coverage, every activation /
// code / scale byte read, every LDS byte written or read, the two units of a block in
// neighbouring lanes of one pass, and every converted unit owned by one thread.
int audit_mx(int N, int K, int M, const MxPlan& p)
{
    const int T = (N + kRowsPerWG - 1) / kRowsPerWG, G = p.grid, tw = p.tw, depth = p.depth, mm = p.mm;
    if ((K & 511) || M < 2 || M > mm || mm > 8 || tw < 1 || tw > kM1MaxWaves || G < 1 || (long)G * tw < T ||
        depth < 2 || depth > 3)
        return 2;
    const int nsteps = K >> 9, nthreads = 64 * tw, rowb = mx_row_bytes(K), xerow = mx_xe_row_bytes(K);
    const size_t xb = (size_t)mx_x_bytes(mm, K), wb = (size_t)m1_wave_bytes(depth, nsteps);
    if (xb + (size_t)tw * wb != p.lds || p.lds > kLdsPerCU) return 3;
    if ((rowb & 255) != kMxRowPad || (xerow & 3)) return 3;
    const size_t wbytes = (size_t)N * (size_t)(K >> 1), sbytes = (size_t)N * (size_t)(K >> 5);
    const size_t xbytes = (size_t)M * (size_t)K * 2;
    // the rows' copies: every LDS byte of the mm rows' first 2K bytes written once, sources in X
    std::vector<unsigned char> lseen((size_t)mm * rowb, 0);
    const int nunits = mm * nsteps;
    for (int w = 0; w < tw; ++w)
        for (int u = w; u < nunits; u += tw)
            for (int lane = 0; lane < 64; ++lane) {
                if (mx_copy_src(K, M, mm, u, lane) + 16 > xbytes) return 4;
                const int d = mx_copy_dst(K, mm, u, lane);
                if (d + 16 > mm * rowb) return 4;
                for (int b = 0; b < 16; ++b) {
                    if (lseen[(size_t)d + b]) return 4;
                    lseen[(size_t)d + b] = 1;
                }
            }
    for (int m = 0; m < mm; ++m)
        for (int b = 0; b < 2 * K; ++b)
            if (!lseen[(size_t)m * rowb + b]) return 4;
    // conversion, chunk by chunk as mx_convert_chunk deals it: the units of a block in lanes
    // 2i, 2i + 1 of one pass, each unit converted once, reads and writes inside the rows, scale
    // bytes inside the scale rows
    const int upr = K >> 4;
    std::vector<unsigned char> useen((size_t)M * upr, 0);
    if (p.cs_log2 < 0 || p.cs_log2 > 6) return 5;
    const int U = 32 << p.cs_log2, total = M * U, nchunks = (nsteps + (1 << p.cs_log2) - 1) >> p.cs_log2;
    for (int j = 0; j < nchunks; ++j) {
        for (int i0 = 0; i0 < total; i0 += nthreads)
            for (int t = 0; t < nthreads; ++t) {
                if (i0 + 64 * (t / 64) >= total) continue;          // the wave skips the pass
                const int i = i0 + t, ip = i ^ 1;
                const int m = i / U, pp = U * j + i % U, mp = ip / U, ppp = U * j + ip % U;
                const bool live = i < total && pp < upr, livep = ip < total && ppp < upr;
                if (live != livep) return 5;                        // a block's halves live or die together
                if (!live) continue;                                // reads unit 0 of row 0, writes nothing
                if (m != mp || (pp >> 1) != (ppp >> 1)) return 5;   // the DPP partner holds the block's other half
                if (m >= M || 32 * pp + 32 > 2 * K) return 5;
                if ((pp >> 1) >= (K >> 5) || m * xerow + m1_xe_pos(pp >> 1) + 1 > mm * xerow) return 5;
                if (useen[(size_t)m * upr + pp]) return 5;
                useen[(size_t)m * upr + pp] = 1;
            }
    }
    for (size_t g = 0; g < useen.size(); ++g)
        if (!useen[g]) return 5;
    // vmcnt: replay each wave's copies in issue order and check that every wait the kernel makes
    // (same count formulas) leaves outstanding only copies younger than the ones the next use needs
    {
        const int cs = 1 << p.cs_log2, nchunks = (nsteps + cs - 1) / cs, nscale = (16 * nsteps + 63) / 64;
        for (int w = 0; w < tw; ++w)
            for (int has = 0; has < 2; ++has) {
                // op kinds: 0 = activation unit (id = chunk), 1 = ring step (id = step), 2 = scale
                std::vector<std::pair<int, int>> ops;
                for (int u = w; u < nunits; u += tw) ops.push_back({0, (u / mm) / cs});
                for (int i = 0; i < 4; ++i) ops.push_back({1, 0});
                for (int k = 0; k < nscale; ++k) ops.push_back({2, 0});
                for (int d = 1; d < depth; ++d)
                    for (int i = 0; i < 4; ++i) ops.push_back({1, std::min(d, nsteps - 1)});
                auto landed_ok = [&](int n, auto need) {
                    for (int i = (int)ops.size() - std::min(n, 63); i < (int)ops.size(); ++i)
                        if (need(ops[(size_t)i])) return false;
                    return true;
                };
                auto chunk_need = [](int c) { return [c](std::pair<int, int> o) { return o.first == 0 && o.second == c; }; };
                if (!landed_ok(mx_after_chunk(mm, nsteps, cs, depth, nscale, 0, w, tw, has != 0), chunk_need(0)))
                    return 14;
                for (int j = 0; j < nchunks; ++j) {
                    if (j + 1 < nchunks &&
                        !landed_ok(mx_after_chunk(mm, nsteps, cs, depth, nscale, j + 1, w, tw, has != 0), chunk_need(j + 1)))
                        return 14;
                    if (!has) continue;
                    for (int st = cs * j; st < std::min(nsteps, cs * (j + 1)); ++st) {
                        if (!landed_ok(4 * std::min(nsteps - 1 - st, depth - 1), [&](std::pair<int, int> o) {
                                return (o.first == 1 && o.second == st) || (st == 0 && o.first == 2); }))
                            return 14;
                        if (st + depth < nsteps)
                            for (int i = 0; i < 4; ++i) ops.push_back({1, st + depth});
                    }
                }
            }
    }
    std::vector<unsigned char> seen((size_t)T, 0);
    for (int b = 0; b < G; ++b)
        for (int w = 0; w < tw; ++w) {
            const int tw_tile = b + w * G;
            const bool has = tw_tile < T;
            if (has) {
                if (seen[(size_t)tw_tile]) return 6;
                seen[(size_t)tw_tile] = 1;
            }
            const int n0 = (has ? tw_tile : b) * kRowsPerWG;
            const size_t ring = xb + (size_t)w * wb, sarea = ring + (size_t)depth * kStepCodeBytes;
            if (ring + wb > p.lds) return 7;
            for (int lane = 0; lane < 64; ++lane) {
                for (int t0 = 0; t0 < 16 * nsteps; t0 += 64) {        // scale slice copies
                    const int t = std::min(t0 + lane, 16 * nsteps - 1);
                    if (stream_s_seg_off(n0, N, K, nsteps, 0, t) + 16 > sbytes) return 8;
                    if (sarea + 16 * (size_t)(t0 + lane) + 16 > ring + wb) return 8;
                }
                for (int s = 0; s < nsteps; ++s)                       // code copies
                    for (int i = 0; i < 4; ++i) {
                        const size_t g = (size_t)n0 * (K >> 1) + (size_t)s * 256 + stream_w_lane_off(n0, N, K, lane, i);
                        if (g + 16 > wbytes) return 9;
                        if ((size_t)(s % depth) * kStepCodeBytes + i * 1024 + 16 * lane + 16 > (size_t)depth * kStepCodeBytes) return 9;
                    }
                const int r = lane & 15, q = lane >> 4, mrow = (r >> 1) & (mm - 1);
                for (int s = 0; s < nsteps; ++s) {                     // fragment reads
                    if ((size_t)((r * nsteps + s) * 16 + 16) > (size_t)m1_scale_bytes(nsteps)) return 10;
                    for (int u = 0; u < 4; ++u) {
                        if (stream_w_read_off(r, q, u) + 16 > kStepCodeBytes) return 11;
                        // unit 32 s + 8 u + q (k 512 s + 128 u + 16 q ..) and + 4 (k + 64 ..)
                        const int unit = 32 * s + 8 * u + q;
                        if (unit + 4 >= upr) return 12;
                        const size_t off = (size_t)mrow * rowb + 32 * (size_t)(unit + 4) + 16 * (r & 1);
                        if (off + 16 > (size_t)mrow * rowb + 2 * (size_t)K) return 12;
                    }
                    if ((size_t)mrow * xerow + 16 * (size_t)s + 4 * q + 4 > (size_t)mrow * xerow + (((K >> 5) + 15) & ~15))
                        return 13;
                }
            }
        }
    for (int t = 0; t < T; ++t)
        if (!seen[(size_t)t]) return 6;
    return 0;
}

}}  // namespace fp8kv::h4mv_detail

extern "C" int fp8kv_h4mv_audit(int N, int K, int M)
{
    using namespace fp8kv::h4mv_detail;
    if (N < 1 || K < 32 || M < 1 || M > 16 || (K & 31)) return 2;
    M1Plan mp;
    if (m1_plan(N, K, M, mp)) return audit_m1(N, K, mp);
    MxPlan xp;
    if (mx_plan(N, K, M, xp)) return audit_mx(N, K, M, xp);
    KsPlan kp;
    if (kslice_plan(N, K, M, kp, true)) return audit_kslice(N, K, M, kp);
    StreamPlan p;
    if (!stream_plan(N, K, M, p)) return 1;
    return audit_stream(N, K, M, p);
}

extern "C" void fp8kv_h4mv_kslice_tune(int mode, int depth, int order, int workgroups)
{
    fp8kv::h4mv_detail::g_kslice_mode = (mode == 1 || mode == 2) ? mode : 0;
    fp8kv::h4mv_detail::g_kslice_depth = depth;
    fp8kv::h4mv_detail::g_kslice_order = (order == 1 || order == 2) ? order : 0;
    fp8kv::h4mv_detail::g_kslice_wgs = workgroups > 0 ? workgroups : 0;
}

extern "C" void fp8kv_h4mv_m1_tune(int mode, int depth, int workgroups)
{
    fp8kv::h4mv_detail::g_m1_mode = (mode == 1 || mode == 2) ? mode : 0;
    fp8kv::h4mv_detail::g_m1_depth = depth;
    fp8kv::h4mv_detail::g_m1_wgs = workgroups > 0 ? workgroups : 0;
}

extern "C" int fp8kv_h4mv_plan(int N, int K, int M, int* out)
{
    using namespace fp8kv::h4mv_detail;
    if (!out) return FP8KV_ERR_ARG;
    if (N < 1 || K < 32 || M < 1) return FP8KV_ERR_ARG;
    if (M > 16 || (K & 31) != 0) return FP8KV_ERR_SHAPE;
    for (int i = 0; i < 6; ++i) out[i] = 0;
    M1Plan mp;
    MxPlan xp;
    KsPlan kp;
    StreamPlan sp;
    if (m1_plan(N, K, M, mp)) {
        const int v[6] = {3, mp.grid, mp.tw, mp.depth, (int)mp.lds, 1};
        for (int i = 0; i < 6; ++i) out[i] = v[i];
    } else if (mx_plan(N, K, M, xp)) {
        const int v[6] = {4, xp.grid, xp.tw, xp.depth, (int)xp.lds, xp.mm};
        for (int i = 0; i < 6; ++i) out[i] = v[i];
    } else if (kslice_plan(N, K, M, kp, true)) {
        const int v[6] = {kp.batched ? 5 : 2, kp.grid, kp.nw, kp.depth, (int)kp.lds, kp.nt_max};
        for (int i = 0; i < 6; ++i) out[i] = v[i];
    } else if (stream_plan(N, K, M, sp)) {
        const int v[6] = {1, (N + kRowsPerWG * sp.rt - 1) / (kRowsPerWG * sp.rt), sp.nw, sp.depth, (int)sp.lds, sp.rt};
        for (int i = 0; i < 6; ++i) out[i] = v[i];
    } else {
        out[0] = 0;
        out[1] = (N + kRowsPerWG - 1) / kRowsPerWG;
        out[2] = 4;
    }
    return FP8KV_OK;
}

extern "C" void fp8kv_h4mv_mx_tune(int mode, int depth, int workgroups)
{
    fp8kv::h4mv_detail::g_mx_mode = (mode == 1 || mode == 2) ? mode : 0;
    fp8kv::h4mv_detail::g_mx_depth = depth;
    fp8kv::h4mv_detail::g_mx_wgs = workgroups > 0 ? workgroups : 0;
}

extern "C" void fp8kv_h4mv_mx_chunk_tune(int steps_log2)
{
    fp8kv::h4mv_detail::g_mx_chunk = (steps_log2 >= 0 && steps_log2 <= 6) ? steps_log2 + 1 : 0;
}

extern "C" void fp8kv_h4mv_tune(int target_waves, int depth, int row_tiles, int x_mode)
{
    fp8kv::h4mv_detail::g_xg_override = (x_mode == 1 || x_mode == 2) ? x_mode : 0;
    fp8kv::h4mv_detail::g_rt_override = (row_tiles == 1 || row_tiles == 2 || row_tiles == 4) ? row_tiles : 0;
    fp8kv::h4mv_detail::g_target_waves = target_waves > 0 ? target_waves : 0;
    fp8kv::h4mv_detail::g_depth_override = depth;
}

extern "C" int h4mv_launch_status(const void* W, const void* St, const void* Xb, void* Out,
                                  int N, int K, int M, void* stream)
{
    return fp8kv::h4mv_detail::launch_h4mv<__bf16>(W, St, Xb, Out, N, K, M, stream);
}

extern "C" int h4mv_f32_launch_status(const void* W, const void* St, const void* Xb, void* Out,
                                      int N, int K, int M, void* stream)
{
    return fp8kv::h4mv_detail::launch_h4mv<float>(W, St, Xb, Out, N, K, M, stream);
}

extern "C" void h4mv_launch(const void* W, const void* St, const void* Xb, void* Out,
                            int N, int K, int M, void* stream)
{
    fp8kv::g_last_status = h4mv_launch_status(W, St, Xb, Out, N, K, M, stream);
}

extern "C" int fp8kv_last_status(void) { return fp8kv::g_last_status; }

extern "C" void fp8kv_time_next_launch(void* start_event, void* stop_event)
{
    fp8kv::g_time_start = static_cast<hipEvent_t>(start_event);
    fp8kv::g_time_stop = static_cast<hipEvent_t>(stop_event);
}

extern "C" int fp8kv_last_hip_error(void) { return fp8kv::g_last_hip_error; }

extern "C" const char* fp8kv_last_hip_error_string(void)
{
    return hipGetErrorString(static_cast<hipError_t>(fp8kv::g_last_hip_error));
}

extern "C" const char* fp8kv_status_string(int status)
{
    switch (status) {
        case FP8KV_OK: return "ok";
        case FP8KV_ERR_ARG: return "invalid argument";
        case FP8KV_ERR_SHAPE: return "unsupported shape";
        case FP8KV_ERR_ALIGN: return "misaligned pointer or stride";
        case FP8KV_ERR_LAUNCH: return "kernel launch failed";
        case FP8KV_ERR_SCRATCH: return "scratch buffer missing or too small";
        default: return "unknown status";
    }
}
