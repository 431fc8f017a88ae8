// MXFP4 x MXFP8 GEMM for M >= 16 (prefill-sized linears) on gfx950's block-scaled MFMA, and the
// MXFP8 activation quantiser that feeds it.
//
//   Out[m, n] = bf16( sum_k  xq[m, k] * 2^(sx[m, k/32] - 127)  *  w[n, k] * 2^(sw[n, k/32] - 127) )
//
// w: e2m1 codes [N, K/2] (low nibble = even k) with e8m0 scales St [N, K/32] - the matvec's layout
// (h4mv/h4mv.cu:1-3 with the scale repack of h4mv/fp8kv_hipw4.py:32-43); xq: e4m3fn [M, K] with
// e8m0 scales Sx [M, K/32] from h4a8_quant_act (OCP MX v1.0: per 32 consecutive k, shared
// exponent floor(log2(max |x|)) - 8, elements x / 2^e rounded to nearest even and saturated to
// +-448).
//
// Reference: the reference engine's prefill runs its vLLM fork's radiance_mxfp4_fp8_gemm (W4A8,
// per-token fp8 activations from dynamic_per_token_scaled_fp8_quant): profiling/prof_engine.txt:3-4,
// profiling/prof_prefill.txt:8, docs/06-w4gemm-hip-roadmap.md:140.  That library is closed and
// absent, so the activation format here is gfx950's native one (MXFP8, whose block scales the
// MFMA applies itself) and parity is against this file's own definition (oracle/w4a8.py).
//
// gfx950 design:
//   * v_mfma_scale_f32_16x16x128_f8f6f4 with A = 16 weight rows (fp4, cbsz 4) and B = 16 token
//     rows (fp8, blgp 0): D[n][m] += sum over 128 k, the e8m0 scales applied by the MFMA.  Lane
//     (r, j) = (lane % 16, lane / 16) supplies A row r, k 32j .. 32j+31 (16 bytes) and B row r,
//     k 16j .. 16j+15 and 64+16j .. 64+16j+15 (two 16-byte pieces); the scale of (row r, k block j)
//     comes from lane (r, j), four tiles' scales packed in one VGPR and picked with op_sel.
//   * A workgroup of 4 waves computes a 128 (n) x 128 (m) tile, each wave 64 x 64 (4 x 4 MFMA
//     tiles, 16 MFMAs per 128-k step).  Fragments are loaded straight from global memory into
//     registers (the weight tile and the activation tile stay in L2 across the workgroups that
//     share them), two k steps in flight: every load is issued unconditionally (row and k indices
//     clamped into the operands) so the compiler's waits are exact.
//   * Tiles are numbered so that each XCD (workgroups w, w + 8, ...) takes a contiguous range of
//     weight-row blocks with all token blocks of each, keeping a weight tile in one L2.
#include "fp8kv_common.h"
#include "fp8kv_status.h"
#include "fp8kv_diag.h"
#include <utility>

namespace fp8kv {
namespace w4a8_detail {

constexpr int kBN = 128, kBM = 128, kBK = 128;
constexpr int kXcds = 8;

// 0: the LDS kernel, fragments double-buffered, 4-step ring, one workgroup per CU; 1: the
// direct-to-register kernel; 2 / 3: as 0 with a 3 / 5-step ring; 4: single-buffered fragments,
// registers capped for two waves per SIMD, 3-step ring; 5: as 4 with a 2-step ring (51 KB of
// LDS, so up to three workgroups share a CU); 6 / 7: as 5 with 8 x 4 / 4 x 8 MFMA tiles per wave;
// 8: 8 waves of 8 x 4 tiles (256 x 256 per workgroup, 3-step ring, 150 KB of LDS).  Measured on
// the configs[4] linears at M = 2048: 6 ~1.22-1.69 PFLOP/s, 5 ~1.27-1.41, 8 ~0.88-1.67 (only
// gate/up fills the GPU), 7 ~1.05-1.27, 4 ~1.33, 0 ~1.01, 1 ~0.40.
// Default (-1): variant 6 (the 8 x 4 wave tile, 256 x 128 per workgroup) when its grid has more
// tiles than the GPU has CUs, else variant 5 (128 x 128, twice the workgroups).  With one
// workgroup per CU, variant 6 has one wave per SIMD and nothing hides its waits.  Measured at
// M = 2048 (MXFP8, us per launch, variant 5 against 6): 224 tiles of 256 x 128 (down, K = 18944)
// 150 against 184, 256 tiles (qkv) 36 against 45, 384 tiles 58-59 against 56-57, 512 tiles 68
// against 60, 1024 tiles 131 against 116, gate/up (2368 tiles) 323 against 285.
constexpr int kDefaultVariant = -1;
thread_local int g_gemm_variant = kDefaultVariant;
constexpr int64_t kGemmCus = 256;

inline int default_variant(int N, int K, int M)
{
    (void)K;
    const int64_t tiles6 = (int64_t)((N + 255) / 256) * ((M + 127) / 128);
    return tiles6 > kGemmCus ? 6 : 5;
}

inline int pick_variant(int N, int K, int M) { return g_gemm_variant >= 0 ? g_gemm_variant : default_variant(N, K, M); }
// 0: XCD split by the traffic model of pick_split (default); 1: XCDs split the weight blocks
// only; 2: XCDs split the token blocks as far as their count allows.
thread_local int g_gemm_order = 0;

typedef int v8i __attribute__((ext_vector_type(8)));

struct Frags {
    u32x4_t a[4];        // weight n-tile i: 16 bytes (32 e2m1 codes)
    v8i b[4];            // token m-tile i: 16 bytes at k 16j (low half) and at 64 + 16j (high half)
    uint32_t sa[4];      // scale dword of (row, k step) per n-tile: 4 blocks, this lane's is byte j
    uint32_t sb[4];
};

__device__ __forceinline__ v8i concat8(u32x4_t lo, u32x4_t hi)
{
    return (v8i){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

struct Params {
    const uint8_t* W;
    const uint8_t* St;
    const uint8_t* Xq;
    const uint8_t* Sx;
    __bf16* Out;
    const float* tok_scale;   // per-token mode: fp32 scale of each activation row (Sx unused)
    int N, K, M;
    int nblk, mblk;
    int gm, gn;          // tile order: the 8 XCDs split the token blocks gm ways and the weight blocks gn ways
};

// Tile of workgroup L, or false when L has none.  Workgroup L runs on XCD L % 8 (round-robin
// dispatch); XCD x = (xm, xn) takes token blocks xm, xm + gm, ... and the xn-th range of weight
// blocks, weight-block major, so each XCD's L2 holds its share of the activations and the
// weight tiles it streams are shared by the workgroups running it at the same time.
__device__ __forceinline__ bool tile_of(const Params& P, int L, int& nb, int& mb)
{
    const int x = L % kXcds, slot = L / kXcds;
    const int xm = x % P.gm, xn = x / P.gm;
    const int my_m = (P.mblk - xm + P.gm - 1) / P.gm;
    const int nper = (P.nblk + P.gn - 1) / P.gn;
    const int n_lo = xn * nper;
    const int n_hi = n_lo + nper < P.nblk ? n_lo + nper : P.nblk;
    if (my_m <= 0 || n_lo >= n_hi || slot >= my_m * (n_hi - n_lo)) return false;
    nb = n_lo + slot / my_m;
    mb = xm + P.gm * (slot % my_m);
    return true;
}

__device__ __forceinline__ uint32_t load_u32(const void* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Fragments of the k step starting at k0 (clamped to the last step) for the wave's rows.
__device__ __forceinline__ void load_frags(Frags& f, const Params& P, const uint8_t* const (&wrow)[4],
                                           const uint8_t* const (&srow)[4], const uint8_t* const (&xrow)[4],
                                           const uint8_t* const (&sxrow)[4], int k0, int j)
{
    const int kk = k0 < P.K ? k0 : P.K - kBK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f.a[i] = load_nt_16(wrow[i] + ((kk + 32 * j) >> 1));
        f.b[i] = concat8(load_16(xrow[i] + kk + 16 * j), load_16(xrow[i] + kk + 64 + 16 * j));
        f.sa[i] = load_u32(srow[i] + (kk >> 5));
        f.sb[i] = load_u32(sxrow[i] + (kk >> 5));
    }
}

template <int I, int J>
__device__ __forceinline__ f32x4_t mfma_tile(const Frags& f, uint32_t sa, uint32_t sb, f32x4_t acc)
{
    const v8i a = {(int)f.a[I][0], (int)f.a[I][1], (int)f.a[I][2], (int)f.a[I][3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, f.b[J], acc, 4, 0, I, (int)sa, J, (int)sb);
}

template <bool TOK = false>
__device__ __forceinline__ void compute(const Frags& f, f32x4_t (&acc)[4][4], int j)
{
    // this lane's scale byte (k block j) of each tile, packed: tile i in byte i (op_sel picks it)
    // v_perm_b32(hi, lo, sel) picks bytes of {hi, lo}; selector bytes j and j + 4 take byte j
    // of lo and of hi
    const uint32_t sel = (uint32_t)j | ((uint32_t)(j + 4) << 8);
    const uint32_t a01 = __builtin_amdgcn_perm(f.sa[1], f.sa[0], sel);
    const uint32_t a23 = __builtin_amdgcn_perm(f.sa[3], f.sa[2], sel);
    const uint32_t b01 = __builtin_amdgcn_perm(f.sb[1], f.sb[0], sel);
    const uint32_t b23 = __builtin_amdgcn_perm(f.sb[3], f.sb[2], sel);
    const uint32_t sa = (a01 & 0xFFFFu) | (a23 << 16);
    // per-token mode: unit block scales (e8m0 127) on the activations
    const uint32_t sb = TOK ? 0x7F7F7F7Fu : (b01 & 0xFFFFu) | (b23 << 16);
    acc[0][0] = mfma_tile<0, 0>(f, sa, sb, acc[0][0]);
    acc[0][1] = mfma_tile<0, 1>(f, sa, sb, acc[0][1]);
    acc[0][2] = mfma_tile<0, 2>(f, sa, sb, acc[0][2]);
    acc[0][3] = mfma_tile<0, 3>(f, sa, sb, acc[0][3]);
    acc[1][0] = mfma_tile<1, 0>(f, sa, sb, acc[1][0]);
    acc[1][1] = mfma_tile<1, 1>(f, sa, sb, acc[1][1]);
    acc[1][2] = mfma_tile<1, 2>(f, sa, sb, acc[1][2]);
    acc[1][3] = mfma_tile<1, 3>(f, sa, sb, acc[1][3]);
    acc[2][0] = mfma_tile<2, 0>(f, sa, sb, acc[2][0]);
    acc[2][1] = mfma_tile<2, 1>(f, sa, sb, acc[2][1]);
    acc[2][2] = mfma_tile<2, 2>(f, sa, sb, acc[2][2]);
    acc[2][3] = mfma_tile<2, 3>(f, sa, sb, acc[2][3]);
    acc[3][0] = mfma_tile<3, 0>(f, sa, sb, acc[3][0]);
    acc[3][1] = mfma_tile<3, 1>(f, sa, sb, acc[3][1]);
    acc[3][2] = mfma_tile<3, 2>(f, sa, sb, acc[3][2]);
    acc[3][3] = mfma_tile<3, 3>(f, sa, sb, acc[3][3]);
}

__global__ void __launch_bounds__(256)
gemm_kernel(Params P)
{
    int nb, mb;
    if (!tile_of(P, blockIdx.x, nb, mb)) return;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, j = lane >> 4;
    const int n0 = nb * kBN + (wave & 1) * 64;
    const int m0 = mb * kBM + (wave >> 1) * 64;
    const int kh = P.K >> 1, ks = P.K >> 5;

    const uint8_t* wrow[4];
    const uint8_t* srow[4];
    const uint8_t* xrow[4];
    const uint8_t* sxrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int n = n0 + 16 * i + r;
        n = n < P.N ? n : P.N - 1;
        int m = m0 + 16 * i + r;
        m = m < P.M ? m : P.M - 1;
        wrow[i] = P.W + (int64_t)n * kh;
        srow[i] = P.St + (int64_t)n * ks;
        xrow[i] = P.Xq + (int64_t)m * P.K;
        sxrow[i] = P.Sx + (int64_t)m * ks;
    }

    f32x4_t acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

    Frags f0, f1;
    load_frags(f0, P, wrow, srow, xrow, sxrow, 0, j);
    load_frags(f1, P, wrow, srow, xrow, sxrow, kBK, j);
    for (int k0 = 0; k0 < P.K; k0 += 2 * kBK) {
        compute(f0, acc, j);
        load_frags(f0, P, wrow, srow, xrow, sxrow, k0 + 2 * kBK, j);
        if (k0 + kBK < P.K) compute(f1, acc, j);
        load_frags(f1, P, wrow, srow, xrow, sxrow, k0 + 3 * kBK, j);
    }

    // D[n][m]: lane (m = r, q = j) holds rows n = 4j .. 4j + 3 of each 16 x 16 tile
#pragma unroll
    for (int im = 0; im < 4; ++im) {
        const int m = m0 + 16 * im + r;
        if (m >= P.M) continue;
        __bf16* orow = P.Out + (int64_t)m * P.N;
#pragma unroll
        for (int in = 0; in < 4; ++in) {
            const int n = n0 + 16 * in + 4 * j;
            if (n >= P.N) continue;
            const f32x4_t v = acc[in][im];
            *reinterpret_cast<u32x2_t*>(orow + n) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
    }
}

// ---- LDS-pipelined variant -------------------------------------------------------------------
// Each 128-k step of the workgroup's tile (weight codes BN x 64 B, activations BM x 128 B stored
// as two [BM][64 B] halves, and both scale sets, 4 B per row) is copied global -> LDS with direct
// DMA (global_load_lds; every wave issues the same number of copies per step, so vmcnt counts
// are exact), S steps in flight in an LDS ring.  After one barrier per step, each wave reads the
// next step's fragments into registers (ds_read_b128: every read covers one contiguous KB) while
// its MFMAs work on the current step.  With K % 512 == 0 the scale bytes of four steps come in one
// 16-byte copy per row instead (GS), into a two-slot scale ring behind the operand ring.
template <int DPW>
__device__ __forceinline__ void wait_stages_ahead(int ahead)
{
    // ahead = stages issued after the one needed, at most 3
    if (ahead >= 3) wait_vmcnt<3 * DPW>();
    else if (ahead == 2) wait_vmcnt<2 * DPW>();
    else if (ahead == 1) wait_vmcnt<DPW>();
    else wait_vmcnt<0>();
}

__device__ __forceinline__ void lds_barrier_all() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Grouped scale copies (GS, K % 512 == 0, scale rows 16-byte aligned): copy c of a wave covers
// rows 64 e .. 64 e + 63 (e = c * NW + wave) of the group's rows - the BN weight rows, then in
// MXFP8 mode the token rows - lane = row, 16 bytes each: the row's scale bytes of four steps.
// Padding copies repeat the last.  The bytes of steps 4g .. 4g + 3 are copied with step 4g's
// operands into slot g % 2 of a two-slot ring at byte BASE of the LDS (16 bytes per row).
template <int DPW_SG>
struct ScaleGroups {
    uint32_t loff[DPW_SG];
    int lds[DPW_SG];
    bool w[DPW_SG];

    template <int NW, int BN, int ROWS, int BASE>
    __device__ __forceinline__ void setup(const Params& P, int wave, int lane, int N0, int M0, int ks)
    {
#pragma unroll
        for (int c = 0; c < DPW_SG; ++c) {
            int e = c * NW + wave;
            if (e >= ROWS / 64) e = ROWS / 64 - 1;
            w[c] = e < BN / 64;
            if (w[c]) {
                int n = 64 * e + lane;
                n = N0 + n < P.N ? n : P.N - 1 - N0;
                loff[c] = (uint32_t)n * (uint32_t)ks;
            } else {
                int m = 64 * e - BN + lane;
                m = M0 + m < P.M ? m : P.M - 1 - M0;
                loff[c] = (uint32_t)m * (uint32_t)ks;
            }
            lds[c] = BASE + 1024 * e;
        }
    }

    // The group copies that go out with step `step`'s operands (none unless step % 4 == 0).
    template <int ROWS>
    __device__ __forceinline__ void issue(int step, unsigned char* smem, const uint8_t* swtile,
                                          const uint8_t* sxtile) const
    {
        if ((step & 3) != 0) return;                   // wave-uniform
        unsigned char* slot = smem + ((step >> 2) & 1) * (16 * ROWS);
#pragma unroll
        for (int c = 0; c < DPW_SG; ++c)
            dma16_to_lds((w[c] ? swtile : sxtile) + (int64_t)step * 4 + loff[c], slot + lds[c]);
    }
};

// Copies issued after step q's under GS: `ahead` steps of dpw operand copies each, plus dpw_sg
// group copies with every one of them that starts a group.
__device__ __forceinline__ int scale_group_later(int q, int ahead, int dpw, int dpw_sg)
{
    int later = ahead * dpw;
    for (int t = q + 1; t <= q + ahead; ++t) later += (t & 3) == 0 ? dpw_sg : 0;
    return later;
}

template <int WN, int WM, int S>
struct LdsGeom {
    static constexpr int NW = WN * WM;
    static constexpr int BN = 64 * WN, BM = 64 * WM;
    static constexpr int W_BYTES = BN * 64;
    static constexpr int X_BYTES = BM * 128;
    static constexpr int SW_BYTES = BN * 4, SX_BYTES = BM * 4;
    static constexpr int STAGE = W_BYTES + X_BYTES + SW_BYTES + SX_BYTES;
    static constexpr int NW_W = W_BYTES / 1024, NW_X = X_BYTES / 1024;
    static constexpr int NW_S = (SW_BYTES + SX_BYTES) / 256;
    static constexpr int NDMA = NW_W + NW_X + NW_S;
    static constexpr int DPW = NDMA / NW;
    static constexpr int LDS = S * STAGE;
    static_assert(NDMA % NW == 0, "copies must split evenly over the waves");
    static_assert(3 * DPW < 64, "vmcnt range");
    // grouped scales, as in BigGeom (a scale slot is refilled four steps after its last read, so
    // S <= 5)
    static constexpr int OPER = W_BYTES + X_BYTES;
    static constexpr int sg_rows(bool tok) { return tok ? BN : BN + BM; }
    static constexpr int dpw_sg(bool tok) { return (sg_rows(tok) / 64 + NW - 1) / NW; }
    static constexpr int lds_gs(bool tok) { return S * OPER + 2 * 16 * sg_rows(tok); }
    static_assert(S <= 5 && lds_gs(false) <= 160 * 1024, "grouped scales");
};

// DB: fragments double-buffered in registers (one workgroup per CU) or single-buffered with two
// workgroups per CU (registers capped at 256 per lane, so two waves share each SIMD and one
// wave's MFMAs cover the other's waits).
// TOK: per-token mode (activation block scales fixed at 2^0, each output row multiplied by
// P.tok_scale[m]); the activation-scale copies then read weight-scale rows of the tile (clamped
// into the operand) so that every wave still issues the same copies and the waits stay exact.
// GS: grouped scale copies (K % 512 == 0), as in gemm_big_kernel.
template <int WN, int WM, int S, bool DB, bool TOK, bool GS>
__device__ __forceinline__ void gemm_lds_body(const Params& P)
{
    using G = LdsGeom<WN, WM, S>;
    constexpr int STAGE = GS ? G::OPER : G::STAGE;
    constexpr int DPW = GS ? (G::NW_W + G::NW_X) / G::NW : G::DPW;      // copies per wave and step
    constexpr int SG_ROWS = G::sg_rows(TOK), DPW_SG = G::dpw_sg(TOK);     // GS: copies per group
    constexpr int SG_BASE = S * G::OPER;
    extern __shared__ __align__(16) unsigned char smem[];
    int nb, mb;
    if (!tile_of(P, blockIdx.x, nb, mb)) return;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, j = lane >> 4;
    const int wn = wave % WN, wm = wave / WN;
    const int N0 = nb * G::BN, M0 = mb * G::BM;
    const int kh = P.K >> 1, ks = P.K >> 5;
    const int nsteps = P.K / kBK;

    // This wave's DMA copies: copy c of wave w is copy d = c * NW + w of the stage, so the kind of
    // every copy (weight codes, activations, scales) is known at compile time (each kind's copy
    // count is a multiple of the wave count).  Sources are a uniform tile base (advanced per step)
    // plus a 32-bit lane offset, the form the copy instruction takes with a scalar base.
    static_assert(G::NW_W % G::NW == 0 && G::NW_X % G::NW == 0 && G::NW_S % G::NW == 0,
                  "copy kinds must split evenly over the waves");
    const uint8_t* const wtile = P.W + (int64_t)N0 * kh;
    const uint8_t* const xtile = P.Xq + (int64_t)M0 * P.K;
    const uint8_t* const swtile = P.St + (int64_t)N0 * ks;
    const uint8_t* const sxtile = TOK ? swtile : P.Sx + (int64_t)M0 * ks;
    uint32_t loff[DPW];
    int ldsoff[DPW];
#pragma unroll
    for (int c = 0; c < DPW; ++c) {
        const int d = c * G::NW + wave;
        if (c < G::NW_W / G::NW) {                           // weight codes: rows 16 d .. 16 d + 15
            int n = 16 * d + (lane >> 2);
            n = N0 + n < P.N ? n : P.N - 1 - N0;
            loff[c] = (uint32_t)n * (uint32_t)kh + 16u * (uint32_t)(lane & 3);
            ldsoff[c] = 1024 * d;
        } else if (c < (G::NW_W + G::NW_X) / G::NW) {        // activations: half e / (BM/16)
            const int e = d - G::NW_W;
            const int half = e / (G::BM / 16), rb = e % (G::BM / 16);
            int m = 16 * rb + (lane >> 2);
            m = M0 + m < P.M ? m : P.M - 1 - M0;
            loff[c] = (uint32_t)m * (uint32_t)P.K + 64u * half + 16u * (uint32_t)(lane & 3);
            ldsoff[c] = G::W_BYTES + 1024 * e;
        } else {                                             // scales: 64 rows per copy
            const int e = d - G::NW_W - G::NW_X;
            if (e < G::BN / 64) {
                int n = 64 * e + lane;
                n = N0 + n < P.N ? n : P.N - 1 - N0;
                loff[c] = (uint32_t)n * (uint32_t)ks;
                ldsoff[c] = G::W_BYTES + G::X_BYTES + 256 * e;
            } else {
                const int e2 = e - G::BN / 64;
                int m = 64 * e2 + lane;
                if constexpr (TOK) m = N0 + m < P.N ? m : P.N - 1 - N0;
                else m = M0 + m < P.M ? m : P.M - 1 - M0;
                loff[c] = (uint32_t)m * (uint32_t)ks;
                ldsoff[c] = G::W_BYTES + G::X_BYTES + G::SW_BYTES + 256 * e2;
            }
        }
    }
    ScaleGroups<GS ? DPW_SG : 1> sg;
    if constexpr (GS) sg.template setup<G::NW, G::BN, SG_ROWS, SG_BASE>(P, wave, lane, N0, M0, ks);
    auto issue = [&](int step) {
        unsigned char* stage = smem + (step % S) * STAGE;
        const uint8_t* wb = wtile + (int64_t)step * 64;
        const uint8_t* xb = xtile + (int64_t)step * 128;
#pragma unroll
        for (int c = 0; c < DPW; ++c) {
            if (c < G::NW_W / G::NW) {
                dma16_to_lds(wb + loff[c], stage + ldsoff[c]);
            } else if (c < (G::NW_W + G::NW_X) / G::NW) {
                dma16_to_lds(xb + loff[c], stage + ldsoff[c]);
            } else {
                const int e = c * G::NW + wave - G::NW_W - G::NW_X;     // uniform
                const uint8_t* sbase = (e < G::BN / 64 ? swtile : sxtile) + (int64_t)step * 4;
                dma4_to_lds(sbase + loff[c], stage + ldsoff[c]);
            }
        }
        if constexpr (GS) sg.template issue<SG_ROWS>(step, smem, swtile, sxtile);
    };
    // fragment reads: one lane base per kind, tiles at constant offsets from it
    const int abase = (wn * 64 + r) * 64 + 16 * j;
    const int bbase = G::W_BYTES + (wm * 64 + r) * 64 + 16 * j;
    const int sabase = GS ? SG_BASE + (wn * 64 + r) * 16 : G::W_BYTES + G::X_BYTES + (wn * 64 + r) * 4;
    const int sbbase = GS ? SG_BASE + (G::BN + wm * 64 + r) * 16
                          : G::W_BYTES + G::X_BYTES + G::SW_BYTES + (wm * 64 + r) * 4;
    constexpr int SROW = GS ? 256 : 64;              // bytes between the scale dwords of tiles i and i + 1
    auto read = [&](Frags& f, int step) {
        const unsigned char* stage = smem + (step % S) * STAGE;
        const unsigned char* sst = GS ? smem + ((step >> 2) & 1) * (16 * SG_ROWS) + 4 * (step & 3) : stage;
        const unsigned char* pa = stage + abase;
        const unsigned char* pb = stage + bbase;
        const unsigned char* psa = sst + sabase;
        const unsigned char* psb = sst + sbbase;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f.a[i] = *reinterpret_cast<const u32x4_t*>(pa + 1024 * i);
            f.b[i] = concat8(*reinterpret_cast<const u32x4_t*>(pb + 1024 * i),
                             *reinterpret_cast<const u32x4_t*>(pb + 1024 * i + G::BM * 64));
            f.sa[i] = *reinterpret_cast<const uint32_t*>(psa + SROW * i);
            if constexpr (!TOK || !GS) f.sb[i] = *reinterpret_cast<const uint32_t*>(psb + SROW * i);
            else f.sb[i] = 0u;
        }
    };

    f32x4_t acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

    // Ring protocol for step q: every wave waits until its own copies of step q have landed (at
    // most min(S - 2, steps left) later steps still in flight), the barrier makes everyone's
    // copies visible and retires step q - 1's buffer (each wave read it, lgkmcnt(0), before the
    // barrier), step q + S - 1 is copied into that buffer, and step q's fragments are read.
    auto sync_read = [&](Frags& f, int q) {
        const int left = nsteps - 1 - q;
        const int ahead = left < S - 2 ? left : S - 2;
        if constexpr (GS) {
            wait_vmcnt_dyn(scale_group_later(q, ahead, DPW, DPW_SG));
        } else {
            wait_stages_ahead<DPW>(ahead);
        }
        lds_barrier_all();
        if (q + S - 1 < nsteps) issue(q + S - 1);
        read(f, q);
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (s < nsteps) issue(s);
    if constexpr (DB) {
        Frags fa, fb;
        sync_read(fa, 0);
        // pairs of steps without an exit in between (the accumulators stay in place), then the
        // odd last step
        for (int s = 0; s + 1 < nsteps; s += 2) {
            sync_read(fb, s + 1);
            compute<TOK>(fa, acc, j);                // MFMAs on step s while step s + 1 is read
            if (s + 2 < nsteps) sync_read(fa, s + 2);
            compute<TOK>(fb, acc, j);
        }
        if (nsteps & 1) compute<TOK>(fa, acc, j);
    } else {
        Frags f;
        for (int s = 0; s < nsteps; ++s) {
            sync_read(f, s);
            compute<TOK>(f, acc, j);
        }
    }

    const int n0 = N0 + wn * 64, m0 = M0 + wm * 64;
    // per-token mode: the wave's row scales are loaded together at clamped rows and applied to
    // every accumulator before the guarded stores (a product the compiler sinks into a guarded
    // store waits there for all earlier memory operations, the stores included)
    if constexpr (TOK) {
        float ts[4];
#pragma unroll
        for (int im = 0; im < 4; ++im) ts[im] = P.tok_scale[min(m0 + 16 * im + r, P.M - 1)];
#pragma unroll
        for (int im = 0; im < 4; ++im) {
#pragma unroll
            for (int in = 0; in < 4; ++in) {
                acc[in][im] = acc[in][im] * ts[im];
                asm volatile("" : "+v"(acc[in][im]));   // keeps the product out of the store branch
            }
        }
    }
#pragma unroll
    for (int im = 0; im < 4; ++im) {
        const int m = m0 + 16 * im + r;
        if (m >= P.M) continue;
        __bf16* orow = P.Out + (int64_t)m * P.N;
#pragma unroll
        for (int in = 0; in < 4; ++in) {
            const int n = n0 + 16 * in + 4 * j;
            if (n >= P.N) continue;
            const f32x4_t v = acc[in][im];
            *reinterpret_cast<u32x2_t*>(orow + n) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
    }
}

template <int WN, int WM, int S, bool GS = false>
__global__ void __launch_bounds__(64 * WN * WM)
gemm_lds_kernel(Params P)
{
    gemm_lds_body<WN, WM, S, true, false, GS>(P);
}

template <int WN, int WM, int S, bool TOK = false, bool GS = false>
__global__ void __launch_bounds__(64 * WN * WM) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_lds2_kernel(Params P)
{
    gemm_lds_body<WN, WM, S, false, TOK, GS>(P);
}

// ---- larger wave tiles -------------------------------------------------------------------------
// Each wave computes TN x TM MFMA tiles (16 x 16 each): TN weight tiles share one activation
// fragment and TM activation tiles one weight fragment, so a 128-k step costs 16 (TN + 2 TM)
// bytes of LDS reads per lane for TN * TM MFMAs.  Scale bytes: four tiles per VGPR (op_sel).
template <int WN, int WM, int TN, int TM, int S>
struct BigGeom {
    static constexpr int NW = WN * WM;
    static constexpr int BN = 16 * TN * WN, BM = 16 * TM * WM;
    static constexpr int W_BYTES = BN * 64;
    static constexpr int X_BYTES = BM * 128;
    static constexpr int SW_BYTES = BN * 4, SX_BYTES = BM * 4;
    static constexpr int STAGE = W_BYTES + X_BYTES + SW_BYTES + SX_BYTES;
    static constexpr int NW_W = W_BYTES / 1024, NW_X = X_BYTES / 1024;
    static constexpr int NW_SW = SW_BYTES / 256, NW_SX = SX_BYTES / 256;
    // scale copies padded to a multiple of the wave count (the extra copies repeat the last one)
    static constexpr int NW_S = ((NW_SW + NW_SX + NW - 1) / NW) * NW;
    static constexpr int NDMA = NW_W + NW_X + NW_S;
    static constexpr int DPW = NDMA / NW;
    static constexpr int LDS = S * STAGE;
    static_assert(NW_W % NW == 0 && NW_X % NW == 0, "copy kinds must split evenly over the waves");
    static_assert(TN % 4 == 0 && TM % 4 == 0, "tiles come in groups of four (one scale VGPR)");
    static_assert((S - 1) * DPW < 64, "vmcnt range");
    // Grouped scales (K % 512 == 0): one 16-byte copy per lane brings a row's scale bytes of four
    // steps into a two-slot scale ring behind the operand ring (weight rows, then in MXFP8 mode the
    // token rows; 16 bytes per row).
    static constexpr int OPER = W_BYTES + X_BYTES;
    static constexpr int sg_rows(bool tok) { return tok ? BN : BN + BM; }
    static constexpr int dpw_sg(bool tok) { return (sg_rows(tok) / 64 + NW - 1) / NW; }
    static constexpr int lds_gs(bool tok) { return S * OPER + 2 * 16 * sg_rows(tok); }
    static_assert(lds_gs(false) <= 160 * 1024, "LDS");
    static_assert((S - 1) * (NW_W + NW_X) / NW + 2 * dpw_sg(false) < 64, "vmcnt range");
};

template <int TN, int TM>
struct BigFrags {
    u32x4_t a[TN];
    v8i b[TM];
    uint32_t sa[TN];
    uint32_t sb[TM];
};

template <int TN, int TM, int... Is>
__device__ __forceinline__ void big_mfmas(const BigFrags<TN, TM>& f, const uint32_t (&sa)[TN / 4],
                                          const uint32_t (&sb)[TM / 4], f32x4_t (&acc)[TN][TM],
                                          std::integer_sequence<int, Is...>)
{
    ((acc[Is / TM][Is % TM] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
          (v8i){(int)f.a[Is / TM][0], (int)f.a[Is / TM][1], (int)f.a[Is / TM][2], (int)f.a[Is / TM][3], 0, 0, 0, 0},
          f.b[Is % TM], acc[Is / TM][Is % TM], 4, 0, (Is / TM) % 4, (int)sa[(Is / TM) / 4], (Is % TM) % 4,
          (int)sb[(Is % TM) / 4])), ...);
}

template <int TN, int TM, bool TOK>
__device__ __forceinline__ void big_compute(const BigFrags<TN, TM>& f, f32x4_t (&acc)[TN][TM], int j)
{
    const uint32_t sel = (uint32_t)j | ((uint32_t)(j + 4) << 8);
    uint32_t sa[TN / 4], sb[TM / 4];
#pragma unroll
    for (int g = 0; g < TN / 4; ++g) {
        const uint32_t lo = __builtin_amdgcn_perm(f.sa[4 * g + 1], f.sa[4 * g], sel);
        const uint32_t hi = __builtin_amdgcn_perm(f.sa[4 * g + 3], f.sa[4 * g + 2], sel);
        sa[g] = (lo & 0xFFFFu) | (hi << 16);
    }
#pragma unroll
    for (int g = 0; g < TM / 4; ++g) {
        const uint32_t lo = __builtin_amdgcn_perm(f.sb[4 * g + 1], f.sb[4 * g], sel);
        const uint32_t hi = __builtin_amdgcn_perm(f.sb[4 * g + 3], f.sb[4 * g + 2], sel);
        sb[g] = TOK ? 0x7F7F7F7Fu : (lo & 0xFFFFu) | (hi << 16);
    }
    big_mfmas<TN, TM>(f, sa, sb, acc, std::make_integer_sequence<int, TN * TM>{});
}

// TOK: per-token mode, as in gemm_lds_body.  GS: grouped scales (BigGeom; K % 512 == 0): the
// scale bytes of steps 4g .. 4g + 3 are copied with step 4g's operands into slot g % 2 of the scale
// ring, a quarter of the per-step scale copies, each lane 16 bytes instead of 4.
template <int WN, int WM, int TN, int TM, int S, bool TOK = false, bool GS = false>
__global__ void __launch_bounds__(64 * WN * WM) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_big_kernel(Params P)
{
    using G = BigGeom<WN, WM, TN, TM, S>;
    constexpr int STAGE = GS ? G::OPER : G::STAGE;
    constexpr int DPW = GS ? (G::NW_W + G::NW_X) / G::NW : G::DPW;      // copies per wave and step
    constexpr int SG_ROWS = G::sg_rows(TOK), DPW_SG = G::dpw_sg(TOK);     // GS: copies per group
    constexpr int SG_BASE = S * G::OPER;
    extern __shared__ __align__(16) unsigned char smem[];
    int nb, mb;
    if (!tile_of(P, blockIdx.x, nb, mb)) return;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, j = lane >> 4;
    const int wn = wave % WN, wm = wave / WN;
    const int N0 = nb * G::BN, M0 = mb * G::BM;
    const int kh = P.K >> 1, ks = P.K >> 5;
    const int nsteps = P.K / kBK;

    const uint8_t* const wtile = P.W + (int64_t)N0 * kh;
    const uint8_t* const xtile = P.Xq + (int64_t)M0 * P.K;
    const uint8_t* const swtile = P.St + (int64_t)N0 * ks;
    const uint8_t* const sxtile = TOK ? swtile : P.Sx + (int64_t)M0 * ks;
    uint32_t loff[DPW];
    int ldsoff[DPW];
    bool from_w[DPW];
#pragma unroll
    for (int c = 0; c < DPW; ++c) {
        const int d = c * G::NW + wave;
        from_w[c] = false;
        if (c < G::NW_W / G::NW) {
            int n = 16 * d + (lane >> 2);
            n = N0 + n < P.N ? n : P.N - 1 - N0;
            loff[c] = (uint32_t)n * (uint32_t)kh + 16u * (uint32_t)(lane & 3);
            ldsoff[c] = 1024 * d;
        } else if (c < (G::NW_W + G::NW_X) / G::NW) {
            const int e = d - G::NW_W;
            const int half = e / (G::BM / 16), rb = e % (G::BM / 16);
            int m = 16 * rb + (lane >> 2);
            m = M0 + m < P.M ? m : P.M - 1 - M0;
            loff[c] = (uint32_t)m * (uint32_t)P.K + 64u * half + 16u * (uint32_t)(lane & 3);
            ldsoff[c] = G::W_BYTES + 1024 * e;
        } else {
            int e = d - G::NW_W - G::NW_X;
            if (e >= G::NW_SW + G::NW_SX) e = G::NW_SW + G::NW_SX - 1;      // padding copy: repeat
            if (e < G::NW_SW) {
                int n = 64 * e + lane;
                n = N0 + n < P.N ? n : P.N - 1 - N0;
                loff[c] = (uint32_t)n * (uint32_t)ks;
                ldsoff[c] = G::W_BYTES + G::X_BYTES + 256 * e;
                from_w[c] = true;
            } else {
                const int e2 = e - G::NW_SW;
                int m = 64 * e2 + lane;
                if constexpr (TOK) m = N0 + m < P.N ? m : P.N - 1 - N0;
                else m = M0 + m < P.M ? m : P.M - 1 - M0;
                loff[c] = (uint32_t)m * (uint32_t)ks;
                ldsoff[c] = G::W_BYTES + G::X_BYTES + G::SW_BYTES + 256 * e2;
            }
        }
    }
    ScaleGroups<GS ? DPW_SG : 1> sg;
    if constexpr (GS) sg.template setup<G::NW, G::BN, SG_ROWS, SG_BASE>(P, wave, lane, N0, M0, ks);
    auto issue = [&](int step) {
        unsigned char* stage = smem + (step % S) * STAGE;
        const uint8_t* wb = wtile + (int64_t)step * 64;
        const uint8_t* xb = xtile + (int64_t)step * 128;
#pragma unroll
        for (int c = 0; c < DPW; ++c) {
            if (c < G::NW_W / G::NW) {
                dma16_to_lds(wb + loff[c], stage + ldsoff[c]);
            } else if (c < (G::NW_W + G::NW_X) / G::NW) {
                dma16_to_lds(xb + loff[c], stage + ldsoff[c]);
            } else {
                const uint8_t* sbase = (from_w[c] ? swtile : sxtile) + (int64_t)step * 4;
                dma4_to_lds(sbase + loff[c], stage + ldsoff[c]);
            }
        }
        if constexpr (GS) sg.template issue<SG_ROWS>(step, smem, swtile, sxtile);
    };
    const int abase = (wn * 16 * TN + r) * 64 + 16 * j;
    const int bbase = G::W_BYTES + (wm * 16 * TM + r) * 64 + 16 * j;
    const int sabase = GS ? SG_BASE + (wn * 16 * TN + r) * 16 : G::W_BYTES + G::X_BYTES + (wn * 16 * TN + r) * 4;
    const int sbbase = GS ? SG_BASE + (G::BN + wm * 16 * TM + r) * 16
                          : G::W_BYTES + G::X_BYTES + G::SW_BYTES + (wm * 16 * TM + r) * 4;
    constexpr int SROW = GS ? 256 : 64;              // bytes between the scale dwords of tiles i and i + 1
    auto read = [&](BigFrags<TN, TM>& f, int step) {
        const unsigned char* stage = smem + (step % S) * STAGE;
        const unsigned char* sst = GS ? smem + ((step >> 2) & 1) * (16 * SG_ROWS) + 4 * (step & 3) : stage;
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            f.a[i] = *reinterpret_cast<const u32x4_t*>(stage + abase + 1024 * i);
            f.sa[i] = *reinterpret_cast<const uint32_t*>(sst + sabase + SROW * i);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            f.b[i] = concat8(*reinterpret_cast<const u32x4_t*>(stage + bbase + 1024 * i),
                             *reinterpret_cast<const u32x4_t*>(stage + bbase + 1024 * i + G::BM * 64));
            if constexpr (!TOK) f.sb[i] = *reinterpret_cast<const uint32_t*>(sst + sbbase + SROW * i);
            else f.sb[i] = 0u;
        }
    };

    f32x4_t acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

    // ring protocol as in gemm_lds_body (wait for step q, barrier, refill the retired buffer, read);
    // under GS the steps issued after q carry DPW_SG more copies each when they start a group
    auto sync_read = [&](BigFrags<TN, TM>& f, int q) {
        const int left = nsteps - 1 - q;
        const int ahead = left < S - 2 ? left : S - 2;
        if constexpr (GS) {
            wait_vmcnt_dyn(scale_group_later(q, ahead, DPW, DPW_SG));
        } else {
            if (ahead >= 2) wait_vmcnt<2 * DPW>();
            else if (ahead == 1) wait_vmcnt<DPW>();
            else wait_vmcnt<0>();
        }
        lds_barrier_all();
        if (q + S - 1 < nsteps) issue(q + S - 1);
        read(f, q);
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (s < nsteps) issue(s);
    BigFrags<TN, TM> f;
    for (int s = 0; s < nsteps; ++s) {
        sync_read(f, s);
        big_compute<TN, TM, TOK>(f, acc, j);
    }

    const int n0 = N0 + wn * 16 * TN, m0 = M0 + wm * 16 * TM;
    if constexpr (TOK) {                           // row scales applied before the guarded stores
        float ts[TM];
#pragma unroll
        for (int im = 0; im < TM; ++im) ts[im] = P.tok_scale[min(m0 + 16 * im + r, P.M - 1)];
#pragma unroll
        for (int im = 0; im < TM; ++im) {
#pragma unroll
            for (int in = 0; in < TN; ++in) {
                acc[in][im] = acc[in][im] * ts[im];
                asm volatile("" : "+v"(acc[in][im]));
            }
        }
    }
#pragma unroll
    for (int im = 0; im < TM; ++im) {
        const int m = m0 + 16 * im + r;
        if (m >= P.M) continue;
        __bf16* orow = P.Out + (int64_t)m * P.N;
#pragma unroll
        for (int in = 0; in < TN; ++in) {
            const int n = n0 + 16 * in + 4 * j;
            if (n >= P.N) continue;
            const f32x4_t v = acc[in][im];
            *reinterpret_cast<u32x2_t*>(orow + n) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
    }
}

// ---- activation quantiser: bf16 [M, K] -> e4m3fn [M, K] + e8m0 [M, K/32] ---------------------
// One thread per 32-element block: four 16-byte loads, the block maximum, two 16-byte stores.
__global__ void __launch_bounds__(256)
quant_kernel(const uint16_t* __restrict__ X, int64_t x_stride, uint8_t* __restrict__ Xq,
             uint8_t* __restrict__ Sx, int M, int K)
{
    const int nb = K >> 5;
    const int64_t items = (int64_t)M * nb;
    for (int64_t it = blockIdx.x * 256 + threadIdx.x; it < items; it += (int64_t)gridDim.x * 256) {
        const int m = (int)(it / nb), b = (int)(it - (int64_t)m * nb);
        const uint16_t* src = X + (int64_t)m * x_stride + 32 * b;
        u32x4_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = load_16(src + 8 * i);
        float amax = 0.f;
        bool bad = false;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float lo = __uint_as_float(v[i][k] << 16), hi = __uint_as_float(v[i][k] & 0xFFFF0000u);
                bad |= !(__builtin_fabsf(lo) <= 3.4e38f) || !(__builtin_fabsf(hi) <= 3.4e38f);
                amax = __builtin_fmaxf(amax, __builtin_fmaxf(__builtin_fabsf(lo), __builtin_fabsf(hi)));
            }
        // shared exponent floor(log2(amax)) - 8 (e4m3's largest exponent), as an e8m0 byte
        // clamped to [0, 254]; 255 (NaN) when the block holds a NaN or an infinity
        int e = 0;
        if (amax > 0.f) {
            const uint32_t bits = __float_as_uint(amax);
            const int be = (int)(bits >> 23);
            e = be > 0 ? be - 127 : -118 - (int)__builtin_clz(bits & 0x7FFFFFu);   // subnormal amax
        }
        int sbyte = e - 8 + 127;
        sbyte = sbyte < 0 ? 0 : (sbyte > 254 ? 254 : sbyte);
        if (amax == 0.f) sbyte = 0;
        if (bad) sbyte = 255;
        // 2^-(sbyte - 127); finite inputs give sbyte <= 246, so this is a normal float
        const float inv = bad ? 1.f : __uint_as_float((uint32_t)(254 - sbyte) << 23);
        u32x4_t q[2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t d0 = v[i][2 * h], d1 = v[i][2 * h + 1];
                float a0 = __uint_as_float(d0 << 16) * inv, a1 = __uint_as_float(d0 & 0xFFFF0000u) * inv;
                float a2 = __uint_as_float(d1 << 16) * inv, a3 = __uint_as_float(d1 & 0xFFFF0000u) * inv;
                a0 = __builtin_fminf(__builtin_fmaxf(a0, -448.f), 448.f);
                a1 = __builtin_fminf(__builtin_fmaxf(a1, -448.f), 448.f);
                a2 = __builtin_fminf(__builtin_fmaxf(a2, -448.f), 448.f);
                a3 = __builtin_fminf(__builtin_fmaxf(a3, -448.f), 448.f);
                const uint32_t p0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a0, a1, 0, false) & 0xFFFFu;
                const uint32_t p1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a2, a3, 0, false) & 0xFFFFu;
                const int o = 2 * i + h;                      // output dword: elements 4 o .. 4 o + 3
                q[o >> 2][o & 3] = p0 | (p1 << 16);
            }
        uint8_t* dst = Xq + (int64_t)m * K + 32 * b;
        *reinterpret_cast<u32x4_t*>(dst) = q[0];
        *reinterpret_cast<u32x4_t*>(dst + 16) = q[1];
        Sx[(int64_t)m * nb + b] = (uint8_t)sbyte;
    }
}

// ---- per-token activation quantiser: bf16 [M, K] -> e4m3fn [M, K] + fp32 scale [M] ------------
// vLLM's dynamic_per_token_scaled_fp8_quant (csrc/quantization/fp8/common.cu, the kernel the
// reference engine runs before its W4A8 GEMM: profiling/prof_engine.txt:8): per row,
// scale = max(max|x| / 448, 1 / (448 * 512)) and q = e4m3fn(clamp(x / scale, -448, 448)), the
// division correctly rounded, max and clamp NaN-ignoring (fmaxf / fminf).  One workgroup of 256
// threads per row.  Rows of up to 2048 R elements stay in registers (R 16-byte pieces per thread:
// one HBM read per element); longer rows take a second pass over the same bytes.
constexpr float kTokFp8Max = 448.f;
constexpr int kTokThreads = 256;
constexpr int kTokMaxR = 16;

__device__ __forceinline__ float amax8(const u32x4_t& v, float amax)
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        amax = fmaxf(amax, fabsf(__uint_as_float(v[i] << 16)));
        amax = fmaxf(amax, fabsf(__uint_as_float(v[i] & 0xFFFF0000u)));
    }
    return amax;
}

// e4m3fn bytes of the 8 bf16 values in v divided by scale
__device__ __forceinline__ u32x2_t token_codes8(const u32x4_t& v, float scale)
{
    uint32_t out[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float a[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a[2 * i] = __uint_as_float(v[2 * h + i] << 16);
            a[2 * i + 1] = __uint_as_float(v[2 * h + i] & 0xFFFF0000u);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = fmaxf(-kTokFp8Max, fminf(__fdiv_rn(a[i], scale), kTokFp8Max));
        const uint32_t p0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a[0], a[1], 0, false) & 0xFFFFu;
        const uint32_t p1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a[2], a[3], 0, false) & 0xFFFFu;
        out[h] = p0 | (p1 << 16);
    }
    return (u32x2_t){out[0], out[1]};
}

// Row maximum over the workgroup, then the row's scale (thread 0 stores it).
__device__ __forceinline__ float token_scale(float amax, float* red, float* scales, int m)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float min_scale = 1.f / (kTokFp8Max * 512.f);
    const float scale = fmaxf(__fdiv_rn(amax, kTokFp8Max), min_scale);
    if (threadIdx.x == 0) scales[m] = scale;
    return scale;
}

// R > 0: the row in registers (K <= 2048 R); R == 0: two passes over the row.
template <int R>
__global__ void __launch_bounds__(kTokThreads)
quant_token_kernel(const uint16_t* __restrict__ X, int64_t x_stride, uint8_t* __restrict__ Xq,
                   float* __restrict__ scales, int K)
{
    __shared__ float red[kTokThreads / 64];
    const int m = blockIdx.x;
    const uint16_t* row = X + (int64_t)m * x_stride;
    uint8_t* qrow = Xq + (int64_t)m * K;
    float amax = 0.f;
    if constexpr (R > 0) {
        u32x4_t v[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int k = 8 * (threadIdx.x + i * kTokThreads);
            v[i] = k < K ? load_16(row + k) : (u32x4_t){0u, 0u, 0u, 0u};     // |0| leaves the max
            amax = amax8(v[i], amax);
        }
        const float scale = token_scale(amax, red, scales, m);
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int k = 8 * (threadIdx.x + i * kTokThreads);
            if (k < K) *reinterpret_cast<u32x2_t*>(qrow + k) = token_codes8(v[i], scale);
        }
    } else {
        for (int k = 8 * threadIdx.x; k < K; k += 8 * kTokThreads) amax = amax8(load_16(row + k), amax);
        const float scale = token_scale(amax, red, scales, m);
        for (int k = 8 * threadIdx.x; k < K; k += 8 * kTokThreads)
            *reinterpret_cast<u32x2_t*>(qrow + k) = token_codes8(load_16(row + k), scale);
    }
}

// Variants the per-token entry point runs (the tuning hook's forced variant applies when it is
// one of them).
inline bool has_token_variant(int v) { return v == 5 || v == 6; }

constexpr int64_t kL2Bytes = (int64_t)4 << 20;        // per XCD
constexpr int kLdsPerCu = 160 * 1024;
constexpr int kCusPerXcd = 32;

// Split of the 8 XCDs between token blocks (gm ways) and weight blocks (gn = 8 / gm ways).  The
// XCDs of one token group read its activations, those of one weight group its weights, so a
// launch fetches about gn * X + gm * W bytes into the L2s (X, W: activation and weight bytes
// with scales).  Pick the gm in {1, 2, 4, 8} dividing the token-block count with the least of
// that, among the splits under which an XCD's activation share is reused from its L2: either all
// the XCD's tiles run in one round of resident workgroups (the tiles of a round stream K together)
// or the share fits half an L2 (it then survives the weight tiles streamed between rounds).
// Measured at the configs[4] linears, M = 2048, against the token-block split as far as the
// count allows (bytes fetched into the L2s, FETCH_SIZE): qkv 70 -> 46 MB, o 53 -> 36 MB, gate/up
// 667 -> 419 MB, down 332 -> 226 MB; kernel time 1-4 % lower (qkv 42.3 -> 40.5 us, down 193.9 ->
// 188.4 us).
int pick_split(const Params& P, int BM, int lds_bytes, bool act_scales)
{
    if (g_gemm_order == 1) return 1;
    int gm_max = 1;
    while (gm_max < kXcds && P.mblk % (2 * gm_max) == 0) gm_max *= 2;
    if (g_gemm_order == 2) return gm_max;
    const int64_t xb = (int64_t)P.M * P.K + (act_scales ? (int64_t)P.M * (P.K / 32) : 0);
    const int64_t wb = (int64_t)P.N * (P.K / 2) + (int64_t)P.N * (P.K / 32);
    const int64_t resident = (int64_t)kCusPerXcd * (lds_bytes > 0 ? kLdsPerCu / lds_bytes : 1);
    int best = gm_max;
    int64_t best_cost = -1;
    for (int gm = 1; gm <= gm_max; gm *= 2) {
        const int gn = kXcds / gm;
        const int64_t tiles = (int64_t)(P.mblk / gm) * ((P.nblk + gn - 1) / gn);
        const int64_t share = (int64_t)(P.mblk / gm) * BM * (P.K + P.K / 32);
        if (tiles > resident && 2 * share > kL2Bytes) continue;
        const int64_t cost = gn * xb + gm * wb;
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = gm;
        }
    }
    return best;
}

int launch_gemm(Params& P, int variant, bool tok, hipStream_t st)
{
    const int BN = variant == 6 ? BigGeom<2, 2, 8, 4, 2>::BN : variant == 7 ? BigGeom<2, 2, 4, 8, 2>::BN
                 : variant == 8 ? BigGeom<2, 4, 8, 4, 3>::BN : 128;
    const int BM = variant == 6 ? BigGeom<2, 2, 8, 4, 2>::BM : variant == 7 ? BigGeom<2, 2, 4, 8, 2>::BM
                 : variant == 8 ? BigGeom<2, 4, 8, 4, 3>::BM : 128;
    P.nblk = (P.N + BN - 1) / BN;
    P.mblk = (P.M + BM - 1) / BM;
    if ((int64_t)P.nblk * P.mblk > 0x7FFFFFFF - kXcds) return FP8KV_ERR_SHAPE;
    // each row's scales of four steps in one 16-byte copy when K % 512 == 0 (rows 16-byte aligned)
    // and the scale operands start 16-byte aligned; the entry points only require 4
    const bool gs = P.K % 512 == 0 && aligned(P.St, 16) && (tok || aligned(P.Sx, 16));
    const int lds = variant == 6 ? (gs ? BigGeom<2, 2, 8, 4, 2>::lds_gs(tok) : BigGeom<2, 2, 8, 4, 2>::LDS)
                  : variant == 7 ? (gs ? BigGeom<2, 2, 4, 8, 2>::lds_gs(tok) : BigGeom<2, 2, 4, 8, 2>::LDS)
                  : variant == 8 ? (gs ? BigGeom<2, 4, 8, 4, 3>::lds_gs(tok) : BigGeom<2, 4, 8, 4, 3>::LDS)
                  : variant == 1 ? 0
                  : variant == 0 ? (gs ? LdsGeom<2, 2, 4>::lds_gs(tok) : LdsGeom<2, 2, 4>::LDS)
                  : variant == 2 || variant == 4 ? (gs ? LdsGeom<2, 2, 3>::lds_gs(tok) : LdsGeom<2, 2, 3>::LDS)
                  : variant == 3 ? (gs ? LdsGeom<2, 2, 5>::lds_gs(tok) : LdsGeom<2, 2, 5>::LDS)
                  : (gs ? LdsGeom<2, 2, 2>::lds_gs(tok) : LdsGeom<2, 2, 2>::LDS);
    const int gm = pick_split(P, BM, lds, !tok);
    P.gm = gm;
    P.gn = kXcds / gm;
    const int64_t per_xcd = (int64_t)((P.mblk + gm - 1) / gm) * ((P.nblk + P.gn - 1) / P.gn);
    const int64_t grid = per_xcd * kXcds;
    begin_launch();
    if (tok) {
        if (variant == 6 && gs)
            launch_kernel(gemm_big_kernel<2, 2, 8, 4, 2, true, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
        else if (variant == 6)
            launch_kernel(gemm_big_kernel<2, 2, 8, 4, 2, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
        else if (gs)
            launch_kernel(gemm_lds2_kernel<2, 2, 2, true, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
        else
            launch_kernel(gemm_lds2_kernel<2, 2, 2, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
        return finish_launch();
    }
    switch (variant) {
        case 1:
            launch_kernel(gemm_kernel, dim3((unsigned)grid), dim3(256), 0, st, P);
            break;
        case 2:
            if (gs) launch_kernel(gemm_lds_kernel<2, 2, 3, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
            else launch_kernel(gemm_lds_kernel<2, 2, 3>, dim3((unsigned)grid), dim3(256), lds, st, P);
            break;
        case 3:
            if (gs) launch_kernel(gemm_lds_kernel<2, 2, 5, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
            else launch_kernel(gemm_lds_kernel<2, 2, 5>, dim3((unsigned)grid), dim3(256), lds, st, P);
            break;
        case 4:
            if (gs) launch_kernel(gemm_lds2_kernel<2, 2, 3, false, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
            else launch_kernel(gemm_lds2_kernel<2, 2, 3>, dim3((unsigned)grid), dim3(256), lds, st, P);
            break;
        case 6:
            if (gs)
                launch_kernel(gemm_big_kernel<2, 2, 8, 4, 2, false, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
            else
                launch_kernel(gemm_big_kernel<2, 2, 8, 4, 2>, dim3((unsigned)grid), dim3(256), lds, st, P);
            break;
        case 7:
            if (gs)
                launch_kernel(gemm_big_kernel<2, 2, 4, 8, 2, false, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
            else
                launch_kernel(gemm_big_kernel<2, 2, 4, 8, 2>, dim3((unsigned)grid), dim3(256), lds, st, P);
            break;
        case 8:
            if (gs)
                launch_kernel(gemm_big_kernel<2, 4, 8, 4, 3, false, true>, dim3((unsigned)grid), dim3(512), lds, st, P);
            else
                launch_kernel(gemm_big_kernel<2, 4, 8, 4, 3>, dim3((unsigned)grid), dim3(512), lds, st, P);
            break;
        default:                                          // 5
            if (gs) launch_kernel(gemm_lds2_kernel<2, 2, 2, false, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
            else launch_kernel(gemm_lds2_kernel<2, 2, 2>, dim3((unsigned)grid), dim3(256), lds, st, P);
            break;
        case 0:
            if (gs) launch_kernel(gemm_lds_kernel<2, 2, 4, true>, dim3((unsigned)grid), dim3(256), lds, st, P);
            else launch_kernel(gemm_lds_kernel<2, 2, 4>, dim3((unsigned)grid), dim3(256), lds, st, P);
            break;
    }
    return finish_launch();
}

Params make_params(const void* W, const void* St, const void* Xq, const void* Sx, const float* tok_scale,
                   void* Out, int N, int K, int M)
{
    Params P;
    P.W = static_cast<const uint8_t*>(W);
    P.St = static_cast<const uint8_t*>(St);
    P.Xq = static_cast<const uint8_t*>(Xq);
    P.Sx = static_cast<const uint8_t*>(Sx);
    P.tok_scale = tok_scale;
    P.Out = static_cast<__bf16*>(Out);
    P.N = N;
    P.K = K;
    P.M = M;
    return P;
}

}  // namespace w4a8_detail
}  // namespace fp8kv

using namespace fp8kv;
using namespace fp8kv::w4a8_detail;

extern "C" int h4a8_quant_act(const void* X, int64_t x_row_stride, void* Xq, void* Sx, int M, int K,
                              void* stream)
{
    if (!X || !Xq || !Sx || M < 0 || K < 32) return FP8KV_ERR_ARG;
    if (M == 0) return FP8KV_OK;
    if (K % 32 != 0) return FP8KV_ERR_SHAPE;
    if (x_row_stride < K) return FP8KV_ERR_ARG;
    if (!aligned(X, 16) || !aligned(Xq, 16) || (x_row_stride & 7)) return FP8KV_ERR_ALIGN;
    const int64_t items = (int64_t)M * (K / 32);
    int64_t blocks = (items + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    begin_launch();
    launch_kernel(quant_kernel, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                  static_cast<const uint16_t*>(X), x_row_stride, static_cast<uint8_t*>(Xq),
                  static_cast<uint8_t*>(Sx), M, K);
    return finish_launch();
}

extern "C" int h4a8_gemm(const void* W, const void* St, const void* Xq, const void* Sx, void* Out,
                         int N, int K, int M, void* stream)
{
    if (!W || !St || !Xq || !Sx || !Out || N < 1 || K < 1 || M < 0) return FP8KV_ERR_ARG;
    if (M == 0) return FP8KV_OK;
    if (K % kBK != 0 || N % 4 != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(W, 16) || !aligned(Xq, 16) || !aligned(St, 4) || !aligned(Sx, 4) || !aligned(Out, 8))
        return FP8KV_ERR_ALIGN;
    Params P = make_params(W, St, Xq, Sx, nullptr, Out, N, K, M);
    return launch_gemm(P, pick_variant(N, K, M), false, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int h4a8_quant_act_token(const void* X, int64_t x_row_stride, void* Xq, float* scales, int M,
                                    int K, void* stream)
{
    if (!X || !Xq || !scales || M < 0 || K < 8) return FP8KV_ERR_ARG;
    if (M == 0) return FP8KV_OK;
    if (K % 8 != 0) return FP8KV_ERR_SHAPE;
    if (x_row_stride < K) return FP8KV_ERR_ARG;
    if (!aligned(X, 16) || !aligned(Xq, 8) || (x_row_stride & 7) || !aligned(scales, 4)) return FP8KV_ERR_ALIGN;
    const int r = (K + 8 * kTokThreads - 1) / (8 * kTokThreads);     // 16-byte pieces per thread
    const dim3 grid((unsigned)M), block(kTokThreads);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const uint16_t* x = static_cast<const uint16_t*>(X);
    uint8_t* xq = static_cast<uint8_t*>(Xq);
    begin_launch();
    if (r <= 1) launch_kernel(quant_token_kernel<1>, grid, block, 0, st, x, x_row_stride, xq, scales, K);
    else if (r <= 2) launch_kernel(quant_token_kernel<2>, grid, block, 0, st, x, x_row_stride, xq, scales, K);
    else if (r <= 4) launch_kernel(quant_token_kernel<4>, grid, block, 0, st, x, x_row_stride, xq, scales, K);
    else if (r <= 8) launch_kernel(quant_token_kernel<8>, grid, block, 0, st, x, x_row_stride, xq, scales, K);
    else if (r <= 12) launch_kernel(quant_token_kernel<12>, grid, block, 0, st, x, x_row_stride, xq, scales, K);
    else if (r <= kTokMaxR) launch_kernel(quant_token_kernel<kTokMaxR>, grid, block, 0, st, x, x_row_stride, xq, scales, K);
    else launch_kernel(quant_token_kernel<0>, grid, block, 0, st, x, x_row_stride, xq, scales, K);
    return finish_launch();
}

extern "C" int h4a8_gemm_token(const void* W, const void* St, const void* Xq, const float* token_scales,
                               void* Out, int N, int K, int M, void* stream)
{
    if (!W || !St || !Xq || !token_scales || !Out || N < 1 || K < 1 || M < 0) return FP8KV_ERR_ARG;
    if (M == 0) return FP8KV_OK;
    if (K % kBK != 0 || N % 4 != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(W, 16) || !aligned(Xq, 16) || !aligned(St, 4) || !aligned(token_scales, 4) || !aligned(Out, 8))
        return FP8KV_ERR_ALIGN;
    Params P = make_params(W, St, Xq, nullptr, token_scales, Out, N, K, M);
    int variant = pick_variant(N, K, M);
    if (!has_token_variant(variant)) variant = default_variant(N, K, M);
    return launch_gemm(P, variant, true, reinterpret_cast<hipStream_t>(stream));
}

extern "C" void fp8kv_gemm_tune(int variant, int order)
{
    fp8kv::w4a8_detail::g_gemm_variant = (variant >= 0 && variant <= 8) ? variant : -1;
    fp8kv::w4a8_detail::g_gemm_order = (order == 1 || order == 2) ? order : 0;
}
