// lm_head over the tied embedding, top-k selection and exact rerank for gfx950.
//
// Reference: the reference engine ends every decode step with an int2 "draft" lm_head over the
// tied embedding (vocab 128167, docs/06-w4gemm-hip-roadmap.md:116; kernel _draft_head_int2,
// profiling/prof_h4mv.txt:6), an exact rerank of its candidates (_rerank_exact,
// profiling/prof_h4mv.txt:19) and torch's top-k (aten::topk / gatherTopK, profiling/prof_h4mv.txt:10,12).
// The int2 format belongs to the reference's closed vLLM fork, so this build defines its own
// draft: the embedding quantised to MXFP4 (the matvec's format, e2m1 codes + e8m0 per 32), whose
// fp32 logits come from the MXFP4 matvec; candidates are then rescored against the bf16
// embedding rows.
//
//   * h4mv_topk: logits[m, n] = X[m] . dequant(W[n])^T in fp32 (h4mv_f32_launch_status, into the
//     workspace), then the k largest per row, in two kernels: every 4096-logit chunk of a row
//     gives its own top k (chunk_topk_kernel), and one workgroup per row picks the top k of those
//     candidates (merge_topk_kernel).  Each selection is a workgroup radix select over 64-bit
//     rank keys held in registers (block_topk), 8 bits per round with an LDS histogram.
//   * rank order: value descending, NaN above every number (as torch.topk), +0 and -0 equal, then
//     index ascending.  Keys are unique (they carry the index), so every round has one winner.
//   * fp8kv_rerank_exact: out = the C candidates of each row rescored as fp32 dot products of X[m]
//     with bf16 embedding rows E[idx] and sorted in rank order; invalid indices sort last with
//     index -1 and value -inf, and repeated indices keep their candidate order.
#include "fp8kv_common.h"
#include "fp8kv_status.h"

namespace fp8kv {
namespace lmhead_detail {

constexpr int kThreads = 256;
constexpr int kChunk = 4096;                 // logits per chunk: 16 per thread
constexpr int kPerThread = kChunk / kThreads;
constexpr int kMaxK = 64;
constexpr int kMaxMergePerThread = 8;        // merge: up to 2048 candidates per row (512 per wave)
constexpr int kMaxCandidates = kMaxMergePerThread * kThreads;
constexpr int kMaxRerank = 64;

// Monotone map of the float order onto uint32 (NaN highest, -0 == +0), then the index inverted so
// that the lower index wins a tie.  Key 0 never comes from a logit: it marks "nothing".
__device__ __forceinline__ uint64_t rank_key(float v, uint32_t idx)
{
    uint32_t b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0u;
    uint32_t o;
    if ((b & 0x7fffffffu) > 0x7f800000u) o = 0xffffffffu;
    else o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - idx);
}
__device__ __forceinline__ float key_value(uint64_t key)
{
    const uint32_t o = (uint32_t)(key >> 32);
    if (o == 0xffffffffu) return __uint_as_float(0x7fc00000u);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ int32_t key_index(uint64_t key)
{
    return (int32_t)(0xffffffffu - (uint32_t)key);
}

// Inclusive prefix sum over the lanes of a wave (lane order).
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v, int lane)
{
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = (uint32_t)__shfl_up((int)v, d);
        if (lane >= d) v += o;
    }
    return v;
}

// The k (<= kMaxK) largest of the kThreads * NPL keys the workgroup holds (unique; 0 = none),
// written in no particular order to out[0 .. k) (0 past the number of non-zero keys).  Radix
// select from the top, 8 bits per round: a 256-bucket LDS histogram of the keys that match the
// digits fixed so far, then one wave finds the bucket holding the k-th largest of them.  The
// search stops as soon as that bucket holds exactly the keys still needed (they are all taken;
// with unique keys this happens by the 8th round, usually after two or three), and every key at
// or above the threshold is written at a position from an LDS counter.
template <int NPL>
__device__ __forceinline__ void block_topk(const uint64_t (&keys)[NPL], int k, uint64_t* out)
{
    static_assert(kThreads == 256, "one histogram bucket per thread");
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit, s_above, s_in_bucket, s_total, s_cnt;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t prefix = 0, mask = 0, T = 0;
    uint32_t need = (uint32_t)k;
    bool found = false;
    if (tid == 0) s_cnt = 0;
    for (int shift = 56; shift >= 0; shift -= 8) {
        hist[tid] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NPL; ++j)
            if (keys[j] != 0 && (keys[j] & mask) == prefix)
                atomicAdd(&hist[(uint32_t)(keys[j] >> shift) & 255u], 1u);
        __syncthreads();
        if (wave == 0) {
            // lane l holds buckets 255 - 4l .. 252 - 4l, so lane order is descending key order
            uint32_t h[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) h[i] = hist[255 - 4 * lane - i];
            const uint32_t tot = (h[0] + h[1]) + (h[2] + h[3]);
            const uint32_t incl = wave_inclusive_sum(tot, lane);
            const uint32_t excl = incl - tot;
            if (lane == 63) s_total = incl;
            if (excl < need && incl >= need) {          // the lane holding the need-th key
                uint32_t cum = excl;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (cum + h[i] >= need) {
                        s_digit = 255u - 4u * (uint32_t)lane - (uint32_t)i;
                        s_above = cum;
                        s_in_bucket = h[i];
                        break;
                    }
                    cum += h[i];
                }
            }
        }
        __syncthreads();
        if (s_total < need) {                          // fewer keys than asked for: take them all
            T = 1;
            found = true;
            break;
        }
        const uint32_t d = s_digit;
        need -= s_above;
        prefix |= (uint64_t)d << shift;
        mask |= (uint64_t)0xffu << shift;
        if (s_in_bucket == need) {                     // the whole bucket is taken
            T = prefix;
            found = true;
            break;
        }
        __syncthreads();                               // everyone has read the bucket state
    }
    if (!found) T = prefix;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
        if (keys[j] != 0 && keys[j] >= T) out[atomicAdd(&s_cnt, 1u)] = keys[j];
    __syncthreads();
    for (uint32_t p = s_cnt + (uint32_t)tid; p < (uint32_t)k; p += kThreads) out[p] = 0;
}

// grid (nchunks, M): the top k of logits[m, 4096 c .. +4096) as keys in cand[m][c][0..k), in no
// particular order.  Loads are unconditional (indices clamped into the row, keys past it masked
// to 0), so all 16 of a thread are in flight together.
__global__ void __launch_bounds__(kThreads)
chunk_topk_kernel(const float* __restrict__ logits, int N, int k, uint64_t* __restrict__ cand)
{
    const int c = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    const float* row = logits + (size_t)m * (size_t)N;
    float v[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) v[j] = row[min(c * kChunk + j * kThreads + tid, N - 1)];
    uint64_t keys[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int n = c * kChunk + j * kThreads + tid;
        keys[j] = n < N ? rank_key(v[j], (uint32_t)n) : 0;
    }
    block_topk<kPerThread>(keys, k, cand + ((size_t)m * gridDim.x + c) * (size_t)k);
}

// grid (M): the top k of a row's ncand (<= 2048) candidate keys, written as values and indices
// in rank order (positions past the valid candidates: index -1, value -inf): the workgroup
// selects them, then each one's position is the number of keys above it.
__global__ void __launch_bounds__(kThreads)
merge_topk_kernel(const uint64_t* __restrict__ cand, int ncand, int k, float* __restrict__ out_val,
                  int32_t* __restrict__ out_idx)
{
    __shared__ uint64_t top[kMaxK];
    const int m = blockIdx.x, tid = threadIdx.x;
    const uint64_t* row = cand + (size_t)m * (size_t)ncand;
    uint64_t keys[kMaxMergePerThread];
#pragma unroll
    for (int j = 0; j < kMaxMergePerThread; ++j) keys[j] = row[min(j * kThreads + tid, ncand - 1)];
#pragma unroll
    for (int j = 0; j < kMaxMergePerThread; ++j)
        if (j * kThreads + tid >= ncand) keys[j] = 0;
    block_topk<kMaxMergePerThread>(keys, k, top);
    __syncthreads();
    if (tid < k) {
        const uint64_t mine = top[tid];
        int rank = 0;
        for (int j = 0; j < k; ++j) {
            const uint64_t o = top[j];
            rank += (o > mine || (o == mine && j < tid)) ? 1 : 0;
        }
        out_val[(size_t)m * k + rank] = mine ? key_value(mine) : -__builtin_inff();
        out_idx[(size_t)m * k + rank] = mine ? key_index(mine) : -1;
    }
}

// grid (M): C candidate rows of E rescored against X[m] (fp32 dot products of bf16 rows, one wave
// per candidate, lanes over 8-element pieces), then sorted in rank order.
__global__ void __launch_bounds__(kThreads)
rerank_kernel(const __bf16* __restrict__ E, int64_t e_stride, int V, const __bf16* __restrict__ X,
              int64_t x_stride, const int32_t* __restrict__ cand, int C, int H,
              float* __restrict__ out_val, int32_t* __restrict__ out_idx)
{
    __shared__ uint64_t keys[kMaxRerank];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const __bf16* x = X + (int64_t)m * x_stride;
    const int32_t* ci = cand + (size_t)m * C;
    for (int c = wave; c < C; c += kThreads / 64) {
        const int32_t idx = ci[c];
        const bool ok = idx >= 0 && idx < V;
        const __bf16* e = E + (int64_t)(ok ? idx : 0) * e_stride;
        float acc = 0.f;
        for (int p = lane; p < H / 8; p += 64) {
            const u32x4_t a = *reinterpret_cast<const u32x4_t*>(x + 8 * p);
            const u32x4_t b = *reinterpret_cast<const u32x4_t*>(e + 8 * p);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                acc = __builtin_fmaf(__uint_as_float(a[w] << 16), __uint_as_float(b[w] << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(a[w] & 0xffff0000u), __uint_as_float(b[w] & 0xffff0000u), acc);
            }
        }
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) acc += __shfl_xor(acc, s);
        if (lane == 0) keys[c] = ok ? rank_key(acc, (uint32_t)idx) : 0;
    }
    __syncthreads();
    if (tid < C) {
        // Position = keys ranked above this one, plus equal keys earlier in the list (repeated
        // indices, and the zero keys of invalid candidates, keep their candidate order).
        const uint64_t mine = keys[tid];
        int rank = 0;
        for (int j = 0; j < C; ++j) rank += (keys[j] > mine || (keys[j] == mine && j < tid)) ? 1 : 0;
        out_val[(size_t)m * C + rank] = mine ? key_value(mine) : -__builtin_inff();
        out_idx[(size_t)m * C + rank] = mine ? key_index(mine) : -1;
    }
}

inline int nchunks(int N) { return (N + kChunk - 1) / kChunk; }

inline size_t logits_bytes(int N, int M) { return ((size_t)M * (size_t)N * 4 + 255) & ~(size_t)255; }

inline size_t workspace_bytes(int N, int M, int k)
{
    return logits_bytes(N, M) + (size_t)M * (size_t)nchunks(N) * (size_t)k * 8;
}

}  // namespace lmhead_detail
}  // namespace fp8kv

using namespace fp8kv;
using namespace fp8kv::lmhead_detail;

extern "C" size_t h4mv_topk_workspace_bytes(int N, int M, int k)
{
    if (N < 1 || M < 1 || k < 1 || k > kMaxK) return 0;
    return workspace_bytes(N, M, k);
}

extern "C" int h4mv_topk(const void* W, const void* St, const void* Xb, int N, int K, int M, int k,
                         float* out_val, int32_t* out_idx, void* workspace, size_t workspace_bytes_given,
                         void* stream)
{
    if (!W || !St || !Xb || !out_val || !out_idx || !workspace) return FP8KV_ERR_ARG;
    if (N < 1 || K < 1 || M < 1 || k < 1) return FP8KV_ERR_ARG;
    if (k > kMaxK || k > N || (int64_t)nchunks(N) * k > kMaxCandidates) return FP8KV_ERR_SHAPE;
    if ((int64_t)M * N > ((int64_t)1 << 31)) return FP8KV_ERR_SHAPE;
    if (!aligned(workspace, 256)) return FP8KV_ERR_ALIGN;
    if (workspace_bytes_given < workspace_bytes(N, M, k)) return FP8KV_ERR_SCRATCH;
    float* logits = static_cast<float*>(workspace);
    uint64_t* cand = reinterpret_cast<uint64_t*>(static_cast<unsigned char*>(workspace) + logits_bytes(N, M));
    int rc = h4mv_f32_launch_status(W, St, Xb, logits, N, K, M, stream);
    if (rc != FP8KV_OK) return rc;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int nc = nchunks(N);
    begin_launch();
    launch_kernel(chunk_topk_kernel, dim3((unsigned)nc, (unsigned)M), dim3(kThreads), 0, st,
                  static_cast<const float*>(logits), N, k, cand);
    rc = finish_launch();
    if (rc != FP8KV_OK) return rc;
    begin_launch();
    launch_kernel(merge_topk_kernel, dim3((unsigned)M), dim3(kThreads), 0, st,
                  static_cast<const uint64_t*>(cand), nc * k, k, out_val, out_idx);
    return finish_launch();
}

extern "C" int fp8kv_rerank_exact(const void* E, int64_t e_row_stride, int V, const void* X,
                                  int64_t x_row_stride, const int32_t* cand_idx, int C, int M, int H,
                                  float* out_val, int32_t* out_idx, void* stream)
{
    if (!E || !X || !cand_idx || !out_val || !out_idx) return FP8KV_ERR_ARG;
    if (V < 1 || C < 1 || M < 1 || H < 1) return FP8KV_ERR_ARG;
    if (C > kMaxRerank || H % 8 != 0) return FP8KV_ERR_SHAPE;
    if (!aligned(E, 16) || !aligned(X, 16) || (e_row_stride & 7) || (x_row_stride & 7)) return FP8KV_ERR_ALIGN;
    begin_launch();
    launch_kernel(rerank_kernel, dim3((unsigned)M), dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream),
                  static_cast<const __bf16*>(E), e_row_stride, V, static_cast<const __bf16*>(X), x_row_stride,
                  cand_idx, C, H, out_val, out_idx);
    return finish_launch();
}
