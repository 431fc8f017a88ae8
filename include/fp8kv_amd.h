/* C ABI of libfp8kv_amd.so: the MI355X (gfx950) kernels of the quantized-inference hot path.
 *
 * Conventions for every entry point:
 *   - all pointers are caller-owned device memory (except where a parameter says "host");
 *   - nothing is allocated, nothing synchronises the host: work is enqueued on `stream`
 *     (a hipStream_t; NULL = the legacy default stream), so calls can be captured in HIP graphs;
 *   - the int-returning entry points return FP8KV_OK or one of the error codes below and
 *     launch nothing when they reject their arguments.
 */
#ifndef FP8KV_AMD_H
#define FP8KV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FP8KV_OK = 0,
    FP8KV_ERR_ARG = 1,      /* null pointer, non-positive size, bad count */
    FP8KV_ERR_SHAPE = 2,    /* geometry this library does not implement (e.g. head_size != 128) */
    FP8KV_ERR_ALIGN = 3,    /* a pointer or stride breaks the alignment the kernel loads need */
    FP8KV_ERR_LAUNCH = 4,   /* hipGetLastError() reported a failure after the launch */
    FP8KV_ERR_SCRATCH = 5   /* scratch buffer missing or smaller than the *_scratch_bytes query */
};

/* Human-readable name of a status code (static string). */
const char* fp8kv_status_string(int status);

/* Status of the last h4mv_launch() call on the calling host thread. */
int fp8kv_last_status(void);

/* HIP error code (and its text) behind the last FP8KV_ERR_LAUNCH returned on this host thread. */
int fp8kv_last_hip_error(void);
const char* fp8kv_last_hip_error_string(void);

/* ---------------------------------------------------------------------------------------------
 * MXFP4 W4A16 matvec:  Out[m, n] = bf16( sum_k X[m, k] * e2m1(W[n, k]) * e8m0(St[n, k / 32]) )
 *   W   uint8 [N, K/2]  two e2m1 codes per byte, low nibble = even k     (16-byte aligned)
 *   St  uint8 [N, K/32] e8m0 scale per 32 k (the [K/32, N] checkpoint tensor transposed)
 *   Xb  bf16  [M, K]    contiguous                                        (16-byte aligned)
 *   Out bf16  [M, N]    contiguous; fp32 accumulation, round-to-nearest-even to bf16
 *   1 <= M <= 16, K % 32 == 0.
 *
 * Replaces: extern "C" void h4mv_launch(const void* W, const void* St, const void* Xb, void* Out,
 *           int N, int K, int M, void* stream)   -- reference h4mv/h4mv.cu:106-122,
 *           bound by ctypes in h4mv/fp8kv_hipw4.py:21-23 (argtypes [c_void_p]*4 + [c_int]*3 + [c_void_p]).
 * Same symbol, same signature, same argument meaning.  Differences: M up to 16 (the reference runs
 * M > 8 silently as M = 8), bf16 rounding is nearest-even (the reference rounds half up), and a
 * rejected call launches nothing and records its status for fp8kv_last_status().
 * Non-finite activations: NaN in X gives NaN outputs of its row (as the reference).  An infinity
 * in X gives NaN in every output of its row on the block-scaled kernels, which run on shapes of at
 * least 1024 row tiles with K % 512 == 0: at M = 1 (cfg1, the configs[4] gate/up shape, the
 * lm_head vocabulary), and at 2 <= M <= 8 where the workgroups fit one round (cfg1, gate/up);
 * there the row is split into e4m3 parts, which have no infinity, and its 32-k block takes the NaN
 * scale.  Everywhere else it gives +-inf (NaN where its weight is zero), as the reference does.
 * fp8kv_h4mv_plan (fp8kv_diag.h) reports which kernel a shape uses.
 */
void h4mv_launch(const void* W, const void* St, const void* Xb, void* Out,
                 int N, int K, int M, void* stream);

/* Same operation as h4mv_launch, returning the status instead of recording it. */
int h4mv_launch_status(const void* W, const void* St, const void* Xb, void* Out,
                       int N, int K, int M, void* stream);

/* Same operation with an fp32 output Out[M, N] (no output rounding).
 * Replaces the fp32-output matvec ABI of the reference's HIP demo,
 * w4-hip-demo/w4_hip_demo.cu:157-171 (w4matvec_v{1,2}_launch(W, St, X, Y, N, K, stream), Y fp32),
 * generalised to 1 <= M <= 16 rows of bf16 X. */
int h4mv_f32_launch_status(const void* W, const void* St, const void* Xb, void* Out,
                           int N, int K, int M, void* stream);

/* Load-time repack of the block scales for h4mv_launch: scale_nk[n, g] = scale_kn[g, n] for the
 * checkpoint's weight_scale uint8 [K/32, N] (contiguous) into uint8 [N, K/32] (contiguous).
 * K % 32 == 0.  Run it once per weight, outside graph capture.
 * Replaces: the scale repack of h4mv/fp8kv_hipw4.py:32-43 (_st_for: weight_scale.t().contiguous()). */
int h4mv_repack_scales(const void* scale_kn, void* scale_nk, int N, int K, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Paged fp8-e4m3 KV decode attention (one query token per sequence, split-context, one launch).
 *
 *   out[qsl[s], h, :] = bf16( v_scale * softmax_t( q[qsl[s], h, :] . K_t * sm_scale * k_scale ) . V_t )
 *   for t in [0, seq_lens[s]), h in [0, num_q_heads); query head h reads kv head h / (HQ / HKV).
 *
 *   q            bf16 [tokens, HQ, 128], row stride q_row_stride elements, heads contiguous (16 B aligned)
 *   k_cache      fp8 e4m3fn bytes; element (block, slot, kv_head, d) at
 *                k_cache + block*sk0 + slot*sk1 + kv_head*sk2 + d   (strides in bytes, multiples of 16)
 *   v_cache      same with sv0..sv2 (multiples of 8).  Both the standalone [NB, PBLK, HKV, D] cache and the
 *                engine's interleaved [NB, HKV, PBLK, 2D] tensor viewed as K | V halves are accepted.
 *   out          bf16 [tokens, HQ, 128], row stride out_row_stride; only rows qsl[s] are written
 *   query_start_loc int32 [NS + 1] (row of sequence s = query_start_loc[s]); seq_lens int32 [NS];
 *   block_table  int32 [NS, bt_stride]; k_scale, v_scale fp32 device scalars (read on the device)
 *   head_size == 128, HQ % HKV == 0, HQ / HKV <= 16, block_size a power of two >= 16 (vLLM's block
 *   sizes), 1 <= num_splits <= 256.
 *   A sequence with seq_len 0 gets zeros.
 *
 * Scratch: fp8kv_decode_scratch_bytes() bytes (0 when num_splits == 1), 256-byte aligned: a fixed
 * 256 KiB region of per-pair merge tickets, then the split records.  It must be zero-filled once
 * after allocation (torch.zeros, or fp8kv_decode_scratch_reset); every completed call leaves the
 * tickets zero again, and the records need no initial state.  Calls sharing one scratch buffer
 * must not overlap in time.  A call that did not complete (a faulted or aborted launch) can leave
 * tickets non-zero, and later calls then skip or misplace the merge: reset the buffer before
 * reusing it.
 *
 * Replaces: vllm-fp8kv/fp8kv_v3.py:116-139, run(q, k_cache, v_cache, out, qsl, slens, bt, kscale,
 * vscale, sm_scale, TILE, warps, stages, nsplit, scratch), which launches the Triton kernels
 * _decode_attn_split (fp8kv_v3.py:3-80) and _decode_attn_reduce (fp8kv_v3.py:83-113) with the cache
 * strides k_cache.stride(0..2) / v_cache.stride(0..2) and block-table stride bt.stride(0).
 */
int fp8kv_decode_attn(const void* q, int64_t q_row_stride,
                      const void* k_cache, const void* v_cache,
                      int64_t sk0, int64_t sk1, int64_t sk2,
                      int64_t sv0, int64_t sv1, int64_t sv2,
                      void* out, int64_t out_row_stride,
                      const int32_t* query_start_loc, const int32_t* seq_lens,
                      const int32_t* block_table, int64_t bt_stride,
                      const float* k_scale, const float* v_scale, float sm_scale,
                      int num_seqs, int num_q_heads, int num_kv_heads, int head_size,
                      int block_size, int num_splits, void* scratch, size_t scratch_bytes,
                      void* stream);

/* fp8kv_decode_attn without a scratch argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).  No
 * counterpart in the reference.  The tickets and split records live in a file-scope device array
 * of 8 MiB inside the library, one copy per GPU, held until the process ends; nothing is allocated
 * or freed.  Same arguments, semantics and results as fp8kv_decode_attn (bit for bit) except that
 * a call needing more than 8 MiB of scratch (fp8kv_decode_scratch_bytes) returns
 * FP8KV_ERR_SCRATCH and launches nothing; every split count the library plans fits at any GQA.
 * The array is zero when the library is loaded and every completed call leaves its tickets at
 * zero, so no call launches anything besides the decode kernel (a captured first call records no
 * extra node).  Every call on one
 * GPU shares that GPU's array: calls that overlap in time on one GPU (different streams, or
 * graphs replayed concurrently) race and must be serialised by the caller. */
int fp8kv_decode_attn_noalloc(const void* q, int64_t q_row_stride,
                              const void* k_cache, const void* v_cache,
                              int64_t sk0, int64_t sk1, int64_t sk2,
                              int64_t sv0, int64_t sv1, int64_t sv2,
                              void* out, int64_t out_row_stride,
                              const int32_t* query_start_loc, const int32_t* seq_lens,
                              const int32_t* block_table, int64_t bt_stride,
                              const float* k_scale, const float* v_scale, float sm_scale,
                              int num_seqs, int num_q_heads, int num_kv_heads, int head_size,
                              int block_size, int num_splits, void* stream);

/* Split count the library would choose for a batch whose longest context is max_seq_len
 * (replaces the fixed NSPLIT = 8 of vllm-fp8kv/fp8kv_override.py:43).  Any value in [1, 256]
 * gives the same result up to rounding; this one fills the GPU. */
int fp8kv_decode_num_splits(int num_seqs, int num_kv_heads, int max_seq_len);

/* Scratch bytes fp8kv_decode_attn needs for this geometry and split count (0 = none; 0 is also
 * returned for a geometry the kernel rejects).  Replaces the scratch sizing of
 * vllm-fp8kv/fp8kv_v3.py:121-124 and vllm-fp8kv/fp8kv_override.py:87-96. */
size_t fp8kv_decode_scratch_bytes(int num_seqs, int num_q_heads, int num_kv_heads, int head_size,
                                  int num_splits);

/* Zero-fills `scratch_bytes` bytes of a decode scratch buffer (256-byte aligned) with a kernel on
 * `stream` (not a memset, so it may be captured in a graph): the state fp8kv_decode_attn expects.
 * For a fresh buffer, and after a call that did not complete.  No counterpart in the reference: its
 * Triton split kernel overwrites every partial before the reduce kernel reads it, so its scratch
 * starts as torch.empty (vllm-fp8kv/fp8kv_v3.py:119-122); this library's one-launch merge keeps
 * its tickets in the scratch and needs them zero between calls. */
int fp8kv_decode_scratch_reset(void* scratch, size_t scratch_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Paged fp8-e4m3 KV causal prefill attention, one sequence.
 *
 *   out[i, h, :] = bf16( v_scale * softmax_{t <= q0 + i}( q[i, h, :] . K_t * sm_scale * k_scale ) . V_t )
 *   for i in [0, qlen): query i is token q0 + i of a sequence whose context (q0 + qlen tokens,
 *   the new ones included) is mapped by block_table row 0.  Layouts, strides, scales and geometry
 *   limits as for fp8kv_decode_attn (out additionally 16-byte aligned with row stride % 8 == 0).
 *   The slot strides sk1 and sv1 must be >= 0 with (block_size - 1) * max(sk1, sv1) + 128 < 2^32
 *   (a row's offset within its cache block is 32-bit), else FP8KV_ERR_SHAPE; this holds for the
 *   varlen entry point as well.
 *
 * Replaces: vllm-fp8kv/fp8kv_prefill.py:124-144, run(q, k_cache, v_cache, out, bt, kscale, vscale,
 * sm_scale, q0, qlen, BM, BN, warps, stages), the launch of the Triton kernel _prefill_attn
 * (fp8kv_prefill.py:31-121).  Any GQA <= 16 is exact (the reference's row packing is not when GQA
 * does not divide its BM).
 */
int fp8kv_prefill_attn(const void* q, int64_t q_row_stride,
                       const void* k_cache, const void* v_cache,
                       int64_t sk0, int64_t sk1, int64_t sk2,
                       int64_t sv0, int64_t sv1, int64_t sv2,
                       void* out, int64_t out_row_stride,
                       const int32_t* block_table, int64_t bt_stride,
                       const float* k_scale, const float* v_scale, float sm_scale,
                       int num_q_heads, int num_kv_heads, int head_size, int block_size,
                       int q0, int qlen, void* stream);

/* Causal prefill of several sequences packed along the token axis (vLLM varlen metadata):
 * sequence s owns q / out rows cu_seqlens_q[s] .. cu_seqlens_q[s+1]-1 (device int32 [NS + 1]),
 * its context is seq_lens[s] tokens (device int32 [NS], new tokens included), so its first query
 * is token seq_lens[s] - qlen_s, and block_table row s maps it.  max_query_len (host) bounds the
 * grid; sequences with no new tokens are skipped.
 *
 * Replaces: the multi-sequence prefill the reference leaves to vLLM's stock path (its hook gates on
 * exactly one sequence, vllm-fp8kv/fp8kv_prefill.py:163, and falls through to
 * TritonAttentionImpl.forward otherwise, :195-196). */
int fp8kv_prefill_attn_varlen(const void* q, int64_t q_row_stride,
                              const void* k_cache, const void* v_cache,
                              int64_t sk0, int64_t sk1, int64_t sk2,
                              int64_t sv0, int64_t sv1, int64_t sv2,
                              void* out, int64_t out_row_stride,
                              const int32_t* cu_seqlens_q, const int32_t* seq_lens,
                              const int32_t* block_table, int64_t bt_stride,
                              const float* k_scale, const float* v_scale, float sm_scale,
                              int num_seqs, int num_q_heads, int num_kv_heads, int head_size,
                              int block_size, int max_query_len, void* stream);

/* ---------------------------------------------------------------------------------------------
 * The same attention over bf16 K/V caches (the reference's K_FP8 = False branch): K and V are
 * used as stored and the scales do not apply,
 *
 *   decode:  out[qsl[s], h, :] = bf16( softmax_t( q . K_t * sm_scale ) . V_t )
 *   prefill: out[i, h, :]      = bf16( softmax_{t <= q0 + i}( q[i, h, :] . K_t * sm_scale ) . V_t )
 *
 * k_scale and v_scale are accepted for a signature identical to the e4m3 entry points and ignored
 * (NULL allowed).  Cache strides are in bf16 elements (the caches' torch strides), each a multiple
 * of 8, caches 16-byte aligned; slot strides at most 2^25 elements.  Everything else (layouts,
 * geometry limits, scratch and its reset for decode, varlen metadata) as for the e4m3 entry points.
 *
 * Replace: vllm-fp8kv/fp8kv_v3.py:116-139 run() with a bf16 cache (K_FP8 = k_cache.dtype !=
 * torch.bfloat16 at :135,139; the kernels' bf16 branches at :44-45,61-66,110) and
 * vllm-fp8kv/fp8kv_prefill.py:124-144 run() with a bf16 cache (:143; kernel branches :57-60,
 * 77-82,117).  The varlen entry point extends the latter as fp8kv_prefill_attn_varlen does. */
int fp8kv_decode_attn_bf16(const void* q, int64_t q_row_stride,
                           const void* k_cache, const void* v_cache,
                           int64_t sk0, int64_t sk1, int64_t sk2,
                           int64_t sv0, int64_t sv1, int64_t sv2,
                           void* out, int64_t out_row_stride,
                           const int32_t* query_start_loc, const int32_t* seq_lens,
                           const int32_t* block_table, int64_t bt_stride,
                           const float* k_scale, const float* v_scale, float sm_scale,
                           int num_seqs, int num_q_heads, int num_kv_heads, int head_size,
                           int block_size, int num_splits, void* scratch, size_t scratch_bytes,
                           void* stream);

int fp8kv_prefill_attn_bf16(const void* q, int64_t q_row_stride,
                            const void* k_cache, const void* v_cache,
                            int64_t sk0, int64_t sk1, int64_t sk2,
                            int64_t sv0, int64_t sv1, int64_t sv2,
                            void* out, int64_t out_row_stride,
                            const int32_t* block_table, int64_t bt_stride,
                            const float* k_scale, const float* v_scale, float sm_scale,
                            int num_q_heads, int num_kv_heads, int head_size, int block_size,
                            int q0, int qlen, void* stream);

int fp8kv_prefill_attn_varlen_bf16(const void* q, int64_t q_row_stride,
                                   const void* k_cache, const void* v_cache,
                                   int64_t sk0, int64_t sk1, int64_t sk2,
                                   int64_t sv0, int64_t sv1, int64_t sv2,
                                   void* out, int64_t out_row_stride,
                                   const int32_t* cu_seqlens_q, const int32_t* seq_lens,
                                   const int32_t* block_table, int64_t bt_stride,
                                   const float* k_scale, const float* v_scale, float sm_scale,
                                   int num_seqs, int num_q_heads, int num_kv_heads, int head_size,
                                   int block_size, int max_query_len, void* stream);

/* ---------------------------------------------------------------------------------------------
 * fp8-e4m3 KV-cache write: quantise new K and V rows and scatter them into the paged cache.
 *
 *   k_cache[block, slot, h, d] = e4m3fn( float(key[i, h, d]) / k_scale )   (V likewise)
 *   for token i whose s = slot_mapping[i] >= 0: block = s / block_size, slot = s % block_size;
 *   negative slots are padding and write nothing.  The division is fp32 and correctly rounded,
 *   the conversion rounds to nearest even, finite values and +-inf saturate to +-448, NaN stays
 *   NaN (0x7F / 0xFF, sign kept).
 *
 *   key, value    bf16 [num_tokens, num_kv_heads, head_size], row strides key_row_stride /
 *                 value_row_stride (elements, multiples of 8), heads contiguous, 16-byte aligned
 *   k_cache       fp8 bytes at k_cache + block*sk0 + slot*sk1 + h*sk2 + d (strides in bytes,
 *                 multiples of 16, cache 16-byte aligned); v_cache likewise with sv0..sv2
 *                 (multiples of 8): the layouts fp8kv_decode_attn reads, standalone or engine
 *   slot_mapping  int64 [num_tokens]; k_scale, v_scale fp32 device scalars
 *   head_size % 16 == 0, block_size a power of two.
 *
 * Replaces: vLLM's reshape_and_cache_flash(key, value, key_cache, value_cache, slot_mapping,
 * "fp8", k_scale, v_scale) - the kernel reshape_and_cache_kernel_flash the reference's engine
 * runs before each attention call (profiling/prof_h4mv.txt:9, profiling/prof_prefill.txt:23) -
 * for the per-tensor fp8 cache that vllm-fp8kv/fp8kv_override.py:82-85 reads.
 */
int fp8kv_cache_write(const void* key, int64_t key_row_stride,
                      const void* value, int64_t value_row_stride,
                      void* k_cache, void* v_cache,
                      int64_t sk0, int64_t sk1, int64_t sk2,
                      int64_t sv0, int64_t sv1, int64_t sv2,
                      const int64_t* slot_mapping,
                      const float* k_scale, const float* v_scale,
                      int num_tokens, int num_kv_heads, int head_size, int block_size,
                      void* stream);

/* ---------------------------------------------------------------------------------------------
 * Layer epilogues around the MXFP4 linears (decode and prefill).
 *
 * The reference engine runs these as compiler-fused kernels of its vLLM model code (listed in
 * profiling/prof_engine.txt:13,15,17 and profiling/prof_h4mv.txt:11,13,15: "fused_add_rms_norm"
 * before the qkv and gate/up linears, "mul silu slice" between gate/up and down).  Two rounding
 * forms are offered, selected by `mode`:
 *   0 - the compiled native form those profiles show (f32 intermediates, one final rounding);
 *   1 - vLLM's custom ops (_C.fused_add_rms_norm, _C.silu_and_mul), which round the residual sum
 *       and the SiLU output to bf16 before using them.
 * ------------------------------------------------------------------------------------------- */

/* residual[t, :] <- bf16(x + residual); out[t, :] = bf16(bf16((x + residual) * rsqrt(mean((x +
 * residual)^2) + eps)) * weight), per token t (mode 1 uses the bf16-rounded sum throughout).
 * bf16 rows, 16-byte aligned, strides in elements (multiples of 8); hidden_size % 8 == 0 and
 * <= 16384; out may be x (in place, as vLLM's op writes it).
 * Replaces: vLLM's fused_add_rms_norm(input, residual, weight, epsilon), the engine's
 * triton_red_fused_fused_add_rms_norm_* kernels (profiling/prof_engine.txt:13,15). */
int fp8kv_fused_add_rmsnorm(const void* x, int64_t x_row_stride, void* residual,
                            int64_t residual_row_stride, const void* weight, void* out,
                            int64_t out_row_stride, int num_tokens, int hidden_size, float eps,
                            int mode, void* stream);

/* out[t, j] = bf16(silu(gate_up[t, j]) * gate_up[t, d + j]) for j < d (mode 1: silu rounded to
 * bf16 first).  bf16, 16-byte aligned, strides in elements (multiples of 8), d % 8 == 0.
 * Replaces: vLLM's silu_and_mul(out, input), the engine's triton_poi_fused_mul_mxfp4_linear_silu_slice
 * kernel (profiling/prof_engine.txt:17). */
int fp8kv_silu_mul(const void* gate_up, int64_t in_row_stride, void* out, int64_t out_row_stride,
                   int num_tokens, int d, int mode, void* stream);

/* Load-time row interleave of a merged gate/up MXFP4 weight for h4mv_silu_mul: row 16 T + i of
 * W_out / St_out is gate row 8 T + i (i < 8) or up row N/2 + 8 T + i - 8 (i >= 8) of W [N, K/2] /
 * St [N, K/32] (the layout h4mv_launch reads).  N % 16 == 0, K % 32 == 0; run once per weight.
 * No counterpart in the reference (its gate/up linear writes both halves and a separate kernel
 * applies SiLU-and-mul). */
int h4mv_interleave_gate_up(const void* W, const void* St, void* W_out, void* St_out, int N, int K,
                            void* stream);

/* Out[M, N/2] = silu_mul(X . dequant(W, St)^T) for a gate/up weight interleaved by
 * h4mv_interleave_gate_up: the same bits as h4mv_launch into a bf16 [M, N] buffer (un-interleaved
 * order) followed by fp8kv_silu_mul(mode), in one launch that never writes the gate and up
 * values.  M <= 8, K % 512 == 0, N % 16 == 0, Out 8-byte aligned.
 * Replaces: the gate/up mxfp4_linear (h4mv/fp8kv_hipw4.py:62-94 with h4mv_launch) followed by the
 * engine's SiLU-and-mul kernel (profiling/prof_engine.txt:17). */
int h4mv_silu_mul(const void* W, const void* St, const void* Xb, void* Out, int N, int K, int M,
                  int mode, void* stream);

/* ---------------------------------------------------------------------------------------------
 * MXFP4 x MXFP8 GEMM for M >= 16 (prefill-sized linears) on gfx950's block-scaled MFMA.
 *
 * The reference engine's prefill linears run its vLLM fork's W4A8 GEMM on per-token fp8
 * activations (radiance_mxfp4_fp8_gemm; profiling/prof_engine.txt:3-4, profiling/prof_prefill.txt:8,
 * docs/06-w4gemm-hip-roadmap.md:140; the activations come from vLLM's
 * dynamic_per_token_scaled_fp8_quant, profiling/prof_engine.txt:8).  That GEMM library is
 * closed, so two activation formats are offered: gfx950's native MXFP8 block format
 * (h4a8_quant_act + h4a8_gemm) and the engine's per-token fp8 (h4a8_quant_act_token +
 * h4a8_gemm_token), whose quantiser restates vLLM's published kernel.
 * ------------------------------------------------------------------------------------------- */

/* Xq[m, k] = e4m3fn(X[m, k] / 2^(Sx[m, k/32] - 127)) per 32-wide block of k, with the e8m0
 * byte Sx = floor(log2(max |block|)) - 8 + 127 clamped to [0, 254] (0 for an all-zero block,
 * 255 = NaN for a block holding NaN or +-inf): OCP MX v1.0 MXFP8, round to nearest even,
 * saturated to +-448.  X bf16 [M, K] (row stride in elements, multiple of 8, 16-byte aligned),
 * Xq uint8 [M, K] (16-byte aligned), Sx uint8 [M, K/32]; K % 32 == 0.
 * Replaces: vLLM's dynamic_per_token_scaled_fp8_quant ahead of the W4A8 GEMM
 * (profiling/prof_engine.txt:8). */
int h4a8_quant_act(const void* X, int64_t x_row_stride, void* Xq, void* Sx, int M, int K, void* stream);

/* Out[m, n] = bf16( sum_k dq(Xq, Sx)[m, k] * dq(W, St)[n, k] ), f32 accumulation; W / St in
 * the layout h4mv_launch reads (uint8 [N, K/2], low nibble = even k; uint8 [N, K/32]).
 * K % 128 == 0, N % 4 == 0, Out bf16 [M, N] 8-byte aligned; any M >= 1 (the matvec is faster
 * for M <= 8).
 * Replaces: radiance_mxfp4_fp8_gemm (the fork's W4A8 prefill GEMM, profiling/prof_prefill.txt:8). */
int h4a8_gemm(const void* W, const void* St, const void* Xq, const void* Sx, void* Out, int N, int K,
              int M, void* stream);

/* Per-token fp8: per row m, scales[m] = max(max_k |X[m, k]| / 448, 1 / (448 * 512)) and
 * Xq[m, k] = e4m3fn(clamp(X[m, k] / scales[m], -448, 448)), the division correctly rounded, the
 * maximum and the clamp ignoring NaN (fmaxf / fminf), round to nearest even.  X bf16 [M, K] (row
 * stride in elements, multiple of 8, 16-byte aligned), Xq uint8 [M, K] (8-byte aligned), scales
 * fp32 [M]; K % 8 == 0.
 * Replaces: vLLM's dynamic_per_token_scaled_fp8_quant (csrc/quantization/fp8/common.cu, no
 * static upper bound), the engine's activation quantiser (profiling/prof_engine.txt:8). */
int h4a8_quant_act_token(const void* X, int64_t x_row_stride, void* Xq, float* scales, int M, int K,
                         void* stream);

/* Out[m, n] = bf16( token_scales[m] * sum_k e4m3(Xq[m, k]) * dq(W, St)[n, k] ), f32 accumulation,
 * the scale applied to the accumulator before the bf16 rounding.  Same W / St layout, shape and
 * alignment rules as h4a8_gemm; token_scales fp32 [M].
 * Replaces: radiance_mxfp4_fp8_gemm on per-token fp8 activations (profiling/prof_prefill.txt:8). */
int h4a8_gemm_token(const void* W, const void* St, const void* Xq, const float* token_scales, void* Out,
                    int N, int K, int M, void* stream);

/* ---------------------------------------------------------------------------------------------
 * lm_head over the tied embedding, top-k and exact rerank (the end of a decode step).
 *
 * The reference engine runs an int2 "draft" lm_head over the tied embedding (vocab 128167), an
 * exact rerank of its candidates and torch's top-k (kernels _draft_head_int2, _rerank_exact,
 * aten::topk in profiling/prof_h4mv.txt:6,10,19; docs/06-w4gemm-hip-roadmap.md:116).  Its int2
 * format is the closed fork's; this library's draft is the embedding in MXFP4 (the layout
 * h4mv_launch reads), and the rerank reads the bf16 embedding rows.
 * Rank order everywhere: value descending, NaN above every number (as torch.topk), +0 == -0,
 * then index ascending.
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes h4mv_topk needs (fp32 logits [M, N] + per-chunk candidates); 0 for k outside
 * [1, 64] or a non-positive size. */
size_t h4mv_topk_workspace_bytes(int N, int M, int k);

/* out_val / out_idx [M, k] = the k largest of logits[m, :] = X[m] . dequant(W, St)^T (fp32
 * accumulation, the fp32 output of h4mv_f32_launch_status), in rank order.  W, St, Xb as for
 * h4mv_launch (1 <= M <= 16); 1 <= k <= min(64, N) and ceil(N / 4096) * k <= 2048 (every k up to
 * 64 at vocab sizes up to 131072); workspace 256-byte aligned, at least
 * h4mv_topk_workspace_bytes(N, M, k) bytes (no initial state).  Three kernels on `stream`.
 * Replaces: the draft lm_head (_draft_head_int2) and aten::topk of the reference engine's decode
 * step (profiling/prof_h4mv.txt:6,10). */
int h4mv_topk(const void* W, const void* St, const void* Xb, int N, int K, int M, int k,
              float* out_val, int32_t* out_idx, void* workspace, size_t workspace_bytes, void* stream);

/* out_val / out_idx [M, C] = the candidates cand_idx[m, 0..C) rescored as fp32 dot products of
 * X[m, :] with bf16 embedding rows E[idx, :] (H elements each, rows row_stride elements apart,
 * multiples of 8, 16-byte aligned) and sorted in rank order; an index outside [0, V) sorts last
 * with index -1 and value -inf, repeated indices keep their candidate order.  1 <= C <= 64,
 * H % 8 == 0.
 * Replaces: the exact rerank of the draft head's candidates (_rerank_exact,
 * profiling/prof_h4mv.txt:19). */
int fp8kv_rerank_exact(const void* E, int64_t e_row_stride, int V, const void* X, int64_t x_row_stride,
                       const int32_t* cand_idx, int C, int M, int H, float* out_val, int32_t* out_idx,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FP8KV_AMD_H */
