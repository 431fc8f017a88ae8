/* Diagnostics exported by libfp8kv_amd.so for the tests and the benchmark (not part of the drop-in ABI in
 * include/fp8kv_amd.h): host-only audits, tuning hooks and the launch-timing hook.  Every tuning hook
 * and the timing hook set state of the calling host thread only (thread_local): "later launches"
 * below means later launches from that thread, and a sweep on one thread never changes the kernels
 * another thread launches.
 *
 * The benchmark's read-only reference launch lives in a library of its own, libfp8kv_measure.so
 * (csrc/stream_read.hip), which the product library does not contain:
 *   int fp8kv_stream_read(const void* src, size_t bytes, void* sink, void* stream,
 *                         void* start_event, void* stop_event);
 * reads `bytes` (a multiple of 16, at most 16 GiB) from the 16-byte aligned `src` once, with 16-byte
 * non-temporal loads all in flight at once, writes one dword per workgroup to `sink` (4096 dwords
 * suffice) and stamps the two hipEvent_t (either may be NULL) at the dispatch's start and end. */
#ifndef FP8KV_DIAG_H
#define FP8KV_DIAG_H
#ifdef __cplusplus
extern "C" {
#endif

/* Enumerate every global and LDS address the MXFP4 matvec's LDS kernel (M = 1, K-slice or
 * streaming, whichever the planner picks) would touch for (N, K, M) and check it against the operand sizes
 * and the LDS allocation.
 * 0 = all in bounds, 1 = the shape uses the register-path kernel instead, >= 2 = violation id. */
int fp8kv_h4mv_audit(int N, int K, int M);

/* Tuning hook for sweeps: waves per launch the matvec's K split aims for, a forced LDS ring depth
 * (one row tile only), a forced row-tile count per workgroup (1, 2 or 4) and the activation path
 * (1: copies through LDS, 2: direct loads); 0 = the built-in defaults.  Affects later launches
 * and audits. */
void fp8kv_h4mv_tune(int target_waves, int depth, int row_tiles, int x_mode);

/* Tuning hook for the matvec's K-slice kernel: mode 0 = used from M = 3 on when every CU gets at
 * least two 16-row tiles (the default), 1 = whenever the shape allows it (N >= 16, K % 512 == 0,
 * K <= 4096, M <= 8), 2 = never; depth = LDS ring slots per wave (3; any other value: 2, the default);
 * order = tile order (1: each workgroup a contiguous range, 2: interleaved; 0: default);
 * workgroups = workgroup count the planner aims for (0: default).  Affects later launches and
 * audits. */
void fp8kv_h4mv_kslice_tune(int mode, int depth, int order, int workgroups);

/* Tuning hook for the matvec's M = 1 kernel (e2m1 codes on the block-scaled MFMA, activations as
 * e4m3 hi + lo): mode 0 = used at M = 1 when N / 16 >= 1024 tiles (the default), 1 = whenever the
 * shape allows it (M = 1, K % 512 == 0), 2 = never; depth = LDS ring slots per wave (3; any other
 * value: 2, the default); workgroups = workgroup count the planner aims for (0: default 256).
 * Affects later launches and audits. */
void fp8kv_h4mv_m1_tune(int mode, int depth, int workgroups);

/* Tuning hook for the matvec's M = 2 .. 8 kernel (the M = 1 kernel's e4m3 hi + lo activations, one
 * column pair per row): mode 0 = used at 2 <= M <= 8 when N / 16 >= 1024 tiles and every workgroup
 * runs in one round (the default), 1 = whenever the shape allows it (2 <= M <= 8, K % 512 == 0),
 * 2 = never; depth = LDS ring slots per wave (3; any other value: 2, the default); workgroups =
 * workgroup count the planner aims for (0: default).  Affects later launches and audits. */
void fp8kv_h4mv_mx_tune(int mode, int depth, int workgroups);

/* Tuning hook for the M = 2 .. 8 kernel's activation conversion: 2^steps_log2 K steps per chunk
 * (0..6; the first chunk is converted before the stream, each later one while the previous one
 * streams); any other value restores the default.  Affects later launches and audits. */
void fp8kv_h4mv_mx_chunk_tune(int steps_log2);

/* Planner query of the matvec launch (host only, no GPU call): the kernel h4mv_launch would run
 * for (N, K, M) under the current tuning hooks.  out[6] = {kernel (0 register path, 1 streaming,
 * 2 K-slice, 3 M = 1, 4 M = 2 .. 8 hi / lo, 5 batched K-slice), grid, waves per workgroup, ring
 * depth, dynamic LDS bytes, activation rows (kernels 3 and 4) / row tiles (1) / tiles per
 * workgroup (2, 5)}.  Returns FP8KV_OK or an argument / shape status. */
int fp8kv_h4mv_plan(int N, int K, int M, int* out);

/* Tuning hook for sweeps of the decode attention launch: kernel variant index (0..6; any other
 * value, e.g. -1, selects the default, variant 5: 8 waves, chunks of 2 groups of 16 keys, 2 chunks
 * in flight per wave, each group's K and V bytes requested together) and the workgroup count its split planner
 * aims for (0 = default 256).  Affects later launches. */
void fp8kv_decode_tune(int variant, int target_wgs);

/* Tuning hook for sweeps of the prefill attention launch: index of the (waves, row-sets per wave,
 * LDS ring depth) shape to use for every GQA (0..7), 8 + s for key-split shape s (0..4, used only
 * at its own GQA: 6, 12, 4, 8, 16) with the default block pairing, 13 + s for the same with paired
 * token blocks (r, n16 - 1 - r) at any grid size, or -1 for the per-GQA default. */
void fp8kv_prefill_tune(int shape);

/* bf16-KV prefill: query heads per wave (1 or 2); any other value restores the default (two where
 * GQA > 1, else one). */
void fp8kv_prefill_bf16_tune(int heads_per_wave);

/* Planner query of the prefill attention launch (host only, no GPU call): the plan the entry
 * points would launch for this shape under the current tuning hook.  ctx_hint is the longest
 * context (q0 + qlen) for fp8kv_prefill_attn and max_query_len for the varlen entry point.
 * out[8] = {kernel (1 key-split, 0 per-wave), shape index, token blocks per workgroup, paired
 * (blocks r and n16 - 1 - r in one workgroup), token-block ranks per kv head, grid x, grid z,
 * threads per workgroup}; all zero sizes when there is nothing to launch. */
int fp8kv_prefill_plan(int num_q_heads, int num_kv_heads, int num_seqs, int max_query_len,
                       int ctx_hint, int* out);

/* Tuning hook for the MXFP4 x MXFP8 GEMM: kernel variant (0..8; any other value selects the
 * default, which picks variant 6 or 5 from the shape; the per-token entry point runs only 5 and 6
 * and takes its default for the others) and XCD split (0 = chosen by the traffic model, the
 * default; 1 = XCDs split the weight blocks only; 2 = XCDs split the token blocks as far as their
 * count allows).  Affects later launches. */
void fp8kv_gemm_tune(int variant, int order);

/* Measurement hook: the next kernel launched by this host thread through any entry point records
 * start_event / stop_event (hipEvent_t, either may be NULL) at its own start and end, via
 * hipExtLaunchKernel.  hipEventElapsedTime between them is then the kernel's execution time.
 * The events are used once; a rejected call leaves them armed for the next launch. */
void fp8kv_time_next_launch(void* start_event, void* stop_event);

#ifdef __cplusplus
}
#endif
#endif
