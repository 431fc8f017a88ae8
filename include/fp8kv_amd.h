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

#ifdef __cplusplus
}
#endif

#endif /* FP8KV_AMD_H */
