"""ctypes binding of libfp8kv_amd.so (declarations: include/fp8kv_amd.h).

The library path is FP8KV_AMD_LIB if set, else the in-tree build next to this package.
Loading fails loudly: there is no CPU or Python fallback for any kernel.
"""
from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH, MEASURE_LIB_PATH

_c_vp = ctypes.c_void_p
_c_i = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_f = ctypes.c_float
_c_sz = ctypes.c_size_t

# name -> (restype, argtypes).  Mirrors include/fp8kv_amd.h.
SIGNATURES: dict[str, tuple] = {
    "fp8kv_status_string": (ctypes.c_char_p, [_c_i]),
    "fp8kv_last_status": (_c_i, []),
    "fp8kv_last_hip_error": (_c_i, []),
    "fp8kv_last_hip_error_string": (ctypes.c_char_p, []),
    # reference ABI, h4mv/h4mv.cu:106-107 / h4mv/fp8kv_hipw4.py:21-23
    "h4mv_launch": (None, [_c_vp] * 4 + [_c_i] * 3 + [_c_vp]),
    "h4mv_launch_status": (_c_i, [_c_vp] * 4 + [_c_i] * 3 + [_c_vp]),
    "h4mv_f32_launch_status": (_c_i, [_c_vp] * 4 + [_c_i] * 3 + [_c_vp]),
    "h4mv_repack_scales": (_c_i, [_c_vp, _c_vp, _c_i, _c_i, _c_vp]),
    # paged fp8 decode attention (csrc/decode_attn.hip)
    "fp8kv_decode_num_splits": (_c_i, [_c_i] * 3),
    "fp8kv_decode_scratch_bytes": (_c_sz, [_c_i] * 5),
    "fp8kv_decode_scratch_reset": (_c_i, [_c_vp, _c_sz, _c_vp]),
    "fp8kv_decode_attn_noalloc": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_i64] * 6 + [_c_vp, _c_i64]
                                  + [_c_vp] * 3 + [_c_i64] + [_c_vp] * 2 + [_c_f] + [_c_i] * 6 + [_c_vp]),
    "fp8kv_decode_attn": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_i64] * 6 + [_c_vp, _c_i64]
                          + [_c_vp] * 3 + [_c_i64] + [_c_vp] * 2 + [_c_f] + [_c_i] * 6
                          + [_c_vp, _c_sz, _c_vp]),
    # paged fp8 causal prefill attention (csrc/prefill_attn.hip)
    "fp8kv_prefill_attn": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_i64] * 6 + [_c_vp, _c_i64]
                           + [_c_vp, _c_i64] + [_c_vp] * 2 + [_c_f] + [_c_i] * 6 + [_c_vp]),
    "fp8kv_prefill_attn_varlen": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_i64] * 6
                                  + [_c_vp, _c_i64] + [_c_vp] * 3 + [_c_i64] + [_c_vp] * 2 + [_c_f]
                                  + [_c_i] * 6 + [_c_vp]),
    # the same attention over bf16 K/V caches (csrc/decode_attn.hip, csrc/prefill_bf16kv.hip)
    "fp8kv_decode_attn_bf16": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_i64] * 6 + [_c_vp, _c_i64]
                               + [_c_vp] * 3 + [_c_i64] + [_c_vp] * 2 + [_c_f] + [_c_i] * 6
                               + [_c_vp, _c_sz, _c_vp]),
    "fp8kv_prefill_attn_bf16": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_i64] * 6 + [_c_vp, _c_i64]
                                + [_c_vp, _c_i64] + [_c_vp] * 2 + [_c_f] + [_c_i] * 6 + [_c_vp]),
    "fp8kv_prefill_attn_varlen_bf16": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_i64] * 6
                                       + [_c_vp, _c_i64] + [_c_vp] * 3 + [_c_i64] + [_c_vp] * 2 + [_c_f]
                                       + [_c_i] * 6 + [_c_vp]),
    # fp8 KV-cache write (csrc/cache_write.hip)
    "fp8kv_cache_write": (_c_i, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp] + [_c_i64] * 6
                          + [_c_vp] * 3 + [_c_i] * 4 + [_c_vp]),
    # layer epilogues (csrc/epilogues.hip, h4mv_silu_mul in csrc/h4mv.hip)
    "fp8kv_fused_add_rmsnorm": (_c_i, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_i, _c_i,
                                       _c_f, _c_i, _c_vp]),
    "fp8kv_silu_mul": (_c_i, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i, _c_i, _c_i, _c_vp]),
    "h4mv_interleave_gate_up": (_c_i, [_c_vp] * 4 + [_c_i] * 2 + [_c_vp]),
    "h4mv_silu_mul": (_c_i, [_c_vp] * 4 + [_c_i] * 4 + [_c_vp]),
    # MXFP4 x MXFP8 GEMM (csrc/w4a8_gemm.hip)
    "h4a8_quant_act": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp, _c_i, _c_i, _c_vp]),
    "h4a8_gemm": (_c_i, [_c_vp] * 5 + [_c_i] * 3 + [_c_vp]),
    "h4a8_quant_act_token": (_c_i, [_c_vp, _c_i64, _c_vp, _c_vp, _c_i, _c_i, _c_vp]),
    "h4a8_gemm_token": (_c_i, [_c_vp] * 5 + [_c_i] * 3 + [_c_vp]),
    # lm_head top-k and exact rerank (csrc/lm_head.hip)
    "h4mv_topk_workspace_bytes": (_c_sz, [_c_i] * 3),
    "h4mv_topk": (_c_i, [_c_vp] * 3 + [_c_i] * 4 + [_c_vp] * 3 + [_c_sz, _c_vp]),
    "fp8kv_rerank_exact": (_c_i, [_c_vp, _c_i64, _c_i, _c_vp, _c_i64, _c_vp, _c_i, _c_i, _c_i, _c_vp, _c_vp,
                                  _c_vp]),
    # host-only diagnostics (csrc/fp8kv_diag.h)
    "fp8kv_h4mv_audit": (_c_i, [_c_i] * 3),
    "fp8kv_h4mv_tune": (None, [_c_i] * 4),
    "fp8kv_h4mv_kslice_tune": (None, [_c_i] * 4),
    "fp8kv_h4mv_m1_tune": (None, [_c_i] * 3),
    "fp8kv_h4mv_mx_tune": (None, [_c_i] * 3),
    "fp8kv_h4mv_mx_chunk_tune": (None, [_c_i]),
    "fp8kv_h4mv_plan": (_c_i, [_c_i, _c_i, _c_i, _c_vp]),
    "fp8kv_decode_tune": (None, [_c_i] * 2),
    "fp8kv_prefill_tune": (None, [_c_i]),
    "fp8kv_prefill_bf16_tune": (None, [_c_i]),
    "fp8kv_prefill_plan": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_vp]),
    "fp8kv_gemm_tune": (None, [_c_i, _c_i]),
    "fp8kv_time_next_launch": (None, [_c_vp, _c_vp]),
}

# libfp8kv_measure.so: the benchmark's read-only reference launch (csrc/stream_read.hip).
MEASURE_SIGNATURES: dict[str, tuple] = {
    "fp8kv_stream_read": (_c_i, [_c_vp, _c_sz, _c_vp, _c_vp, _c_vp, _c_vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_measure: ctypes.CDLL | None = None


class Fp8kvError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed: status {status} ({msg})")
        self.status = status


def lib_path() -> str:
    return os.environ.get("FP8KV_AMD_LIB") or LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and type the library; raises if it is missing."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        # Load torch first when it is installed: its wheel bundles a HIP runtime with the same
        # soname as /opt/rocm's, and whichever is loaded first serves the whole process.  Loading
        # this library first would bind torch to the system runtime instead of its own.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        path = lib_path()
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: build it with fp8kv_amd.build.build() (no fallback path exists)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def load_measure() -> ctypes.CDLL:
    """Load (once) the benchmark's measurement library (fp8kv_stream_read); not part of the path."""
    global _measure
    load()
    with _lock:
        if _measure is None:
            if not os.path.exists(MEASURE_LIB_PATH):
                raise FileNotFoundError(f"{MEASURE_LIB_PATH} is missing: build it with fp8kv_amd.build.build()")
            lib = ctypes.CDLL(MEASURE_LIB_PATH)
            for name, (res, args) in MEASURE_SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _measure = lib
        return _measure


def check(fn_name: str, status: int) -> None:
    if status != 0:
        lib = load()
        msg = lib.fp8kv_status_string(status).decode()
        if status == 4:
            msg += f": HIP error {lib.fp8kv_last_hip_error()} ({lib.fp8kv_last_hip_error_string().decode()})"
        raise Fp8kvError(fn_name, status, msg)
