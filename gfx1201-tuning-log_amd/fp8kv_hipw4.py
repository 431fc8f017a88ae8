"""Route small-M MXFP4 linear layers through the gfx950 matvec (vLLM op-level hook).

Drop-in for h4mv/fp8kv_hipw4.py.  With FP8KV_HIPW4=1, importing this module starts a poller
thread (fp8kv_hipw4.py:45-58, 98) that waits for the engine's ``radiance_mxfp4`` module, stands
down when ``radiance_mxfp4.WPERM`` is set (:50-52), steals the current CUDA body of
``radiance::mxfp4_linear`` - ``_backend_fns["cuda"]`` or ``_init_fn`` (:54); calling the module
attribute instead would recurse - and re-registers the op's CUDA implementation (:62).  The new
implementation takes the fast path when the reference's gate holds (:70-76): x is a contiguous
2-D bf16 tensor with 1 <= M <= FP8KV_HIPW4_MAX_M (default 4; clamped to the kernel's 16),
K % 32 == 0, N >= 8, weight_scale has K / 32 rows and the weight pointer is 16-byte aligned.  It
then repacks weight_scale [K/32, N] -> [N, K/32] once per tensor with the library's
h4mv_repack_scales (cached by data pointer and shape, cache cleared above 512 entries, never
during graph capture: :32-43) and calls
``h4mv_launch`` of libfp8kv_amd.so through ctypes with the reference's exact binding (:21-23,
81-83), returning a fresh bf16 [M, N] tensor (bias is applied outside, :9-10).  The void
launcher records its status; the hook reads it (fp8kv_last_status) after each launch, so a
rejected call falls back instead of returning an unwritten tensor.  Anything else, or any
exception, runs the stolen body (:91-94).

With FP8KV_HIPW4_GEMM=1 as well, larger batches (M > FP8KV_HIPW4_MAX_M, the prefill-sized
linears the reference leaves to its fork's W4A8 GEMM) take the library's own GEMM path when its
gate holds (contiguous 2-D bf16 x, K % 128 == 0, N % 4 == 0, K / 32 scale rows, 16-byte aligned
weight): x is quantised to fp8 and multiplied on the block-scaled MFMA.  FP8KV_HIPW4_GEMM_ACT
picks the activation format: "token" (the default; per-token fp8 as the engine's
dynamic_per_token_scaled_fp8_quant makes it, h4a8_quant_act_token + h4a8_gemm_token) or "mx"
(MXFP8 blocks of 32, h4a8_quant_act + h4a8_gemm).  The fork's GEMM library is closed, so even the
per-token path matches it only to fp32-accumulation rounding, not bit for bit.

The library path is FP8KV_AMD_LIB if set, else the in-tree build (the reference hard-codes
/opt/fp8kv/libh4mv.so).
"""
from __future__ import annotations

import ctypes
import os
import sys
import threading
import time

_PKG = os.path.dirname(os.path.abspath(__file__))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

TAG = "[hipw4]"
STATS = {"fast": 0, "gemm": 0, "slow": 0, "logged": False, "calls": 0}
_STATE = {"installed": False, "body": None, "patched": None}


def _log(msg: str) -> None:
    sys.stderr.write(f"{TAG} {msg}\n")


def load_launcher(path: str | None = None):
    """ctypes handle of ``h4mv_launch`` bound exactly as the reference binds it."""
    import torch  # noqa: F401  - bind the library to torch's HIP runtime (see fp8kv_amd._lib.load)
    if path is None:
        from fp8kv_amd import _lib
        path = _lib.lib_path()
    lib = ctypes.CDLL(path)
    lib.h4mv_launch.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 3 + [ctypes.c_void_p]
    lib.h4mv_launch.restype = None
    return lib.h4mv_launch


def load_status(path: str | None = None):
    """ctypes handle of ``fp8kv_last_status``: the status the last ``h4mv_launch`` on this host
    thread recorded (the reference's void entry point cannot return it)."""
    import torch  # noqa: F401
    if path is None:
        from fp8kv_amd import _lib
        path = _lib.lib_path()
    lib = ctypes.CDLL(path)
    lib.fp8kv_last_status.argtypes = []
    lib.fp8kv_last_status.restype = ctypes.c_int
    return lib.fp8kv_last_status


# The matvec kernels take 1 <= M <= 16; h4mv_launch rejects anything larger and launches nothing.
KERNEL_MAX_M = 16


def clamp_max_m(value: str) -> int:
    """FP8KV_HIPW4_MAX_M as an int in [1, KERNEL_MAX_M] (logged when clamped)."""
    m = int(value)
    c = min(max(m, 1), KERNEL_MAX_M)
    if c != m:
        _log(f"FP8KV_HIPW4_MAX_M={m} clamped to {c} (the matvec takes 1 <= M <= {KERNEL_MAX_M})")
    return c


def load_gemm(path: str | None = None, act: str = "token"):
    """Callable gemm(x, weight, st, out, stream) running an activation quantiser then the GEMM
    through ctypes (status checked; quantised activations in fresh torch buffers): ``act``
    "token" (h4a8_quant_act_token + h4a8_gemm_token) or "mx" (h4a8_quant_act + h4a8_gemm)."""
    import torch
    if act not in ("token", "mx"):
        raise ValueError(f"unknown activation format {act!r}")
    if path is None:
        from fp8kv_amd import _lib
        path = _lib.lib_path()
    lib = ctypes.CDLL(path)
    vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.h4a8_quant_act.argtypes = [vp, i64, vp, vp, ci, ci, vp]
    lib.h4a8_quant_act.restype = ci
    lib.h4a8_gemm.argtypes = [vp] * 5 + [ci] * 3 + [vp]
    lib.h4a8_gemm.restype = ci
    lib.h4a8_quant_act_token.argtypes = [vp, i64, vp, vp, ci, ci, vp]
    lib.h4a8_quant_act_token.restype = ci
    lib.h4a8_gemm_token.argtypes = [vp] * 5 + [ci] * 3 + [vp]
    lib.h4a8_gemm_token.restype = ci

    def gemm_token(x, weight, st, out, stream):
        M, K = x.shape
        N = weight.shape[0]
        xq = torch.empty((M, K), dtype=torch.uint8, device=x.device)
        sc = torch.empty((M,), dtype=torch.float32, device=x.device)
        rc = lib.h4a8_quant_act_token(x.data_ptr(), K, xq.data_ptr(), sc.data_ptr(), M, K, stream)
        if rc != 0:
            raise RuntimeError(f"h4a8_quant_act_token status {rc}")
        rc = lib.h4a8_gemm_token(weight.data_ptr(), st.data_ptr(), xq.data_ptr(), sc.data_ptr(), out.data_ptr(),
                                 N, K, M, stream)
        if rc != 0:
            raise RuntimeError(f"h4a8_gemm_token status {rc}")

    if act == "token":
        return gemm_token

    def gemm(x, weight, st, out, stream):
        M, K = x.shape
        N = weight.shape[0]
        xq = torch.empty((M, K), dtype=torch.uint8, device=x.device)
        sx = torch.empty((M, K // 32), dtype=torch.uint8, device=x.device)
        rc = lib.h4a8_quant_act(x.data_ptr(), K, xq.data_ptr(), sx.data_ptr(), M, K, stream)
        if rc != 0:
            raise RuntimeError(f"h4a8_quant_act status {rc}")
        rc = lib.h4a8_gemm(weight.data_ptr(), st.data_ptr(), xq.data_ptr(), sx.data_ptr(), out.data_ptr(),
                           N, K, M, stream)
        if rc != 0:
            raise RuntimeError(f"h4a8_gemm status {rc}")

    return gemm


def _device_repack(s):
    from fp8kv_amd import ops
    return ops.repack_scales(s)


class ScaleRepack:
    """weight_scale [K/32, N] -> contiguous [N, K/32], cached by (data_ptr, shape).

    ``transpose`` does the repack: the library's h4mv_repack_scales (a device kernel, the default)
    or, in tests on fake tensors, any callable with the same result."""

    def __init__(self, is_capturing, limit: int = 512, transpose=_device_repack):
        self.cache: dict = {}
        self.is_capturing = is_capturing
        self.limit = limit
        self.transpose = transpose

    def __call__(self, s):
        key = (s.data_ptr(), tuple(s.shape))
        ent = self.cache.get(key)
        if ent is not None:
            return ent
        if self.is_capturing():
            return None                      # never allocate or launch helper work during capture
        st = self.transpose(s)
        if len(self.cache) > self.limit:
            self.cache.clear()
        self.cache[key] = st
        return st


def fast_path_ok(x, weight, weight_scale, maxm: int, torch) -> bool:
    """The reference's gate (h4mv/fp8kv_hipw4.py:70-76)."""
    if not (torch.is_tensor(x) and x.dim() == 2 and x.is_contiguous()
            and 1 <= x.shape[0] <= maxm and x.dtype == torch.bfloat16):
        return False
    N = weight.shape[0]
    K = weight.shape[1] * 2
    return (K % 32 == 0 and N >= 8 and weight_scale.shape[0] == K // 32
            and weight.data_ptr() % 16 == 0)


def gemm_path_ok(x, weight, weight_scale, maxm: int, torch) -> bool:
    """Gate of the opt-in GEMM path for batches above the matvec's M limit."""
    if not (torch.is_tensor(x) and x.dim() == 2 and x.is_contiguous() and x.shape[0] > maxm
            and x.dtype == torch.bfloat16):
        return False
    N = weight.shape[0]
    K = weight.shape[1] * 2
    return (K % 128 == 0 and N % 4 == 0 and N >= 8 and weight_scale.shape[0] == K // 32
            and weight.is_contiguous() and weight.data_ptr() % 16 == 0)


def make_patched(body, launch, repack, maxm: int, torch, stream_ptr, gemm=None, last_status=None):
    """The replacement op body: fast path through ``launch`` (h4mv_launch), the opt-in GEMM path
    through ``gemm`` for larger batches, else ``body``.  ``last_status()`` (fp8kv_last_status)
    is read after every launch: a call the library rejected wrote nothing, so ``body`` runs
    instead.  ``maxm`` is clamped to the kernel's limit."""
    maxm = min(max(int(maxm), 1), KERNEL_MAX_M)

    def _patched(x, weight, weight_scale, wref):
        try:
            if STATS["calls"] < 3:
                STATS["calls"] += 1
                _log(f"call#{STATS['calls']} x={tuple(x.shape)}/{x.dtype}/c={x.is_contiguous()} "
                     f"w={tuple(weight.shape)}/{weight.dtype} s={tuple(weight_scale.shape)}")
            if fast_path_ok(x, weight, weight_scale, maxm, torch):
                st = repack(weight_scale)
                if st is not None:
                    M, N, K = x.shape[0], weight.shape[0], weight.shape[1] * 2
                    out = torch.empty((M, N), device=x.device, dtype=torch.bfloat16)
                    launch(weight.data_ptr(), st.data_ptr(), x.data_ptr(), out.data_ptr(), N, K, M,
                           ctypes.c_void_p(stream_ptr()))
                    rc = last_status() if last_status is not None else 0
                    if rc != 0:
                        raise RuntimeError(f"h4mv_launch status {rc} (N={N} K={K} M={M})")
                    STATS["fast"] += 1
                    if not STATS["logged"]:
                        STATS["logged"] = True
                        _log(f"ENGAGED N={N} K={K} M={M} (x={tuple(x.shape)} w={tuple(weight.shape)} "
                             f"s={tuple(weight_scale.shape)})")
                    return out
            elif gemm is not None and gemm_path_ok(x, weight, weight_scale, maxm, torch):
                st = repack(weight_scale)
                if st is not None:
                    M, N = x.shape[0], weight.shape[0]
                    out = torch.empty((M, N), device=x.device, dtype=torch.bfloat16)
                    gemm(x, weight, st, out, ctypes.c_void_p(stream_ptr()))
                    STATS["gemm"] += 1
                    return out
        except Exception as e:
            _log(f"fast path failed ({e!r}), falling back")
        STATS["slow"] += 1
        return body(x, weight, weight_scale, wref)

    return _patched


def steal_body(rm):
    """The op's current CUDA body, taken before re-registering (h4mv/fp8kv_hipw4.py:53-54)."""
    f = rm.mxfp4_linear
    return f._backend_fns.get("cuda") or f._init_fn


def register(patched, torch):
    torch.library.impl("radiance::mxfp4_linear", "CUDA")(patched)


def _poll(launch, maxm, tries: int = 1500, delay: float = 0.2, gemm=None, last_status=None):
    import torch
    body = None
    for _ in range(tries):
        try:
            import radiance_mxfp4 as rm
            if getattr(rm, "WPERM", False):
                _log("WPERM=1, standing down")
                return
            body = steal_body(rm)
            break
        except Exception:
            time.sleep(delay)
    if body is None:
        _log("radiance module never appeared")
        return
    repack = ScaleRepack(torch.cuda.is_current_stream_capturing)
    patched = make_patched(body, launch, repack, maxm, torch,
                           lambda: torch.cuda.current_stream().cuda_stream, gemm=gemm,
                           last_status=last_status)
    register(patched, torch)
    _STATE.update(body=body, patched=patched)
    _log("op impl overridden")


def _install() -> bool:
    if os.environ.get("FP8KV_HIPW4", "0") != "1":
        return False
    try:
        launch = load_launcher()
        last_status = load_status()
    except Exception as e:
        _log(f"lib load fail: {e}")
        return False
    maxm = clamp_max_m(os.environ.get("FP8KV_HIPW4_MAX_M", "4"))
    gemm = None
    if os.environ.get("FP8KV_HIPW4_GEMM", "0") == "1":
        try:
            gemm = load_gemm(act=os.environ.get("FP8KV_HIPW4_GEMM_ACT", "token"))
        except Exception as e:
            _log(f"gemm path unavailable: {e}")
    threading.Thread(target=_poll, args=(launch, maxm), kwargs={"gemm": gemm, "last_status": last_status},
                     daemon=True).start()
    _STATE["installed"] = True
    _log("installed")
    return True


_install()
