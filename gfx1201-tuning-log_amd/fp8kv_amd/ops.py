"""Torch-facing wrappers over the C ABI (device memory and streams come from PyTorch-ROCm).

Every wrapper validates shapes/dtypes/devices on the host, launches on the current stream and
raises ``Fp8kvError`` if the library rejects the call.  Nothing here computes on the CPU.
"""
from __future__ import annotations

import torch

from . import _lib


def _stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def repack_scales(weight_scale: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Checkpoint scales uint8 [K/32, N] -> kernel layout [N, K/32] on the device
    (h4mv_repack_scales; the reference's weight_scale.t().contiguous(), h4mv/fp8kv_hipw4.py:32-43)."""
    _require(weight_scale.is_cuda and weight_scale.dim() == 2 and weight_scale.is_contiguous()
             and weight_scale.element_size() == 1, "weight_scale must be a contiguous 1-byte [K/32, N] device tensor")
    G, N = weight_scale.shape
    if out is None:
        out = torch.empty((N, G), dtype=weight_scale.dtype, device=weight_scale.device)
    _require(out.shape == (N, G) and out.is_contiguous() and out.element_size() == 1
             and out.device == weight_scale.device, "out must be a contiguous [N, K/32] byte tensor")
    lib = _lib.load()
    st = lib.h4mv_repack_scales(weight_scale.data_ptr(), out.data_ptr(), N, 32 * G,
                                _stream_ptr(weight_scale))
    _lib.check("h4mv_repack_scales", st)
    return out


def h4mv(x: torch.Tensor, weight: torch.Tensor, scales_nk: torch.Tensor,
         out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """[M, N] = x [M, K] . dequant(weight [N, K/2], scales_nk [N, K/32])^T in bf16 (or fp32).

    Same contract as the reference's ``lib.h4mv_launch`` call in h4mv/fp8kv_hipw4.py:78-83;
    ``out_dtype=torch.float32`` selects the unrounded fp32-output entry point.
    """
    _require(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(),
             "x must be a contiguous 2-D bf16 device tensor")
    M, K = x.shape
    _require(weight.dtype == torch.uint8 and weight.dim() == 2 and weight.is_contiguous(),
             "weight must be contiguous uint8 [N, K/2]")
    N = weight.shape[0]
    _require(weight.shape[1] * 2 == K, f"weight {tuple(weight.shape)} does not match K={K}")
    _require(scales_nk.dtype == torch.uint8 and tuple(scales_nk.shape) == (N, K // 32)
             and scales_nk.is_contiguous(), f"scales must be contiguous uint8 [{N}, {K // 32}]")
    _require(weight.device == x.device == scales_nk.device, "tensors on different devices")
    _require(out_dtype in (torch.bfloat16, torch.float32), "out_dtype must be bf16 or fp32")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    else:
        _require(out.dtype == out_dtype and tuple(out.shape) == (M, N) and out.is_contiguous(),
                 f"out must be contiguous {out_dtype} [M, N]")
    lib = _lib.load()
    fn = lib.h4mv_launch_status if out_dtype == torch.bfloat16 else lib.h4mv_f32_launch_status
    st = fn(weight.data_ptr(), scales_nk.data_ptr(), x.data_ptr(), out.data_ptr(), N, K, M,
            _stream_ptr(x))
    _lib.check("h4mv_launch_status", st)
    return out


# ------------------------------------------------------------------------------ decode attention

_scratch_cache: dict = {}
# Buffers replaced by a larger one stay alive for the life of the process: a graph captured while
# one of them was current replays with its address, so freeing it would hand the graph's tickets
# and records to whatever the allocator puts there next.
_scratch_retired: list = []
# First allocation per device.  The split planner's plans need at most
# counters (256 KiB) + (2 * 256 - 1) records of 16 * 130 floats (4.25 MB at GQA 16), so a buffer of
# this size never grows for planned splits; only explicit larger split counts grow it.
DECODE_SCRATCH_MIN_BYTES = 8 << 20


def decode_num_splits(num_seqs: int, num_kv_heads: int, max_seq_len: int) -> int:
    return int(_lib.load().fp8kv_decode_num_splits(num_seqs, num_kv_heads, max_seq_len))


def decode_scratch_bytes(num_seqs: int, num_q_heads: int, num_kv_heads: int, num_splits: int,
                         head_size: int = 128) -> int:
    return int(_lib.load().fp8kv_decode_scratch_bytes(num_seqs, num_q_heads, num_kv_heads,
                                                     head_size, num_splits))


def decode_scratch(nbytes: int, device, allow_alloc: bool = True) -> torch.Tensor | None:
    """Zero-filled scratch of at least ``nbytes`` for ``device``, reused across calls.

    The kernel leaves its tickets zero again after every completed call, so it is zeroed only
    when allocated.  The first buffer has DECODE_SCRATCH_MIN_BYTES; a larger request replaces it, and
    the replaced buffer is kept alive (graphs captured with it keep replaying into it).  With
    ``allow_alloc=False`` (e.g. during graph capture) a too-small cache returns None.
    """
    if nbytes <= 0:
        return None
    dev = torch.device(device)
    idx = dev.index
    if idx is None:
        idx = torch.cuda.current_device() if dev.type == "cuda" else 0
    key = (dev.type, idx)
    buf = _scratch_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        if not allow_alloc:
            return None
        size = max(nbytes, 2 * buf.numel() if buf is not None else DECODE_SCRATCH_MIN_BYTES)
        if buf is not None:
            _scratch_retired.append(buf)
        buf = torch.zeros(size, dtype=torch.uint8, device=dev)
        _scratch_cache[key] = buf
    return buf


def decode_scratch_reset(scratch: torch.Tensor) -> None:
    """Zero a decode scratch buffer on the current stream with the library's fill kernel
    (fp8kv_decode_scratch_reset): for a buffer whose last call did not complete."""
    _require(scratch.is_cuda and scratch.is_contiguous(), "scratch must be a contiguous device tensor")
    st = _lib.load().fp8kv_decode_scratch_reset(scratch.data_ptr(), scratch.numel() * scratch.element_size(),
                                                _stream_ptr(scratch))
    _lib.check("fp8kv_decode_scratch_reset", st)


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _scale_tensor(x, device) -> torch.Tensor:
    if torch.is_tensor(x):
        _require(x.dtype == torch.float32 and x.numel() >= 1 and x.device == device,
                 "k/v scales must be fp32 device tensors")
        return x
    return torch.tensor([float(x)], dtype=torch.float32, device=device)


def _fp8_cache_check(c: torch.Tensor, name: str) -> None:
    _require(c.is_cuda and c.dim() == 4, f"{name} must be a 4-D device tensor [NB, PBLK, HKV, D]")
    _require(c.dtype in (torch.float8_e4m3fn, torch.uint8), f"{name} must be float8_e4m3fn (or raw uint8)")
    _require(c.stride(3) == 1, f"{name} must be contiguous along head_size")


def _kv_caches_bf16(k_cache: torch.Tensor, v_cache: torch.Tensor) -> bool:
    """True for bf16 K/V caches (the reference's K_FP8 = False branch, scales ignored), False for
    e4m3 ones (float8_e4m3fn or raw uint8); both caches must agree."""
    if k_cache.dtype == torch.bfloat16 or v_cache.dtype == torch.bfloat16:
        for c, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
            _require(c.is_cuda and c.dim() == 4 and c.dtype == torch.bfloat16 and c.stride(3) == 1,
                     f"{n} must be a 4-D bf16 device tensor [NB, PBLK, HKV, D] contiguous along "
                     "head_size (both caches bf16, or both e4m3)")
        return True
    _fp8_cache_check(k_cache, "k_cache")
    _fp8_cache_check(v_cache, "v_cache")
    return False


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     out: torch.Tensor, query_start_loc: torch.Tensor, seq_lens: torch.Tensor,
                     block_table: torch.Tensor, k_scale, v_scale, sm_scale: float,
                     num_splits: int | None = None, max_seq_len: int | None = None,
                     scratch: torch.Tensor | None = None) -> torch.Tensor:
    """Paged decode attention; writes ``out[query_start_loc[s]]`` for every sequence s.

    Contract of vllm-fp8kv/fp8kv_v3.py:116-139 (q [T, HQ, D] bf16, caches [NB, PBLK, HKV, D] fp8
    views with arbitrary block/slot/head strides, int32 metadata, device fp32 scales).  bf16
    caches take the reference's K_FP8 = False branch (fp8kv_v3.py:135): the scales are ignored.
    ``num_splits`` defaults to the library's plan for ``max_seq_len`` (read from ``seq_lens`` when
    not given, which synchronises).  ``scratch`` defaults to a per-device cached buffer.
    """
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and q.stride(2) == 1
             and q.stride(1) == q.shape[2], "q must be bf16 [T, HQ, D] with contiguous heads")
    _require(out.dtype == torch.bfloat16 and out.dim() == 3 and out.stride(2) == 1
             and out.stride(1) == out.shape[2] and out.shape[1:] == q.shape[1:],
             "out must be bf16 [T, HQ, D] with contiguous heads")
    bf16_kv = _kv_caches_bf16(k_cache, v_cache)
    for t, n in ((query_start_loc, "query_start_loc"), (seq_lens, "seq_lens"),
                 (block_table, "block_table")):
        _require(t.dtype == torch.int32 and t.is_cuda, f"{n} must be an int32 device tensor")
    _require(block_table.dim() == 2 and block_table.stride(1) == 1, "block_table must be [NS, max_blocks]")
    NS = block_table.shape[0]
    HQ, D = q.shape[1], q.shape[2]
    HKV = k_cache.shape[2]
    PBLK = k_cache.shape[1]
    dev = q.device
    ks = None if bf16_kv else _scale_tensor(k_scale, dev)
    vs = None if bf16_kv else _scale_tensor(v_scale, dev)
    if num_splits is None:
        if max_seq_len is None:
            max_seq_len = int(seq_lens.max().item()) if NS > 0 else 0
        num_splits = decode_num_splits(NS, HKV, int(max_seq_len))
    need = decode_scratch_bytes(NS, HQ, HKV, num_splits, D)
    if scratch is None:
        scratch = decode_scratch(need, dev)
    elif need > 0:
        _require(scratch.is_cuda and scratch.numel() * scratch.element_size() >= need,
                 f"scratch needs {need} bytes")
    sbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    lib = _lib.load()
    name = "fp8kv_decode_attn_bf16" if bf16_kv else "fp8kv_decode_attn"
    st = getattr(lib, name)(
        q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        v_cache.stride(0), v_cache.stride(1), v_cache.stride(2),
        out.data_ptr(), out.stride(0), query_start_loc.data_ptr(), seq_lens.data_ptr(),
        block_table.data_ptr(), block_table.stride(0), _ptr(ks), _ptr(vs),
        float(sm_scale), NS, HQ, HKV, D, PBLK, int(num_splits),
        None if scratch is None else scratch.data_ptr(), sbytes, _stream_ptr(q))
    _lib.check(name, st)
    return out


# ------------------------------------------------------------------------------ prefill attention

def _prefill_common(q, k_cache, v_cache, out, block_table):
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and q.stride(2) == 1
             and q.stride(1) == q.shape[2], "q must be bf16 [T, HQ, D] with contiguous heads")
    _require(out.dtype == torch.bfloat16 and out.dim() == 3 and out.stride(2) == 1
             and out.stride(1) == out.shape[2] and out.shape[1:] == q.shape[1:],
             "out must be bf16 [T, HQ, D] with contiguous heads")
    bf16_kv = _kv_caches_bf16(k_cache, v_cache)
    _require(block_table.dtype == torch.int32 and block_table.is_cuda and block_table.dim() == 2
             and block_table.stride(1) == 1, "block_table must be int32 [NS, max_blocks] on the device")
    return bf16_kv


def prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      out: torch.Tensor, block_table: torch.Tensor, k_scale, v_scale,
                      sm_scale: float, q0: int, qlen: int) -> torch.Tensor:
    """Single-sequence causal prefill: query i of q[:qlen] is token q0 + i (sees keys <= q0 + i).

    Contract of vllm-fp8kv/fp8kv_prefill.py:124-144 run(q, k_cache, v_cache, out, bt, kscale,
    vscale, sm_scale, q0, qlen): block-table row 0 holds the sequence, scales are device fp32.
    bf16 caches take the reference's K_FP8 = False branch (fp8kv_prefill.py:143): no scales.
    """
    bf16_kv = _prefill_common(q, k_cache, v_cache, out, block_table)
    _require(0 <= qlen <= q.shape[0] and qlen <= out.shape[0] and q0 >= 0, "bad q0 / qlen")
    dev = q.device
    ks = None if bf16_kv else _scale_tensor(k_scale, dev)
    vs = None if bf16_kv else _scale_tensor(v_scale, dev)
    name = "fp8kv_prefill_attn_bf16" if bf16_kv else "fp8kv_prefill_attn"
    st = getattr(_lib.load(), name)(
        q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        v_cache.stride(0), v_cache.stride(1), v_cache.stride(2),
        out.data_ptr(), out.stride(0), block_table.data_ptr(), block_table.stride(0),
        _ptr(ks), _ptr(vs), float(sm_scale), q.shape[1], k_cache.shape[2], q.shape[2],
        k_cache.shape[1], int(q0), int(qlen), _stream_ptr(q))
    _lib.check(name, st)
    return out


def prefill_attention_varlen(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             out: torch.Tensor, cu_seqlens_q: torch.Tensor, seq_lens: torch.Tensor,
                             block_table: torch.Tensor, k_scale, v_scale, sm_scale: float,
                             max_query_len: int | None = None) -> torch.Tensor:
    """Causal prefill of sequences packed along the token axis (vLLM varlen metadata).

    Sequence s owns q rows cu_seqlens_q[s] .. cu_seqlens_q[s+1]-1; its context has seq_lens[s]
    tokens (new ones included), so its q0 is seq_lens[s] - qlen_s; block_table row s maps it.
    ``max_query_len`` sizes the grid (read from ``cu_seqlens_q`` when not given, which syncs).
    """
    bf16_kv = _prefill_common(q, k_cache, v_cache, out, block_table)
    for t, n in ((cu_seqlens_q, "cu_seqlens_q"), (seq_lens, "seq_lens")):
        _require(t.dtype == torch.int32 and t.is_cuda, f"{n} must be an int32 device tensor")
    NS = block_table.shape[0]
    _require(cu_seqlens_q.numel() == NS + 1 and seq_lens.numel() == NS, "metadata sizes differ")
    if max_query_len is None:
        max_query_len = int((cu_seqlens_q[1:] - cu_seqlens_q[:-1]).max().item()) if NS else 0
    dev = q.device
    ks = None if bf16_kv else _scale_tensor(k_scale, dev)
    vs = None if bf16_kv else _scale_tensor(v_scale, dev)
    name = "fp8kv_prefill_attn_varlen_bf16" if bf16_kv else "fp8kv_prefill_attn_varlen"
    st = getattr(_lib.load(), name)(
        q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        v_cache.stride(0), v_cache.stride(1), v_cache.stride(2),
        out.data_ptr(), out.stride(0), cu_seqlens_q.data_ptr(), seq_lens.data_ptr(),
        block_table.data_ptr(), block_table.stride(0), _ptr(ks), _ptr(vs),
        float(sm_scale), NS, q.shape[1], k_cache.shape[2], q.shape[2], k_cache.shape[1],
        int(max_query_len), _stream_ptr(q))
    _lib.check(name, st)
    return out


# ------------------------------------------------------------------------------ fp8 KV-cache write

def cache_write(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                v_cache: torch.Tensor, slot_mapping: torch.Tensor, k_scale, v_scale) -> None:
    """Quantise key / value [T, HKV, D] bf16 to e4m3fn (x / scale, SATFINITE) and write token i
    at slot_mapping[i] (negative: skipped) of the paged caches [NB, PBLK, HKV, D] (fp8 views with
    any block / slot / head strides, the layouts the attention wrappers take).  The semantics of
    vLLM's reshape_and_cache_flash with an fp8 cache."""
    for t, n in ((key, "key"), (value, "value")):
        _require(t.is_cuda and t.dtype == torch.bfloat16 and t.dim() == 3 and t.stride(2) == 1
                 and t.stride(1) == t.shape[2], f"{n} must be bf16 [T, HKV, D] with contiguous heads")
    _require(key.shape == value.shape, "key and value must have the same shape")
    _fp8_cache_check(k_cache, "k_cache")
    _fp8_cache_check(v_cache, "v_cache")
    _require(k_cache.shape[1:] == v_cache.shape[1:] and k_cache.shape[2:] == key.shape[1:],
             "caches must be [NB, PBLK, HKV, D] matching key")
    _require(slot_mapping.is_cuda and slot_mapping.dtype == torch.int64 and slot_mapping.dim() == 1
             and slot_mapping.shape[0] == key.shape[0] and slot_mapping.stride(0) == 1,
             "slot_mapping must be an int64 device tensor [T]")
    dev = key.device
    ks = _scale_tensor(k_scale, dev)
    vs = _scale_tensor(v_scale, dev)
    T, HKV, D = key.shape
    lib = _lib.load()
    st = lib.fp8kv_cache_write(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        v_cache.stride(0), v_cache.stride(1), v_cache.stride(2),
        slot_mapping.data_ptr(), ks.data_ptr(), vs.data_ptr(), T, HKV, D, k_cache.shape[1],
        _stream_ptr(key))
    _lib.check("fp8kv_cache_write", st)


# ------------------------------------------------------------------------------ layer epilogues

def _bf16_rows(t: torch.Tensor, name: str) -> None:
    _require(t.is_cuda and t.dtype == torch.bfloat16 and t.dim() == 2 and t.stride(1) == 1,
             f"{name} must be a 2-D bf16 device tensor with contiguous rows")


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
                      out: torch.Tensor | None = None, mode: int = 0) -> torch.Tensor:
    """residual <- x + residual (bf16, in place); returns rmsnorm(x + residual) * weight in bf16.

    mode 0: the compiled vLLM native form the reference engine runs (f32 sum used for the mean
    and the scaling); mode 1: vLLM's _C.fused_add_rms_norm (bf16-rounded sum).  ``out`` may be
    ``x`` (vLLM's op writes the result into its input).  fp8kv_fused_add_rmsnorm.
    """
    _bf16_rows(x, "x")
    _bf16_rows(residual, "residual")
    M, H = x.shape
    _require(tuple(residual.shape) == (M, H), "residual must match x")
    _require(weight.is_cuda and weight.dtype == torch.bfloat16 and tuple(weight.shape) == (H,)
             and weight.is_contiguous(), "weight must be a contiguous bf16 [H] device tensor")
    if out is None:
        out = torch.empty_like(x)
    _bf16_rows(out, "out")
    _require(tuple(out.shape) == (M, H), "out must match x")
    st = _lib.load().fp8kv_fused_add_rmsnorm(x.data_ptr(), x.stride(0), residual.data_ptr(),
                                             residual.stride(0), weight.data_ptr(), out.data_ptr(),
                                             out.stride(0), M, H, float(eps), int(mode), _stream_ptr(x))
    _lib.check("fp8kv_fused_add_rmsnorm", st)
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None, mode: int = 0) -> torch.Tensor:
    """[M, d] = silu(gate_up[:, :d]) * gate_up[:, d:] in bf16 (mode 0: one rounding, as the
    compiled vLLM native form; mode 1: SiLU rounded first, as vLLM's _C.silu_and_mul)."""
    _bf16_rows(gate_up, "gate_up")
    M, d2 = gate_up.shape
    _require(d2 % 2 == 0, "gate_up width must be even")
    d = d2 // 2
    if out is None:
        out = torch.empty((M, d), dtype=torch.bfloat16, device=gate_up.device)
    _bf16_rows(out, "out")
    _require(tuple(out.shape) == (M, d), f"out must be [{M}, {d}]")
    st = _lib.load().fp8kv_silu_mul(gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(), out.stride(0),
                                    M, d, int(mode), _stream_ptr(gate_up))
    _lib.check("fp8kv_silu_mul", st)
    return out


def interleave_gate_up(weight: torch.Tensor, scales_nk: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Load-time row interleave of a merged gate/up weight (rows [gate; up]) for h4mv_silu_mul:
    each 16-row tile becomes 8 gate rows then the up rows of the same 8 features."""
    _require(weight.is_cuda and weight.dtype == torch.uint8 and weight.dim() == 2 and weight.is_contiguous(),
             "weight must be contiguous uint8 [N, K/2] on the device")
    N, KH = weight.shape
    K = 2 * KH
    _require(scales_nk.dtype == torch.uint8 and tuple(scales_nk.shape) == (N, K // 32)
             and scales_nk.is_contiguous() and scales_nk.device == weight.device,
             f"scales must be contiguous uint8 [{N}, {K // 32}]")
    w_out = torch.empty_like(weight)
    s_out = torch.empty_like(scales_nk)
    st = _lib.load().h4mv_interleave_gate_up(weight.data_ptr(), scales_nk.data_ptr(), w_out.data_ptr(),
                                             s_out.data_ptr(), N, K, _stream_ptr(weight))
    _lib.check("h4mv_interleave_gate_up", st)
    return w_out, s_out


def h4mv_silu_mul(x: torch.Tensor, weight_il: torch.Tensor, scales_il: torch.Tensor,
                  out: torch.Tensor | None = None, mode: int = 0) -> torch.Tensor:
    """[M, N/2] = silu_mul(x . dequant(W)^T) for a gate/up weight from interleave_gate_up, in one
    launch (the same bits as h4mv into [M, N] followed by silu_mul(mode))."""
    _require(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(),
             "x must be a contiguous 2-D bf16 device tensor")
    M, K = x.shape
    N = weight_il.shape[0]
    _require(weight_il.dtype == torch.uint8 and tuple(weight_il.shape) == (N, K // 2)
             and weight_il.is_contiguous(), f"weight must be contiguous uint8 [N, {K // 2}]")
    _require(scales_il.dtype == torch.uint8 and tuple(scales_il.shape) == (N, K // 32)
             and scales_il.is_contiguous(), f"scales must be contiguous uint8 [{N}, {K // 32}]")
    _require(weight_il.device == x.device == scales_il.device, "tensors on different devices")
    if out is None:
        out = torch.empty((M, N // 2), dtype=torch.bfloat16, device=x.device)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (M, N // 2) and out.is_contiguous(),
             f"out must be contiguous bf16 [{M}, {N // 2}]")
    st = _lib.load().h4mv_silu_mul(weight_il.data_ptr(), scales_il.data_ptr(), x.data_ptr(), out.data_ptr(),
                                   N, K, M, int(mode), _stream_ptr(x))
    _lib.check("h4mv_silu_mul", st)
    return out


# ------------------------------------------------------------------------------ MXFP4 x MXFP8 GEMM

def quant_mxfp8(x: torch.Tensor, out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """bf16 [M, K] -> (e4m3fn codes uint8 [M, K], e8m0 scale bytes uint8 [M, K/32]) per 32-wide
    block of K (OCP MX, shared exponent floor(log2 max|x|) - 8).  h4a8_quant_act."""
    _bf16_rows(x, "x")
    M, K = x.shape
    if out is None:
        out = (torch.empty((M, K), dtype=torch.uint8, device=x.device),
               torch.empty((M, K // 32), dtype=torch.uint8, device=x.device))
    xq, sx = out
    _require(xq.dtype == torch.uint8 and tuple(xq.shape) == (M, K) and xq.is_contiguous(), "codes must be uint8 [M, K]")
    _require(sx.dtype == torch.uint8 and tuple(sx.shape) == (M, K // 32) and sx.is_contiguous(),
             "scales must be uint8 [M, K/32]")
    st = _lib.load().h4a8_quant_act(x.data_ptr(), x.stride(0), xq.data_ptr(), sx.data_ptr(), M, K, _stream_ptr(x))
    _lib.check("h4a8_quant_act", st)
    return xq, sx


def h4a8_gemm(xq: torch.Tensor, sx: torch.Tensor, weight: torch.Tensor, scales_nk: torch.Tensor,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 [M, N] = dequant(xq, sx) . dequant(weight, scales_nk)^T on the block-scaled MFMA."""
    M, K = xq.shape
    N = weight.shape[0]
    _require(xq.is_cuda and xq.dtype == torch.uint8 and xq.is_contiguous(), "xq must be contiguous uint8 [M, K]")
    _require(sx.dtype == torch.uint8 and tuple(sx.shape) == (M, K // 32) and sx.is_contiguous(), "sx must be uint8 [M, K/32]")
    _require(weight.dtype == torch.uint8 and tuple(weight.shape) == (N, K // 2) and weight.is_contiguous(),
             "weight must be contiguous uint8 [N, K/2]")
    _require(scales_nk.dtype == torch.uint8 and tuple(scales_nk.shape) == (N, K // 32) and scales_nk.is_contiguous(),
             "scales must be contiguous uint8 [N, K/32]")
    _require(xq.device == sx.device == weight.device == scales_nk.device, "tensors on different devices")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=xq.device)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (M, N) and out.is_contiguous(),
             "out must be contiguous bf16 [M, N]")
    st = _lib.load().h4a8_gemm(weight.data_ptr(), scales_nk.data_ptr(), xq.data_ptr(), sx.data_ptr(),
                               out.data_ptr(), N, K, M, _stream_ptr(xq))
    _lib.check("h4a8_gemm", st)
    return out


def quant_fp8_per_token(x: torch.Tensor, out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """bf16 [M, K] -> (e4m3fn codes uint8 [M, K], fp32 scales [M]), one scale per row:
    max(max|x| / 448, 1 / (448 * 512)), codes e4m3fn(clamp(x / scale)).  h4a8_quant_act_token
    (vLLM's dynamic_per_token_scaled_fp8_quant)."""
    _bf16_rows(x, "x")
    M, K = x.shape
    if out is None:
        out = (torch.empty((M, K), dtype=torch.uint8, device=x.device),
               torch.empty((M,), dtype=torch.float32, device=x.device))
    xq, sc = out
    _require(xq.dtype == torch.uint8 and tuple(xq.shape) == (M, K) and xq.is_contiguous(), "codes must be uint8 [M, K]")
    _require(sc.dtype == torch.float32 and tuple(sc.shape) == (M,) and sc.is_contiguous(), "scales must be fp32 [M]")
    st = _lib.load().h4a8_quant_act_token(x.data_ptr(), x.stride(0), xq.data_ptr(), sc.data_ptr(), M, K,
                                          _stream_ptr(x))
    _lib.check("h4a8_quant_act_token", st)
    return xq, sc


def h4a8_gemm_token(xq: torch.Tensor, token_scales: torch.Tensor, weight: torch.Tensor,
                    scales_nk: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 [M, N] = token_scales[:, None] * (e4m3(xq) . dequant(weight, scales_nk)^T)."""
    M, K = xq.shape
    N = weight.shape[0]
    _require(xq.is_cuda and xq.dtype == torch.uint8 and xq.is_contiguous(), "xq must be contiguous uint8 [M, K]")
    _require(token_scales.dtype == torch.float32 and tuple(token_scales.shape) == (M,) and token_scales.is_contiguous(),
             "token scales must be fp32 [M]")
    _require(weight.dtype == torch.uint8 and tuple(weight.shape) == (N, K // 2) and weight.is_contiguous(),
             "weight must be contiguous uint8 [N, K/2]")
    _require(scales_nk.dtype == torch.uint8 and tuple(scales_nk.shape) == (N, K // 32) and scales_nk.is_contiguous(),
             "scales must be contiguous uint8 [N, K/32]")
    _require(xq.device == token_scales.device == weight.device == scales_nk.device, "tensors on different devices")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=xq.device)
    _require(out.dtype == torch.bfloat16 and tuple(out.shape) == (M, N) and out.is_contiguous(),
             "out must be contiguous bf16 [M, N]")
    st = _lib.load().h4a8_gemm_token(weight.data_ptr(), scales_nk.data_ptr(), xq.data_ptr(), token_scales.data_ptr(),
                                     out.data_ptr(), N, K, M, _stream_ptr(xq))
    _lib.check("h4a8_gemm_token", st)
    return out


def mxfp4_linear(x: torch.Tensor, weight: torch.Tensor, scales_nk: torch.Tensor,
                 act: str = "mx") -> torch.Tensor:
    """x [M, K] bf16 -> [M, N] bf16 through an fp8 activation quantiser and the block-scaled GEMM:
    ``act`` "mx" (MXFP8 blocks of 32) or "token" (per-token fp8, the engine's format)."""
    if act == "token":
        xq, sc = quant_fp8_per_token(x)
        return h4a8_gemm_token(xq, sc, weight, scales_nk)
    _require(act == "mx", f"unknown activation format {act!r}")
    xq, sx = quant_mxfp8(x)
    return h4a8_gemm(xq, sx, weight, scales_nk)


# ------------------------------------------------------------------------------ lm_head, top-k, rerank

_topk_ws: dict = {}
# Workspaces replaced by a larger one stay alive for the life of the process, as the decode
# scratch does: a graph captured while one was current replays its logits and candidates into it.
_topk_ws_retired: list = []


def topk_workspace(nbytes: int, device, allow_alloc: bool = True) -> torch.Tensor | None:
    """The per-device cached lm_head workspace, grown to at least ``nbytes``.  A replaced buffer
    is kept alive; with ``allow_alloc=False`` (graph capture) a too-small cache returns None.
    Every call on a device shares this buffer, so calls that overlap on different streams race:
    pass an explicit workspace per stream instead."""
    dev = torch.device(device)
    idx = dev.index
    if idx is None:
        idx = torch.cuda.current_device() if dev.type == "cuda" else 0
    key = (dev.type, idx)
    buf = _topk_ws.get(key)
    if buf is None or buf.numel() < nbytes:
        if not allow_alloc:
            return None
        if buf is not None:
            _topk_ws_retired.append(buf)
        buf = torch.empty(max(nbytes, 2 * buf.numel() if buf is not None else nbytes), dtype=torch.uint8,
                          device=dev)
        _topk_ws[key] = buf
    return buf


def lm_head_topk(x: torch.Tensor, weight: torch.Tensor, scales_nk: torch.Tensor, k: int,
                 workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(values fp32 [M, k], indices int32 [M, k]) of the k largest logits x . dequant(W)^T per row,
    in rank order (value descending, NaN first, ties by lower index).  h4mv_topk; the workspace
    defaults to the per-device cached buffer of ``topk_workspace``, which calls on one device
    share (calls overlapping on different streams must pass their own).  During graph capture
    the cache is not grown: capture a call whose workspace is already large enough, or pass one."""
    _require(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(),
             "x must be a contiguous 2-D bf16 device tensor")
    M, K = x.shape
    N = weight.shape[0]
    _require(weight.dtype == torch.uint8 and tuple(weight.shape) == (N, K // 2) and weight.is_contiguous(),
             "weight must be contiguous uint8 [N, K/2]")
    _require(scales_nk.dtype == torch.uint8 and tuple(scales_nk.shape) == (N, K // 32)
             and scales_nk.is_contiguous(), f"scales must be contiguous uint8 [{N}, {K // 32}]")
    lib = _lib.load()
    need = int(lib.h4mv_topk_workspace_bytes(N, M, int(k)))
    _require(need > 0, f"k={k} outside [1, 64]")
    if workspace is None:
        workspace = topk_workspace(need, x.device, allow_alloc=not torch.cuda.is_current_stream_capturing())
        _require(workspace is not None,
                 f"lm_head_topk during graph capture needs {need} workspace bytes: pass a workspace")
    vals = torch.empty((M, k), dtype=torch.float32, device=x.device)
    idx = torch.empty((M, k), dtype=torch.int32, device=x.device)
    st = lib.h4mv_topk(weight.data_ptr(), scales_nk.data_ptr(), x.data_ptr(), N, K, M, int(k),
                       vals.data_ptr(), idx.data_ptr(), workspace.data_ptr(),
                       workspace.numel() * workspace.element_size(), _stream_ptr(x))
    _lib.check("h4mv_topk", st)
    return vals, idx


def rerank_exact(embedding: torch.Tensor, x: torch.Tensor, candidates: torch.Tensor
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """(values fp32 [M, C], indices int32 [M, C]): candidates[m] rescored as fp32 dot products of
    x[m] with the bf16 embedding rows and sorted in rank order (fp8kv_rerank_exact)."""
    _bf16_rows(embedding, "embedding")
    _bf16_rows(x, "x")
    V, H = embedding.shape
    M = x.shape[0]
    _require(x.shape[1] == H, "x and embedding widths differ")
    _require(candidates.is_cuda and candidates.dtype == torch.int32 and candidates.dim() == 2
             and candidates.shape[0] == M and candidates.is_contiguous(), "candidates must be int32 [M, C]")
    C = candidates.shape[1]
    vals = torch.empty((M, C), dtype=torch.float32, device=x.device)
    idx = torch.empty((M, C), dtype=torch.int32, device=x.device)
    st = _lib.load().fp8kv_rerank_exact(embedding.data_ptr(), embedding.stride(0), V, x.data_ptr(), x.stride(0),
                                        candidates.data_ptr(), C, M, H, vals.data_ptr(), idx.data_ptr(),
                                        _stream_ptr(x))
    _lib.check("fp8kv_rerank_exact", st)
    return vals, idx

