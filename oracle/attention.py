"""Paged fp8-KV attention (decode and causal prefill) restated on the CPU (torch, fp64 default).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Cache model (both reference kernels): logical token t of sequence s lives in physical block
``block_table[s, t // PBLK]`` at in-block slot ``t % PBLK`` (vllm-fp8kv/fp8kv_v3.py:55-60,
fp8kv_prefill.py:73-76); the caches are indexed ``[block, slot, kv_head, d]`` through arbitrary
strides, so both the standalone ``[NB, PBLK, HKV, D]`` tensor and the engine's transposed
K|V-interleaved view (vllm-fp8kv/fp8kv_override.py:82-85) are accepted as torch views.
fp8 values are decoded with the e4m3fn table (exact), k_scale folds into the score scale and
v_scale multiplies the output (fp8kv_v3.py:43-45,110-111; fp8kv_prefill.py:57-58,117-118).
bf16 caches (the reference's K_FP8 = False branch, fp8kv_v3.py:44-45,61-66,110,135 and
fp8kv_prefill.py:57-60,77-82,117,143) are used as stored and both scales are ignored.

  * ``decode_attention``  - fp8kv_v3.py:3-113 semantics; the reference's own oracle is
    fp8kv_v3.py:158-177 (also fp8kv_kernel.py:109-122, profiling/mb_stock.py:41-53).
    One query token per sequence at row ``qsl[s]``; it attends to all ``seq_lens[s]`` tokens.
    A sequence with no context yields zeros (the reference kernel yields NaN there: its merge
    computes 0 * exp(-inf - -inf), fp8kv_v3.py:100-111).
  * ``prefill_attention`` - single sequence, fp8kv_prefill.py:31-121 semantics; the reference's
    own oracle is vllm-fp8kv/prefill_test.py:23-38.  Query i is token q0 + i and sees keys
    t <= q0 + i (fp8kv_prefill.py:108).
  * ``varlen_prefill_attention`` - several sequences packed along the token axis with
    ``cu_seqlens_q``; q0 of sequence s is seq_lens[s] - qlen_s (the rule of
    fp8kv_prefill.py:179 applied per sequence).

Pinned by (tests/test_oracle.py): context 1 gives v_scale * V_0 exactly; identical keys give
v_scale * mean(V); torch's scaled_dot_product_attention (fp64, explicit causal mask) on the
gathered dequantised cache; a brute-force pure-Python loop on a tiny case; the scale fold
checked against pre-scaled K/V; block-table permutation invariance; decode == the last row of a
prefill over the same context; varlen == independent per-sequence runs; planted mistakes
(k_scale dropped, off-by-one causal mask, wrong GQA head mapping) failing those checks.  bf16
caches: SDPA on the stored values with the scales left out, a bf16 cache holding an e4m3 cache's
values times power-of-two scales reproducing the e4m3 path exactly, and a planted use of the
scales failing the SDPA check.
"""
from __future__ import annotations

import torch

from .formats import E4M3FN

_E4M3_T = torch.tensor(E4M3FN, dtype=torch.float64)


def _as_u8(cache: torch.Tensor) -> torch.Tensor:
    if cache.dtype == torch.uint8:
        return cache
    if cache.dtype == torch.float8_e4m3fn:
        return cache.view(torch.uint8)
    raise TypeError(f"expected uint8 or float8_e4m3fn cache, got {cache.dtype}")


def gather_kv(cache: torch.Tensor, bt_row: torch.Tensor, ctx: int, kh: int,
              dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """Dequantised (unscaled) [ctx, D] rows of kv head ``kh`` for tokens 0..ctx-1 (bf16 caches:
    the stored values)."""
    pblk = cache.shape[1]
    t = torch.arange(ctx)
    blk = bt_row.long()[t // pblk]
    slot = t % pblk
    if cache.dtype == torch.bfloat16:
        return cache[blk, slot, kh, :].to(dtype)
    codes = _as_u8(cache)[blk, slot, kh, :]                        # [ctx, D] uint8
    return _E4M3_T.to(dtype)[codes.long()]


def _scales(cache: torch.Tensor, k_scale: float, v_scale: float) -> tuple[float, float]:
    """The scales that apply: none for bf16 caches (fp8kv_v3.py:44-45,110; fp8kv_prefill.py:57-60,117)."""
    return (1.0, 1.0) if cache.dtype == torch.bfloat16 else (k_scale, v_scale)


def _attend(qh: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, v_scale: float,
            q_pos: torch.Tensor | None) -> torch.Tensor:
    """softmax(qh k^T * scale [causal on q_pos]) v * v_scale; qh [R, D], k/v [ctx, D]."""
    s = (qh @ k.T) * scale
    if q_pos is not None:
        mask = torch.arange(k.shape[0])[None, :] > q_pos[:, None]
        s = s.masked_fill(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return (p @ v) * v_scale


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     qsl: torch.Tensor, seq_lens: torch.Tensor, block_table: torch.Tensor,
                     k_scale: float, v_scale: float, sm_scale: float,
                     dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """Output [NS, HQ, D] (row s = token qsl[s]) of one-token-per-sequence paged decode."""
    NS = block_table.shape[0]
    HQ, D = q.shape[1], q.shape[2]
    HKV = k_cache.shape[2]
    gqa = HQ // HKV
    k_scale, v_scale = _scales(k_cache, k_scale, v_scale)
    out = torch.zeros(NS, HQ, D, dtype=dtype)
    for s in range(NS):
        ctx = int(seq_lens[s])
        if ctx <= 0:
            continue
        tok = int(qsl[s])
        for kh in range(HKV):
            k = gather_kv(k_cache, block_table[s], ctx, kh, dtype)
            v = gather_kv(v_cache, block_table[s], ctx, kh, dtype)
            qh = q[tok, kh * gqa:(kh + 1) * gqa, :].to(dtype)
            out[s, kh * gqa:(kh + 1) * gqa] = _attend(qh, k, v, sm_scale * k_scale, v_scale, None)
    return out


def prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      bt_row: torch.Tensor, k_scale: float, v_scale: float, sm_scale: float,
                      q0: int, qlen: int, dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """Output [qlen, HQ, D] of causal prefill: query i = token q0 + i sees keys 0..q0+i."""
    HQ, D = q.shape[1], q.shape[2]
    HKV = k_cache.shape[2]
    gqa = HQ // HKV
    k_scale, v_scale = _scales(k_cache, k_scale, v_scale)
    ctx = q0 + qlen
    pos = torch.arange(qlen) + q0
    out = torch.empty(qlen, HQ, D, dtype=dtype)
    for kh in range(HKV):
        k = gather_kv(k_cache, bt_row, ctx, kh, dtype)
        v = gather_kv(v_cache, bt_row, ctx, kh, dtype)
        for g in range(gqa):
            h = kh * gqa + g
            out[:, h] = _attend(q[:qlen, h].to(dtype), k, v, sm_scale * k_scale, v_scale, pos)
    return out


def varlen_prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             cu_seqlens_q: torch.Tensor, seq_lens: torch.Tensor,
                             block_table: torch.Tensor, k_scale: float, v_scale: float,
                             sm_scale: float, dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """Output [T, HQ, D] for sequences packed along tokens; q0_s = seq_lens[s] - qlen_s."""
    T, HQ, D = q.shape
    out = torch.zeros(T, HQ, D, dtype=dtype)
    for s in range(block_table.shape[0]):
        a, b = int(cu_seqlens_q[s]), int(cu_seqlens_q[s + 1])
        qlen = b - a
        if qlen <= 0:
            continue
        q0 = int(seq_lens[s]) - qlen
        out[a:b] = prefill_attention(q[a:b], k_cache, v_cache, block_table[s], k_scale, v_scale,
                                     sm_scale, q0, qlen, dtype)
    return out
