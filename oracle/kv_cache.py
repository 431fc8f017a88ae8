"""fp8 KV-cache write (quantise + scatter into the paged cache), restated on the CPU (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference does not implement this step: its engine runs vLLM's
``reshape_and_cache_flash`` (kernel ``reshape_and_cache_kernel_flash``, listed in the reference's
profiles at profiling/prof_h4mv.txt:9, profiling/prof_prefill.txt:23, profiling/prof_engine.txt:11)
from the vLLM 0.28 fork shipped in the image the reference runs (serve-fp8kv-best.sh; the fork is
pinned only by that image tag and is absent here).  Its published algorithm (vLLM
csrc/cache_kernels.cu, reshape_and_cache_flash_kernel, with the fp8 ``scaled_convert`` of
csrc/quantization/fp8): for token i with slot = slot_mapping[i] >= 0 (negative slots are padding
and skipped), block = slot // block_size, offset = slot % block_size, and every (head, d):

    cache[block, offset, head, d] = e4m3fn_satfinite( float32(x[i, head, d]) / scale )

with the division in fp32, round-to-nearest-even into e4m3fn and saturation of finite values to
+-448 (the SATFINITE mode).  The read side of this format is what the attention kernels consume
(vllm-fp8kv/fp8kv_override.py:82-85 views the same bytes as fp8).

Functions and what pins them (tests/test_oracle_kv_cache.py):
  * ``encode_e4m3fn_satfinite`` - float32 -> e4m3fn byte.  Pinned by torch's float8_e4m3fn cast
    (a library routine; round to nearest even) on every bf16 value whose quotient it does not
    turn into NaN, by the round trip of every finite code, by the midpoints between adjacent codes
    (ties to the even code), by brute-force nearest-value search on the whole bf16 range, and by
    the saturation rules (finite overflow and +-inf give +-448, NaN keeps its sign: 0x7F / 0xFF).
  * ``cache_write`` - the scatter.  Pinned by the addressing identities checked in the tests
    (every written byte decodes to the quantised input at the slot's (block, offset), unwritten
    bytes keep their previous value, negative slots write nothing).
"""
from __future__ import annotations

import numpy as np

from .formats import E4M3FN

E4M3_MAX = 448.0
_FINITE_POS = E4M3FN[:0x7F]                     # codes 0x00 .. 0x7E, increasing


def encode_e4m3fn_satfinite(y: np.ndarray) -> np.ndarray:
    """float32 array -> uint8 e4m3fn codes: RNE, finite values and +-inf saturate to +-448,
    NaN -> 0x7F with the input's sign bit, -0.0 -> 0x80."""
    y = np.asarray(y, dtype=np.float32)
    flat = y.ravel()
    a = np.abs(flat).astype(np.float64)
    nan = np.isnan(flat)
    a = np.where(nan, 0.0, np.minimum(a, E4M3_MAX))
    idx = np.searchsorted(_FINITE_POS, a)                           # vals[idx-1] < a <= vals[idx]
    idx = np.clip(idx, 1, len(_FINITE_POS) - 1)
    lo, hi = _FINITE_POS[idx - 1], _FINITE_POS[idx]
    pick_hi = (a - lo) > (hi - a)
    tie = (a - lo) == (hi - a)
    pick_hi = pick_hi | (tie & ((idx % 2) == 0))                    # the even code wins ties
    code = np.where(pick_hi, idx, idx - 1)
    code = np.where(a == 0.0, 0, code)
    code = np.where(nan, 0x7F, code).astype(np.uint8)
    sign = np.signbit(flat).astype(np.uint8) << 7
    return (code | sign).reshape(y.shape)


def quantize_rows(x: np.ndarray, scale: float) -> np.ndarray:
    """x (bf16 values given as float32) / scale in fp32, then e4m3fn (SATFINITE)."""
    q = np.asarray(x, dtype=np.float32) / np.float32(scale)
    return encode_e4m3fn_satfinite(q)


def cache_write(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                slot_mapping: np.ndarray, k_scale: float, v_scale: float, block_size: int) -> None:
    """In place: key/value float32 [T, HKV, D] (bf16 values); caches uint8 [NB, block_size, HKV, D]
    (standalone layout; other layouts are views with the same indexing); slot_mapping int64 [T]."""
    kq = quantize_rows(key, k_scale)
    vq = quantize_rows(value, v_scale)
    for i, slot in enumerate(np.asarray(slot_mapping, dtype=np.int64)):
        if slot < 0:
            continue
        b, o = divmod(int(slot), block_size)
        k_cache[b, o] = kq[i]
        v_cache[b, o] = vq[i]
