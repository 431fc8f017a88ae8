"""MXFP4 x MXFP8 GEMM and the MXFP8 activation quantiser, restated on the CPU (numpy, fp64).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference engine's prefill linears run its vLLM fork's W4A8 GEMM (radiance_mxfp4_fp8_gemm,
profiling/prof_engine.txt:3-4, profiling/prof_prefill.txt:8) on per-token fp8 activations; that
library is closed and absent, so this build defines its own operator on gfx950's native block
format and this module is its definition:

  quant_mxfp8 (OCP MX v1.0, MXFP8 E4M3, block 32 along K): for each block, shared exponent
      e = floor(log2(max |x|)) - 8, scale byte clip(e + 127, 0, 254) (0 for an all-zero block,
      255 = NaN for a block holding NaN or +-inf), elements e4m3fn(x / 2^(byte - 127)) rounded
      to nearest even and saturated to +-448;
  gemm: Out[m, n] = sum_k dq(xq)[m, k] * dq(w)[n, k] with dq(w) = e2m1 * 2^(St - 127) in the
      matvec's [N, K/2] / [N, K/32] layout (oracle/matvec.py, h4mv/h4mv.cu:1-3).

  quant_fp8_per_token (vLLM's dynamic_per_token_scaled_fp8_quant, csrc/quantization/fp8/common.cu
      of vLLM, the engine's activation quantiser at profiling/prof_engine.txt:8; vLLM is not in
      this container, so this restates its published kernel): per row, scale = max(amax / 448,
      1 / (448 * 512)) in fp32, codes e4m3fn(fmax(-448, fmin(x / scale, 448))) with the fp32
      division correctly rounded and NaN-ignoring min / max;
  gemm_token: Out[m, n] = scale[m] * sum_k e4m3(codes)[m, k] * dq(w)[n, k].

Pins (tests/test_oracle_w4a8.py): the element encoder is the pinned kv_cache encoder (torch's
float8 cast, midpoints, brute force); the quantiser against torch's float8_e4m3fn cast of
x / 2^e per block and the OCP rule that the block maximum lands in e4m3's top binade; exact
round trips of representable blocks; the GEMM against exact integer arithmetic (integer-valued
operands, unit scales) and against the matvec oracle on dequantised activations; planted
mistakes (exponent off by one, scales applied to the wrong block) fail the checks.
"""
from __future__ import annotations

import numpy as np

from .formats import E4M3FN
from .kv_cache import encode_e4m3fn_satfinite
from .matvec import dequant_w4


def quant_mxfp8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x [M, K] float32 (bf16 values) -> (codes uint8 [M, K], scale bytes uint8 [M, K/32])."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    blk = x.reshape(M, K // 32, 32)
    with np.errstate(invalid="ignore"):
        amax = np.max(np.abs(blk), axis=-1)
    bad = ~np.isfinite(amax) | np.any(~np.isfinite(blk), axis=-1)
    _, E = np.frexp(np.where(bad, 1.0, amax).astype(np.float64))     # amax = f 2^E, f in [0.5, 1)
    e = E - 1
    sbyte = np.clip(e - 8 + 127, 0, 254)
    sbyte = np.where(amax == 0, 0, sbyte)
    sbyte = np.where(bad, 255, sbyte).astype(np.uint8)
    inv = np.where(bad, 1.0, np.ldexp(1.0, -(sbyte.astype(np.int64) - 127)))
    q = (blk.astype(np.float64) * inv[..., None]).astype(np.float32)
    codes = encode_e4m3fn_satfinite(q).reshape(M, K)
    return codes, sbyte


def dequant_mxfp8(codes: np.ndarray, sbyte: np.ndarray) -> np.ndarray:
    M, K = codes.shape
    v = E4M3FN[codes].astype(np.float64).reshape(M, K // 32, 32)
    s = np.where(sbyte == 255, np.nan, np.ldexp(1.0, sbyte.astype(np.int64) - 127))
    return (v * s[..., None]).reshape(M, K)


def gemm(W: np.ndarray, St: np.ndarray, codes: np.ndarray, sbyte: np.ndarray) -> np.ndarray:
    """float64 [M, N] = dequant_mxfp8(codes, sbyte) @ dequant_w4(W, St)^T."""
    return dequant_mxfp8(codes, sbyte) @ dequant_w4(W, St).T


FP8_MAX = np.float32(448.0)
TOKEN_MIN_SCALE = np.float32(1.0) / np.float32(448.0 * 512.0)


def quant_fp8_per_token(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x [M, K] float32 (bf16 values) -> (codes uint8 [M, K], scales float32 [M])."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        amax = np.fmax.reduce(np.abs(x), axis=1, initial=np.float32(0.0)).astype(np.float32)
    scale = np.fmax(amax / FP8_MAX, TOKEN_MIN_SCALE).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        q = (x / scale[:, None]).astype(np.float32)               # IEEE fp32 division
    q = np.fmax(-FP8_MAX, np.fmin(q, FP8_MAX))
    return encode_e4m3fn_satfinite(q), scale


def gemm_token(W: np.ndarray, St: np.ndarray, codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """float64 [M, N] = scales[:, None] * (e4m3(codes) @ dequant_w4(W, St)^T)."""
    v = E4M3FN[codes].astype(np.float64)
    return (v @ dequant_w4(W, St).T) * np.asarray(scales, dtype=np.float64)[:, None]
