"""MXFP4 W4A16 matvec restated on the CPU (numpy, fp64 accumulation).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows the reference's torch oracle h4mv/h4mv_test.py:19-32 (LUT dequant, per-32 scale,
x @ W^T) and the kernel contract of h4mv/h4mv.cu:1-3,43-104 (W [N,K/2] low nibble = even k,
St [N,K/32] e8m0, x [M,K] bf16, out [M,N]).  The scale tensor is taken in the kernel's
[N, K/32] layout; ``repack_scales`` restates the load-time transpose of h4mv/fp8kv_hipw4.py:32-43.

Pinned by (tests/test_oracle.py):
  * the one-hot probes of h4mv/h4mv_test.py:38-52 (weight 1.0 at one k, x one-hot at that k,
    M = 8 rows, every k of a 32-group: result exactly 1.0),
  * the integer full-row probe of w4-hip-demo/probe_w4hip.py:33-47 (random codes, scale byte
    127, x = (k mod 7) - 3: every product and partial sum is exact in fp32, so the result is
    compared with exact integer arithmetic on doubled values),
  * a brute-force pure-Python loop on a tiny random case with random scales,
  * planted mistakes (nibble order swapped, scale applied to the wrong group) failing the above.
"""
from __future__ import annotations

import numpy as np

from .formats import E2M1, E8M0, unpack_e2m1


def repack_scales(weight_scale: np.ndarray) -> np.ndarray:
    """[K/32, N] checkpoint scale tensor -> [N, K/32] contiguous (h4mv/fp8kv_hipw4.py:32-43)."""
    return np.ascontiguousarray(np.asarray(weight_scale, dtype=np.uint8).T)


def dequant_w4(W: np.ndarray, St: np.ndarray, rows: slice | None = None) -> np.ndarray:
    """float64 [n, K] weights = e2m1(W) * e8m0(St) broadcast over each 32-wide group."""
    W = np.asarray(W, dtype=np.uint8)
    St = np.asarray(St, dtype=np.uint8)
    if rows is not None:
        W, St = W[rows], St[rows]
    n, kh = W.shape
    K = kh * 2
    assert St.shape == (n, K // 32), (St.shape, n, K)
    w = E2M1[unpack_e2m1(W)]                                   # [n, K]
    s = E8M0[St]                                               # [n, K/32]
    return (w.reshape(n, K // 32, 32) * s[:, :, None]).reshape(n, K)


def w4mv(W: np.ndarray, St: np.ndarray, X: np.ndarray, chunk: int = 2048) -> np.ndarray:
    """float64 [M, N] = X[M, K] @ dequant(W, St)^T, accumulated in fp64.

    ``X`` may be any float array (bf16 inputs should be passed already widened to float32).
    """
    X = np.asarray(X, dtype=np.float64)
    N = W.shape[0]
    out = np.empty((X.shape[0], N), dtype=np.float64)
    for r0 in range(0, N, chunk):
        r1 = min(N, r0 + chunk)
        out[:, r0:r1] = X @ dequant_w4(W, St, slice(r0, r1)).T
    return out


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values (8 significant bits) in the binade of each |v|; 0 maps to 2^-133."""
    v = np.abs(np.asarray(v, dtype=np.float64))
    _, e = np.frexp(v)                                  # v = f * 2^e, f in [0.5, 1)
    ulp = np.ldexp(1.0, e - 8)
    return np.where(v == 0, 2.0 ** -133, ulp)


def bf16_excess_error(y: np.ndarray, ref: np.ndarray) -> float:
    """max over elements of (|y - ref| - ulp_bf16(ref)/2) / max|ref|, floored at 0.

    A bf16 output can be no closer to the exact result than half a bf16 ulp, so this is the
    error a bf16-output kernel adds on top of the unavoidable output rounding (0 for a
    correctly rounded result, ~1e-6 for fp32 accumulation).
    """
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    ex = np.max(np.abs(y - ref) - 0.5 * bf16_ulp(ref))
    return max(0.0, float(ex / den)) if den > 0 else float(max(0.0, ex))


def rel_to_max_error(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| / max |ref|: the matvec error measure of h4mv/h4mv_test.py:74."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / den) if den > 0 else float(np.max(np.abs(y - ref)))
