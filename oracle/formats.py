"""Number formats of the hot path, restated from their definitions (CPU, numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Functions and what pins them (tests/test_oracle.py):
  * ``e4m3fn_table``  - KV-cache element, OCP FP8 E4M3 ("fn": no inf, 0x7F/0xFF NaN, max 448).
    The reference casts e4m3fn -> bf16 directly and relies on that being exact
    (vllm-fp8kv/fp8kv_v3.py:61-63, docs/03-fp8kv-pathology-and-kernel.md:33).
    Pinned by: torch's float8_e4m3fn -> float32 conversion on all 256 bytes, OCP spot values
    (448, 2^-9, 2^-6, 1.0, -0.0, NaN codes) and the bf16 round trip of every finite value.
  * ``e2m1_table``    - MXFP4 element.  Reference LUT: h4mv/h4mv_test.py:16-17, bit rules
    h4mv/h4mv.cu:33-41 (zero iff (v & 7) == 0, subnormal 0.5 has mantissa 0).
    Pinned by: the literal LUT of h4mv_test.py:16-17 and the bit rules above checked code by
    code (torch 2.10 has the float4_e2m1fn_x2 dtype but no CPU conversion for it).
  * ``e8m0_table``    - MX block scale 2^(b-127) (docs/04-w4a8-matvec-wall.md:12,
    h4mv/h4mv.cu:72).  Byte 255 is NaN per OCP MX v1.0; the reference kernel turns it into +inf
    and its torch oracle into 2^128 (h4mv_test.py:20) - this restatement follows the OCP spec.
    Pinned by: torch's float8_e8m0fnu -> float32 conversion on bytes 0..254 and the NaN code.
  * ``pack_e2m1`` / ``unpack_e2m1`` - two codes per byte, low nibble = even k
    (h4mv/h4mv.cu:2, w4-hip-demo/w4_hip_demo.cu:3-6).  Pinned by the one-hot probes of
    h4mv_test.py:38-52 run through the matvec oracle.
  * ``quantize_e4m3`` - per-tensor KV quantisation x / (amax/448) -> e4m3fn used to build the
    BASELINE inputs.  Pinned by the e4m3 table (every output code decodes to within half an ulp).
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def e4m3fn_table() -> np.ndarray:
    """float64[256]: value of each e4m3fn byte (sign | 4-bit exponent, bias 7 | 3-bit mantissa)."""
    out = np.empty(256, dtype=np.float64)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 0x7
        if e == 0xF and m == 0x7:
            out[b] = np.nan
        elif e == 0:
            out[b] = s * (m / 8.0) * 2.0 ** -6
        else:
            out[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


def e2m1_table() -> np.ndarray:
    """float64[16]: value of each e2m1 code (sign | 2-bit exponent, bias 1 | 1-bit mantissa)."""
    out = np.empty(16, dtype=np.float64)
    for v in range(16):
        s = -1.0 if v & 0x8 else 1.0
        e = (v >> 1) & 0x3
        m = v & 0x1
        out[v] = s * (0.5 * m if e == 0 else (1.0 + 0.5 * m) * 2.0 ** (e - 1))
    return out


def e8m0_table() -> np.ndarray:
    """float64[256]: 2^(b-127) for b in 0..254, NaN for b = 255."""
    out = np.array([2.0 ** (b - 127) for b in range(256)], dtype=np.float64)
    out[255] = np.nan
    return out


E4M3FN = e4m3fn_table()
E2M1 = e2m1_table()
E8M0 = e8m0_table()


def pack_e2m1(codes: np.ndarray) -> np.ndarray:
    """uint8 codes [..., K] (values 0..15) -> uint8 [..., K/2], low nibble = even k."""
    codes = np.asarray(codes, dtype=np.uint8)
    assert codes.shape[-1] % 2 == 0
    return (codes[..., 0::2] & 0xF) | ((codes[..., 1::2] & 0xF) << 4)


def unpack_e2m1(packed: np.ndarray) -> np.ndarray:
    """uint8 [..., K/2] -> uint8 codes [..., K]."""
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 0xF
    out[..., 1::2] = packed >> 4
    return out


def decode_e4m3(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float64 values (table lookup)."""
    return E4M3FN[np.asarray(codes, dtype=np.uint8)]


def quantize_e4m3(x: np.ndarray, scale: float) -> np.ndarray:
    """float array -> uint8 e4m3fn codes of x / scale, round to nearest (ties to even code).

    Values are clamped to +-448 first (the per-tensor scale amax/448 keeps them in range).
    Nearest-value search over the finite table, ties to the even mantissa code, which is
    the IEEE-style rounding torch's float8_e4m3fn cast applies.
    """
    y = np.clip(np.asarray(x, dtype=np.float64) / scale, -E4M3_MAX, E4M3_MAX)
    pos = np.array([b for b in range(0x7F)], dtype=np.uint8)          # 0x00..0x7E, all finite
    vals = E4M3FN[pos]                                                  # increasing
    a = np.abs(y).ravel()
    idx = np.searchsorted(vals, a)                                      # vals[idx-1] < a <= vals[idx]
    idx = np.clip(idx, 1, len(vals) - 1)
    lo, hi = vals[idx - 1], vals[idx]
    pick_hi = (a - lo) > (hi - a)
    tie = (a - lo) == (hi - a)
    pick_hi = pick_hi | (tie & ((idx % 2) == 0))                        # even code wins ties
    code = np.where(pick_hi, idx, idx - 1).astype(np.uint8)
    code = np.where(a == 0, 0, code).astype(np.uint8)
    sign = (np.signbit(y.ravel()) & (code != 0)).astype(np.uint8) << 7
    return (code | sign).reshape(np.shape(y)).astype(np.uint8)
