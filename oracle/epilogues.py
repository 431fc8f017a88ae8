"""Layer epilogues around the MXFP4 linears, restated on the CPU (numpy, float32 steps).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference engine runs these as compiler-fused kernels of its vLLM model code, listed in its
profiles: profiling/prof_engine.txt:13,15 (triton_red_fused_fused_add_rms_norm_*: residual add +
RMSNorm ahead of the qkv and gate/up linears) and :17 (triton_poi_fused_mul_..._silu_slice:
SiLU(gate) * up between gate/up and down); also profiling/prof_h4mv.txt:11,13,15.  vLLM (the
0.28 fork pinned only by the image tag in serve-fp8kv-best.sh) is absent here, so the arithmetic
is restated from vLLM's published RMSNorm / SiluAndMul in two forms (``mode``):

  mode 0 - the compiled native form (RMSNorm.forward_static / SiluAndMul.forward_native traced
           by the compiler, the kernels the profiles list):
      z = f32(x) + f32(res); res' = bf16(z); var = mean(z^2); y = bf16(z * rsqrt(var + eps));
      out = bf16(f32(y) * f32(w));   silu_mul: out = bf16(silu(f32(g)) * f32(u))
  mode 1 - vLLM's custom ops (_C.fused_add_rms_norm, _C.silu_and_mul):
      z = bf16(f32(x) + f32(res)) used for var and y;  silu_mul: out = bf16(f32(bf16(silu(g))) * f32(u))

Parity at the vLLM boundary itself is unpinned (vLLM absent).  Pins (tests/test_oracle_epilogues.py):
  * ``bf16_round`` - against torch's float32 -> bfloat16 conversion on every bf16 neighbourhood
    (a library routine) including ties, infinities and NaN;
  * ``fused_add_rmsnorm`` - against the same steps written with torch CPU library routines
    (torch.rsqrt, .to(torch.bfloat16)), and against the closed form for constant rows
    (eps = 0: y = sign(c) exactly, out = sign(c) * w);
  * ``silu_mul`` - against torch.nn.functional.silu on the CPU in both rounding forms, and the
    special values silu(0) = 0, silu(+big) = big, silu(-big) = -0;
  * ``interleave_gate_up`` - against its row map written out per row, and as a permutation (the
    inverse map restores the input);
  * planted mistakes (mean over H - 1, residual not added, gate/up halves swapped) failing the above.
"""
from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value (ties to even), returned as float32; NaN stays NaN."""
    x = np.asarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def fused_add_rmsnorm(x: np.ndarray, residual: np.ndarray, weight: np.ndarray, eps: float,
                      mode: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """x, residual [M, H] and weight [H] (bf16 values as float32) -> (out, new_residual), float32
    arrays holding bf16 values."""
    x = np.asarray(x, dtype=np.float32)
    res = np.asarray(residual, dtype=np.float32)
    w = np.asarray(weight, dtype=np.float32)
    z = (x + res).astype(np.float32)
    new_res = bf16_round(z)
    if mode == 1:
        z = new_res
    H = z.shape[-1]
    ss = np.sum(z.astype(np.float64) ** 2, axis=-1, keepdims=True)
    var = (ss / H).astype(np.float32)
    r = (1.0 / np.sqrt((var + np.float32(eps)).astype(np.float64))).astype(np.float32)
    y = bf16_round((z * r).astype(np.float32))
    out = bf16_round((y * w).astype(np.float32))
    return out, new_res


def silu_f32(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def silu_mul(gate_up: np.ndarray, mode: int = 0) -> np.ndarray:
    """gate_up [M, 2d] (bf16 values as float32) -> [M, d] float32 holding bf16 values."""
    gu = np.asarray(gate_up, dtype=np.float32)
    d = gu.shape[-1] // 2
    s = silu_f32(gu[..., :d])
    if mode == 1:
        s = bf16_round(s)
    with np.errstate(over="ignore", invalid="ignore"):
        return bf16_round((s * gu[..., d:]).astype(np.float32))


def interleave_rows(N: int) -> np.ndarray:
    """Source row of each interleaved row: row 16 T + i <- gate row 8 T + i (i < 8) or up row
    N/2 + 8 T + i - 8 (i >= 8)."""
    R = np.arange(N)
    T, i = R // 16, R % 16
    return np.where(i < 8, 8 * T + i, N // 2 + 8 * T + (i - 8))


def interleave_gate_up(W: np.ndarray, St: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    src = interleave_rows(W.shape[0])
    return np.ascontiguousarray(W[src]), np.ascontiguousarray(St[src])
