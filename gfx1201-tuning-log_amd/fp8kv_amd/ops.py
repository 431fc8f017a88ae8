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


def repack_scales(weight_scale: torch.Tensor) -> torch.Tensor:
    """Checkpoint scales [K/32, N] -> kernel layout [N, K/32] (h4mv/fp8kv_hipw4.py:32-43)."""
    return weight_scale.t().contiguous()


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
