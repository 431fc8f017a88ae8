"""GPU parity of the layer epilogues (csrc/epilogues.hip, h4mv_silu_mul) against the CPU oracle.

Bars: the new residual is bit-exact (an f32 add of two bf16 values, then one rounding); the
RMSNorm and SiLU-and-mul outputs are within one bf16 step of the oracle (the GPU's rsqrt / exp
and the order of the sum of squares differ from numpy's in the last f32 bit, which can move a
bf16 rounding by one step) with at least 99% bit-exact; the interleave is bit-exact; the fused
matvec epilogue equals the two-step path (matvec into bf16, then the SiLU-and-mul kernel) bit
for bit, and the oracle's fp64 matvec followed by SiLU-and-mul within the matvec bar.
"""
import numpy as np
import pytest
import torch

from fp8kv_amd import ops, workloads
from oracle import epilogues as ep, matvec

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _steps_apart(a: torch.Tensor, b: np.ndarray) -> np.ndarray:
    ia = a.cpu().view(torch.int16).numpy().astype(np.int64)
    ib = torch.from_numpy(np.asarray(b, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().astype(np.int64)
    return np.abs(ia - ib)


def _rows(M, H, seed, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, H, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("M,H", [(1, 3584), (8, 3584), (300, 4096), (5, 16384), (3, 8), (2, 5120), (7, 2056),
                                 (2048, 3584), (1537, 1032)])
def test_rmsnorm_parity(mode, M, H):
    """The output is rounded twice, bf16(bf16(z * r) * w), so a last-bit difference in r (rsqrt and
    the order of the sum of squares) that moves bf16(z * r) by one step can end two steps away;
    at millions of elements that happens a few times in a million."""
    x, res, w = _rows(M, H, 1), _rows(M, H, 2, 5.0), _rows(1, H, 3, 1.0)[0]
    xd, rd, wd = x.to(DEV), res.to(DEV), w.to(DEV)
    out = ops.fused_add_rmsnorm(xd, rd, wd, 1e-6, mode=mode)
    torch.cuda.synchronize()
    r_out, r_res = ep.fused_add_rmsnorm(x.float().numpy(), res.float().numpy(), w.float().numpy(), 1e-6, mode)
    assert np.array_equal(rd.cpu().float().numpy(), r_res)
    d = _steps_apart(out, r_out)
    assert d.max() <= 2 and (d > 1).mean() < 1e-4 and (d == 0).mean() >= 0.99, \
        (d.max(), (d > 1).mean(), (d == 0).mean())


def test_rmsnorm_strided_rows_in_place():
    """x as the first half of wider rows, the result written over x (vLLM's in-place form)."""
    M, H = 6, 1024
    big = _rows(M, 2 * H, 4)
    res, w = _rows(M, H, 5), _rows(1, H, 6, 1.0)[0]
    bd = big.to(DEV)
    xd = bd[:, :H]
    rd = res.to(DEV)
    ops.fused_add_rmsnorm(xd, rd, w.to(DEV), 1e-5, out=xd)
    torch.cuda.synchronize()
    r_out, r_res = ep.fused_add_rmsnorm(big[:, :H].float().numpy(), res.float().numpy(), w.float().numpy(), 1e-5)
    assert np.array_equal(rd.cpu().float().numpy(), r_res)
    assert _steps_apart(bd[:, :H].contiguous(), r_out).max() <= 1
    assert torch.equal(bd[:, H:].cpu(), big[:, H:])              # the other half untouched


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("M,d", [(8, 18944), (1, 8), (33, 1000)])
def test_silu_mul_parity(mode, M, d):
    gu = _rows(M, 2 * d, 7 + M)
    out = ops.silu_mul(gu.to(DEV), mode=mode)
    torch.cuda.synchronize()
    ref = ep.silu_mul(gu.float().numpy(), mode)
    dd = _steps_apart(out, ref)
    assert dd.max() <= 1 and (dd == 0).mean() >= 0.99


def test_silu_mul_strided_rows():
    M, d = 5, 256
    big = _rows(M, 3 * d, 8)
    out = torch.zeros(M, 2 * d, dtype=torch.bfloat16, device=DEV)
    ops.silu_mul(big.to(DEV)[:, d:], out=out[:, :d])
    torch.cuda.synchronize()
    ref = ep.silu_mul(big[:, d:].float().numpy())
    assert _steps_apart(out[:, :d].contiguous(), ref).max() <= 1
    assert torch.count_nonzero(out[:, d:]) == 0


def test_interleave_bit_exact():
    c = workloads.w4_case(128, 1024, 1, seed=9)
    wi, si = ops.interleave_gate_up(c["W"].to(DEV), c["St"].to(DEV))
    rw, rs = ep.interleave_gate_up(c["W"].numpy(), c["St"].numpy())
    assert np.array_equal(wi.cpu().numpy(), rw) and np.array_equal(si.cpu().numpy(), rs)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("N,K,M", [(512, 1024, 1), (512, 1024, 3), (1024, 2048, 8), (37888, 3584, 8), (37888, 3584, 1)])
def test_fused_silu_epilogue_equals_two_step(mode, N, K, M):
    c = workloads.w4_case(N, K, M, seed=N + M)
    W, St, X = c["W"].to(DEV), c["St"].to(DEV), c["X"].to(DEV)
    wi, si = ops.interleave_gate_up(W, St)
    fused = ops.h4mv_silu_mul(X, wi, si, mode=mode)
    two = ops.silu_mul(ops.h4mv(X, W, St), mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(fused, two)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("depth", [2, 3])
def test_fused_silu_epilogue_kslice(mode, depth):
    """The fused epilogue on the K-slice kernel forced through its tuning hook (one and several
    tiles per workgroup) equals the two-step path on the same kernel."""
    from fp8kv_amd import _lib
    lib = _lib.load()
    try:
        lib.fp8kv_h4mv_kslice_tune(1, depth, 0, 0)
        lib.fp8kv_h4mv_mx_tune(2, 0, 0)
        for N, K, M in ((512, 1024, 3), (8224, 2048, 8), (28672, 4096, 5), (28672, 4096, 3)):
            c = workloads.w4_case(N, K, M, seed=N + M + depth)
            W, St, X = c["W"].to(DEV), c["St"].to(DEV), c["X"].to(DEV)
            wi, si = ops.interleave_gate_up(W, St)
            fused = ops.h4mv_silu_mul(X, wi, si, mode=mode)
            two = ops.silu_mul(ops.h4mv(X, W, St), mode=mode)
            torch.cuda.synchronize()
            assert torch.equal(fused, two), (N, K, M)
    finally:
        lib.fp8kv_h4mv_kslice_tune(0, 0, 0, 0)
        lib.fp8kv_h4mv_mx_tune(0, 0, 0)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("depth", [2, 3])
def test_fused_silu_epilogue_mx(mode, depth):
    """The fused epilogue on the M = 2 .. 8 hi / lo kernel forced through its tuning hook equals
    the two-step path on the same kernel (one tile, several tiles per workgroup, cfg1's shape at
    two, four and eight activation rows)."""
    from fp8kv_amd import _lib
    lib = _lib.load()
    try:
        lib.fp8kv_h4mv_mx_tune(1, depth, 0)
        for N, K, M in ((16, 512, 2), (8224, 2048, 3), (28672, 4096, 4), (28672, 4096, 8), (37888, 3584, 7)):
            c = workloads.w4_case(N, K, M, seed=N + M + depth)
            W, St, X = c["W"].to(DEV), c["St"].to(DEV), c["X"].to(DEV)
            wi, si = ops.interleave_gate_up(W, St)
            fused = ops.h4mv_silu_mul(X, wi, si, mode=mode)
            two = ops.silu_mul(ops.h4mv(X, W, St), mode=mode)
            torch.cuda.synchronize()
            assert torch.equal(fused, two), (N, K, M)
    finally:
        lib.fp8kv_h4mv_mx_tune(0, 0, 0)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("depth", [2, 3])
def test_fused_silu_epilogue_m1(mode, depth):
    """The fused epilogue on the M = 1 kernel forced through its tuning hook equals the two-step
    path on the same kernel (one tile, several tiles per workgroup, cfg1's shape)."""
    from fp8kv_amd import _lib
    lib = _lib.load()
    try:
        lib.fp8kv_h4mv_m1_tune(1, depth, 0)
        for N, K in ((16, 512), (8224, 2048), (28672, 4096)):
            c = workloads.w4_case(N, K, 1, seed=N + depth)
            W, St, X = c["W"].to(DEV), c["St"].to(DEV), c["X"].to(DEV)
            wi, si = ops.interleave_gate_up(W, St)
            fused = ops.h4mv_silu_mul(X, wi, si, mode=mode)
            two = ops.silu_mul(ops.h4mv(X, W, St), mode=mode)
            torch.cuda.synchronize()
            assert torch.equal(fused, two), (N, K)
    finally:
        lib.fp8kv_h4mv_m1_tune(0, 0, 0)


def test_fused_silu_epilogue_vs_oracle():
    N, K, M = 1024, 2048, 4
    c = workloads.w4_case(N, K, M, seed=11)
    wi, si = ops.interleave_gate_up(c["W"].to(DEV), c["St"].to(DEV))
    got = ops.h4mv_silu_mul(c["X"].to(DEV), wi, si).float().cpu().numpy()
    y = matvec.w4mv(c["W"].numpy(), c["St"].numpy(), c["X"].float().numpy())
    ref = ep.silu_mul(ep.bf16_round(y.astype(np.float32)))
    assert matvec.rel_to_max_error(got, ref) < 1e-2
