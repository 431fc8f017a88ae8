"""GPU parity of the MXFP8 quantiser (h4a8_quant_act) and the MXFP4 x MXFP8 GEMM (h4a8_gemm).

The per-token fp8 path (h4a8_quant_act_token, h4a8_gemm_token) meets the same bars: codes and
fp32 scales bit-exact, the GEMM on the same operands within the bf16 bar, end to end within 5e-2.

Bars: quantiser codes and scale bytes bit-exact against the oracle; GEMM output (on the same
quantised operands) within half a bf16 ulp of the fp64 oracle plus 1e-4 * max|ref| (fp32
accumulation inside the MFMA, the matvec's bf16 bar); end to end (bf16 x through the quantiser
and the GEMM) against the unquantised W4A16 product, the error MXFP8 activations cost, < 5e-2
relative to the largest output.
"""
import numpy as np
import pytest
import torch

from fp8kv_amd import _lib, ops, workloads
from oracle import matvec, w4a8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _x(M, K, seed, spread=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if spread:
        x = x * torch.exp(torch.empty(M, K // 32, 1).uniform_(-spread, spread, generator=g)).expand(M, K // 32, 32).reshape(M, K)
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("M,K,spread", [(1, 32, 0), (16, 512, 0), (300, 3584, 20.0), (7, 18944, 5.0)])
def test_quant_bit_exact(M, K, spread):
    x = _x(M, K, M + K, spread)
    xq, sx = ops.quant_mxfp8(x.to(DEV))
    torch.cuda.synchronize()
    rc, rs = w4a8.quant_mxfp8(x.float().numpy())
    assert np.array_equal(sx.cpu().numpy(), rs)
    assert np.array_equal(xq.cpu().numpy(), rc)


def test_quant_special_blocks():
    x = torch.zeros(2, 128)
    x[0, 40] = float("inf")
    x[0, 70] = 2.0 ** -130
    x[1, 0:32] = torch.linspace(-1000, 1000, 32)
    x[1, 96] = float("nan")
    x = x.to(torch.bfloat16)
    xq, sx = ops.quant_mxfp8(x.to(DEV))
    rc, rs = w4a8.quant_mxfp8(x.float().numpy())
    assert np.array_equal(sx.cpu().numpy(), rs)
    finite = np.repeat(rs != 255, 32, axis=1)
    assert np.array_equal(xq.cpu().numpy()[finite], rc[finite])


def _gemm_case(N, K, M, seed):
    c = workloads.w4_case(N, K, M, seed=seed)
    rc, rs = w4a8.quant_mxfp8(c["X"].float().numpy())
    return c, rc, rs


@pytest.mark.parametrize("variant,order", [(-1, 0), (0, 0), (0, 1), (1, 0), (2, 0), (3, 1), (4, 0), (5, 1), (6, 0), (6, 1), (7, 0), (8, 0)])
@pytest.mark.parametrize("N,K,M", [(256, 512, 16), (200, 1024, 37), (4096, 3584, 300), (512, 18944, 64),
                                   (128, 128, 1), (1024, 3072, 129), (384, 256, 200), (128, 384, 64)])
def test_gemm_parity(N, K, M, variant, order):
    lib = _lib.load()
    c, rc, rs = _gemm_case(N, K, M, seed=N + M)
    try:
        lib.fp8kv_gemm_tune(variant, order)
        out = ops.h4a8_gemm(torch.from_numpy(rc).to(DEV), torch.from_numpy(rs).to(DEV), c["W"].to(DEV), c["St"].to(DEV))
        torch.cuda.synchronize()
    finally:
        lib.fp8kv_gemm_tune(-1, 0)
    ref = w4a8.gemm(c["W"].numpy(), c["St"].numpy(), rc, rs)
    got = out.float().cpu().numpy()
    assert matvec.bf16_excess_error(got, ref) < 1e-4


@pytest.mark.parametrize("variant", [-1, 5, 6, 8])
def test_gemm_scales_only_4_byte_aligned(variant):
    """Scale operands that start 4 bytes past a 16-byte boundary (the entry point requires 4): the
    kernels that copy four steps' scales per lane at once (K % 512 == 0) must fall back to per-step
    copies and still meet the bar."""
    N, K, M = 512, 3584, 200
    lib = _lib.load()
    c, rc, rs = _gemm_case(N, K, M, seed=77)

    def offset_view(a):
        buf = torch.zeros(a.size + 16, dtype=torch.uint8, device=DEV)
        v = buf[4:4 + a.size].view(a.shape)
        v.copy_(torch.from_numpy(np.ascontiguousarray(a)).to(DEV))
        assert v.data_ptr() % 16 == 4
        return v

    try:
        lib.fp8kv_gemm_tune(variant, 0)
        out = ops.h4a8_gemm(torch.from_numpy(rc).to(DEV), offset_view(rs), c["W"].to(DEV), offset_view(c["St"].numpy()))
        torch.cuda.synchronize()
    finally:
        lib.fp8kv_gemm_tune(-1, 0)
    ref = w4a8.gemm(c["W"].numpy(), c["St"].numpy(), rc, rs)
    assert matvec.bf16_excess_error(out.float().cpu().numpy(), ref) < 1e-4


@pytest.mark.parametrize("variant,act", [(-1, "mx"), (5, "mx"), (6, "mx"), (8, "mx"), (2, "mx"), (5, "token"),
                                         (6, "token")])
def test_gemm_repeats_bitwise(variant, act):
    """Ten calls on the same operands give the same bits (the ring's waits are counted by hand: a
    wait that retired early would read a copy still in flight), at a shape with many tiles per
    XCD and K % 512 == 0 (grouped scale copies), and meet the oracle bar."""
    N, K, M = 2048, 3584, 512
    lib = _lib.load()
    if act == "token":
        c, rc, rs = _token_case(N, K, M, seed=91)
        xs = torch.from_numpy(rs).to(DEV)
        run = lambda: ops.h4a8_gemm_token(xq, xs, w, st)            # noqa: E731
        ref = w4a8.gemm_token(c["W"].numpy(), c["St"].numpy(), rc, rs)
    else:
        c, rc, rs = _gemm_case(N, K, M, seed=91)
        xs = torch.from_numpy(rs).to(DEV)
        run = lambda: ops.h4a8_gemm(xq, xs, w, st)                  # noqa: E731
        ref = w4a8.gemm(c["W"].numpy(), c["St"].numpy(), rc, rs)
    xq, w, st = torch.from_numpy(rc).to(DEV), c["W"].to(DEV), c["St"].to(DEV)
    try:
        lib.fp8kv_gemm_tune(variant, 0)
        outs = [run().clone() for _ in range(10)]
        torch.cuda.synchronize()
    finally:
        lib.fp8kv_gemm_tune(-1, 0)
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert matvec.bf16_excess_error(outs[0].float().cpu().numpy(), ref) < 1e-4


def _random_shapes(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        K = 128 * int(rng.integers(1, 48))                 # half of them K % 512 == 0 on average
        if rng.random() < 0.5:
            K = 512 * max(1, K // 512)
        N = 4 * int(rng.integers(1, 1200))
        M = int(rng.integers(1, 700))
        out.append((N, K, M))
    return out


@pytest.mark.parametrize("N,K,M", _random_shapes(12, 2026))
@pytest.mark.parametrize("act", ["mx", "token"])
def test_gemm_random_shapes(N, K, M, act):
    """Seeded random shapes through the default planner (every tile size, ring, XCD split and the
    grouped scale copies where K % 512 == 0), against the oracle."""
    if act == "token":
        c, rc, rs = _token_case(N, K, M, seed=N + K + M)
        out = ops.h4a8_gemm_token(torch.from_numpy(rc).to(DEV), torch.from_numpy(rs).to(DEV), c["W"].to(DEV),
                                  c["St"].to(DEV))
        ref = w4a8.gemm_token(c["W"].numpy(), c["St"].numpy(), rc, rs)
    else:
        c, rc, rs = _gemm_case(N, K, M, seed=N + K + M)
        out = ops.h4a8_gemm(torch.from_numpy(rc).to(DEV), torch.from_numpy(rs).to(DEV), c["W"].to(DEV),
                            c["St"].to(DEV))
        ref = w4a8.gemm(c["W"].numpy(), c["St"].numpy(), rc, rs)
    torch.cuda.synchronize()
    assert matvec.bf16_excess_error(out.float().cpu().numpy(), ref) < 1e-4


def test_end_to_end_against_w4a16_product():
    N, K, M = 1024, 3584, 64
    c = workloads.w4_case(N, K, M, seed=21)
    got = ops.mxfp4_linear(c["X"].to(DEV), c["W"].to(DEV), c["St"].to(DEV)).float().cpu().numpy()
    ref = matvec.w4mv(c["W"].numpy(), c["St"].numpy(), c["X"].float().numpy())
    assert matvec.rel_to_max_error(got, ref) < 5e-2


def test_nan_scale_block_gives_nan_rows():
    N, K, M = 128, 256, 16
    c = workloads.w4_case(N, K, M, seed=22)
    x = c["X"].clone()
    x[3, 100] = float("inf")
    got = ops.mxfp4_linear(x.to(DEV), c["W"].to(DEV), c["St"].to(DEV)).float().cpu()
    assert torch.isnan(got[3]).all()
    assert torch.isfinite(torch.cat([got[:3], got[4:]])).all()


@pytest.mark.parametrize("act", ["token", "mx"])
def test_linear_hook_gemm_path_matches_ops(act):
    """The opt-in large-batch path of the MXFP4 linear hook (ctypes into the quantiser and the
    GEMM of either activation format, scales repacked on the device) gives the same bits as
    ops.mxfp4_linear."""
    import fp8kv_hipw4 as h
    N, K, M = 512, 1024, 40
    c = workloads.w4_case(N, K, M, seed=23)
    x, w, s_kn = c["X"].to(DEV), c["W"].to(DEV), c["S_kn"].to(DEV)
    repack = h.ScaleRepack(lambda: False)
    patched = h.make_patched(lambda *a: None, h.load_launcher(), repack, 8, torch,
                             lambda: torch.cuda.current_stream().cuda_stream, gemm=h.load_gemm(act=act))
    got = patched(x, w, s_kn, None)
    want = ops.mxfp4_linear(x, w, c["St"].to(DEV), act=act)
    torch.cuda.synchronize()
    assert got is not None and torch.equal(got, want)


# ---- per-token fp8 activations -----------------------------------------------------------------

@pytest.mark.parametrize("M,K,spread", [(1, 8, 0), (16, 512, 0), (300, 3584, 20.0), (7, 18944, 5.0), (33, 2056, 40.0),
                                         (5, 8192, 3.0), (3, 16384, 0), (2, 32768, 1.0), (3, 40000, 2.0)])
def test_token_quant_bit_exact(M, K, spread):
    """Row lengths for every register-resident variant (2048 R elements, R = 1, 2, 4, 8, 12, 16)
    and the two-pass fallback above 32768."""
    g = torch.Generator().manual_seed(M * 7 + K)
    x = torch.randn(M, K, generator=g)
    if spread:
        x = x * torch.exp(torch.empty(M, 1).uniform_(-spread, spread, generator=g))
    x = x.to(torch.bfloat16)
    xq, sc = ops.quant_fp8_per_token(x.to(DEV))
    torch.cuda.synchronize()
    rc, rs = w4a8.quant_fp8_per_token(x.float().numpy())
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(xq.cpu().numpy(), rc)


def test_token_quant_special_rows():
    """All-zero and tiny rows (scale floor), a NaN element, an infinite element, a strided input."""
    x = torch.ones(6, 256)
    x[0] = 0
    x[1] = 1e-7
    x[2, 17] = float("nan")
    x[3, 200] = float("inf")
    x[4, 9] = -float("inf")
    x[5] = torch.linspace(-3000, 3000, 256)
    xb = x.to(torch.bfloat16)
    big = torch.zeros(6, 264, dtype=torch.bfloat16)
    big[:, :256] = xb
    xq, sc = ops.quant_fp8_per_token(big.to(DEV)[:, :256])
    torch.cuda.synchronize()
    rc, rs = w4a8.quant_fp8_per_token(xb.float().numpy())
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(xq.cpu().numpy(), rc)


def _token_case(N, K, M, seed):
    c = workloads.w4_case(N, K, M, seed=seed)
    rc, rs = w4a8.quant_fp8_per_token(c["X"].float().numpy())
    return c, rc, rs


@pytest.mark.parametrize("variant,order", [(-1, 0), (5, 0), (5, 1), (6, 0), (6, 1), (2, 0)])
@pytest.mark.parametrize("N,K,M", [(256, 512, 16), (200, 1024, 37), (4096, 3584, 300), (512, 18944, 64),
                                   (128, 128, 1), (1024, 3072, 129), (384, 256, 200)])
def test_token_gemm_parity(N, K, M, variant, order):
    """Forced variants outside the per-token set (2) fall back to the default choice."""
    lib = _lib.load()
    c, rc, rs = _token_case(N, K, M, seed=N + 3 * M)
    try:
        lib.fp8kv_gemm_tune(variant, order)
        out = ops.h4a8_gemm_token(torch.from_numpy(rc).to(DEV), torch.from_numpy(rs).to(DEV), c["W"].to(DEV),
                                  c["St"].to(DEV))
        torch.cuda.synchronize()
    finally:
        lib.fp8kv_gemm_tune(-1, 0)
    ref = w4a8.gemm_token(c["W"].numpy(), c["St"].numpy(), rc, rs)
    got = out.float().cpu().numpy()
    assert matvec.bf16_excess_error(got, ref) < 1e-4


def test_token_end_to_end_against_w4a16_product():
    N, K, M = 1024, 3584, 64
    c = workloads.w4_case(N, K, M, seed=31)
    got = ops.mxfp4_linear(c["X"].to(DEV), c["W"].to(DEV), c["St"].to(DEV), act="token").float().cpu().numpy()
    ref = matvec.w4mv(c["W"].numpy(), c["St"].numpy(), c["X"].float().numpy())
    assert matvec.rel_to_max_error(got, ref) < 5e-2
