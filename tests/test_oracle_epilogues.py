"""Pins for the layer-epilogue oracle (CPU only): RMSNorm with residual add, SiLU-and-mul, and
the gate/up row interleave, checked against torch CPU library routines, closed forms and the
row map; the ``planted_*`` tests plant a plausible mistake in the oracle and show a check fails."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import epilogues as ep

ALL_BF16 = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def _bf(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16)


def _ulps_apart(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 steps between two arrays of bf16 values (same sign assumed near zero)."""
    ia = torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().astype(np.int64)
    ib = torch.from_numpy(np.asarray(b, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().astype(np.int64)
    return np.abs(ia - ib)


def test_bf16_round_matches_torch_everywhere():
    base = ALL_BF16.float().numpy()
    fin = np.isfinite(base)
    # every bf16 value, the midpoints above it, and points just either side of the midpoints
    bits = base[fin].view(np.uint32)
    cands = np.concatenate([bits, bits + 0x8000, bits + 0x7FFF, bits + 0x8001, bits + 0x1234]).astype(np.uint32)
    x = cands.view(np.float32)
    ours = ep.bf16_round(x)
    lib = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    same = (ours == lib) | (np.isnan(ours) & np.isnan(lib))
    assert same.all()


def _torch_rmsnorm(x, res, w, eps, mode):
    xb, rb, wb = _bf(x), _bf(res), _bf(w)
    if mode == 0:
        z = xb.float() + rb.float()
        new_res = z.to(torch.bfloat16)
    else:
        new_res = (xb + rb)                                   # bf16 add: f32 sum rounded once
        z = new_res.float()
    var = z.double().pow(2).mean(-1, keepdim=True).float()
    y = (z * torch.rsqrt(var + eps)).to(torch.bfloat16)
    out = y * wb                                              # bf16 x bf16: f32 product rounded
    return out.float().numpy(), new_res.float().numpy()


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("H", [8, 256, 3584, 5120])
def test_rmsnorm_matches_torch_pipeline(mode, H):
    rng = np.random.default_rng(H + mode)
    M = 17
    x = ep.bf16_round(rng.standard_normal((M, H)).astype(np.float32) * 3)
    res = ep.bf16_round(rng.standard_normal((M, H)).astype(np.float32) * 5)
    w = ep.bf16_round(rng.standard_normal(H).astype(np.float32))
    out, new_res = ep.fused_add_rmsnorm(x, res, w, 1e-6, mode)
    t_out, t_res = _torch_rmsnorm(x, res, w, 1e-6, mode)
    assert np.array_equal(new_res, t_res)
    d = _ulps_apart(out, t_out)
    assert d.max() <= 1 and (d == 0).mean() > 0.99


def test_rmsnorm_constant_rows_closed_form():
    """eps = 0, a row of one power of two c: z * rsqrt(mean z^2) = sign(c) exactly, out = sign(c) w."""
    H = 64
    w = ep.bf16_round(np.linspace(-3, 3, H).astype(np.float32))
    for c in (2.0 ** -20, 0.25, 1.0, -8.0, 2.0 ** 30):
        x = np.full((1, H), c, np.float32)
        res = np.zeros((1, H), np.float32)
        for mode in (0, 1):
            out, new_res = ep.fused_add_rmsnorm(x, res, w, 0.0, mode)
            assert np.array_equal(new_res[0], x[0])
            assert np.array_equal(out[0], np.sign(c) * w)


@pytest.mark.parametrize("mode", [0, 1])
def test_silu_mul_matches_torch(mode):
    g = ALL_BF16.float()
    fin = torch.isfinite(g)
    g = g[fin][::3][:16000].reshape(1, -1)
    u = torch.from_numpy(np.random.default_rng(3).standard_normal(g.shape).astype(np.float32)).to(torch.bfloat16).float()
    gu = torch.cat([g, u], 1).numpy()
    ours = ep.silu_mul(gu, mode)
    gb, ub = g.to(torch.bfloat16), u.to(torch.bfloat16)
    if mode == 0:
        lib = (F.silu(gb.float()) * ub.float()).to(torch.bfloat16).float().numpy()
    else:
        lib = (F.silu(gb) * ub).float().numpy()               # bf16 SiLU, then bf16 x bf16
    d = _ulps_apart(ours, lib)
    assert d.max() <= 1 and (d == 0).mean() > 0.999


def test_silu_special_values():
    s = ep.silu_f32(np.array([0.0, 100.0, -100.0, -1e30, 1e30], np.float32))
    assert s[0] == 0.0 and s[1] == 100.0 and s[2] == 0.0 and np.signbit(s[2]) and s[4] == 1e30
    assert s[3] == 0.0


def test_interleave_row_map():
    N = 64
    src = ep.interleave_rows(N)
    for R in range(N):
        T, i = divmod(R, 16)
        want = 8 * T + i if i < 8 else N // 2 + 8 * T + i - 8
        assert src[R] == want
    assert sorted(src.tolist()) == list(range(N))            # a permutation
    W = np.arange(N * 4, dtype=np.uint8).reshape(N, 4)
    S = np.arange(N, dtype=np.uint8).reshape(N, 1)
    Wi, Si = ep.interleave_gate_up(W, S)
    inv = np.argsort(src)
    assert np.array_equal(Wi[inv], W) and np.array_equal(Si[inv], S)


def test_planted_mean_over_h_minus_1_fails_closed_form(monkeypatch):
    def bad(x, residual, weight, eps, mode=0):
        z = (np.asarray(x, np.float32) + np.asarray(residual, np.float32))
        H = z.shape[-1]
        var = (np.sum(z.astype(np.float64) ** 2, -1, keepdims=True) / (H - 1)).astype(np.float32)
        y = ep.bf16_round(z / np.sqrt(var + eps))
        return ep.bf16_round(y * weight), ep.bf16_round(z)
    monkeypatch.setattr(ep, "fused_add_rmsnorm", bad)
    w = np.ones(64, np.float32)
    out, _ = ep.fused_add_rmsnorm(np.full((1, 64), 0.25, np.float32), np.zeros((1, 64), np.float32), w, 0.0)
    assert not np.array_equal(out[0], w)


def test_planted_swapped_halves_fails_torch_check():
    rng = np.random.default_rng(5)
    gu = ep.bf16_round(rng.standard_normal((2, 64)).astype(np.float32))
    swapped = np.concatenate([gu[:, 32:], gu[:, :32]], 1)
    lib = (F.silu(_bf(gu[:, :32]).float()) * _bf(gu[:, 32:]).float()).to(torch.bfloat16).float().numpy()
    assert not np.array_equal(ep.silu_mul(swapped), lib)
    assert np.array_equal(_ulps_apart(ep.silu_mul(gu), lib).max() <= 1, True)
