"""Pins for the MXFP8 quantiser and the MXFP4 x MXFP8 GEMM oracle (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import formats, matvec, w4a8
from fp8kv_amd import workloads


def _bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def test_quant_matches_torch_cast_per_block():
    """codes = torch's float8_e4m3fn cast of x / 2^(byte - 127) wherever torch does not overflow
    to NaN (|q| >= 464, which the OCP rule saturates to 448)."""
    rng = np.random.default_rng(0)
    x = _bf16(rng.standard_normal((64, 256)) * np.exp(rng.uniform(-20, 20, (64, 1))))
    codes, sb = w4a8.quant_mxfp8(x)
    q = x.reshape(64, 8, 32) / np.ldexp(1.0, sb.astype(np.int64) - 127)[..., None]
    lib = torch.from_numpy(q.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy().reshape(64, 256)
    ok = (lib & 0x7F) != 0x7F
    assert ok.mean() > 0.95
    assert np.array_equal(codes[ok], lib[ok])
    assert np.all(codes[~ok] & 0x7F == 0x7E)                     # saturated to +-448


def test_block_max_lands_in_top_binade():
    rng = np.random.default_rng(1)
    x = _bf16(rng.standard_normal((32, 512)) * 1e-3)
    codes, sb = w4a8.quant_mxfp8(x)
    v = np.abs(formats.E4M3FN[codes].reshape(32, 16, 32)).max(-1)
    assert np.all((v >= 256) & (v <= 448))                       # 2^8 <= max|q| < 2^9, saturating at 448


def test_representable_blocks_round_trip():
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 256, (8, 128), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x40
    codes[:, ::32] = 0x78                                        # every block holds 256 (e4m3 exponent 8)
    e = rng.integers(-30, 30, (8, 4))
    x = (formats.E4M3FN[codes].reshape(8, 4, 32) * np.ldexp(1.0, e)[..., None]).reshape(8, 128).astype(np.float32)
    c2, sb = w4a8.quant_mxfp8(x)
    assert np.array_equal(w4a8.dequant_mxfp8(c2, sb), x.astype(np.float64))
    assert np.array_equal(sb.astype(np.int64) - 127, e)


def test_special_blocks():
    x = np.zeros((1, 96), np.float32)
    x[0, 40] = np.inf
    x[0, 70] = 2.0 ** -130                                      # tiny: the scale clamps to 2^-127
    x[0, 71] = 2.0 ** -140                                      # below the clamped scale's range: 0
    c, sb = w4a8.quant_mxfp8(x)
    assert sb[0, 0] == 0 and np.all(c[0, :32] == 0)             # all-zero block
    assert sb[0, 1] == 255                                      # non-finite -> NaN scale
    d = w4a8.dequant_mxfp8(c, sb)
    assert sb[0, 2] == 0 and d[0, 70] == 2.0 ** -130 and d[0, 71] == 0.0


def test_gemm_exact_integer_case():
    """Integer-valued operands with unit scales: every product and sum is exact."""
    rng = np.random.default_rng(3)
    N, K, M = 16, 256, 8
    wc = rng.integers(0, 16, (N, K))
    W = formats.pack_e2m1(wc.astype(np.uint8))
    St = np.full((N, K // 32), 127, np.uint8)
    xi = rng.integers(-8, 9, (M, K)).astype(np.float32)
    codes = np.array([[int(np.nonzero(formats.E4M3FN == v)[0][0]) for v in row] for row in xi], np.uint8)
    sb = np.full((M, K // 32), 127, np.uint8)
    got = w4a8.gemm(W, St, codes, sb)
    want = xi.astype(np.int64) @ (formats.E2M1[wc] * 2).astype(np.int64).T
    assert np.array_equal(got * 2, want.astype(np.float64))


def test_gemm_equals_matvec_oracle_on_dequantised_activations():
    c = workloads.w4_case(64, 512, 5, seed=4)
    W, St = c["W"].numpy(), c["St"].numpy()
    codes, sb = w4a8.quant_mxfp8(c["X"].float().numpy())
    a = w4a8.gemm(W, St, codes, sb)
    b = matvec.w4mv(W, St, w4a8.dequant_mxfp8(codes, sb))
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_planted_exponent_off_by_one_fails_top_binade(monkeypatch):
    real = w4a8.quant_mxfp8

    def bad(x):
        c, sb = real(x)
        return c, (sb + 1).astype(np.uint8)
    rng = np.random.default_rng(5)
    x = _bf16(rng.standard_normal((4, 64)))
    c, sb = bad(x)
    q = np.abs(x.reshape(4, 2, 32) / np.ldexp(1.0, sb.astype(np.int64) - 127)[..., None]).max(-1)
    assert not np.all((q >= 256) & (q <= 512))


# ---- per-token fp8 (vLLM's dynamic_per_token_scaled_fp8_quant) --------------------------------

def test_token_codes_match_torch_cast():
    """codes = torch's float8_e4m3fn cast (a library routine, round to nearest even) of
    x / scale, the quotient rounded to fp32 first."""
    rng = np.random.default_rng(10)
    x = _bf16(rng.standard_normal((48, 512)) * np.exp(rng.uniform(-30, 30, (48, 1))))
    codes, sc = w4a8.quant_fp8_per_token(x)
    q = (x / sc[:, None]).astype(np.float32)
    lib = torch.from_numpy(q).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes, lib)


def test_token_scale_and_row_max():
    """scale = amax / 448 (fp32) for rows above the floor, and each row's largest element lands on
    +-448 (code 0x7E / 0xFE); rows below the floor take 1 / (448 * 512)."""
    rng = np.random.default_rng(11)
    x = _bf16(rng.standard_normal((64, 300)) * np.exp(rng.uniform(-10, 10, (64, 1))))
    codes, sc = w4a8.quant_fp8_per_token(x)
    amax = np.abs(x).max(axis=1)
    floor = np.float32(1) / np.float32(229376)
    above = (amax / np.float32(448)).astype(np.float32) > floor
    assert 16 < above.sum() < 64
    assert np.array_equal(sc[above], (amax[above] / np.float32(448)).astype(np.float32))
    assert np.all(sc[~above] == floor)
    at = np.abs(x).argmax(axis=1)
    assert np.all(codes[np.arange(64), at][above] & 0x7F == 0x7E)
    tiny = np.full((2, 64), 1e-7, np.float32)
    tiny[1] = 0
    tc, ts = w4a8.quant_fp8_per_token(_bf16(tiny))
    assert np.all(ts == floor)
    assert np.all(tc[1] == 0)
    assert np.all(formats.E4M3FN[tc[0]] * floor <= 1.07e-7)


def test_token_dequant_error_bound():
    """|x - e4m3(code) * scale| <= 2^-4 |x| in e4m3's normal range (3 mantissa bits, round to
    nearest) and <= 2^-10 scale below it."""
    rng = np.random.default_rng(12)
    x = _bf16(rng.standard_normal((32, 1024)) * 3.0)
    codes, sc = w4a8.quant_fp8_per_token(x)
    dq = formats.E4M3FN[codes] * sc[:, None].astype(np.float64)
    err = np.abs(dq - x)
    normal = np.abs(x) / sc[:, None] >= 2.0 ** -6
    assert np.all(err[normal] <= 2.0 ** -4 * np.abs(x[normal]) * (1 + 1e-6))
    assert np.all(err[~normal] <= 2.0 ** -10 * np.broadcast_to(sc[:, None], x.shape)[~normal] * (1 + 1e-6))


def test_token_nonfinite_rows():
    """fmaxf / fminf semantics: a NaN element is skipped by the maximum and clamps to +448; an
    infinite element makes the scale infinite, every finite element 0 and the infinite ones
    +448 (inf / inf is NaN)."""
    x = np.ones((2, 16), np.float32)
    x[0, 3] = np.nan
    x[1, 5] = np.inf
    codes, sc = w4a8.quant_fp8_per_token(x)
    assert sc[0] == np.float32(1) / np.float32(448)
    assert codes[0, 3] == 0x7E and np.all(np.delete(codes[0], 3) == 0x7E)
    assert np.isinf(sc[1]) and codes[1, 5] == 0x7E and np.all(np.delete(codes[1], 5) == 0)


def test_token_gemm_exact_integer_case():
    """Integer-valued e4m3 activations and e2m1 weights with unit weight scales: the product is an
    exact integer matrix (numpy int64), times the row scale."""
    rng = np.random.default_rng(13)
    M, N, K = 5, 24, 256
    ints = np.array([0x38, 0x40, 0x44, 0x48, 0xB8, 0xC0, 0x00])       # 1, 2, 3, 4, -1, -2, 0
    codes = rng.choice(ints, (M, K)).astype(np.uint8)
    W = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    St = np.full((N, K // 32), 127, np.uint8)
    sc = np.array([1.0, 2.0, 0.5, 0.125, 3.0], np.float32)
    xi = formats.E4M3FN[codes].astype(np.int64)
    w2 = (matvec.dequant_w4(W, St) * 2).astype(np.int64)             # e2m1 values times 2 are integers
    want = (xi @ w2.T).astype(np.float64) / 2 * sc[:, None]
    assert np.array_equal(w4a8.gemm_token(W, St, codes, sc), want)


def test_planted_fp8_max_240_fails_row_max(monkeypatch):
    """The fnuz bound (240) in place of e4m3fn's 448 moves the row maximum off code 0x7E."""
    rng = np.random.default_rng(14)
    x = _bf16(rng.standard_normal((8, 64)))
    monkeypatch.setattr(w4a8, "FP8_MAX", np.float32(240.0))
    codes, _ = w4a8.quant_fp8_per_token(x)
    at = np.abs(x).argmax(axis=1)
    assert not np.all(codes[np.arange(8), at] & 0x7F == 0x7E)
