"""Pins for the fp8 KV-cache write oracle (CPU only).

The encoder is checked against torch's float8_e4m3fn cast (a library conversion), against the
e4m3fn table (round trip and midpoints), against brute-force nearest-value search, and against the
saturation rules of vLLM's SATFINITE conversion; the scatter against its addressing identities.
The ``planted_*`` tests plant a plausible mistake in the oracle and show that a check catches it.
"""
import numpy as np
import pytest
import torch

from oracle import formats, kv_cache

ALL_BF16 = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
SCALES = [1.0, 0.5, 0.0123, 3.7, 2.0 ** -7]


def _torch_cast(y32: torch.Tensor) -> np.ndarray:
    return y32.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


@pytest.mark.parametrize("scale", SCALES)
def test_encoder_matches_torch_cast_where_torch_is_finite(scale):
    """torch's cast rounds to nearest even but turns finite overflow (|y| >= 464) into NaN; on every
    other bf16 quotient the two agree bit for bit (signed zeros included)."""
    y = (ALL_BF16.float() / torch.tensor(scale, dtype=torch.float32))
    ours = kv_cache.encode_e4m3fn_satfinite(y.numpy())
    lib = _torch_cast(y)
    lib_nan = (lib & 0x7F) == 0x7F
    in_nan = torch.isnan(y).numpy()
    keep = ~lib_nan & ~in_nan
    assert keep.sum() > 30000                       # the whole e4m3 range and everything below it
    assert np.array_equal(ours[keep], lib[keep])
    # NaN inputs: NaN code with the input's sign, as torch gives.
    assert np.array_equal(ours[in_nan], lib[in_nan])


def test_encoder_round_trips_every_finite_code():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    vals = formats.E4M3FN[codes].astype(np.float32)
    assert np.array_equal(kv_cache.encode_e4m3fn_satfinite(vals), codes)


def test_encoder_midpoints_go_to_even_code():
    pos = formats.E4M3FN[:0x7F]
    mid = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)        # exact in fp32
    got = kv_cache.encode_e4m3fn_satfinite(mid).astype(int)
    lo = np.arange(0x7E)
    want = np.where(lo % 2 == 0, lo, lo + 1)
    assert np.array_equal(got, want)
    assert np.array_equal(kv_cache.encode_e4m3fn_satfinite(-mid).astype(int), want | 0x80)


def test_encoder_saturation_rules():
    y = np.array([448, 463.9, 464, 500, 1e30, np.inf, -np.inf, -1e30, np.nan, -np.nan],
                 dtype=np.float32)
    got = kv_cache.encode_e4m3fn_satfinite(y).tolist()
    assert got == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE, 0x7F, 0xFF]
    assert kv_cache.encode_e4m3fn_satfinite(np.float32(-0.0)) == 0x80
    assert kv_cache.encode_e4m3fn_satfinite(np.float32(-1e-6)) == 0x80      # underflow keeps sign


def test_encoder_brute_force_nearest_on_all_bf16():
    with np.errstate(invalid="ignore"):
        y = ALL_BF16.float().numpy() / np.float32(0.37)
    fin = np.isfinite(y)
    a = np.minimum(np.abs(y[fin]).astype(np.float64), 448.0)
    vals = formats.E4M3FN[:0x7F]
    dist = np.abs(a[:, None] - vals[None, :])
    best = dist.min(axis=1)
    got = kv_cache.encode_e4m3fn_satfinite(y[fin]).astype(int) & 0x7F
    assert np.array_equal(dist[np.arange(len(a)), got], best)       # always a nearest code
    ties = (dist == best[:, None]).sum(axis=1) > 1
    assert np.all(got[ties] % 2 == 0)                               # even code on ties


def test_quantize_rows_matches_torch_fp32_pipeline():
    """quantize_rows = torch's own fp32 pipeline (bf16 -> fp32, fp32 division by the fp32 scale,
    float8_e4m3fn cast) wherever torch's cast is finite."""
    rng = np.random.default_rng(0)
    xb = torch.from_numpy(rng.standard_normal(200000).astype(np.float32) * 4).to(torch.bfloat16)
    for scale in (0.0123, 0.37, 1.0 / 3.0):
        s32 = torch.tensor(scale, dtype=torch.float32)
        lib = _torch_cast(xb.float() / s32)
        ours = kv_cache.quantize_rows(xb.float().numpy(), scale)
        ok = (lib & 0x7F) != 0x7F
        assert ok.sum() > 150000                     # most quotients stay below 464
        assert np.array_equal(ours[ok], lib[ok])


def test_cache_write_addressing():
    rng = np.random.default_rng(1)
    T, HKV, D, PB, NB = 7, 2, 32, 16, 5
    key = torch.from_numpy(rng.standard_normal((T, HKV, D)).astype(np.float32)).to(torch.bfloat16).float().numpy()
    val = torch.from_numpy(rng.standard_normal((T, HKV, D)).astype(np.float32)).to(torch.bfloat16).float().numpy()
    kc = rng.integers(0, 256, (NB, PB, HKV, D), dtype=np.uint8)
    vc = rng.integers(0, 256, (NB, PB, HKV, D), dtype=np.uint8)
    kc0, vc0 = kc.copy(), vc.copy()
    slots = np.array([0, 17, -1, 79, 33, -5, 48], dtype=np.int64)
    kv_cache.cache_write(key, val, kc, vc, slots, 0.05, 0.07, PB)
    written = np.zeros((NB, PB), dtype=bool)
    for i, s in enumerate(slots):
        if s < 0:
            continue
        b, o = divmod(int(s), PB)
        written[b, o] = True
        assert np.array_equal(kc[b, o], kv_cache.encode_e4m3fn_satfinite(key[i] / np.float32(0.05)))
        assert np.allclose(formats.E4M3FN[vc[b, o]], val[i] / 0.07, rtol=2 ** -3, atol=2 ** -9)
    assert np.array_equal(kc[~written], kc0[~written])
    assert np.array_equal(vc[~written], vc0[~written])


def test_planted_truncation_fails_midpoints(monkeypatch):
    """Round-toward-zero instead of nearest-even: the midpoint check catches it."""
    def trunc(y):
        y = np.asarray(y, dtype=np.float32)
        a = np.minimum(np.abs(y).astype(np.float64), 448.0)
        code = np.searchsorted(formats.E4M3FN[:0x7F], a, side="right") - 1
        return (code.astype(np.uint8) | (np.signbit(y).astype(np.uint8) << 7))
    monkeypatch.setattr(kv_cache, "encode_e4m3fn_satfinite", trunc)
    pos = formats.E4M3FN[:0x7F]
    mid = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    got = kv_cache.encode_e4m3fn_satfinite(mid).astype(int)
    lo = np.arange(0x7E)
    assert not np.array_equal(got, np.where(lo % 2 == 0, lo, lo + 1))
