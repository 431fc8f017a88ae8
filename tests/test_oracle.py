"""Pins for the CPU oracle (CPU only).

Every oracle function is checked here against something it was not derived from: a library
conversion, a literal table from the reference's own tests, a closed form, a special case, or a
brute-force loop on a tiny input.  The ``planted_*`` tests plant a plausible mistake in the
oracle (monkeypatched on the CPU) and show that one of those checks catches it.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention, formats, matvec

# The reference's literal e2m1 table, h4mv/h4mv_test.py:16-17 (also bench_w4hip.py:39-40).
REF_E2M1_LUT = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


# ----------------------------------------------------------------------------------- formats

def test_e4m3_table_matches_torch_conversion():
    b = torch.arange(256, dtype=torch.uint8)
    lib = b.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    ours = formats.E4M3FN
    assert np.array_equal(np.isnan(ours), np.isnan(lib))
    fin = ~np.isnan(ours)
    assert np.array_equal(ours[fin], lib[fin])
    assert np.array_equal(np.signbit(ours[fin]), np.signbit(lib[fin]))


def test_e4m3_spot_values_from_spec():
    t = formats.E4M3FN
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert t[0x01] == 2.0 ** -9 and t[0x07] == 7 * 2.0 ** -9
    assert t[0x08] == 2.0 ** -6 and t[0x38] == 1.0
    assert t[0x80] == 0.0 and np.signbit(t[0x80])
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert np.sum(np.isnan(t)) == 2


def test_e4m3_values_exact_in_bf16():
    v = formats.E4M3FN[~np.isnan(formats.E4M3FN)]
    rt = torch.tensor(v).to(torch.bfloat16).to(torch.float64).numpy()
    assert np.array_equal(rt, v)


def test_quantize_e4m3_matches_torch_cast():
    g = np.random.default_rng(3)
    x = g.standard_normal(20000) * 3
    scale = float(np.abs(x).max()) / 448.0
    ours = formats.decode_e4m3(formats.quantize_e4m3(x, scale))
    lib = torch.tensor(x / scale).clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.float64).numpy()
    assert np.array_equal(ours, lib)


def test_e2m1_table_matches_reference_lut():
    assert np.array_equal(formats.E2M1, np.array(REF_E2M1_LUT))
    assert np.array_equal(np.signbit(formats.E2M1), np.signbit(np.array(REF_E2M1_LUT)))


def test_e2m1_bit_rules():
    for v in range(16):
        val = formats.E2M1[v]
        assert (val == 0.0) == ((v & 7) == 0)                  # h4mv.cu:35
        e, m = (v >> 1) & 3, v & 1
        if e == 0 and m == 1:
            assert abs(val) == 0.5                              # subnormal, h4mv.cu:39
        assert np.signbit(val) == bool(v & 8)


def test_e8m0_table_matches_torch_conversion():
    b = torch.arange(256, dtype=torch.uint8)
    lib = b.view(torch.float8_e8m0fnu).to(torch.float64).numpy()
    ours = formats.E8M0
    assert np.array_equal(ours[:255], lib[:255])
    assert np.isnan(ours[255]) and np.isnan(lib[255])
    assert ours[127] == 1.0 and ours[0] == 2.0 ** -127


def test_pack_unpack_roundtrip_and_nibble_order():
    codes = np.arange(32, dtype=np.uint8) % 16
    packed = formats.pack_e2m1(codes)
    assert packed[0] == (0 | (1 << 4))                          # low nibble = even k
    assert np.array_equal(formats.unpack_e2m1(packed), codes)


# ----------------------------------------------------------------------------------- matvec

def _one_hot_probe(k: int, M: int = 8, N: int = 4):
    """h4mv/h4mv_test.py:38-52: weight code 2 (= 1.0) at k, x one-hot at k, scale byte 127."""
    W = np.zeros((N, 16), dtype=np.uint8)
    W[:, k // 2] = 2 if k % 2 == 0 else (2 << 4)
    St = np.full((N, 1), 127, dtype=np.uint8)
    X = np.zeros((M, 32), dtype=np.float32)
    X[:, k] = 1.0
    return W, St, X


def test_matvec_one_hot_probes():
    for k in range(32):
        W, St, X = _one_hot_probe(k)
        assert np.array_equal(matvec.w4mv(W, St, X), np.ones((8, 4)))


def test_matvec_integer_full_row_exact():
    """w4-hip-demo/probe_w4hip.py:33-47: scale 127, x = (k mod 7) - 3, exact in any order."""
    rng = np.random.default_rng(0)
    N, K = 8, 4096
    W = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    St = np.full((N, K // 32), 127, dtype=np.uint8)
    x = (np.arange(K) % 7) - 3
    y = matvec.w4mv(W, St, x[None, :].astype(np.float32))[0]
    twice = [int(round(2 * v)) for v in REF_E2M1_LUT]
    for n in range(N):
        acc = 0
        for b in range(K // 2):
            byte = int(W[n, b])
            acc += twice[byte & 15] * int(x[2 * b]) + twice[byte >> 4] * int(x[2 * b + 1])
        assert y[n] == acc / 2


def _brute_matvec(W, St, X):
    N, M, K = W.shape[0], X.shape[0], W.shape[1] * 2
    out = [[0.0] * N for _ in range(M)]
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                byte = int(W[n, k // 2])
                code = (byte & 15) if k % 2 == 0 else (byte >> 4)
                s += float(X[m, k]) * REF_E2M1_LUT[code] * math.ldexp(1.0, int(St[n, k // 32]) - 127)
            out[m][n] = s
    return np.array(out)


def _tiny_random_matvec(seed=1):
    rng = np.random.default_rng(seed)
    N, K, M = 3, 96, 2
    W = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    St = rng.integers(110, 140, (N, K // 32), dtype=np.uint8)
    X = rng.standard_normal((M, K)).astype(np.float32)
    return W, St, X


def test_matvec_brute_force_random_scales():
    W, St, X = _tiny_random_matvec()
    np.testing.assert_allclose(matvec.w4mv(W, St, X), _brute_matvec(W, St, X), rtol=1e-12, atol=0)


def test_matvec_repack_is_transpose():
    S = np.arange(12, dtype=np.uint8).reshape(3, 4)             # [K/32=3, N=4]
    St = matvec.repack_scales(S)
    assert St.shape == (4, 3) and St.flags["C_CONTIGUOUS"] and St[2, 1] == S[1, 2]


def test_bf16_ulp_matches_torch_rounding():
    rng = np.random.default_rng(7)
    v = rng.standard_normal(5000) * np.exp2(rng.integers(-30, 30, 5000))
    u = matvec.bf16_ulp(v)
    b = torch.tensor(v).to(torch.bfloat16).to(torch.float64).numpy()
    assert np.all(np.abs(b - v) <= u / 2)                       # RNE lands within half an ulp
    up = np.abs(b) + matvec.bf16_ulp(b)                         # next value up from b
    same_binade = np.frexp(up)[1] == np.frexp(np.abs(b))[1]
    rt = torch.tensor(up[same_binade]).to(torch.bfloat16).to(torch.float64).numpy()
    assert np.array_equal(rt, up[same_binade])                  # ... and is representable
    assert matvec.bf16_excess_error(b, v) == 0.0


def test_planted_nibble_swap_fails_probe(monkeypatch):
    def swapped(p):
        p = np.asarray(p, dtype=np.uint8)
        out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
        out[..., 0::2] = p >> 4
        out[..., 1::2] = p & 0xF
        return out
    monkeypatch.setattr(matvec, "unpack_e2m1", swapped)
    W, St, X = _one_hot_probe(5)
    assert not np.array_equal(matvec.w4mv(W, St, X), np.ones((8, 4)))


def test_planted_scale_bias_fails_brute_force(monkeypatch):
    monkeypatch.setattr(matvec, "E8M0", np.array([2.0 ** (b - 126) for b in range(256)]))
    W, St, X = _tiny_random_matvec()
    assert not np.allclose(matvec.w4mv(W, St, X), _brute_matvec(W, St, X), rtol=1e-6)


# -------------------------------------------------------------------------------- attention

def _lib_gather(cache, bt_row, ctx, kh):
    """Gather through torch's own fp8 conversion and explicit per-token indexing."""
    rows = []
    pblk = cache.shape[1]
    for t in range(ctx):
        rows.append(cache[int(bt_row[t // pblk]), t % pblk, kh].to(torch.float64))
    return torch.stack(rows)


def _sdpa_reference(q, kc, vc, bt_row, ks, vs, sm, q0, qlen):
    """torch SDPA in fp64 with an explicit causal mask (token q0+i sees keys <= q0+i)."""
    HQ, D = q.shape[1], q.shape[2]
    HKV = kc.shape[2]
    ctx = q0 + qlen
    out = torch.empty(qlen, HQ, D, dtype=torch.float64)
    allow = torch.arange(ctx)[None, :] <= (torch.arange(qlen) + q0)[:, None]
    for h in range(HQ):
        kh = h // (HQ // HKV)
        k = _lib_gather(kc, bt_row, ctx, kh) * ks
        v = _lib_gather(vc, bt_row, ctx, kh) * vs
        out[:, h] = F.scaled_dot_product_attention(
            q[:qlen, h].to(torch.float64)[None], k[None], v[None], attn_mask=allow[None], scale=sm)[0]
    return out


def _small_case(ctx=(37, 5, 20), layout="standalone", seed=0, HQ=6, HKV=2, D=16):
    from fp8kv_amd import workloads
    return workloads.decode_case(ctx, HQ=HQ, HKV=HKV, D=D, PBLK=4, pool_blocks=24, seed=seed,
                                 layout=layout)


@pytest.mark.parametrize("layout", ["standalone", "engine"])
def test_decode_matches_sdpa(layout):
    c = _small_case(layout=layout)
    ks, vs = 0.5, 2.0                                          # fp8kv_v3.py:170-177 scale case
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], ks, vs, c["sm_scale"])
    for s in range(3):
        ctx = int(c["seq_lens"][s])
        ref = _sdpa_reference(c["q"][s:s + 1], c["k_cache"], c["v_cache"], c["block_table"][s],
                              ks, vs, c["sm_scale"], ctx - 1, 1)
        torch.testing.assert_close(out[s], ref[0], rtol=1e-12, atol=1e-12)


def test_decode_context_one_is_scaled_v0():
    c = _small_case(ctx=(1, 1, 1))
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 0.7, 1.75, c["sm_scale"])
    for s in range(3):
        blk = int(c["block_table"][s, 0])
        for h in range(6):
            v0 = c["v_cache"][blk, 0, h // 3].to(torch.float64) * 1.75
            assert torch.equal(out[s, h], v0)


def test_decode_identical_keys_give_mean_v():
    c = _small_case(ctx=(9, 4, 13))
    kc = c["k_cache"].clone()
    kc.view(torch.uint8)[:] = 0x3C                             # every key element = 1.5
    out = attention.decode_attention(c["q"], kc, c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 1.0, 3.0, c["sm_scale"])
    for s in range(3):
        ctx = int(c["seq_lens"][s])
        for h in range(6):
            v = _lib_gather(c["v_cache"], c["block_table"][s], ctx, h // 3)
            torch.testing.assert_close(out[s, h], 3.0 * v.mean(0), rtol=1e-12, atol=1e-12)


def test_decode_zero_context_gives_zeros():
    c = _small_case(ctx=(0, 6, 3))
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 1.0, 1.0, c["sm_scale"])
    assert torch.count_nonzero(out[0]) == 0 and torch.isfinite(out).all()


def test_decode_brute_force_tiny():
    c = _small_case(ctx=(5, 3, 1), HQ=2, HKV=1, D=4)
    ks, vs, sm = 0.25, 1.5, 0.5
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], ks, vs, sm)
    kb = c["k_cache"].view(torch.uint8)
    vb = c["v_cache"].view(torch.uint8)
    for s in range(3):
        ctx = int(c["seq_lens"][s])
        for h in range(2):
            scores = []
            for t in range(ctx):
                blk = int(c["block_table"][s, t // 4])
                kv = [REF_E4M3(int(kb[blk, t % 4, 0, d])) for d in range(4)]
                scores.append(sum(float(c["q"][s, h, d]) * kv[d] for d in range(4)) * sm * ks)
            mx = max(scores)
            w = [math.exp(x - mx) for x in scores]
            for d in range(4):
                num = sum(w[t] * REF_E4M3(int(vb[int(c["block_table"][s, t // 4]), t % 4, 0, d]))
                          for t in range(ctx))
                assert abs(out[s, h, d].item() - vs * num / sum(w)) < 1e-12


def REF_E4M3(b: int) -> float:
    """e4m3fn decode written from the OCP spec with math.ldexp (independent of the table code)."""
    sign = -1.0 if b & 0x80 else 1.0
    exp, man = (b >> 3) & 15, b & 7
    if exp == 0:
        return sign * math.ldexp(man, -9)
    return sign * math.ldexp(8 + man, exp - 10)


def test_decode_block_permutation_invariance():
    c = _small_case()
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 1.0, 1.0, c["sm_scale"])
    perm = torch.randperm(24, generator=torch.Generator().manual_seed(5))
    inv = torch.argsort(perm)
    kc = c["k_cache"][perm]                                     # new block i holds old block perm[i]
    vc = c["v_cache"][perm]
    bt = inv[c["block_table"].long()].to(torch.int32)
    out2 = attention.decode_attention(c["q"], kc, vc, c["qsl"], c["seq_lens"], bt, 1.0, 1.0,
                                      c["sm_scale"])
    assert torch.equal(out, out2)


def test_prefill_matches_sdpa_and_row0():
    from fp8kv_amd import workloads
    c = workloads.prefill_case([19], [0], HQ=6, HKV=2, D=16, PBLK=4, pool_blocks=8, seed=2)
    out = attention.prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0],
                                      0.5, 2.0, c["sm_scale"], 0, 19)
    ref = _sdpa_reference(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0], 0.5, 2.0,
                          c["sm_scale"], 0, 19)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)
    blk = int(c["block_table"][0, 0])
    for h in range(6):                                          # q0 = 0: row 0 sees key 0 only
        assert torch.equal(out[0, h], c["v_cache"][blk, 0, h // 3].to(torch.float64) * 2.0)


# ---- bf16 caches: the reference's K_FP8 = False branch (vllm-fp8kv/fp8kv_v3.py:44-45,61-66,110;
# fp8kv_prefill.py:57-60,77-82,117): values used as stored, k_scale and v_scale ignored.

def _bf16_case(layout="standalone", ctx=(37, 5, 20), seed=4):
    from fp8kv_amd import workloads
    return workloads.decode_case(ctx, HQ=6, HKV=2, D=16, PBLK=4, pool_blocks=24, seed=seed,
                                 layout=layout, kv_gen="bf16")


@pytest.mark.parametrize("layout", ["standalone", "engine"])
def test_bf16_decode_matches_sdpa_without_scales(layout):
    c = _bf16_case(layout)
    assert c["k_cache"].dtype == torch.bfloat16
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 0.5, 2.0, c["sm_scale"])   # scales ignored
    for s in range(3):
        ctx = int(c["seq_lens"][s])
        ref = _sdpa_reference(c["q"][s:s + 1], c["k_cache"], c["v_cache"], c["block_table"][s],
                              1.0, 1.0, c["sm_scale"], ctx - 1, 1)
        torch.testing.assert_close(out[s], ref[0], rtol=1e-12, atol=1e-12)


def test_bf16_prefill_matches_sdpa_without_scales():
    from fp8kv_amd import workloads
    c = workloads.prefill_case([19], [7], HQ=6, HKV=2, D=16, PBLK=4, pool_blocks=8, seed=5, kv_gen="bf16")
    out = attention.prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0],
                                      0.25, 3.0, c["sm_scale"], 7, 19)
    ref = _sdpa_reference(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0], 1.0, 1.0,
                          c["sm_scale"], 7, 19)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)


def test_bf16_cache_of_scaled_e4m3_values_equals_the_e4m3_path():
    """A bf16 cache holding an e4m3 cache's values times power-of-two scales (exact in bf16) gives
    what the e4m3 path gives with those scales; the bf16 call's own scales play no part."""
    c = _small_case(seed=6)
    ks, vs = 0.5, 4.0
    k16 = (c["k_cache"].to(torch.float64) * ks).to(torch.bfloat16)
    v16 = (c["v_cache"].to(torch.float64) * vs).to(torch.bfloat16)
    assert torch.equal(k16.to(torch.float64), c["k_cache"].to(torch.float64) * ks)
    a = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                   c["block_table"], ks, vs, c["sm_scale"])
    b = attention.decode_attention(c["q"], k16, v16, c["qsl"], c["seq_lens"], c["block_table"],
                                   123.0, 0.01, c["sm_scale"])
    torch.testing.assert_close(a, b, rtol=1e-13, atol=0)


def test_bf16_planted_scale_use_fails_the_pin(monkeypatch):
    """An oracle that applied the scales to bf16 caches fails the SDPA pin above."""
    monkeypatch.setattr(attention, "_scales", lambda cache, ks, vs: (ks, vs))
    c = _bf16_case()
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 0.5, 2.0, c["sm_scale"])
    ref = _sdpa_reference(c["q"][0:1], c["k_cache"], c["v_cache"], c["block_table"][0], 1.0, 1.0,
                          c["sm_scale"], int(c["seq_lens"][0]) - 1, 1)
    assert not torch.allclose(out[0], ref[0], rtol=1e-6, atol=1e-6)


def test_prefill_continuation_matches_sdpa():
    from fp8kv_amd import workloads
    c = workloads.prefill_case([11], [13], HQ=6, HKV=2, D=16, PBLK=4, pool_blocks=8, seed=4,
                               layout="engine")
    out = attention.prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0],
                                      1.0, 1.0, c["sm_scale"], 13, 11)
    ref = _sdpa_reference(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0], 1.0, 1.0,
                          c["sm_scale"], 13, 11)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)


def test_decode_equals_last_prefill_row():
    from fp8kv_amd import workloads
    c = workloads.prefill_case([7], [9], HQ=6, HKV=2, D=16, PBLK=4, pool_blocks=8, seed=6)
    pre = attention.prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0],
                                      0.8, 1.2, c["sm_scale"], 9, 7)
    qsl = torch.tensor([6, 7], dtype=torch.int32)
    dec = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], qsl,
                                     torch.tensor([16], dtype=torch.int32), c["block_table"],
                                     0.8, 1.2, c["sm_scale"])
    torch.testing.assert_close(dec[0], pre[6], rtol=1e-12, atol=1e-12)


def test_varlen_equals_independent_runs():
    from fp8kv_amd import workloads
    c = workloads.prefill_case([5, 9, 3], [0, 4, 11], HQ=6, HKV=2, D=16, PBLK=4, pool_blocks=24,
                               seed=8)
    out = attention.varlen_prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["cu_seqlens_q"],
                                             c["seq_lens"], c["block_table"], 1.0, 1.0,
                                             c["sm_scale"])
    cu = c["cu_seqlens_q"]
    for s, (ql, q0) in enumerate(zip(c["qlens"], c["q0s"])):
        ref = _sdpa_reference(c["q"][int(cu[s]):int(cu[s + 1])], c["k_cache"], c["v_cache"],
                              c["block_table"][s], 1.0, 1.0, c["sm_scale"], q0, ql)
        torch.testing.assert_close(out[int(cu[s]):int(cu[s + 1])], ref, rtol=1e-12, atol=1e-12)


def test_planted_dropped_k_scale_fails_sdpa(monkeypatch):
    c = _small_case()
    real = attention._attend
    monkeypatch.setattr(attention, "_attend",
                        lambda qh, k, v, scale, vs, pos: real(qh, k, v, scale / 0.5, vs, pos))
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 0.5, 2.0, c["sm_scale"])
    ref = _sdpa_reference(c["q"][0:1], c["k_cache"], c["v_cache"], c["block_table"][0], 0.5, 2.0,
                          c["sm_scale"], int(c["seq_lens"][0]) - 1, 1)
    assert not torch.allclose(out[0], ref[0], rtol=1e-3, atol=1e-3)


def test_planted_causal_off_by_one_fails_row0(monkeypatch):
    from fp8kv_amd import workloads
    c = workloads.prefill_case([6], [0], HQ=6, HKV=2, D=16, PBLK=4, pool_blocks=8, seed=2)

    def shifted(qh, k, v, scale, vs, pos):
        return attention.__dict__["_attend_real"](qh, k, v, scale, vs, pos + 1)
    monkeypatch.setitem(attention.__dict__, "_attend_real", attention._attend)
    monkeypatch.setattr(attention, "_attend", shifted)
    out = attention.prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0],
                                      1.0, 1.0, c["sm_scale"], 0, 6)
    blk = int(c["block_table"][0, 0])
    assert not torch.equal(out[0, 0], c["v_cache"][blk, 0, 0].to(torch.float64))


def test_planted_gqa_mapping_fails_sdpa(monkeypatch):
    c = _small_case()
    real_gather = attention.gather_kv
    monkeypatch.setattr(attention, "gather_kv",
                        lambda cache, bt, ctx, kh, dtype=torch.float64:
                        real_gather(cache, bt, ctx, (kh + 1) % cache.shape[2], dtype))
    out = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 1.0, 1.0, c["sm_scale"])
    ref = _sdpa_reference(c["q"][0:1], c["k_cache"], c["v_cache"], c["block_table"][0], 1.0, 1.0,
                          c["sm_scale"], int(c["seq_lens"][0]) - 1, 1)
    assert not torch.allclose(out[0], ref[0], rtol=1e-3, atol=1e-3)
