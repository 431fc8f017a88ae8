"""Seeded synthetic inputs for the benchmark configurations (built on the CPU, then moved).

All generators use a CPU ``torch.Generator`` so the same seed gives the same bytes on any
machine; the bench's cache-defeating rotation copies are generated on the device instead.

  * ``w4_case``      MXFP4 matvec: codes uniform over all 16 values (uniform bytes), e8m0 scale
                     bytes uniform in [119, 123] (2^-8 .. 2^-4), x ~ N(0,1) bf16.
  * ``decode_case``  paged fp8 decode: K, V ~ N(0,1) quantised per tensor with scale amax/448
                     (``kv_gen="ref"``: N(0,1) * 2 cast straight to e4m3 with scale 1, the
                     reference's self-test data),
                     a pool of blocks handed out by a seeded permutation, one query per sequence.
  * ``prefill_case`` paged fp8 prefill, single sequence or varlen (cu_seqlens).
Layouts: ``"standalone"`` caches are [NB, PBLK, HKV, D]; ``"engine"`` caches are views of one
uint8 tensor [NB, HKV, PBLK, 2D] (K then V per token row) exactly as the attention hook sees
them after ``kv_cache.transpose(1, 2).split(D, -1)`` (vllm-fp8kv/fp8kv_override.py:82-85).
"""
from __future__ import annotations

import math

import torch

E4M3_MAX = 448.0


def w4_case(N: int, K: int, M: int, seed: int = 0, scale_lo: int = 119, scale_hi: int = 123):
    g = torch.Generator().manual_seed(seed)
    W = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, generator=g)
    S_kn = torch.randint(scale_lo, scale_hi + 1, (K // 32, N), dtype=torch.uint8, generator=g)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16)
    return {"W": W, "S_kn": S_kn, "St": S_kn.t().contiguous(), "X": X}


def quantize_per_tensor(x: torch.Tensor):
    """fp32 tensor -> (float8_e4m3fn tensor, scale) with scale = amax / 448."""
    amax = float(x.abs().max())
    scale = amax / E4M3_MAX if amax > 0 else 1.0
    q = (x / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q, scale


def _make_cache(nb: int, pblk: int, hkv: int, d: int, g: torch.Generator, layout: str,
                kv_gen: str = "amax"):
    k = torch.randn(nb, pblk, hkv, d, generator=g)
    v = torch.randn(nb, pblk, hkv, d, generator=g)
    if kv_gen == "bf16":
        # bf16 caches, stored as they are (the reference's K_FP8 = False branch: no scales)
        kb, vb = k.to(torch.bfloat16), v.to(torch.bfloat16)
        if layout == "standalone":
            return kb, vb, None, 1.0, 1.0
        if layout == "engine":
            kv = torch.empty(nb, hkv, pblk, 2 * d, dtype=torch.bfloat16)
            kv[..., :d] = kb.transpose(1, 2)
            kv[..., d:] = vb.transpose(1, 2)
            kc, vc = engine_views(kv, d)
            return kc, vc, kv, 1.0, 1.0
        raise ValueError(layout)
    if kv_gen == "amax":
        kq, ks = quantize_per_tensor(k)
        vq, vs = quantize_per_tensor(v)
    elif kv_gen == "ref":
        # the reference's self-test data: N(0,1) * 2 cast straight to e4m3 (vllm-fp8kv/fp8kv_v3.py:150-151)
        kq, ks = (k * 2).to(torch.float8_e4m3fn), 1.0
        vq, vs = (v * 2).to(torch.float8_e4m3fn), 1.0
    else:
        raise ValueError(kv_gen)
    if layout == "standalone":
        return kq, vq, None, ks, vs
    if layout == "engine":
        kv = torch.empty(nb, hkv, pblk, 2 * d, dtype=torch.uint8)
        kv[..., :d] = kq.view(torch.uint8).transpose(1, 2)
        kv[..., d:] = vq.view(torch.uint8).transpose(1, 2)
        kc, vc = engine_views(kv, d)
        return kc, vc, kv, ks, vs
    raise ValueError(layout)


def engine_pool_amax(nb: int, hkv: int, pblk: int, d: int, generator: torch.Generator,
                     device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """An engine-layout fp8 KV pool [nb, hkv, pblk, 2d] (K | V) built on `device` the way
    BASELINE.json configs[0] specifies the cache: K and V ~ N(0,1), each quantised to e4m3 with a
    per-tensor scale amax / 448.  Returns (pool, k_scale, v_scale), the scales as fp32 [1]
    device tensors (the form the attention hooks pass)."""
    pool = torch.empty(nb, hkv, pblk, 2 * d, dtype=torch.uint8, device=device)
    scales = []
    for half in (slice(0, d), slice(d, 2 * d)):
        x = torch.randn(nb, hkv, pblk, d, device=device, generator=generator)
        amax = x.abs().max()
        scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
        pool[..., half] = (x / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8)
        scales.append(scale.reshape(1).to(torch.float32))
        del x
    return pool, scales[0], scales[1]


def engine_views(kv_cache: torch.Tensor, head_size: int):
    """The K and V fp8 views the attention hook builds (vllm-fp8kv/fp8kv_override.py:82-85); a
    bf16 pool gives bf16 views."""
    kc = kv_cache.transpose(1, 2)
    key_cache, value_cache = kc.split(head_size, dim=-1)
    if kv_cache.dtype == torch.bfloat16:
        return key_cache, value_cache
    return key_cache.view(torch.float8_e4m3fn), value_cache.view(torch.float8_e4m3fn)


def decode_case(ctx_lens, HQ: int = 24, HKV: int = 4, D: int = 128, PBLK: int = 16,
                pool_blocks: int | None = None, seed: int = 0, layout: str = "standalone",
                contiguous_bt: bool = False, kv_gen: str = "amax"):
    ctx_lens = [int(c) for c in ctx_lens]
    NS = len(ctx_lens)
    need = [math.ceil(c / PBLK) for c in ctx_lens]
    if pool_blocks is None:
        pool_blocks = max(1, sum(need))
    assert sum(need) <= pool_blocks, "pool too small"
    g = torch.Generator().manual_seed(seed)
    kc, vc, kv, ks, vs = _make_cache(pool_blocks, PBLK, HKV, D, g, layout, kv_gen)
    max_blocks = max(1, max(need))
    bt = torch.zeros(NS, max_blocks, dtype=torch.int32)
    ids = torch.arange(pool_blocks) if contiguous_bt else torch.randperm(pool_blocks, generator=g)
    o = 0
    for s, n in enumerate(need):
        bt[s, :n] = ids[o:o + n].to(torch.int32)
        o += n
    q = torch.randn(NS, HQ, D, generator=g).to(torch.bfloat16)
    return {
        "q": q, "k_cache": kc, "v_cache": vc, "kv_cache": kv, "k_scale": ks, "v_scale": vs,
        "qsl": torch.arange(NS + 1, dtype=torch.int32),
        "seq_lens": torch.tensor(ctx_lens, dtype=torch.int32),
        "block_table": bt, "sm_scale": 1.0 / math.sqrt(D),
    }


def prefill_case(qlens, q0s, HQ: int = 24, HKV: int = 4, D: int = 128, PBLK: int = 16,
                 pool_blocks: int | None = None, seed: int = 0, layout: str = "standalone",
                 contiguous_bt: bool = False, kv_gen: str = "amax"):
    """Packed varlen prefill: sequence s has qlens[s] new tokens after q0s[s] cached ones."""
    qlens = [int(x) for x in qlens]
    q0s = [int(x) for x in q0s]
    ctx = [a + b for a, b in zip(qlens, q0s)]
    case = decode_case(ctx, HQ, HKV, D, PBLK, pool_blocks, seed, layout, contiguous_bt, kv_gen)
    g = torch.Generator().manual_seed(seed + 7919)
    T = sum(qlens)
    case["q"] = torch.randn(T, HQ, D, generator=g).to(torch.bfloat16)
    cu = [0]
    for n in qlens:
        cu.append(cu[-1] + n)
    case["cu_seqlens_q"] = torch.tensor(cu, dtype=torch.int32)
    case["qsl"] = case["cu_seqlens_q"]
    case["q0s"] = q0s
    case["qlens"] = qlens
    return case


def to_device(case: dict, device) -> dict:
    out = {}
    for k, v in case.items():
        out[k] = v.to(device) if isinstance(v, torch.Tensor) else v
    if case.get("kv_cache") is not None:
        kv = case["kv_cache"].to(device)
        out["kv_cache"] = kv
        out["k_cache"], out["v_cache"] = engine_views(kv, case["q"].shape[-1])
    return out
