"""GPU parity of the fp8 KV-cache write (fp8kv_cache_write) against the CPU oracle.

Bar: bit-exact (integer/byte output).  Every bf16 bit pattern goes through the kernel at several
scales; layouts (standalone [NB, PBLK, HKV, D] and the engine's [NB, HKV, PBLK, 2D] K|V view),
padding slots, an 8-byte-aligned V cache, untouched bytes, and a write -> decode round trip.
"""
import math

import numpy as np
import pytest
import torch

from fp8kv_amd import ops, workloads
from oracle import attention, kv_cache

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

ALL_BF16 = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def _caches(layout, NB, PBLK, HKV, D, fill):
    g = torch.Generator().manual_seed(fill)
    if layout == "engine":
        kv = torch.randint(0, 256, (NB, HKV, PBLK, 2 * D), dtype=torch.uint8, generator=g).to(DEV)
        kc, vc = workloads.engine_views(kv, D)
        return kc, vc, kv
    kc = torch.randint(0, 256, (NB, PBLK, HKV, D), dtype=torch.uint8, generator=g).to(DEV)
    vc = torch.randint(0, 256, (NB, PBLK, HKV, D), dtype=torch.uint8, generator=g).to(DEV)
    return kc.view(torch.float8_e4m3fn), vc.view(torch.float8_e4m3fn), None


def _check(key, value, slots, ks, vs, layout="standalone", PBLK=16, NB=None, seed=0):
    T, HKV, D = key.shape
    if NB is None:
        NB = max(1, (int(slots.max()) // PBLK) + 1 if slots.numel() else 1)
    kc, vc, _ = _caches(layout, NB, PBLK, HKV, D, seed)
    k0 = kc.view(torch.uint8).cpu().numpy().copy()
    v0 = vc.view(torch.uint8).cpu().numpy().copy()
    ops.cache_write(key.to(DEV), value.to(DEV), kc, vc, slots.to(DEV), ks, vs)
    torch.cuda.synchronize()
    k_ref, v_ref = k0.copy(), v0.copy()
    kv_cache.cache_write(key.float().numpy(), value.float().numpy(), k_ref, v_ref,
                         slots.numpy(), ks, vs, PBLK)
    got_k = kc.view(torch.uint8).cpu().numpy()
    got_v = vc.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got_k, k_ref)
    assert np.array_equal(got_v, v_ref)
    return kc, vc


@pytest.mark.parametrize("scale", [1.0, 0.5, 0.0123, 3.7, 2.0 ** -7])
def test_every_bf16_pattern_bit_exact(scale):
    """All 65536 bf16 values (NaNs, infinities, subnormals, both zeros) as K, reversed as V."""
    HKV, D = 4, 128
    T = 65536 // (HKV * D)
    key = ALL_BF16.view(T, HKV, D)
    value = ALL_BF16.flip(0).view(T, HKV, D)
    slots = torch.randperm(T, generator=torch.Generator().manual_seed(1)).to(torch.int64)
    _check(key, value, slots, scale, scale * 0.75, NB=T // 16)


@pytest.mark.parametrize("layout", ["standalone", "engine"])
@pytest.mark.parametrize("PBLK", [16, 32])
def test_layouts_and_padding_slots(layout, PBLK):
    g = torch.Generator().manual_seed(2)
    T, HKV, D, NB = 300, 4, 128, 40
    key = (torch.randn(T, HKV, D, generator=g) * 3).to(torch.bfloat16)
    value = (torch.randn(T, HKV, D, generator=g) * 3).to(torch.bfloat16)
    slots = torch.randperm(NB * PBLK, generator=g)[:T].to(torch.int64)
    slots[::7] = -1                                    # padding tokens write nothing
    _check(key, value, slots, 0.02, 0.03, layout=layout, PBLK=PBLK, NB=NB, seed=3)


def test_other_geometries():
    g = torch.Generator().manual_seed(4)
    for HKV, D, T in ((1, 16, 5), (8, 64, 33), (2, 256, 17), (6, 128, 1)):
        key = torch.randn(T, HKV, D, generator=g).to(torch.bfloat16)
        value = torch.randn(T, HKV, D, generator=g).to(torch.bfloat16)
        slots = torch.arange(T, dtype=torch.int64) * 3
        _check(key, value, slots, 0.05, 0.01, PBLK=16, NB=(3 * T) // 16 + 1, seed=HKV)


def test_strided_token_rows_and_8_byte_aligned_v_cache():
    """key / value as slices of wider rows (vLLM's qkv split), V cache at an 8-byte offset."""
    g = torch.Generator().manual_seed(5)
    T, HKV, D, PBLK, NB = 40, 2, 64, 16, 4
    qkv = torch.randn(T, 3 * HKV * D, generator=g).to(torch.bfloat16)
    qkv_d = qkv.to(DEV)
    key_d = qkv_d[:, HKV * D:2 * HKV * D].view(T, HKV, D)            # row stride 3 HKV D
    value_d = qkv_d[:, 2 * HKV * D:].view(T, HKV, D)
    assert key_d.stride(0) == 3 * HKV * D
    key, value = key_d.cpu(), value_d.cpu()
    kc = torch.zeros(NB, PBLK, HKV, D, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
    raw = torch.zeros(NB * PBLK * HKV * D + 8, dtype=torch.uint8, device=DEV)
    vc = raw[8:].view(NB, PBLK, HKV, D).view(torch.float8_e4m3fn)
    slots = torch.arange(T, dtype=torch.int64)
    ops.cache_write(key_d, value_d, kc, vc, slots.to(DEV), 0.1, 0.2)
    torch.cuda.synchronize()
    k_ref = np.zeros((NB, PBLK, HKV, D), dtype=np.uint8)
    v_ref = np.zeros((NB, PBLK, HKV, D), dtype=np.uint8)
    kv_cache.cache_write(key.float().numpy(), value.float().numpy(), k_ref, v_ref, slots.numpy(),
                         0.1, 0.2, PBLK)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), k_ref)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), v_ref)
    assert int(raw[:8].sum()) == 0


def test_write_then_decode_round_trip():
    """Tokens written by the kernel and read by the decode kernel give the oracle's attention over
    the dequantised cache (the format contract between the two entry points)."""
    g = torch.Generator().manual_seed(6)
    HQ, HKV, D, PBLK, ctx = 24, 4, 128, 16, 700
    NB = math.ceil(ctx / PBLK) + 3
    kv = torch.zeros(NB, HKV, PBLK, 2 * D, dtype=torch.uint8, device=DEV)
    kc, vc = workloads.engine_views(kv, D)
    key = torch.randn(ctx, HKV, D, generator=g).to(torch.bfloat16)
    value = torch.randn(ctx, HKV, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(NB, generator=g)[:math.ceil(ctx / PBLK)].to(torch.int32)
    slots = (perm.repeat_interleave(PBLK)[:ctx].to(torch.int64) * PBLK
             + torch.arange(ctx, dtype=torch.int64) % PBLK)
    ks, vs = 0.01, 0.012
    ops.cache_write(key.to(DEV), value.to(DEV), kc, vc, slots.to(DEV), ks, vs)
    q = torch.randn(1, HQ, D, generator=g).to(torch.bfloat16)
    out = torch.zeros(1, HQ, D, dtype=torch.bfloat16, device=DEV)
    bt = perm.view(1, -1)
    ops.decode_attention(q.to(DEV), kc, vc, out, torch.tensor([0, 1], dtype=torch.int32, device=DEV),
                         torch.tensor([ctx], dtype=torch.int32, device=DEV), bt.to(DEV), ks, vs,
                         1 / math.sqrt(D), max_seq_len=ctx)
    torch.cuda.synchronize()
    kpool = np.zeros((NB * PBLK, HKV, D), dtype=np.uint8)
    vpool = np.zeros((NB * PBLK, HKV, D), dtype=np.uint8)
    kpool[slots.numpy()] = kv_cache.quantize_rows(key.float().numpy(), ks)
    vpool[slots.numpy()] = kv_cache.quantize_rows(value.float().numpy(), vs)
    kpool = torch.from_numpy(kpool).view(NB, PBLK, HKV, D).view(torch.float8_e4m3fn)
    vpool = torch.from_numpy(vpool).view(NB, PBLK, HKV, D).view(torch.float8_e4m3fn)
    # the kernel's cache bytes are the oracle's bytes at every written slot
    got = kv.cpu().view(NB, HKV, PBLK, 2 * D).transpose(1, 2).reshape(NB * PBLK, HKV, 2 * D)
    assert torch.equal(got[slots, :, :D], kpool.view(torch.uint8).view(-1, HKV, D)[slots])
    ref = attention.decode_attention(q, kpool, vpool, torch.tensor([0, 1]), torch.tensor([ctx]),
                                     bt, ks, vs, 1 / math.sqrt(D))
    torch.testing.assert_close(out.cpu().double(), ref.double(), rtol=1e-2, atol=1e-2)
