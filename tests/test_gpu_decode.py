"""GPU parity of the paged fp8 decode attention (fp8kv_decode_attn) against the CPU oracle.

Bar (BASELINE): bf16 output vs the fp64 oracle within rtol = atol = 1e-2 elementwise; the
reference's own self-test bar (max-abs < 0.05, vllm-fp8kv/fp8kv_v3.py:168,177) is implied.
Inputs come from seeded CPU generators (fp8kv_amd.workloads) and are copied to the device.
"""
import math

import pytest
import torch

from fp8kv_amd import _lib, ops, workloads
from oracle import attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
RTOL = ATOL = 1e-2


def _oracle(c, ks=None, vs=None):
    ks = c["k_scale"] if ks is None else ks
    vs = c["v_scale"] if vs is None else vs
    return attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                      c["block_table"], ks, vs, c["sm_scale"])


def _run(c, ks=None, vs=None, num_splits=None, out=None):
    d = workloads.to_device(c, DEV)
    ks = c["k_scale"] if ks is None else ks
    vs = c["v_scale"] if vs is None else vs
    if out is None:
        out = torch.zeros_like(d["q"])
    ops.decode_attention(d["q"], d["k_cache"], d["v_cache"], out, d["qsl"], d["seq_lens"],
                         d["block_table"], torch.tensor([ks], device=DEV),
                         torch.tensor([vs], device=DEV), c["sm_scale"], num_splits=num_splits)
    torch.cuda.synchronize()
    return out


def _rows(c, out):
    """Output rows qsl[s] of every sequence, as [NS, HQ, D] fp64 on the CPU."""
    idx = c["qsl"][:-1].long()
    return out.cpu()[idx].to(torch.float64)


def _check(c, ks=None, vs=None, num_splits=None):
    ref = _oracle(c, ks, vs)
    got = _rows(c, _run(c, ks, vs, num_splits))
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=ATOL)
    err = (got - ref).abs().max().item()
    assert err < 0.05 * max(1.0, ref.abs().max().item())
    return err


@pytest.mark.parametrize("num_splits", [None, 1, 2, 5])
def test_config0_cpu_parity_case(num_splits):
    """batch 1, 24/4 heads, ctx 512, block 16, contiguous block table."""
    c = workloads.decode_case([512], contiguous_bt=True, seed=0)
    _check(c, num_splits=num_splits)


def test_scale_fold_case():
    """k_scale = 0.5, v_scale = 2.0 (vllm-fp8kv/fp8kv_v3.py:170-177)."""
    c = workloads.decode_case([512, 1000], seed=1, kv_gen="ref")
    err = _check(c, ks=0.5, vs=2.0)
    assert err < 0.05


@pytest.mark.parametrize("layout", ["standalone", "engine"])
def test_config2_batch8(layout):
    """batch 8, ctx ~ U[1024, 4096], 5060-block pool, random block permutation."""
    g = torch.Generator().manual_seed(2)
    ctx = torch.randint(1024, 4097, (8,), generator=g).tolist()
    c = workloads.decode_case(ctx, pool_blocks=5060, seed=2, layout=layout)
    err = _check(c)
    print(f"cfg2 {layout}: max-abs {err:.2e}")


def test_b8_at_4k():
    c = workloads.decode_case([4096] * 8, pool_blocks=5060, seed=3, layout="engine")
    _check(c)


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (16, 2), (32, 2), (6, 1), (15, 5), (20, 4)])
def test_other_head_geometries(hq, hkv):
    """(32, 8) is the reference's own geometry (vllm-fp8kv/fp8kv_v3.py:144); GQA 1 .. 16."""
    c = workloads.decode_case([777, 2048, 5], HQ=hq, HKV=hkv, seed=4)
    _check(c)


def test_edge_context_lengths():
    ctx = [1, 2, 15, 16, 17, 31, 33, 63, 64, 65, 127, 255, 257, 1000, 4097]
    c = workloads.decode_case(ctx, seed=5)
    _check(c)
    _check(c, num_splits=1)
    _check(c, num_splits=256)


def test_context_one_is_scaled_v0():
    c = workloads.decode_case([1, 1], seed=6)
    got = _rows(c, _run(c, 1.0, 1.75))
    for s in range(2):
        blk = int(c["block_table"][s, 0])
        for h in range(24):
            v0 = (c["v_cache"][blk, 0, h // 6].to(torch.float64) * 1.75).to(torch.bfloat16)
            assert torch.equal(got[s, h].to(torch.bfloat16), v0)


def test_zero_context_gives_zeros():
    c = workloads.decode_case([0, 300, 0], seed=7)
    got = _rows(c, _run(c))
    assert torch.count_nonzero(got[0]) == 0 and torch.count_nonzero(got[2]) == 0
    torch.testing.assert_close(got[1], _oracle(c)[1], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("splits", [1, 3, 8, 9, 16, 17, 24, 32, 33, 64, 256])
def test_split_count_invariance(splits):
    c = workloads.decode_case([3000, 1500, 4096], seed=8)
    _check(c, num_splits=splits)


def test_block_size_32():
    c = workloads.decode_case([700, 64, 1025], PBLK=32, seed=9, layout="engine")
    _check(c)


def test_query_rows_and_canary():
    """Sequence s reads q row qsl[s] and writes only out row qsl[s]."""
    c = workloads.decode_case([300, 90, 1200], seed=10)
    T = 9
    g = torch.Generator().manual_seed(11)
    q_all = torch.randn(T, 24, 128, generator=g).to(torch.bfloat16)
    qsl = torch.tensor([1, 4, 8, 9], dtype=torch.int32)
    c2 = dict(c, q=q_all, qsl=qsl)
    ref = _oracle(c2)
    canary = torch.full((T, 24, 128), 3.0, dtype=torch.bfloat16, device=DEV)
    out = _run(c2, out=canary)
    got = out.cpu()
    rows = [1, 4, 8]
    torch.testing.assert_close(got[rows].to(torch.float64), ref, rtol=RTOL, atol=ATOL)
    others = [r for r in range(T) if r not in rows]
    assert torch.all(got[others] == 3.0)


def test_repeat_calls_bitwise_identical():
    """The merge ticket returns to zero after every call, so repeated calls agree bit for bit."""
    c = workloads.decode_case([4096, 2000, 3333, 17], seed=12)
    a = _run(c, num_splits=16).clone()
    for _ in range(3):
        assert torch.equal(_run(c, num_splits=16), a)
    b = _run(c, num_splits=7)                      # other shape on the same scratch buffer
    torch.testing.assert_close(b.float(), a.float(), rtol=RTOL, atol=ATOL)
    assert torch.equal(_run(c, num_splits=16), a)


def test_graph_capture_replay():
    """Captured in a HIP graph and replayed with changing inputs; every replay equals eager."""
    c = workloads.decode_case([2048, 4000], seed=13)
    d = workloads.to_device(c, DEV)
    ks = torch.tensor([c["k_scale"]], device=DEV)
    vs = torch.tensor([c["v_scale"]], device=DEV)
    out = torch.zeros_like(d["q"])
    args = (d["q"], d["k_cache"], d["v_cache"], out, d["qsl"], d["seq_lens"], d["block_table"], ks, vs,
            c["sm_scale"])
    ops.decode_attention(*args, num_splits=16)                 # allocates the scratch outside capture
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            ops.decode_attention(*args, num_splits=16)
    torch.cuda.current_stream().wait_stream(s)
    for it in range(4):
        d["q"].copy_(torch.randn(d["q"].shape, generator=torch.Generator().manual_seed(100 + it))
                     .to(torch.bfloat16).to(DEV))
        d["seq_lens"].copy_(torch.tensor([2048 - 100 * it, 4000 - 7 * it], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = torch.zeros_like(out)
        ops.decode_attention(d["q"], d["k_cache"], d["v_cache"], eager, d["qsl"], d["seq_lens"],
                             d["block_table"], ks, vs, c["sm_scale"], num_splits=16)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {it}"


def test_rejects_unsupported_geometry():
    c = workloads.decode_case([64], D=64, seed=14)
    d = workloads.to_device(c, DEV)
    out = torch.zeros_like(d["q"])
    with pytest.raises(_lib.Fp8kvError) as e:
        ops.decode_attention(d["q"], d["k_cache"], d["v_cache"], out, d["qsl"], d["seq_lens"],
                             d["block_table"], 1.0, 1.0, 1 / math.sqrt(64))
    assert e.value.status == 2


@pytest.mark.parametrize("variant", list(range(7)))
def test_every_launch_variant(variant):
    """Each (waves, chunk, depth) variant the tuning hook can select meets the same bar."""
    lib = _lib.load()
    c = workloads.decode_case([4096, 1500, 33, 2900], seed=15, layout="engine")
    try:
        lib.fp8kv_decode_tune(variant, 0)
        for splits in (1, 4, 8, 13, 32, 37):
            _check(c, num_splits=splits)
    finally:
        lib.fp8kv_decode_tune(-1, 0)


def test_graph_replay_after_scratch_grows():
    """A graph captured with the cached scratch keeps replaying correctly after an eager call
    needs a larger buffer (the old one is kept alive, tickets and records zero)."""
    c = workloads.decode_case([2048, 4000], seed=16)
    d = workloads.to_device(c, DEV)
    ks = torch.tensor([c["k_scale"]], device=DEV)
    vs = torch.tensor([c["v_scale"]], device=DEV)
    out = torch.zeros_like(d["q"])
    args = (d["q"], d["k_cache"], d["v_cache"], out, d["qsl"], d["seq_lens"], d["block_table"], ks, vs,
            c["sm_scale"])
    ops.decode_attention(*args, num_splits=16)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            ops.decode_attention(*args, num_splits=16)
    torch.cuda.current_stream().wait_stream(s)
    before = ops._scratch_cache[("cuda", torch.cuda.current_device())]
    # 64 sequences x 4 kv heads x 64 splits of GQA-6 records: about 51 MB, beyond the cached buffer
    big = workloads.decode_case([300] * 64, seed=17)
    ref_big = _oracle(big)
    torch.testing.assert_close(_rows(big, _run(big, num_splits=64)), ref_big, rtol=RTOL, atol=ATOL)
    assert ops._scratch_cache[("cuda", torch.cuda.current_device())] is not before
    for it in range(3):
        d["q"].copy_(torch.randn(d["q"].shape, generator=torch.Generator().manual_seed(200 + it))
                     .to(torch.bfloat16).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = torch.zeros_like(out)
        ops.decode_attention(d["q"], d["k_cache"], d["v_cache"], eager, d["qsl"], d["seq_lens"],
                             d["block_table"], ks, vs, c["sm_scale"], num_splits=16)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {it}"


def test_scratch_reset_recovers_a_dirty_buffer():
    """Non-zero tickets (as a launch that never completed would leave) misplace the merge;
    fp8kv_decode_scratch_reset restores the zero state and the next calls are exact."""
    c = workloads.decode_case([3000, 1500, 4096], seed=18)
    ref = _oracle(c)
    d = workloads.to_device(c, DEV)
    ks = torch.tensor([c["k_scale"]], device=DEV)
    vs = torch.tensor([c["v_scale"]], device=DEV)
    need = ops.decode_scratch_bytes(3, 24, 4, 8)
    scratch = torch.full((need + 100,), 0x5A, dtype=torch.uint8, device=DEV)
    ops.decode_scratch_reset(scratch)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(scratch)) == 0
    for _ in range(2):
        out = torch.zeros_like(d["q"])
        ops.decode_attention(d["q"], d["k_cache"], d["v_cache"], out, d["qsl"], d["seq_lens"],
                             d["block_table"], ks, vs, c["sm_scale"], num_splits=8, scratch=scratch)
        torch.cuda.synchronize()
        torch.testing.assert_close(_rows(c, out), ref, rtol=RTOL, atol=ATOL)
        assert int(torch.count_nonzero(scratch[:256 << 10])) == 0   # every call leaves the tickets zero


def test_merge_is_independent_of_the_merging_split():
    """The merging workgroup is whichever split of a pair finishes last, which varies from call to
    call; the merge runs in split order, so 20 calls agree bit for bit."""
    c = workloads.decode_case([4096] * 8, pool_blocks=5060, seed=19, layout="engine")
    a = _run(c, num_splits=8).clone()
    for _ in range(20):
        assert torch.equal(_run(c, num_splits=8), a)


# ---- bf16 caches (the reference's K_FP8 = False branch, vllm-fp8kv/fp8kv_v3.py:44-45,61-66,110,135):
# fp8kv_decode_attn_bf16, values used as stored, scales ignored.

@pytest.mark.parametrize("layout", ["standalone", "engine"])
@pytest.mark.parametrize("num_splits", [None, 1, 3, 8, 33])
def test_bf16_kv_batch(layout, num_splits):
    """bf16 K/V, 8 sequences of mixed length (edge lengths included), both cache layouts; the scales
    passed (0.5, 2.0) must play no part."""
    c = workloads.decode_case([1, 15, 16, 17, 100, 511, 2048, 3001], pool_blocks=400, seed=21,
                              layout=layout, kv_gen="bf16")
    ref = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], 1.0, 1.0, c["sm_scale"])
    got = _rows(c, _run(c, ks=0.5, vs=2.0, num_splits=num_splits))
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (16, 4), (32, 8), (16, 1), (28, 4)])
def test_bf16_kv_head_geometries(hq, hkv):
    c = workloads.decode_case([700, 64, 2500], HQ=hq, HKV=hkv, pool_blocks=300, seed=hq + hkv,
                              kv_gen="bf16")
    torch.testing.assert_close(_rows(c, _run(c)), _oracle(c), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("pblk", [32, 64])
def test_bf16_kv_block_sizes(pblk):
    c = workloads.decode_case([1000, 77], PBLK=pblk, seed=pblk, kv_gen="bf16", layout="engine")
    torch.testing.assert_close(_rows(c, _run(c)), _oracle(c), rtol=RTOL, atol=ATOL)


def test_bf16_kv_b8_4k_and_zero_context():
    """b8@4k over a 5060-block bf16 pool, plus a batch whose first sequence has no context (zeros)."""
    c = workloads.decode_case([4096] * 8, pool_blocks=5060, seed=22, layout="engine", kv_gen="bf16")
    torch.testing.assert_close(_rows(c, _run(c)), _oracle(c), rtol=RTOL, atol=ATOL)
    c = workloads.decode_case([0, 300], seed=23, kv_gen="bf16")
    got = _rows(c, _run(c))
    assert torch.count_nonzero(got[0]) == 0
    torch.testing.assert_close(got, _oracle(c), rtol=RTOL, atol=ATOL)


def test_bf16_kv_through_the_reference_run():
    """fp8kv_v3.run (the reference's signature) takes bf16 caches as the reference does."""
    import fp8kv_v3
    c = workloads.decode_case([64, 100], seed=20, kv_gen="bf16")
    d = workloads.to_device(c, DEV)
    out = torch.full_like(d["q"], 5.0)
    fp8kv_v3.run(d["q"], d["k_cache"], d["v_cache"], out, d["qsl"], d["seq_lens"], d["block_table"],
                 0.3, 7.0, c["sm_scale"])
    torch.cuda.synchronize()
    torch.testing.assert_close(_rows(c, out), _oracle(c), rtol=RTOL, atol=ATOL)


def test_mixed_cache_dtypes_are_rejected():
    """K bf16 with V e4m3 (or the reverse) is refused before anything is launched."""
    c = workloads.decode_case([64], seed=24)
    d = workloads.to_device(c, DEV)
    kb = d["k_cache"].to(torch.bfloat16)
    out = torch.full_like(d["q"], 5.0)
    with pytest.raises(ValueError, match="both caches bf16"):
        ops.decode_attention(d["q"], kb, d["v_cache"], out, d["qsl"], d["seq_lens"], d["block_table"],
                             1.0, 1.0, c["sm_scale"])
    torch.cuda.synchronize()
    assert torch.all(out == 5.0)
