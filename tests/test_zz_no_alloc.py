"""fp8kv_decode_attn_noalloc (the decode entry point that allocates nothing, its scratch a device
array inside the library) against fp8kv_decode_attn with a caller scratch, through the C ABI.

The two run the same kernel with the same split count, so their outputs must agree bit for bit;
both are also held to the fp64 oracle at the attention bar (rtol = atol = 1e-2).  Two calls in a
row, the second smaller, check that the shared array carries nothing from one call into the
next.  Collected last (test_zz_*): the round's end runs the GPU suite with -x.
"""
import ctypes
import math

import pytest
import torch

from fp8kv_amd import _lib, ops, workloads
from oracle import attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
RTOL = ATOL = 1e-2
NOALLOC_MAX = 8 << 20


def _args(d, c, out, num_splits):
    kc, vc, q = d["k_cache"], d["v_cache"], d["q"]
    ks = torch.tensor([c["k_scale"]], dtype=torch.float32, device=DEV)
    vs = torch.tensor([c["v_scale"]], dtype=torch.float32, device=DEV)
    d["_keep"] = (ks, vs)
    NS, HQ, HKV, PBLK = d["block_table"].shape[0], q.shape[1], kc.shape[2], kc.shape[1]
    return [q.data_ptr(), q.stride(0), kc.data_ptr(), vc.data_ptr(),
            kc.stride(0), kc.stride(1), kc.stride(2), vc.stride(0), vc.stride(1), vc.stride(2),
            out.data_ptr(), out.stride(0), d["qsl"].data_ptr(), d["seq_lens"].data_ptr(),
            d["block_table"].data_ptr(), d["block_table"].stride(0), ks.data_ptr(), vs.data_ptr(),
            ctypes.c_float(c["sm_scale"]), NS, HQ, HKV, q.shape[2], PBLK, num_splits]


def _both(c, num_splits):
    lib = _lib.load()
    d = workloads.to_device(c, DEV)
    stream = torch.cuda.current_stream().cuda_stream
    NS, HQ, HKV = d["block_table"].shape[0], d["q"].shape[1], d["k_cache"].shape[2]
    need = ops.decode_scratch_bytes(NS, HQ, HKV, num_splits)
    assert 0 < need <= NOALLOC_MAX
    scratch = torch.zeros(need, dtype=torch.uint8, device=DEV)
    ref_out = torch.full_like(d["q"], 5.0)
    st = lib.fp8kv_decode_attn(*_args(d, c, ref_out, num_splits), scratch.data_ptr(), need, stream)
    assert st == 0, st
    out = torch.full_like(d["q"], 5.0)
    st = lib.fp8kv_decode_attn_noalloc(*_args(d, c, out, num_splits), stream)
    assert st == 0, st
    torch.cuda.synchronize()
    return ref_out, out


def _check(c, num_splits):
    ref_out, out = _both(c, num_splits)
    assert torch.equal(out, ref_out)
    rows = c["qsl"][:-1].long()
    ref = attention.decode_attention(c["q"], c["k_cache"], c["v_cache"], c["qsl"], c["seq_lens"],
                                     c["block_table"], c["k_scale"], c["v_scale"], c["sm_scale"])
    torch.testing.assert_close(out.cpu()[rows].to(torch.float64), ref, rtol=RTOL, atol=ATOL)


def test_noalloc_matches_scratch_entry_point_two_calls():
    """b8@4k with the planned 8 splits, then a smaller batch with other lengths and splits."""
    big = workloads.decode_case([4096] * 8, pool_blocks=5060, seed=31, layout="engine")
    _check(big, ops.decode_num_splits(8, 4, 4096))
    small = workloads.decode_case([700, 33, 1], seed=32)
    _check(small, 5)


def test_noalloc_rejects_scratch_beyond_its_array():
    """64 sequences x 4 kv heads x 64 splits need ~51 MB: refused with FP8KV_ERR_SCRATCH and
    nothing launched (the output keeps its canary)."""
    lib = _lib.load()
    c = workloads.decode_case([64] * 64, seed=33)
    d = workloads.to_device(c, DEV)
    assert ops.decode_scratch_bytes(64, 24, 4, 64) > NOALLOC_MAX
    out = torch.full_like(d["q"], 5.0)
    st = lib.fp8kv_decode_attn_noalloc(*_args(d, c, out, 64), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st == 5 and torch.all(out == 5.0)
    # a split count that fits on the same batch still works right after the refusal
    _check(c, 2)


def test_noalloc_graph_replays():
    """The no-allocation call captured in a HIP graph: every replay, with new query values copied
    into the captured input between replays (and eager calls of the other entry point in
    between), equals an eager fp8kv_decode_attn call on the same inputs bit for bit."""
    lib = _lib.load()
    c = workloads.decode_case([1500, 4096, 77, 2048], pool_blocks=2000, seed=34, layout="engine")
    d = workloads.to_device(c, DEV)
    NS, HQ, HKV = 4, d["q"].shape[1], d["k_cache"].shape[2]
    nsplit = ops.decode_num_splits(NS, HKV, 4096)
    out = torch.zeros_like(d["q"])
    args = _args(d, c, out, nsplit)
    keep = d["_keep"]                   # the captured call's scale tensors stay alive
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            assert lib.fp8kv_decode_attn_noalloc(*args, s.cuda_stream) == 0
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    need = ops.decode_scratch_bytes(NS, HQ, HKV, nsplit)
    scratch = torch.zeros(need, dtype=torch.uint8, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(35)
    for rep in range(4):
        d["q"].copy_(torch.randn(d["q"].shape, device=DEV, generator=gen).to(torch.bfloat16))
        out.fill_(5.0)
        g.replay()
        torch.cuda.synchronize()
        ref_out = torch.full_like(d["q"], 7.0)
        st = lib.fp8kv_decode_attn(*_args(d, c, ref_out, nsplit), scratch.data_ptr(), need,
                                   torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert st == 0
        assert torch.equal(out, ref_out), f"replay {rep}"
    del g, keep
