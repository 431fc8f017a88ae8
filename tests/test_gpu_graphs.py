"""HIP-graph capture and replay of the hot-path entry points (the engine replays decode-step
graphs: the reference captures its decode launches, fp8kv_override.py:90 and
docs/03-fp8kv-pathology-and-kernel.md:34-35, and the linear hook runs inside compiled graphs,
docs/04-w4a8-matvec-wall.md:74).

Each test captures one call on a side stream, then, several times, rewrites the inputs in place,
replays, and checks the replay's output bit for bit against an eager call on the same inputs
(every kernel here is deterministic), with eager work and synchronisations between replays.
"""
import math

import pytest
import torch

from fp8kv_amd import ops, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _capture(fn):
    fn()                                              # eager first: nothing lazy inside capture
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    return graph


@pytest.mark.parametrize("N,K,M", [(28672, 4096, 1), (37888, 3584, 1), (37888, 3584, 8), (4096, 3584, 8),
                                   (3584, 18944, 8), (4096, 3584, 1), (40003, 3584, 8), (70000, 4096, 8)])
def test_matvec_replay(N, K, M):
    """M = 1 kernel (cfg1 and gate/up at M = 1), K-slice kernel (gate/up, M = 8; a partial last
    tile at N = 40003), its batched form (N = 70000: more tiles than one round of the plain
    kernel holds) and streaming kernel (the small-N shapes)."""
    c = workloads.w4_case(N=N, K=K, M=M, seed=N + M)
    X, W, St = c["X"].to(DEV), c["W"].to(DEV), c["St"].to(DEV)
    Y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    graph = _capture(lambda: ops.h4mv(X, W, St, out=Y))
    for it in range(3):
        X.copy_(torch.randn(M, K, generator=torch.Generator().manual_seed(it)).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(Y, ops.h4mv(X, W, St)), f"replay {it}"


@pytest.mark.parametrize("M", [8, 1])
def test_fused_silu_replay(M):
    """The fused gate/up + SiLU-and-mul matvec on the K-slice kernel (M = 8) and the M = 1 kernel."""
    N, K = 37888, 3584
    c = workloads.w4_case(N=N, K=K, M=M, seed=3)
    wi, si = ops.interleave_gate_up(c["W"].to(DEV), c["St"].to(DEV))
    X = c["X"].to(DEV)
    Y = torch.empty(M, N // 2, dtype=torch.bfloat16, device=DEV)
    graph = _capture(lambda: ops.h4mv_silu_mul(X, wi, si, out=Y))
    for it in range(3):
        X.copy_(torch.randn(M, K, generator=torch.Generator().manual_seed(10 + it)).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(Y, ops.h4mv_silu_mul(X, wi, si)), f"replay {it}"


def test_cache_write_replay():
    T, HKV, D, PBLK, NB = 8, 4, 128, 16, 64
    kv = torch.zeros(NB, HKV, PBLK, 2 * D, dtype=torch.uint8, device=DEV)
    kc, vc = workloads.engine_views(kv, D)
    key = torch.empty(T, HKV, D, dtype=torch.bfloat16, device=DEV)
    value = torch.empty_like(key)
    slots = torch.empty(T, dtype=torch.int64, device=DEV)
    ks = torch.tensor([0.02], device=DEV)
    vs = torch.tensor([0.03], device=DEV)

    def fill(it):
        g = torch.Generator().manual_seed(20 + it)
        key.copy_(torch.randn(T, HKV, D, generator=g).to(torch.bfloat16))
        value.copy_(torch.randn(T, HKV, D, generator=g).to(torch.bfloat16))
        slots.copy_(torch.randperm(NB * PBLK, generator=g)[:T])

    fill(0)
    graph = _capture(lambda: ops.cache_write(key, value, kc, vc, slots, ks, vs))
    for it in range(3):
        fill(it + 1)
        kv.zero_()
        graph.replay()
        torch.cuda.synchronize()
        got = kv.clone()
        kv.zero_()
        ops.cache_write(key, value, kc, vc, slots, ks, vs)
        torch.cuda.synchronize()
        assert torch.equal(got, kv), f"replay {it}"


def test_prefill_replay():
    qlen, q0 = 600, 1100                                   # split kernel (context >= 1024)
    c = workloads.prefill_case([qlen], [q0], seed=5, layout="engine")
    d = workloads.to_device(c, DEV)
    ks = torch.tensor([c["k_scale"]], device=DEV)
    vs = torch.tensor([c["v_scale"]], device=DEV)
    out = torch.zeros_like(d["q"])

    def call(o):
        ops.prefill_attention(d["q"], d["k_cache"], d["v_cache"], o, d["block_table"], ks, vs,
                              c["sm_scale"], q0, qlen)

    graph = _capture(lambda: call(out))
    for it in range(3):
        d["q"].copy_(torch.randn(d["q"].shape, generator=torch.Generator().manual_seed(30 + it))
                     .to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        eager = torch.zeros_like(out)
        call(eager)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {it}"
