"""GPU parity of the lm_head top-k (h4mv_topk) and the exact rerank (fp8kv_rerank_exact) against
the CPU oracle (oracle/lm_head.py).

Bars: top-k values within the matvec bar of the fp64 oracle (2e-3 of the row's largest |logit|),
indices equal to the oracle's at every rank whose neighbours are farther apart than twice that
bar (closer values may swap legitimately under fp32 accumulation); ties of bit-identical logits
ordered by index (exact); the rerank's values within 1e-4 of the row's largest |score| and its
order equal to the oracle's wherever the margins allow.  The vocabulary case uses the reference
model's lm_head shape (vocab 128167, hidden 3584; docs/06-w4gemm-hip-roadmap.md:116).
"""
import numpy as np
import pytest
import torch

from fp8kv_amd import _lib, ops, workloads
from oracle import lm_head, matvec

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
TOL = 2e-3


def _check_topk(vals, idx, rv, ri, scale, tol):
    vals, idx = vals.cpu().numpy().astype(np.float64), idx.cpu().numpy().astype(np.int64)
    M, k = rv.shape
    assert np.all(np.abs(vals - rv) <= tol * scale[:, None]), np.abs(vals - rv).max()
    for m in range(M):
        gap = np.abs(np.diff(rv[m]))
        for r in range(k):
            left = gap[r - 1] if r > 0 else np.inf
            right = gap[r] if r < k - 1 else np.inf
            if min(left, right) > 2 * tol * scale[m]:
                assert idx[m, r] == ri[m, r], (m, r, idx[m, :r + 2], ri[m, :r + 2])


def _case_topk(N, K, M, k, seed):
    c = workloads.w4_case(N=N, K=K, M=M, seed=seed)
    vals, idx = ops.lm_head_topk(c["X"].to(DEV), c["W"].to(DEV), c["St"].to(DEV), k)
    torch.cuda.synchronize()
    rv, ri, logits = lm_head.w4_topk(c["W"].numpy(), c["St"].numpy(), c["X"].float().numpy(), k)
    # the boundary: the (k+1)-th value must not be closer to the k-th than the bar either
    _check_topk(vals, idx, rv, ri, np.abs(logits).max(axis=1), TOL)
    return vals, idx, rv, ri


@pytest.mark.parametrize("M,k", [(1, 1), (1, 64), (2, 64), (4, 8), (8, 50)])
def test_vocab_topk(M, k):
    """The reference model's lm_head: vocab 128167 (not a multiple of 16), hidden 3584."""
    _case_topk(128167, 3584, M, k, seed=600 + M + k)


@pytest.mark.parametrize("N,K,M,k", [(100, 256, 2, 64), (64, 256, 1, 64), (4096, 512, 1, 33), (4097, 512, 3, 64),
                                     (17, 64, 1, 5), (40000, 1024, 16, 64)])
def test_topk_shapes(N, K, M, k):
    """k = N, one chunk, exactly one chunk, one logit past a chunk, tiny N, M = 16."""
    _case_topk(N, K, M, k, seed=N + K + M + k)


def test_argmax_equals_full_logits_argmax():
    c = workloads.w4_case(N=128167, K=3584, M=2, seed=77)
    vals, idx = ops.lm_head_topk(c["X"].to(DEV), c["W"].to(DEV), c["St"].to(DEV), 1)
    full = ops.h4mv(c["X"].to(DEV), c["W"].to(DEV), c["St"].to(DEV), out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = torch.topk(full.cpu(), 1)
    assert torch.equal(idx.cpu().long(), ref.indices) and torch.equal(vals.cpu(), ref.values)


def test_ties_break_by_lower_index_and_nan_first():
    """Rows 10, 4000, 70000 and 127999 are copies of the strongest row (bit-identical fp32 logits):
    they rank in index order; a row with scale byte 255 (NaN) ranks above everything."""
    N, K = 128167, 512
    c = workloads.w4_case(N=N, K=K, M=1, seed=78)
    W, St = c["W"].clone(), c["St"].clone()
    logits = matvec.w4mv(W.numpy(), St.numpy(), c["X"].float().numpy())[0]
    top = int(np.argmax(logits))
    for r in (10, 4000, 70000, 127999):
        W[r] = W[top]
        St[r] = St[top]
    St[55] = 255
    vals, idx = ops.lm_head_topk(c["X"].to(DEV), W.to(DEV), St.to(DEV), 6)
    torch.cuda.synchronize()
    got = idx.cpu().tolist()[0]
    assert got[0] == 55 and np.isnan(vals[0, 0].item())
    assert got[1:6] == sorted([10, 4000, 70000, 127999, top])
    assert len(set(vals[0, 1:6].tolist())) == 1


def test_topk_rejects_bad_k():
    """k above 64 is refused on the host; k above N by the library (FP8KV_ERR_SHAPE)."""
    c = workloads.w4_case(N=64, K=64, M=1, seed=1)
    with pytest.raises(ValueError):
        ops.lm_head_topk(c["X"].to(DEV), c["W"].to(DEV), c["St"].to(DEV), 65)
    c = workloads.w4_case(N=20, K=64, M=1, seed=2)
    with pytest.raises(_lib.Fp8kvError) as e:
        ops.lm_head_topk(c["X"].to(DEV), c["W"].to(DEV), c["St"].to(DEV), 21)
    assert e.value.status == 2


def _emb(V, H, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(V, H, generator=g) * 0.05).to(torch.bfloat16)


def test_rerank_exact_against_oracle():
    V, H, M, C = 5000, 3584, 3, 64
    E = _emb(V, H, 90)
    g = torch.Generator().manual_seed(91)
    X = torch.randn(M, H, generator=g).to(torch.bfloat16)
    cand = torch.randint(0, V, (M, C), generator=g, dtype=torch.int32)
    cand[0, 5] = -1
    cand[0, 9] = V + 3
    cand[1, 7] = cand[1, 2]                     # a repeated index
    vals, idx = ops.rerank_exact(E.to(DEV), X.to(DEV), cand.to(DEV))
    torch.cuda.synchronize()
    rv, ri = lm_head.rerank(E.float().numpy(), X.float().numpy(), cand.numpy())
    scale = np.abs(np.where(np.isfinite(rv), rv, 0)).max(axis=1)
    v = vals.cpu().numpy().astype(np.float64)
    fin = np.isfinite(rv)
    assert np.array_equal(np.isfinite(v), fin)
    assert np.all(np.abs(v[fin] - rv[fin]) <= 1e-4 * np.repeat(scale[:, None], C, 1)[fin])
    _check_topk(vals.masked_fill(~torch.from_numpy(fin).to(DEV), 0), idx, np.where(fin, rv, 0), ri, scale, 1e-4)
    assert idx[0, -2:].tolist() == [-1, -1]


def test_draft_then_rerank_recovers_the_exact_argmax():
    """The chain the reference runs: an approximate head proposes candidates, the exact rows rank
    them.  W is a random MXFP4 head, E = dequant(W) + small bf16 noise: the draft's top 64 holds
    E's true best row, and the rerank puts it first (where the margin allows)."""
    V, H, M = 40000, 3584, 2
    c = workloads.w4_case(N=V, K=H, M=M, seed=92)
    Wd = matvec.dequant_w4(c["W"].numpy(), c["St"].numpy())
    g = np.random.default_rng(93)
    E = torch.from_numpy((Wd + g.standard_normal(Wd.shape) * 1e-3 * np.abs(Wd).mean()).astype(np.float32)).to(torch.bfloat16)
    del Wd
    x = c["X"]
    _, cand = ops.lm_head_topk(x.to(DEV), c["W"].to(DEV), c["St"].to(DEV), 64)
    vals, idx = ops.rerank_exact(E.to(DEV), x.to(DEV), cand)
    torch.cuda.synchronize()
    exact = (E.double() @ x.double().T).T.numpy()
    for m in range(M):
        o = lm_head.rank_order(exact[m])
        if exact[m, o[0]] - exact[m, o[1]] > 1e-4 * np.abs(exact[m]).max():
            assert int(idx[m, 0]) == int(o[0])
