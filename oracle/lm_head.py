"""lm_head top-k and exact rerank restated on the CPU (numpy, fp64).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference engine ends a decode step with a draft lm_head over the tied embedding, an exact
rerank of its candidates and torch's top-k (profiling/prof_h4mv.txt:6,10,19;
docs/06-w4gemm-hip-roadmap.md:116).  The draft's int2 format is closed; this build's draft is the
embedding in MXFP4, so its logits are the matvec oracle's (``matvec.w4mv``).

Rank order: value descending, NaN above every number, +0 == -0, then index ascending (and, in a
rerank, candidate position for a repeated index).

Pinned by (tests/test_oracle_lm_head.py):
  * ``rank_order`` against torch.sort(descending=True, stable=True) - a library routine - on
    values with NaN, +-inf, +-0 and many ties, and against a pure-Python sorted() on small cases;
  * a planted mistake (ties broken by the higher index) failing the same checks;
  * ``rerank`` against torch's fp64 matmul of the gathered rows, sorted by ``rank_order``.
"""
from __future__ import annotations

import numpy as np

from . import matvec


def rank_order(values: np.ndarray, tiebreak: np.ndarray | None = None) -> np.ndarray:
    """Indices of ``values`` (1-D) in rank order; ``tiebreak`` (default: the position) orders
    equal values, ascending."""
    v = np.asarray(values, dtype=np.float64)
    n = v.shape[0]
    pos = np.arange(n)
    tb = pos if tiebreak is None else np.asarray(tiebreak)
    nan = np.isnan(v)
    w = np.where(nan, 0.0, v)
    # lexsort: the last key is the primary one.
    return np.lexsort((pos, tb, -w, ~nan))


def topk_rows(logits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """(values, indices) [M, k] of the k top logits of each row, in rank order."""
    L = np.asarray(logits, dtype=np.float64)
    idx = np.stack([rank_order(row)[:k] for row in L])
    vals = np.take_along_axis(L, idx, axis=1)
    return vals, idx


def w4_topk(W: np.ndarray, St: np.ndarray, X: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(values, indices, logits) of the MXFP4 draft head: logits = X . dequant(W, St)^T in fp64."""
    logits = matvec.w4mv(W, St, X)
    v, i = topk_rows(logits, k)
    return v, i, logits


def rerank(E: np.ndarray, X: np.ndarray, cand: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(values, indices) [M, C]: candidate rows of E (bf16 values as float) rescored against X in
    fp64 and put in rank order; indices outside [0, V) go last (value -inf, index -1) in
    candidate order, a repeated index keeps its candidate order."""
    E = np.asarray(E, dtype=np.float64)
    X = np.asarray(X, dtype=np.float64)
    cand = np.asarray(cand, dtype=np.int64)
    V = E.shape[0]
    M, C = cand.shape
    vals = np.full((M, C), -np.inf)
    idx = np.full((M, C), -1, dtype=np.int64)
    for m in range(M):
        ok = (cand[m] >= 0) & (cand[m] < V)
        good = np.nonzero(ok)[0]
        sc = E[cand[m, good]] @ X[m]
        order = rank_order(sc, tiebreak=cand[m, good])
        n = len(good)
        vals[m, :n] = sc[order]
        idx[m, :n] = cand[m, good][order]
    return vals, idx
