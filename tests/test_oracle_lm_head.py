"""Pins of the lm_head top-k / rerank oracle (oracle/lm_head.py) on the CPU."""
import functools
import math

import numpy as np
import pytest
import torch

from oracle import lm_head


def _torch_order(v):
    return torch.sort(torch.from_numpy(np.asarray(v, np.float64)), descending=True, stable=True).indices.numpy()


def _brute(v):
    def cmp(a, b):
        va, vb = v[a], v[b]
        na, nb = math.isnan(va), math.isnan(vb)
        if na != nb:
            return -1 if na else 1
        if not na and va != vb:
            return -1 if va > vb else 1
        return -1 if a < b else (1 if a > b else 0)
    return np.array(sorted(range(len(v)), key=functools.cmp_to_key(cmp)))


def _values(seed, n=500):
    g = np.random.default_rng(seed)
    v = g.integers(-5, 6, n).astype(np.float64) * 0.5          # many ties
    v[g.integers(0, n, 7)] = np.nan
    v[g.integers(0, n, 3)] = np.inf
    v[g.integers(0, n, 3)] = -np.inf
    v[g.integers(0, n, 5)] = -0.0
    v[g.integers(0, n, 5)] = 0.0
    return v


@pytest.mark.parametrize("seed", range(5))
def test_rank_order_matches_torch_stable_sort(seed):
    v = _values(seed)
    assert np.array_equal(lm_head.rank_order(v), _torch_order(v))


@pytest.mark.parametrize("seed", range(5))
def test_rank_order_matches_brute_force(seed):
    v = _values(seed, n=60)
    assert np.array_equal(lm_head.rank_order(v), _brute(list(v)))


def test_planted_reversed_tiebreak_fails():
    v = _values(7)
    planted = np.lexsort((-np.arange(len(v)), -np.where(np.isnan(v), 0, v), ~np.isnan(v)))
    assert not np.array_equal(planted, _torch_order(v))


def test_topk_rows_prefix_of_rank_order():
    g = np.random.default_rng(3)
    L = g.standard_normal((3, 1000))
    vals, idx = lm_head.topk_rows(L, 10)
    for m in range(3):
        t = torch.topk(torch.from_numpy(L[m]), 10)
        assert np.array_equal(idx[m], t.indices.numpy()) and np.allclose(vals[m], t.values.numpy())


def test_rerank_against_torch_matmul():
    g = np.random.default_rng(4)
    E = g.standard_normal((300, 64))
    X = g.standard_normal((2, 64))
    cand = np.array([[5, 17, 299, 5, -1, 300, 42, 0], [1, 2, 3, 4, 5, 6, 7, 8]])
    vals, idx = lm_head.rerank(E, X, cand)
    for m in range(2):
        c = cand[m]
        ok = (c >= 0) & (c < 300)
        sc = (torch.from_numpy(E[c[ok]]) @ torch.from_numpy(X[m])).numpy()
        order = np.argsort(-sc, kind="stable")
        assert np.array_equal(idx[m, :ok.sum()], c[ok][order])
        assert np.allclose(vals[m, :ok.sum()], sc[order])
        assert np.all(idx[m, ok.sum():] == -1) and np.all(np.isneginf(vals[m, ok.sum():]))
    # the repeated index 5 keeps both entries, adjacent
    assert list(idx[0]).count(5) == 2
