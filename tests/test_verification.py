"""The reference harness helpers prepare_queries_from_meta and compute_recall_exact
(src/run_correctness_verification.py:87-125), on the CPU: hand-made cases with
known answers, brute force over Python sorts and sets, and the drop-in import."""
import importlib
import os
import sys

import numpy as np
import pytest
import torch

import gpusparse
from gpusparse.verification import compute_recall_exact, prepare_queries_from_meta

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_prepare_queries_hand_made():
    dense = np.zeros((4, 10), dtype=np.float32)
    dense[0, [2, 7, 5]] = [0.5, 2.0, 1.0]
    dense[1, [9, 0, 4, 3]] = [0.25, 0.25, 3.0, 0.25]  # a tie: which two of the three is numpy's order
    dense[3, 1] = -1.5  # negative weights are nonzeros too, ranked by value
    ti, ts, back = prepare_queries_from_meta({"query_dense": dense}, max_terms=3, device="cpu")
    assert ti.dtype == torch.int32 and ts.dtype == torch.float32 and ti.shape == (4, 3)
    ti, ts = ti.tolist(), ts.tolist()
    assert ti[0] == [7, 5, 2] and ti[2] == [-1, -1, -1] and ti[3] == [1, -1, -1]
    assert ti[1][0] == 4 and set(ti[1][1:]) < {0, 3, 9} and len(set(ti[1][1:])) == 2
    assert ts == [[2.0, 1.0, 0.5], [3.0, 0.25, 0.25], [0.0, 0.0, 0.0], [-1.5, 0.0, 0.0]]
    assert back is dense


@pytest.mark.parametrize("max_terms", [1, 7, 128])
def test_prepare_queries_brute_force(max_terms):
    """Distinct weights: each row is its nonzeros sorted by weight, heaviest first,
    cut at max_terms (Python's sorted over (weight, term) pairs); torch input."""
    rng = np.random.default_rng(max_terms)
    n, V = 30, 3000
    dense = np.zeros((n, V), dtype=np.float32)
    for q in range(n):
        nnz = int(rng.integers(0, 200))
        terms = rng.choice(V, nnz, replace=False)
        dense[q, terms] = rng.permutation(np.arange(1, nnz + 1, dtype=np.float32)) / 8.0
    ti, ts, back = prepare_queries_from_meta({"query_dense": torch.from_numpy(dense)}, max_terms, device="cpu")
    assert isinstance(back, np.ndarray) and np.array_equal(back, dense)
    for q in range(n):
        pairs = sorted(((float(dense[q, t]), t) for t in range(V) if dense[q, t] != 0), reverse=True)[:max_terms]
        want_t = [t for _, t in pairs] + [-1] * (max_terms - len(pairs))
        want_w = [w for w, _ in pairs] + [0.0] * (max_terms - len(pairs))
        assert ti[q].tolist() == want_t and ts[q].tolist() == want_w


def test_prepare_queries_ties_in_long_rows():
    """Rows of many equal weights: weights descending, and the kept weights are
    the row's max_terms largest as a multiset; every kept term holds its weight."""
    rng = np.random.default_rng(5)
    dense = np.zeros((12, 2000), dtype=np.float32)
    for q in range(12):
        terms = rng.choice(2000, 300, replace=False)
        dense[q, terms] = rng.integers(1, 6, 300) / 4.0
    ti, ts, _ = prepare_queries_from_meta({"query_dense": dense}, 100, device="cpu")
    ti, ts = ti.numpy(), ts.numpy()
    for q in range(12):
        assert np.all(np.diff(ts[q]) <= 0)
        assert np.array_equal(ts[q], np.sort(dense[q][dense[q] != 0])[::-1][:100])
        assert np.array_equal(dense[q, ti[q]], ts[q]) and len(set(ti[q].tolist())) == 100


def test_prepare_queries_rejects_bad_input():
    with pytest.raises(ValueError):
        prepare_queries_from_meta({"query_dense": np.zeros(5)}, device="cpu")
    with pytest.raises(ValueError):
        prepare_queries_from_meta({"query_dense": np.zeros((2, 5))}, max_terms=0, device="cpu")


def test_recall_hand_made():
    gpu = np.array([[1, 2, 3, 4], [5, 5, 6, 7]])
    cpu = np.array([[1, 2, 9, 8], [5, 6, 6, 6]])
    r = compute_recall_exact(gpu, cpu, k_values=[2, 4, 10])
    # k=2: {1,2} vs {1,2} -> 2 of 2; {5,6} vs {5} -> 1 of 2.  k=4: 2 of 4; {5,6} vs {5,6,7} -> 2 of 2
    assert r == {"recall@2": 0.75, "recall@4": 4 / 6}
    assert compute_recall_exact(gpu, cpu) == {}  # default ks 10/100/1000 are all wider than 4
    assert compute_recall_exact(np.zeros((0, 5)), np.zeros((0, 5)), [3]) == {"recall@3": 0.0}
    with pytest.raises(ValueError):
        compute_recall_exact(gpu, cpu[:1])


def test_recall_brute_force():
    rng = np.random.default_rng(11)
    gpu = torch.from_numpy(rng.integers(-1, 60, (40, 120)))
    cpu = rng.integers(-1, 60, (40, 100))
    got = compute_recall_exact(gpu, cpu, k_values=[1, 10, 100, 120])
    assert set(got) == {"recall@1", "recall@10", "recall@100"}
    for k in (1, 10, 100):
        hit = total = 0
        for q in range(40):
            truth = set(cpu[q, :k].tolist())
            hit += len(truth & set(gpu[q, :k].tolist()))
            total += len(truth)
        assert got[f"recall@{k}"] == hit / total


def test_helpers_served_by_dropin_module():
    d = os.path.join(ROOT, "gpu-sparse_amd", "dropin")
    sys.path.insert(0, d)
    try:
        mod = importlib.import_module("run_correctness_verification")
        assert mod.prepare_queries_from_meta is gpusparse.prepare_queries_from_meta
        assert mod.compute_recall_exact is gpusparse.compute_recall_exact
        assert mod.VOCAB_SIZE == 30522
    finally:
        sys.path.remove(d)
