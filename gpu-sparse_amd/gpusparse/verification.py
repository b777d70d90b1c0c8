"""Helpers of the reference's correctness harness (src/run_correctness_verification.py):
query tensors from cached dense query metadata, and recall of one ranking against
another.  Host-side numpy; the searches they feed run on the GPU."""
from __future__ import annotations

import numpy as np
import torch


def _host_array(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def prepare_queries_from_meta(meta, max_terms: int = 128, device="cuda:0"):
    """(term_ids int32 [n, max_terms], term_scores float32 [n, max_terms], query_dense)
    from meta["query_dense"], a dense [n, vocab] query-weight matrix (numpy or
    torch), as src/run_correctness_verification.py:87-107 builds them.

    Each row keeps its nonzero terms in descending weight order, at most
    max_terms of them (the heaviest), padded with term -1 / weight 0.  Equal
    weights keep the order numpy's default argsort of the negated weights gives
    them (over the row's nonzeros in ascending term order), which is the order
    the reference harness produces, so the arrays match it element for element.
    The third item is meta["query_dense"] as a numpy array."""
    if max_terms < 1:
        raise ValueError(f"max_terms must be positive, got {max_terms}")
    dense = _host_array(meta["query_dense"])
    if dense.ndim != 2:
        raise ValueError(f"query_dense must be 2-D [queries, vocab], got shape {dense.shape}")
    n = dense.shape[0]
    term_ids = np.full((n, max_terms), -1, dtype=np.int32)
    term_scores = np.zeros((n, max_terms), dtype=np.float32)
    rows, cols = np.nonzero(dense)  # row-major: each row's terms ascending
    bounds = np.searchsorted(rows, np.arange(n + 1))
    for q in range(n):
        c = cols[bounds[q]:bounds[q + 1]]
        if c.size == 0:
            continue
        w = dense[q, c]
        keep = np.argsort(-w)[:max_terms]
        term_ids[q, :keep.size] = c[keep]
        term_scores[q, :keep.size] = w[keep]
    return torch.from_numpy(term_ids).to(device), torch.from_numpy(term_scores).to(device), dense


def compute_recall_exact(gpu_ids, cpu_ids, k_values=(10, 100, 1000)) -> dict:
    """{"recall@k": r} of the ranking gpu_ids [n, >=k] against cpu_ids [n, >=k]
    (src/run_correctness_verification.py:110-125): per k, the distinct ids of each
    row's first k in both, summed over rows, over the distinct ids of the truth's
    first k (0.0 when there are none).  A k wider than either ranking is left out."""
    g = _host_array(gpu_ids)
    c = _host_array(cpu_ids)
    if g.ndim != 2 or c.ndim != 2 or g.shape[0] != c.shape[0]:
        raise ValueError(f"rankings must be 2-D with the same number of rows, got {g.shape} and {c.shape}")
    out = {}
    for k in k_values:
        if k > g.shape[1] or k > c.shape[1]:
            continue
        hit = total = 0
        for q in range(g.shape[0]):
            truth = np.unique(c[q, :k])
            hit += np.intersect1d(truth, np.unique(g[q, :k]), assume_unique=True).size
            total += truth.size
        out[f"recall@{k}"] = hit / total if total > 0 else 0.0
    return out
