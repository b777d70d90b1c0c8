"""Chunk boundaries and the reference's chunked scoring entry points.

``build_chunk_boundaries`` keeps the reference's contract
(src/triton_kernel_chunked.py:83-122): an int64 ``[n_chunks + 1, vocab]`` tensor of
absolute posting indices, ValueError when a list is not ascending.  It runs on
the GPU (``gs_check_lists`` + ``gs_chunk_bounds``) instead of copying the whole
index to the host.

``triton_chunked_score`` / ``triton_chunked_score_fused`` (triton_kernel_chunked.py:
125-170, fused_topk.py:106-160) bounded score memory by scoring one doc chunk at
a time.  Here the doc-tile pipeline of ``gs_search`` already keeps score memory
at O(B * candidates) with no chunk loop or host sync per chunk, so both return
the same exact top-k as :func:`gpusparse.search.search`.
"""
from __future__ import annotations

import torch

from . import _lib
from .index import _device_of, require_ascending
from .search import _check_pow2, search


def build_chunk_boundaries(index, doc_chunk: int) -> torch.Tensor:
    """Per-(term, chunk) posting sub-ranges: bounds[c, t] is the posting index at
    which chunk c begins in list t; row n_chunks holds the list ends."""
    doc_chunk = int(doc_chunk)
    if doc_chunk <= 0:
        raise ValueError(f"doc_chunk must be positive, got {doc_chunk}")
    dev = _lib.require_gpu(_device_of(index))
    require_ascending(index)
    V = int(index.vocab_size)
    N = int(index.num_docs)
    n_chunks = (N + doc_chunk - 1) // doc_chunk
    bounds = torch.empty((n_chunks + 1, V), dtype=torch.int64, device=dev)
    _lib.check(_lib.lib().gs_chunk_bounds(_lib.ptr(index.doc_ids), _lib.ptr(index.offsets), _lib.ptr(index.lengths),
                                          V, N, doc_chunk, _lib.ptr(bounds), _lib.stream_ptr(dev)),
               "gs_chunk_bounds")
    return bounds


def _check_bounds(index, chunk_bounds, doc_chunk):
    if chunk_bounds is None:
        require_ascending(index)
        return
    N = int(index.num_docs)
    n_chunks = (N + int(doc_chunk) - 1) // int(doc_chunk)
    if tuple(chunk_bounds.shape) != (n_chunks + 1, int(index.vocab_size)):
        raise ValueError(f"chunk_bounds has shape {tuple(chunk_bounds.shape)}, expected "
                         f"({n_chunks + 1}, {int(index.vocab_size)}) for doc_chunk={doc_chunk}")


def triton_chunked_score(index, query_term_ids, query_term_scores, top_k=10, doc_chunk=131072, block_pl=128,
                         chunk_bounds=None):
    """Drop-in for triton_chunked_score (src/triton_kernel_chunked.py:125-170)."""
    _check_pow2(block_pl)
    _check_bounds(index, chunk_bounds, doc_chunk)
    return search(index, (query_term_ids, query_term_scores), top_k, path="fused")


def triton_chunked_score_fused(index, query_term_ids, query_term_scores, top_k=10, doc_chunk=131072, block_pl=128,
                               chunk_bounds=None, max_cand=8192):
    """Drop-in for triton_chunked_score_fused (src/fused_topk.py:106-160)."""
    _check_pow2(block_pl)
    _check_bounds(index, chunk_bounds, doc_chunk)
    return search(index, (query_term_ids, query_term_scores), top_k, path="fused")
