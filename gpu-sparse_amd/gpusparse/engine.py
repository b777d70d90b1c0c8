"""The lsr-benchmark engine plug-in surface (lsr_benchmark_engine/gpusparse_retrieval.py).

Host-side formatting functions keep the reference's semantics; index build and
retrieval run on the GPU through this package.  ``lsr_benchmark`` and
``tirex_tracker`` (the TIRA harness) are optional: without them ``main`` raises
and :func:`run_engine` offers the same pipeline on in-memory embeddings.
"""
from __future__ import annotations

import gzip
import os

import numpy as np
import torch

from . import _lib
from .chunked import _check_bounds, build_chunk_boundaries
from .index import CSR, _device_of, build_index  # noqa: F401  (re-exported: gpusparse_retrieval.build_index)
from .search import search_async

BLOCK = 32          # posting lists are padded to a multiple of this
VOCAB_PAD = 1       # vocabulary is sized from the data, plus one


def to_csr(embeddings, dim):
    """(ids, CSR) from (id, tokens, values) triples (gpusparse_retrieval.py:56-69)."""
    ids, lens, indices, data = [], [], [], []
    for emb_id, tokens, values in embeddings:
        ids.append(emb_id)
        t = np.asarray([int(x) for x in tokens], dtype=np.int64)
        v = np.asarray([float(x) for x in values], dtype=np.float64)
        indices.append(t)
        data.append(v)
        lens.append(t.shape[0])
    indptr = np.zeros(len(ids) + 1, dtype=np.int64)
    np.cumsum(np.asarray(lens, dtype=np.int64), out=indptr[1:])
    ind = np.concatenate(indices).astype(np.int32) if indices else np.zeros(0, np.int32)
    dat = np.concatenate(data).astype(np.float32) if data else np.zeros(0, np.float32)
    return ids, CSR(indptr, ind, dat, (len(ids), int(dim)))


def determine_dimension(*embedding_sets):
    """Largest term id + 1 + VOCAB_PAD (gpusparse_retrieval.py:72-78)."""
    d = 0
    for embeddings in embedding_sets:
        for _, tokens, _ in embeddings:
            if len(tokens):
                d = max(d, max(int(t) for t in tokens) + 1)
    return d + VOCAB_PAD


def to_query_tensors(q_csr, device, *, weight_dtype=torch.float32):
    """Dense [nq, max_nnz] term-id / weight tensors, -1 / 0 padded, no truncation
    (gpusparse_retrieval.py:118-132).  Weights are float32 as in the reference
    (:124); ``weight_dtype=None`` keeps uint8 query weights as uint8 (the native
    form a uint8 index takes, which then needs no conversion per search)."""
    if not isinstance(q_csr, CSR):
        q_csr = CSR(np.asarray(q_csr.indptr), np.asarray(q_csr.indices), np.asarray(q_csr.data),
                    tuple(q_csr.shape))
    if weight_dtype not in (None, torch.float32):
        raise ValueError(f"weight_dtype must be torch.float32 or None, got {weight_dtype}")
    indptr = np.asarray(q_csr.indptr, dtype=np.int64)
    nq = indptr.shape[0] - 1
    nnz = np.diff(indptr)
    max_nnz = int(nnz.max()) if nq else 1
    wdt = np.uint8 if (weight_dtype is None and q_csr.data.dtype == np.uint8) else np.float32
    ti = np.full((nq, max_nnz), -1, dtype=np.int32)
    ts = np.zeros((nq, max_nnz), dtype=wdt)
    if nq and indptr[-1]:
        rows = np.repeat(np.arange(nq), nnz)
        cols = np.arange(indptr[-1]) - np.repeat(indptr[:-1], nnz)
        ti[rows, cols] = q_csr.indices
        ts[rows, cols] = q_csr.data
    return (torch.from_numpy(ti).to(device), torch.from_numpy(ts).to(device), max_nnz)


def retrieve(index, q_ids, q_ti, q_ts, doc_ids, k, batch_size=200, doc_chunk=131072, streams=2):
    """Batched retrieval with the reference's output format (gpusparse_retrieval.py:
    135-172): per query a list of (qid, score, docno) for the top k with score > 0.

    Each batch is scored as the reference's call scores it: triton_fused_score
    (path "auto") or, above doc_chunk docs, triton_chunked_score_fused (the fused
    path; its chunk boundaries built and checked once).  Both are `search`; here
    each batch is queued with `search_async` on one of `streams` streams in turn,
    so that the next batches run on the GPU while the host builds this one's
    rankings.  The rankings are the same for any `streams` >= 1."""
    results = []
    n = q_ti.shape[0]
    kk = min(k, index.num_docs)
    chunked = index.num_docs > doc_chunk
    if chunked:
        bounds = build_chunk_boundaries(index, doc_chunk)
        _check_bounds(index, bounds, doc_chunk)  # what triton_chunked_score_fused checks per call
    path = "fused" if chunked else "auto"
    dev = _device_of(index)
    cur = torch.cuda.current_stream(dev)
    # side streams are kept with the index, so that repeated calls reuse them and
    # their workspaces (one per stream) instead of adding new ones
    side = index.aux().setdefault("retrieve_streams", [])
    while len(side) < int(streams):
        side.append(torch.cuda.Stream(dev))
    pool = [cur] if streams <= 1 else side[:int(streams)]
    for st in pool:
        st.wait_stream(cur)  # the query tensors were written on the current stream
    starts = list(range(0, n, batch_size))

    def launch(i):
        s0 = starts[i]
        s1 = min(s0 + batch_size, n)
        with torch.cuda.stream(pool[i % len(pool)]):
            return search_async(index, (q_ti[s0:s1].contiguous(), q_ts[s0:s1].contiguous()), kk, path=path)

    pending = [launch(i) for i in range(min(len(pool), len(starts)))] if len(pool) > 1 else []
    for i, s0 in enumerate(starts):
        s1 = min(s0 + batch_size, n)
        p = pending.pop(0) if pending else launch(i)
        scores, ids = p.result()
        scores = scores.cpu().numpy()
        ids = ids.cpu().numpy()
        if len(pool) > 1 and i + len(pool) < len(starts):
            pending.append(launch(i + len(pool)))
        for r in range(s1 - s0):
            ranking = [(q_ids[s0 + r], float(scores[r, j]), doc_ids[ids[r, j]])
                       for j in range(kk) if scores[r, j] > 0]
            results.append(ranking)
    return results


def write_run(results, path, tag="gpusparse"):
    """gzipped TREC run, one line per (query, rank) (gpusparse_retrieval.py:219-222)."""
    with gzip.open(path, "wt") as f:
        for ranking in results:
            for rank, (qid, score, docno) in enumerate(ranking, start=1):
                f.write(f"{qid} Q0 {docno} {rank} {score} {tag}\n")


def run_engine(doc_embeddings, query_embeddings, output, k, device="cuda:0", batch_size=200, doc_chunk=131072):
    """The body of the plug-in's main without the TIRA tracking: index the docs,
    retrieve for every query, write ``output/run.txt.gz``.  Returns the results."""
    os.makedirs(output, exist_ok=True)
    dev = _lib.require_gpu(device)
    dim = determine_dimension(doc_embeddings, query_embeddings)
    doc_ids, doc_csr = to_csr(doc_embeddings, dim)
    index = build_index(doc_csr, dev)
    torch.cuda.synchronize(dev)
    q_ids, q_csr = to_csr(query_embeddings, dim)
    q_ti, q_ts, _ = to_query_tensors(q_csr, dev)
    results = retrieve(index, q_ids, q_ti, q_ts, doc_ids, k, batch_size=batch_size, doc_chunk=doc_chunk)
    torch.cuda.synchronize(dev)
    write_run(results, os.path.join(output, "run.txt.gz"))
    return results


def _main(dataset, embedding, output, k):
    """gpusparse_retrieval.py:175-222 on this package."""
    import lsr_benchmark
    from lsr_benchmark.irds import embeddings as load_embeddings
    from tirex_tracker import ExportFormat, register_metadata, tracking

    output.mkdir(parents=True, exist_ok=True)
    lsr_benchmark.register_to_ir_datasets(dataset)
    dev = _lib.require_gpu("cuda:0")
    register_metadata({
        "actor": {"team": "gpusparse"},
        "tag": f"gpusparse-{embedding.replace('/', '-')}-{k}",
        "description": ("Exact GPU-native learned sparse retrieval on MI355X: term-major inverted index in "
                        "HBM, LDS doc-tile scatter-add scoring with fused threshold selection, fp64-exact "
                        f"scores. Device: {torch.cuda.get_device_name(0)}."),
    })
    d_emb = load_embeddings(dataset, embedding, "doc")
    q_emb = load_embeddings(dataset, embedding, "query")
    dim = determine_dimension(d_emb, q_emb)
    with tracking(export_file_path=output / "index-metadata.yml", export_format=ExportFormat.IR_METADATA):
        doc_ids, doc_csr = to_csr(d_emb, dim)
        index = build_index(doc_csr, dev)
        torch.cuda.synchronize()
    q_ids, q_csr = to_csr(q_emb, dim)
    q_ti, q_ts, _ = to_query_tensors(q_csr, dev)
    with tracking(export_file_path=output / "retrieval-metadata.yml", export_format=ExportFormat.IR_METADATA):
        results = retrieve(index, q_ids, q_ti, q_ts, doc_ids, k)
        torch.cuda.synchronize()
    write_run(results, output / "run.txt.gz")


try:  # the TIRA harness is not vendored; wrap only when it is installed
    from lsr_benchmark.click import retrieve_command as _retrieve_command
    main = _retrieve_command()(_main)
except ImportError:
    def main(*args, **kwargs):
        raise ImportError("lsr_benchmark / tirex_tracker are not installed; use gpusparse.engine.run_engine")
