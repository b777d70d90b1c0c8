"""Writes tests/golden/golden.npz: small seeded inputs and the expected outputs of
the scoring path (index arrays, chunk bounds, exact top-k) for fp32, fp16 and
uint8 weights.

Expected outputs come from the CPU oracle and are cross-checked here against
brute force (dict-of-lists index, dense products, full sorts) before they are
written.  Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys
from dataclasses import replace

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "gpu-sparse_amd"))
sys.path.insert(0, ROOT)

from gpusparse import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

VOCAB = 1500
DOCS = synth.RowSpec(n_rows=400, vocab=VOCAB, nnz_mean=25.0, nnz_min=4, nnz_max=80)
QUERIES = synth.RowSpec(n_rows=12, vocab=VOCAB, nnz_mean=8.0, nnz_min=2, nnz_max=20)
SEED = 2026
CHUNK = 128
KS = (10, 400)


def brute_topk(D, ti, tw, k):
    Q = np.zeros((ti.shape[0], D.shape[1]))
    for q in range(ti.shape[0]):
        for t, w in zip(ti[q], tw[q]):
            if t >= 0:
                Q[q, t] += float(w)
    S = Q @ D.T
    ids = np.stack([np.array(sorted(range(D.shape[0]), key=lambda d: (-S[q, d], d))[:k]) for q in range(Q.shape[0])])
    return S, ids


def build(weights):
    docs = synth.generate_rows(replace(DOCS, weights=weights), SEED, synth.STREAM_DOCS)
    qspec = replace(QUERIES, weights="u8" if weights == "u8" else "f32")
    queries = synth.generate_rows(qspec, SEED, synth.STREAM_QUERIES)
    ix = O.build_index(docs.indptr, docs.indices, docs.data, DOCS.n_rows, VOCAB)
    ti, tw, _ = O.to_query_tensors(queries.indptr, queries.indices, queries.data)
    out = {"doc_indptr": docs.indptr, "doc_indices": docs.indices, "doc_data": docs.data,
           "q_terms": ti, "q_weights": tw}
    for f in ("doc_ids", "scores", "offsets", "lengths", "padded_lengths", "max_scores"):
        out["ix_" + f] = ix[f]
    out["chunk_bounds"] = O.chunk_bounds(ix["doc_ids"], ix["offsets"], ix["lengths"], VOCAB, DOCS.n_rows, CHUNK)
    D = np.zeros((DOCS.n_rows, VOCAB))
    rows = np.repeat(np.arange(DOCS.n_rows), np.diff(docs.indptr))
    np.add.at(D, (rows, docs.indices), docs.data.astype(np.float64))
    for k in KS:
        v, i = O.search(ix, ti, tw, k)
        S, bi = brute_topk(D, ti, tw, k)
        assert np.array_equal(i, bi), "oracle top-k disagrees with brute force"
        assert np.allclose(v.astype(np.float64), np.take_along_axis(S, bi, 1), rtol=1e-6, atol=1e-9)
        out[f"top{k}_scores"] = v
        out[f"top{k}_ids"] = i
    return out


def main():
    arrays = {}
    for w in ("f32", "f16", "u8"):
        for name, arr in build(w).items():
            arrays[f"{w}/{name}"] = arr
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {len(arrays)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
