"""Test-only stand-in for lsr_benchmark.irds.embeddings
(lsr_benchmark_engine/gpusparse_retrieval.py:194-195): `dataset` names an .npz
fixture holding doc and query embeddings as (ids, indptr, tokens, values)."""
import numpy as np

CALLS = []


def embeddings(dataset, embedding, kind):
    CALLS.append((dataset, embedding, kind))
    with np.load(dataset, allow_pickle=False) as z:
        ids = [str(x) for x in z[f"{kind}_ids"]]
        indptr = z[f"{kind}_indptr"]
        tokens = z[f"{kind}_tokens"]
        values = z[f"{kind}_values"]
    return [(ids[i], tokens[indptr[i]:indptr[i + 1]].tolist(), values[indptr[i]:indptr[i + 1]].tolist())
            for i in range(len(ids))]
