"""Writes the committed fixtures under tests/golden/.

golden.npz: small seeded inputs and the expected outputs of the scoring path
(index arrays, chunk bounds, exact top-k) for fp32, fp16 and uint8 weights.
Expected outputs come from the CPU oracle and are cross-checked here against
brute force (dict-of-lists index, dense products, full sorts) before they are
written.

engine_embeddings.npz + engine_run.txt: sparse doc and query embeddings for the
plug-in's entry point (lsr_benchmark_engine/gpusparse_retrieval.py:175-222) and
the TREC run it must write at k = 10.  The run comes from a brute-force ranking
written here independently of the oracle and the library: per (query, doc) a
Python float (fp64) sum of products in query-term order, docs ordered by (score
descending, doc index ascending), scores printed as float32, only scores > 0
kept (:169-170).  Run from the repository root:  python tests/golden/make_golden.py
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


ENGINE_K = 10


def engine_embeddings(seed=77, n_docs=400, n_queries=20, vocab=600):
    """(doc, query) embeddings as lists of (id, tokens, values) with float32
    values.  Includes two identical docs that tie at the top of one query, a
    query whose tokens no doc holds (empty ranking), a query with fewer than k
    matching docs and a query that repeats a token."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, vocab - 10 + 1) ** 1.05
    p /= p.sum()

    def row(n):
        toks = rng.choice(vocab - 10, size=n, replace=False, p=p)
        vals = rng.lognormal(-0.5, 0.8, size=n).astype(np.float32)
        return [int(t) for t in toks], [float(v) for v in vals]

    docs = [(f"D{i:04d}",) + row(int(rng.integers(3, 41))) for i in range(n_docs)]
    docs[17] = ("D0017", docs[17][1] + [vocab - 8], docs[17][2] + [2.5])
    docs[240] = ("D0240", list(docs[17][1]), list(docs[17][2]))
    rare = [t for t in range(vocab - 10) if sum(t in d[1] for d in docs) == 3][0]
    queries = [(f"Q{i:03d}",) + row(int(rng.integers(2, 13))) for i in range(n_queries)]
    queries[5] = ("Q005", [vocab - 5, vocab - 3], [0.5, 1.25])
    queries[7] = ("Q007", [rare], [0.75])
    t9, v9 = queries[9][1], queries[9][2]
    queries[9] = ("Q009", t9 + [t9[0]], v9 + [0.3125])
    queries[11] = ("Q011", [vocab - 8, docs[17][1][0]], [1.0, 0.5])  # D0017 and D0240 tie on top
    return docs, queries


def brute_run(docs, queries, k, tag="gpusparse"):
    """TREC lines of the exact top-k by brute force over the embeddings."""
    lines = []
    for qid, qt, qv in queries:
        scored = []
        for di, (_, dt, dv) in enumerate(docs):
            s = 0.0
            for t, w in zip(qt, qv):
                for t2, w2 in zip(dt, dv):
                    if t2 == t:
                        s += w * w2
            scored.append((s, di))
        scored.sort(key=lambda x: (-x[0], x[1]))
        rank = 0
        for s, di in scored[:k]:
            if np.float32(s) > 0:
                rank += 1
                lines.append(f"{qid} Q0 {docs[di][0]} {rank} {float(np.float32(s))} {tag}")
    return lines


def pack_embeddings(emb):
    indptr = np.zeros(len(emb) + 1, np.int64)
    indptr[1:] = np.cumsum([len(e[1]) for e in emb])
    return (np.array([e[0] for e in emb]), indptr, np.array([t for e in emb for t in e[1]], np.int64),
            np.array([v for e in emb for v in e[2]], np.float32))


def write_engine_fixture(here):
    docs, queries = engine_embeddings()
    arrays = {}
    for kind, emb in (("doc", docs), ("query", queries)):
        ids, indptr, toks, vals = pack_embeddings(emb)
        arrays.update({f"{kind}_ids": ids, f"{kind}_indptr": indptr, f"{kind}_tokens": toks,
                       f"{kind}_values": vals})
    np.savez_compressed(os.path.join(here, "engine_embeddings.npz"), **arrays)
    lines = brute_run(docs, queries, ENGINE_K)
    with open(os.path.join(here, "engine_run.txt"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote engine fixture: {len(docs)} docs, {len(queries)} queries, {len(lines)} run lines")


def main():
    write_engine_fixture(os.path.dirname(os.path.abspath(__file__)))
    arrays = {}
    for w in ("f32", "f16", "u8"):
        for name, arr in build(w).items():
            arrays[f"{w}/{name}"] = arr
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {len(arrays)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
