"""Small input builders shared by the CPU and GPU tests."""
import numpy as np

from gpusparse.index import CSR


def random_csr(rng, n_docs, vocab, max_len=12, dtype=np.float32, dup_rate=0.0, empty_rate=0.1, sort_rows=False):
    """Random doc-major CSR; rows may be empty, unsorted, and (dup_rate > 0) may
    repeat a term id inside a row."""
    indptr = [0]
    idx, val = [], []
    for _ in range(n_docs):
        n = 0 if rng.random() < empty_rate else int(rng.integers(1, max_len + 1))
        n = min(n, vocab)
        terms = rng.choice(vocab, size=n, replace=False)
        if sort_rows:
            terms = np.sort(terms)
        terms = list(terms)
        if dup_rate and n:
            for _ in range(int(rng.binomial(n, dup_rate))):
                terms.insert(int(rng.integers(0, len(terms) + 1)), terms[int(rng.integers(0, len(terms)))])
        idx.extend(terms)
        indptr.append(len(idx))
        if dtype == np.uint8:
            val.extend(rng.integers(1, 256, size=len(terms)))
        else:
            val.extend(rng.lognormal(-0.5, 0.8, size=len(terms)))
    data = np.asarray(val).astype(dtype)
    return CSR(np.asarray(indptr, np.int64), np.asarray(idx, np.int32), data, (n_docs, vocab))


def random_queries(rng, n, vocab, max_len=10, dtype=np.float32, invalid_rate=0.0, pad_to=None):
    """[n, T] term ids (-1 padded, optionally with out-of-range ids) and weights."""
    lens = rng.integers(0, max_len + 1, size=n)
    T = max(int(lens.max()) if n else 1, 1) if pad_to is None else pad_to
    ti = np.full((n, T), -1, np.int32)
    tw = np.zeros((n, T), dtype)
    for q in range(n):
        L = min(int(lens[q]), T)
        ti[q, :L] = rng.choice(vocab, size=L, replace=False)
        if invalid_rate:
            bad = rng.random(L) < invalid_rate
            ti[q, :L][bad] = np.where(rng.random(int(bad.sum())) < 0.5, -5, vocab + 3)
        if dtype == np.uint8:
            tw[q, :L] = rng.integers(1, 256, size=L)
        else:
            tw[q, :L] = rng.lognormal(-0.5, 0.8, size=L)
    return ti, tw


def dense_docs(csr: CSR, dtype=np.float64):
    """Dense [n_docs, vocab] matrix summing duplicate entries."""
    D = np.zeros(csr.shape, dtype=dtype)
    rows = np.repeat(np.arange(csr.shape[0]), np.diff(csr.indptr))
    np.add.at(D, (rows, csr.indices), csr.data.astype(dtype))
    return D


def dense_queries(ti, tw, vocab, dtype=np.float64):
    Q = np.zeros((ti.shape[0], vocab), dtype=dtype)
    for q in range(ti.shape[0]):
        for t, w in zip(ti[q], tw[q]):
            if 0 <= t < vocab:
                Q[q, t] += dtype(w)
    return Q
