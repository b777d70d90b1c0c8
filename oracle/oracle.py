"""CPU oracle for the exact SPLADE scoring path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module or the C library next to it (liboracle.so), and only as the checker
or as the timed CPU baseline -- never as part of the product path.

Each function restates one piece of the reference (ashutoshuiuc/gpu-sparse) in
plain numpy, citing the file:line it follows.  The reference has no test suite
and no golden vectors; every function here is pinned in tests/test_oracle.py
against an independent computation (brute force over Python lists, dense matrix
products, exhaustive sorting, closed forms):

  build_index            pinned: dict-of-lists builder + layout invariants
  chunk_bounds           pinned: linear scan per list + partition invariant
  forward_index          pinned: the CSR rows sorted stably by column
  tile_bounds            pinned: linear scan per list
  heavy_terms            pinned: Python sorted() over all terms on small vocabularies
  pack_shift             pinned: closed forms at powers of two and scaled cases
  pack_postings          pinned: per-slot decoding + a scalar loop with exact
                         rational rounding (fractions.Fraction, half to even)
  head_limbs             pinned: 128 * high + low == the packed weight of every
                         heavy posting, zero cells exactly where a doc lacks the
                         term, limbs in range, on hand-made and random lists
  scores_f64 / _u32      pinned: dense Q @ D^T (float64 / int64) on small inputs
  scores_f32_sequential  pinned: scalar float32 loop of gpu_scoring.py:246-251
  topk                   pinned: Python sorted() with the same key
  compacted_topk         pinned: topk of the thresholded row
  to_query_tensors       pinned: explicit per-row loop
  fp16 / u8 codes        pinned: numpy float16 cast / closed-form values
  checksum_csr / _index  pinned: equal on an index and its CSR, different after
                         any single planted change (moved, altered, lost posting)
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

BLOCK = 32
HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


# ------------------------------------------------------------------ index build


def build_index(indptr, indices, data, n_docs: int, vocab: int) -> dict:
    """Term-major padded index of a doc-major CSR.

    Follows lsr_benchmark_engine/gpusparse_retrieval.py:81-115 (stable argsort of
    the COO column, bincount lengths, padding to 32, exclusive cumsum offsets,
    copy of each list, pads -1 / 0) and adds max_scores as
    src/run_correctness_verification.py:63,71 does (per-list max, 0 if empty)."""
    indptr = np.asarray(indptr, dtype=np.int64)
    cols = np.asarray(indices, dtype=np.int64)
    vals = np.asarray(data)
    rows = np.repeat(np.arange(n_docs, dtype=np.int64), np.diff(indptr))
    if cols.size and (cols.min() < 0 or cols.max() >= vocab):
        raise IndexError(f"term id outside [0, {vocab})")
    order = np.argsort(cols, kind="stable")
    terms, docs, scores = cols[order], rows[order], vals[order]
    lengths = np.bincount(terms, minlength=vocab).astype(np.int32)
    padded = ((lengths + BLOCK - 1) // BLOCK) * BLOCK
    offsets = np.zeros(vocab, dtype=np.int64)
    if vocab > 1:
        np.cumsum(padded[:-1], out=offsets[1:])
    total = int(offsets[-1] + padded[-1])
    all_docs = np.full(total, -1, dtype=np.int32)
    all_scores = np.zeros(total, dtype=vals.dtype)
    max_scores = np.zeros(vocab, dtype=np.float32)
    pos = 0
    for t in np.nonzero(lengths)[0]:
        L = int(lengths[t])
        o = int(offsets[t])
        all_docs[o:o + L] = docs[pos:pos + L]
        all_scores[o:o + L] = scores[pos:pos + L]
        max_scores[t] = scores[pos:pos + L].astype(np.float32).max()
        pos += L
    return {"doc_ids": all_docs, "scores": all_scores, "offsets": offsets, "lengths": lengths,
            "padded_lengths": padded.astype(np.int32), "max_scores": max_scores,
            "num_docs": int(n_docs), "vocab_size": int(vocab)}


def forward_index(index: dict):
    """Doc-major copy of a term-major index: (row_ptr [N+1] int64, terms int32,
    weights) with each doc's postings in ascending term order and the entries of a
    repeated (doc, term) pair in list order.  The layout of the forward index of
    src/triton_kernel_v4.py:92-158 (doc-major term ids + weights per doc), taken
    from the inverted index instead of a dense matrix."""
    V, N = index["vocab_size"], index["num_docs"]
    lengths = index["lengths"].astype(np.int64)
    docs = np.concatenate([index["doc_ids"][index["offsets"][t]:index["offsets"][t] + lengths[t]]
                           for t in range(V)] or [np.zeros(0, np.int32)]).astype(np.int64)
    terms = np.repeat(np.arange(V, dtype=np.int64), lengths)
    w = np.concatenate([index["scores"][index["offsets"][t]:index["offsets"][t] + lengths[t]]
                        for t in range(V)] or [np.zeros(0, index["scores"].dtype)])
    keep = (docs >= 0) & (docs < N)
    docs, terms, w = docs[keep], terms[keep], w[keep]
    order = np.argsort(docs, kind="stable")
    row_ptr = np.zeros(N + 1, dtype=np.int64)
    np.cumsum(np.bincount(docs, minlength=N), out=row_ptr[1:])
    return row_ptr, terms[order].astype(np.int32), w[order]


def tile_bounds(index: dict, tile_log2: int) -> np.ndarray:
    """[V][n_tiles + 1] list-relative first posting of each doc tile: the
    per-(term, chunk) sub-ranges of src/triton_kernel_chunked.py:110-121 at
    tile granularity (np.searchsorted 'left' of the tile edges)."""
    V, N = index["vocab_size"], index["num_docs"]
    n_tiles = (N + (1 << tile_log2) - 1) >> tile_log2
    edges = np.arange(n_tiles + 1, dtype=np.int64) << tile_log2
    out = np.zeros((V, n_tiles + 1), dtype=np.int32)
    for t in range(V):
        o, n = int(index["offsets"][t]), int(index["lengths"][t])
        out[t] = np.searchsorted(index["doc_ids"][o:o + n], edges, side="left")
    return out


def heavy_terms(lengths, n: int = 64) -> np.ndarray:
    """gs_heavy_terms (no reference counterpart): the n non-empty posting lists
    with the most postings, as term ids by (length desc, term asc), -1 padded."""
    L = np.asarray(lengths, dtype=np.int64)
    nz = np.nonzero(L > 0)[0]
    order = nz[np.lexsort((nz, -L[nz]))][:n]
    out = np.full(n, -1, np.int32)
    out[:len(order)] = order
    return out


def pack_shift(max_abs: float) -> int:
    """gs_pack_shift (no reference counterpart): the largest s with
    max_abs * 2^s <= 8191, 0 for max_abs == 0."""
    m = float(max_abs)
    if not np.isfinite(m) or m < 0:
        raise ValueError(f"max_abs {m} must be finite and >= 0")
    if m == 0:
        return 0
    s = 0
    while np.ldexp(m, s) > 8191.0:
        s -= 1
    while np.ldexp(m, s + 1) <= 8191.0:
        s += 1
    return s


ARRANGE_BLOCK = 1024  # postings per block of the packed copy's bank-aware order


def pack_postings(index: dict, tile_log2: int, shift: int | None = None, arrange: bool = True) -> np.ndarray:
    """Packed scoring copy (gs_pack_postings; no reference counterpart: a layout of
    its posting arrays), int32 [n]: per slot (doc mod 2^tile_log2) * 4 in bits 0-15
    and the weight in bits 16-31 -- the uint8 weight, or for float weights the
    int16 rint(w * 2^shift) (half to even, clamped to +-32767), shift defaulting to
    pack_shift of the largest |w|; padding slots (doc < 0) are 0.
    arrange: each (term, tile) sub-range is cut into blocks of ARRANGE_BLOCK
    postings from its start, and each block of n > 64 postings is rewritten in the
    order arrange_order gives (the sums over a sub-range do not depend on it)."""
    doc = index["doc_ids"].astype(np.int64)
    w = index["scores"]
    ok = doc >= 0
    off = np.where(ok, (doc & ((1 << tile_log2) - 1)) << 2, 0).astype(np.uint32)
    if w.dtype == np.uint8:
        bits = w.astype(np.uint32)
    else:
        wf = w.astype(np.float64)
        if shift is None:
            shift = pack_shift(np.max(np.abs(wf[ok])) if ok.any() else 0.0)
        q = np.clip(np.rint(np.ldexp(wf, shift)), -32767, 32767).astype(np.int16)
        bits = q.view(np.uint16).astype(np.uint32)
    words = (off | (np.where(ok, bits, 0).astype(np.uint32) << 16)).view(np.int32)
    if not arrange:
        return words
    out = words.copy()
    n_docs = int(index["num_docs"])
    edges = np.arange(((n_docs + (1 << tile_log2) - 1) >> tile_log2) + 1, dtype=np.int64) << tile_log2
    for t in np.nonzero(index["lengths"] > 64)[0]:
        o, L = int(index["offsets"][t]), int(index["lengths"][t])
        lst = doc[o:o + L]
        b = np.searchsorted(lst, edges, side="left")
        for lo, hi in zip(b[:-1], b[1:]):
            for a in range(int(lo), int(hi), ARRANGE_BLOCK):
                z = min(a + ARRANGE_BLOCK, int(hi))
                if z - a > 64:
                    out[o + a: o + z] = words[o + a + arrange_order(lst[a:z])]
    return out


def head_limbs(index: dict, heavy, n_rows: int, shift: int | None = None) -> np.ndarray:
    """Dense copy of the heavy terms' packed weights (gs_head_fill; no reference
    counterpart: the B operand of the hybrid scorer's int8 products), int8
    [n_rows, 2, len(heavy)]: for h with heavy[h] >= 0 and each posting (d, w) of
    that list, the packed copy's integer weight wq (pack_postings' weight half)
    as wq & 127 at [d, 0, h] and wq >> 7 (floor) at [d, 1, h]; zero elsewhere."""
    words = pack_postings(index, 0, shift, arrange=False).view(np.uint32)
    out = np.zeros((n_rows, 2, len(heavy)), dtype=np.int8)
    u8 = index["scores"].dtype == np.uint8
    for h, t in enumerate(heavy):
        if t < 0:
            continue
        o, L = int(index["offsets"][t]), int(index["lengths"][t])
        d = index["doc_ids"][o:o + L].astype(np.int64)
        half = (words[o:o + L] >> 16).astype(np.uint16)
        wq = half.astype(np.int64) if u8 else half.view(np.int16).astype(np.int64)
        out[d, 0, h] = (wq & 127).astype(np.int8)
        out[d, 1, h] = (wq >> 7).astype(np.int8)
    return out


def arrange_order(docs: np.ndarray) -> np.ndarray:
    """Bank-aware order of one block of n > 64 postings of a (term, tile) sub-range
    (docs ascending): element i of the result is the block index of the posting
    placed at position i.  G = ceil(n / 64) groups of 64 positions, the last one
    n_last = n - 64 (G - 1) long.  The postings sorted by (doc mod 64, doc) are
    dealt out in turn: the k-th to group k mod G, position k // G while
    k < n_last * G, after that to group k' mod (G - 1), position n_last +
    k' // (G - 1) (k' = k - n_last * G).  Checked in tests against the invariants
    that fix it: a permutation of the sub-range, every residue in ceil(count / G)
    groups' worth at most per group, and the deal order itself on small cases."""
    n = len(docs)
    G = (n + 63) // 64
    nl = n - 64 * (G - 1)
    by_res = np.argsort(docs & 63, kind="stable")  # (residue, doc) order
    k = np.arange(n)
    first = k < nl * G
    k2 = k - nl * G
    grp = np.where(first, k % G, k2 % max(G - 1, 1))
    pos = np.where(first, k // G, nl + k2 // max(G - 1, 1))
    order = np.empty(n, dtype=np.int64)
    order[grp * 64 + pos] = by_res
    return order


def chunk_bounds(doc_ids, offsets, lengths, vocab: int, n_docs: int, doc_chunk: int) -> np.ndarray:
    """[n_chunks + 1, vocab] posting bounds, src/triton_kernel_chunked.py:89-122,
    including its ValueError for non-ascending lists (:99-108)."""
    n_chunks = (n_docs + doc_chunk - 1) // doc_chunk
    n_bad = 0
    for t in np.nonzero(lengths)[0]:
        seg = doc_ids[offsets[t]: offsets[t] + lengths[t]]
        if np.any(np.diff(seg) < 0):
            n_bad += 1
    if n_bad:
        raise ValueError(
            f"{n_bad} of {int((lengths > 0).sum())} posting lists are not ascending in "
            f"doc_id. Chunked scoring requires ascending lists (build the index with "
            f"np.argsort(..., kind='stable')); otherwise results are silently wrong.")
    bounds = np.zeros((n_chunks + 1, vocab), dtype=np.int64)
    edges = [c * doc_chunk for c in range(n_chunks)] + [n_docs]
    for t in range(vocab):
        L = int(lengths[t])
        if L == 0:
            bounds[:, t] = offsets[t]
            continue
        seg = doc_ids[offsets[t]: offsets[t] + L]
        first = int(np.searchsorted(seg, 0, side="left"))
        rel = np.searchsorted(seg[first:], edges, side="left")
        bounds[:, t] = offsets[t] + first + rel
    return bounds


# ------------------------------------------------------------------ scoring


def decode_weights(scores: np.ndarray) -> np.ndarray:
    """Stored weights as float64 (fp16 and uint8 decode exactly)."""
    return scores.astype(np.float64)


def _postings(index, t):
    o = int(index["offsets"][t])
    L = int(index["lengths"][t])
    return index["doc_ids"][o:o + L], index["scores"][o:o + L]


def scores_f64(index: dict, q_terms: np.ndarray, q_weights: np.ndarray) -> np.ndarray:
    """Exhaustive fp64 scatter-add, query terms in order and postings in list order:
    the sum of src/triton_kernel.py:142-156 (out[q, doc] += wq * w) accumulated in
    float64 (products of fp32/fp16/u8 values are exact in float64).  [B, N]."""
    B, T = q_terms.shape
    N, V = index["num_docs"], index["vocab_size"]
    out = np.zeros((B, N), dtype=np.float64)
    for q in range(B):
        acc = out[q]
        for j in range(T):
            t = int(q_terms[q, j])
            if t < 0 or t >= V:          # skipped as in triton_kernel.py:126-128
                continue
            d, w = _postings(index, t)
            np.add.at(acc, d, float(q_weights[q, j]) * decode_weights(w))
    return out


def scores_u32(index: dict, q_terms: np.ndarray, q_weights: np.ndarray) -> np.ndarray:
    """Integer scatter-add of uint8 impacts and uint8 query weights, [B, N] uint32."""
    B, T = q_terms.shape
    N, V = index["num_docs"], index["vocab_size"]
    out = np.zeros((B, N), dtype=np.uint64)
    for q in range(B):
        for j in range(T):
            t = int(q_terms[q, j])
            if t < 0 or t >= V:
                continue
            d, w = _postings(index, t)
            np.add.at(out[q], d, np.uint64(q_weights[q, j]) * w.astype(np.uint64))
    assert out.max(initial=0) < 2 ** 32
    return out.astype(np.uint32)


def scores_f32_sequential(index: dict, q_terms: np.ndarray, q_weights: np.ndarray) -> np.ndarray:
    """The reference CPU path's accumulation (src/gpu_scoring.py:241-251): float32
    accumulator per query, doc_scores[doc] += q * w in query-term then posting order."""
    B, T = q_terms.shape
    N, V = index["num_docs"], index["vocab_size"]
    out = np.zeros((B, N), dtype=np.float32)
    for q in range(B):
        for j in range(T):
            t = int(q_terms[q, j])
            if t < 0 or t >= V:
                continue
            d, w = _postings(index, t)
            prod = (np.float32(q_weights[q, j]) * w.astype(np.float32)).astype(np.float32)
            np.add.at(out[q], d, prod)
    return out


def topk(scores: np.ndarray, k: int):
    """Top-k of each row ordered by score descending, then doc id ascending:
    the tie rule of this implementation (torch.topk's tie order is unspecified).
    Returns (values [B, k] in the input dtype, ids [B, k] int64)."""
    B, N = scores.shape
    k = min(k, N)
    ids = np.empty((B, k), dtype=np.int64)
    for q in range(B):
        order = np.lexsort((np.arange(N), -scores[q].astype(np.float64) if scores.dtype != np.uint32
                            else -scores[q].astype(np.int64)))
        ids[q] = order[:k]
    vals = np.take_along_axis(scores, ids, axis=1)
    return vals, ids


def search(index: dict, q_terms: np.ndarray, q_weights: np.ndarray, k: int):
    """Exact top-k of the scatter-add: float indexes -> (fp32 of the fp64 score,
    ids); uint8 indexes -> (int32 uint32-sum, ids)."""
    if index["scores"].dtype == np.uint8:
        s = scores_u32(index, q_terms, q_weights)
        v, i = topk(s, k)
        return v.astype(np.int32), i
    s = scores_f64(index, q_terms, q_weights)
    v, i = topk(s, k)
    return v.astype(np.float32), i


def compacted_topk(scores: np.ndarray, tau, k: int, max_cand: int = 8192):
    """src/fused_topk.py:71-103: top kk = min(k, L) of the entries >= tau[b] (all
    entries when tau is None), descending, missing slots (-inf, 0); the result
    does not depend on max_cand (overflow rows are redone in full, :96-102)."""
    B, L = scores.shape
    kk = min(k, L)
    vals = np.full((B, kk), -np.inf, dtype=np.float32)
    idx = np.zeros((B, kk), dtype=np.int64)
    for b in range(B):
        row = scores[b]
        cand = np.arange(L) if tau is None else np.nonzero(row >= tau[b])[0]
        order = cand[np.lexsort((cand, -row[cand].astype(np.float64)))][:kk]
        vals[b, :order.size] = row[order]
        idx[b, :order.size] = order
    return vals, idx


def cpu_sequential_score(doc_term_ids, doc_term_scores, query_term_ids_list, query_term_scores_list,
                         num_docs, top_k=10):
    """src/gpu_scoring.py:221-259 restated: dict inverted index, float32 per-query
    accumulator, argpartition + argsort top-k.  Pure Python: small inputs only."""
    inv = {}
    for doc_id in range(num_docs):
        for term_id, score in zip(doc_term_ids[doc_id], doc_term_scores[doc_id]):
            inv.setdefault(term_id, []).append((doc_id, score))
    all_s, all_i = [], []
    for q_terms, q_scores in zip(query_term_ids_list, query_term_scores_list):
        acc = np.zeros(num_docs, dtype=np.float32)
        for term_id, q_score in zip(q_terms, q_scores):
            for doc_id, d_score in inv.get(term_id, ()):
                acc[doc_id] += q_score * d_score
        top = np.argpartition(acc, -top_k)[-top_k:]
        top = top[np.argsort(acc[top])[::-1]]
        all_s.append(acc[top].tolist())
        all_i.append(top.tolist())
    return all_s, all_i


# ------------------------------------------------------------------ host formatting


def to_query_tensors(indptr, indices, data):
    """Dense [nq, max_nnz] ids (-1 pad) and weights (0 pad): gpusparse_retrieval.py:118-132."""
    nq = len(indptr) - 1
    max_nnz = int(np.diff(indptr).max()) if nq else 1
    ti = np.full((nq, max_nnz), -1, dtype=np.int32)
    ts = np.zeros((nq, max_nnz), dtype=np.uint8 if np.asarray(data).dtype == np.uint8 else np.float32)
    for i in range(nq):
        s, e = indptr[i], indptr[i + 1]
        ti[i, :e - s] = indices[s:e]
        ts[i, :e - s] = data[s:e]
    return ti, ts, max_nnz


def rankings(q_ids, scores, ids, doc_ids, k):
    """Per-query [(qid, score, docno)] keeping score > 0 (gpusparse_retrieval.py:168-171)."""
    out = []
    for r in range(scores.shape[0]):
        out.append([(q_ids[r], float(scores[r, j]), doc_ids[ids[r, j]]) for j in range(min(k, scores.shape[1]))
                    if scores[r, j] > 0])
    return out


# ------------------------------------------------------------------ C scorer


_clib = None


def clib():
    """liboracle.so (oracle/oracle_score.c), built by oracle/Makefile."""
    global _clib
    if _clib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run make -C oracle")
        L = C.CDLL(LIB_PATH)
        P, I32, I64 = C.c_void_p, C.c_int32, C.c_int64
        L.orc_search.restype = C.c_int
        L.orc_search.argtypes = [P, P, C.c_int, P, P, I32, I64, P, P, I32, I32, I32, P, P, P, C.c_int]
        L.orc_checksum_csr.restype = C.c_uint64
        L.orc_checksum_csr.argtypes = [P, P, P, C.c_int, I64, C.c_int]
        L.orc_checksum_index.restype = C.c_uint64
        L.orc_checksum_index.argtypes = [P, P, C.c_int, P, P, P, I32, C.c_int, P]
        L.orc_cpu_sequential.restype = C.c_int
        L.orc_cpu_sequential.argtypes = [P, P, C.c_int, P, P, I32, I64, P, P, I32, I32, I32, P, P, C.c_int]
        _clib = L
    return _clib


_WT = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.uint8): 2}


def _c_args(index, q_terms, q_weights):
    doc = np.ascontiguousarray(index["doc_ids"], dtype=np.int32)
    w = np.ascontiguousarray(index["scores"])
    off = np.ascontiguousarray(index["offsets"], dtype=np.int64)
    ln = np.ascontiguousarray(index["lengths"], dtype=np.int32)
    qt = np.ascontiguousarray(q_terms, dtype=np.int32)
    qw = np.ascontiguousarray(q_weights, dtype=np.uint8 if w.dtype == np.uint8 else np.float32)
    return doc, w, off, ln, qt, qw


def c_search(index: dict, q_terms, q_weights, k: int, threads: int = 0):
    """C version of :func:`search` (same definition; OpenMP over queries).
    Returns (scores f32 or int32 [B, k], fp64 scores [B, k], ids int64 [B, k])."""
    doc, w, off, ln, qt, qw = _c_args(index, q_terms, q_weights)
    B, T = qt.shape
    k = min(k, index["num_docs"])
    s64 = np.empty((B, k), dtype=np.float64)
    ids = np.empty((B, k), dtype=np.int64)
    rc = clib().orc_search(doc.ctypes.data, w.ctypes.data, _WT[w.dtype], off.ctypes.data, ln.ctypes.data,
                           int(index["vocab_size"]), int(index["num_docs"]), qt.ctypes.data, qw.ctypes.data, B, T,
                           k, s64.ctypes.data, ids.ctypes.data, None, int(threads))
    if rc:
        raise RuntimeError(f"orc_search failed ({rc})")
    vals = s64.astype(np.int32) if w.dtype == np.uint8 else s64.astype(np.float32)
    return vals, s64, ids


def c_cpu_sequential(index: dict, q_terms, q_weights, k: int, threads: int = 1):
    """The reference CPU path (float32 accumulator per query, cpu_sequential_score
    src/gpu_scoring.py:221-259) in C; the timed CPU baseline."""
    doc, w, off, ln, qt, qw = _c_args(index, q_terms, q_weights)
    B, T = qt.shape
    k = min(k, index["num_docs"])
    vals = np.empty((B, k), dtype=np.float32)
    ids = np.empty((B, k), dtype=np.int64)
    rc = clib().orc_cpu_sequential(doc.ctypes.data, w.ctypes.data, _WT[w.dtype], off.ctypes.data, ln.ctypes.data,
                                   int(index["vocab_size"]), int(index["num_docs"]), qt.ctypes.data,
                                   qw.ctypes.data, B, T, k, vals.ctypes.data, ids.ctypes.data, int(threads))
    if rc:
        raise RuntimeError(f"orc_cpu_sequential failed ({rc})")
    return vals, ids


def checksum_csr(indptr, indices, data, threads: int = 8) -> int:
    """Order-independent checksum of the (doc, term, weight bits) triples of a
    doc-major CSR (orc_checksum_csr); equal to checksum_index of an index built
    from it when the index holds exactly its postings."""
    ip = np.ascontiguousarray(indptr, dtype=np.int64)
    ix = np.ascontiguousarray(indices, dtype=np.int32)
    d = np.ascontiguousarray(data)
    return int(clib().orc_checksum_csr(ip.ctypes.data, ix.ctypes.data, d.ctypes.data, _WT[d.dtype],
                                       ip.shape[0] - 1, int(threads)))


def checksum_index(index: dict, threads: int = 8) -> tuple[int, int]:
    """(checksum of the index's postings, padding / list slots out of layout)."""
    doc = np.ascontiguousarray(index["doc_ids"], dtype=np.int32)
    w = np.ascontiguousarray(index["scores"])
    off = np.ascontiguousarray(index["offsets"], dtype=np.int64)
    ln = np.ascontiguousarray(index["lengths"], dtype=np.int32)
    pd = np.ascontiguousarray(index["padded_lengths"], dtype=np.int32)
    bad = C.c_int64(0)
    s = clib().orc_checksum_index(doc.ctypes.data, w.ctypes.data, _WT[w.dtype], off.ctypes.data, ln.ctypes.data,
                                  pd.ctypes.data, int(index["vocab_size"]), int(threads), C.byref(bad))
    return int(s), int(bad.value)
