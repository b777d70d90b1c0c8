"""Term-major GPU inverted index and its builders.

The index type keeps the reference's fields and layout
(src/gpu_inverted_index.py:21-35): postings of term t occupy
``[offsets[t], offsets[t] + lengths[t])`` of ``doc_ids`` / ``scores``, ascending
in doc id, each list padded with (-1, 0) to a multiple of 32 slots.  Every
builder here funnels into one GPU pipeline (``gs_index_count`` then
``gs_index_fill``: a stable radix transpose of the doc-major CSR), replacing the
host numpy builders of lsr_benchmark_engine/gpusparse_retrieval.py:81-115 and
src/run_correctness_verification.py:32-84.

Posting weights are stored as float32 (the reference), float16 or uint8.  Query
weights are float32 for float indexes and uint8 for uint8 indexes.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, NamedTuple

import ctypes as C
import math

import numpy as np
import torch

from . import _lib

BLOCK_SIZE = 32          # posting lists are padded to a multiple of this (gpu_inverted_index.py:18)
VOCAB_SIZE = 30522       # fixed vocabulary of the harness builder (run_correctness_verification.py:28)
DEFAULT_TILE_LOG2 = 12          # 4096 docs per LDS tile: postings read from the index arrays
DEFAULT_TILE_LOG2_PACKED = 13   # 8192 docs per LDS tile: postings read from the packed copy
DEFAULT_TILE_LOG2_HYBRID = 14   # 16384 docs per LDS tile, one query each: the hybrid search


def default_tile_log2(index) -> int:
    """Doc-tile size (log2) used when a search names none: 8192 docs (the scorer
    reads one packed word per posting, and its per-tile set-up weighs more than the
    9-query groups of 4096-doc tiles save)."""
    return DEFAULT_TILE_LOG2_PACKED


class CSR(NamedTuple):
    """Doc-major sparse matrix as plain arrays (scipy's csr_matrix also accepted)."""

    indptr: np.ndarray   # int64 [n_rows + 1]
    indices: np.ndarray  # int32 [nnz]
    data: np.ndarray     # float32 / float16 / uint8 [nnz]
    shape: tuple

    @property
    def nnz(self) -> int:
        return int(self.indices.shape[0])

    def to_scipy(self):
        import scipy.sparse as sp
        return sp.csr_matrix((self.data, self.indices, self.indptr), shape=self.shape)


@dataclass
class GPUInvertedIndex:
    """GPU-resident inverted index with block-aligned posting lists
    (src/gpu_inverted_index.py:21-35)."""

    doc_ids: torch.Tensor          # [n_slots] int32, -1 padding
    scores: torch.Tensor           # [n_slots] float32 / float16 / uint8, 0 padding
    offsets: torch.Tensor          # [vocab] int64
    lengths: torch.Tensor          # [vocab] int32
    padded_lengths: torch.Tensor   # [vocab] int32
    max_scores: torch.Tensor       # [vocab] float32
    num_docs: int
    vocab_size: int
    device: torch.device
    # derived data this library schedules by (built lazily when missing)
    _aux: dict = field(default_factory=dict, repr=False, compare=False)

    # -------------------------------------------------------------- derived data
    def aux(self) -> dict:
        a = self.__dict__.get("_aux")
        if a is None:                       # built through __new__ (gpusparse_retrieval.py:107-114)
            a = {}
            self.__dict__["_aux"] = a
        return a

    @property
    def wtype(self) -> int:
        w = _lib.WTYPE_OF_DTYPE.get(self.scores.dtype)
        if w is None:
            raise ValueError(f"posting weights must be float32, float16 or uint8, got {self.scores.dtype}")
        return w

    def search(self, query_batch, k: int = 10, **opts):
        """Exact top-k for a batch of queries: ``(scores [B, k], doc ids [B, k])``.

        ``query_batch`` is ``(term_ids [B, T] int32, term_weights [B, T])`` or a
        query CSR (scipy / :class:`CSR`).  See :func:`gpusparse.search.search`."""
        from .search import search
        return search(self, query_batch, k, **opts)


def _device_of(index) -> torch.device:
    dev = getattr(index, "device", None)
    if dev is None:
        dev = index.doc_ids.device
    return torch.device(dev)


def _as_csr(m) -> CSR:
    if isinstance(m, CSR):
        return m
    import scipy.sparse as sp
    if not sp.issparse(m):
        raise TypeError(f"expected a CSR matrix, got {type(m).__name__}")
    m = m.tocsr()
    return CSR(np.asarray(m.indptr), np.asarray(m.indices), np.asarray(m.data), tuple(m.shape))


def _weights_of(data: np.ndarray, weight_dtype) -> np.ndarray:
    """Posting weights in the storage type.  ``weight_dtype=None`` keeps float16 /
    uint8 data as it is and makes anything else float32; torch.float32 converts
    every type to float32, as the reference builders do
    (gpusparse_retrieval.py:98, run_correctness_verification.py:41)."""
    if weight_dtype is None:
        if data.dtype in (np.float16, np.uint8):
            return np.ascontiguousarray(data)
        return np.ascontiguousarray(data, dtype=np.float32)
    if weight_dtype not in (torch.float32, torch.float16, torch.uint8):
        raise ValueError(f"weight_dtype must be torch.float32, torch.float16 or torch.uint8, got {weight_dtype}")
    want = {torch.float32: np.float32, torch.float16: np.float16, torch.uint8: np.uint8}[weight_dtype]
    if data.dtype == want:
        return np.ascontiguousarray(data)
    if want == np.uint8:
        raise ValueError("uint8 impacts must be quantized by the caller (see gpusparse.synth.quantize_u8)")
    return np.ascontiguousarray(data.astype(np.float32).astype(want))


def build_from_csr(csr, device=None, *, vocab_size: int | None = None, weight_dtype=None,
                   index_error: bool = False, timing: dict | None = None) -> GPUInvertedIndex:
    """GPU index build from a doc-major CSR (rows = documents, columns = terms).

    The native builder: float16 and uint8 CSR data are stored as they are unless
    ``weight_dtype`` names another type (the reference-named builders below store
    float32 by default).  ``vocab_size`` defaults to the number of columns.  Term
    ids outside ``[0, vocab_size)`` raise (IndexError when ``index_error``, as
    numpy does in run_correctness_verification.py:54, else ValueError).
    ``timing``: optional dict; receives ("count", "fill") pairs of events on the
    launch stream around gs_index_count and gs_index_fill (the device-side build,
    the CSR already in HBM)."""
    dev = _lib.require_gpu(device)
    c = _as_csr(csr)
    n_docs = int(c.shape[0])
    V = int(c.shape[1] if vocab_size is None else vocab_size)
    if V <= 0:
        raise ValueError(f"vocabulary size must be positive, got {V}")
    indptr = np.ascontiguousarray(c.indptr, dtype=np.int64)
    indices = np.ascontiguousarray(c.indices, dtype=np.int32)
    data = _weights_of(np.asarray(c.data), weight_dtype)
    nnz = int(indices.shape[0])
    if indptr.shape[0] != n_docs + 1 or indptr[0] != 0 or indptr[-1] != nnz or np.any(np.diff(indptr) < 0):
        raise ValueError("malformed CSR indptr")
    if data.shape[0] != nnz:
        raise ValueError("CSR data and indices differ in length")
    L = _lib.lib()
    s = _lib.stream_ptr(dev)
    indptr_d = torch.from_numpy(indptr).to(dev)
    indices_d = torch.from_numpy(indices).to(dev)
    data_d = torch.from_numpy(data).to(dev)
    lengths = torch.empty(V, dtype=torch.int32, device=dev)
    padded = torch.empty(V, dtype=torch.int32, device=dev)
    offsets = torch.empty(V, dtype=torch.int64, device=dev)
    info = torch.zeros(2, dtype=torch.int64, device=dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)] if timing is not None else None
    if ev:
        ev[0].record()
    _lib.check(L.gs_index_count(_lib.ptr(indices_d) if nnz else None, nnz, V, _lib.ptr(lengths),
                                _lib.ptr(padded), _lib.ptr(offsets), _lib.ptr(info), s), "gs_index_count")
    if ev:
        ev[1].record()
    n_slots, n_bad = (int(x) for x in info.cpu())
    if n_bad:
        msg = f"{n_bad} postings have term ids outside [0, {V})"
        raise IndexError(msg) if index_error else ValueError(msg)
    wdt = {np.float32: torch.float32, np.float16: torch.float16, np.uint8: torch.uint8}[data.dtype.type]
    doc_ids = torch.empty(n_slots, dtype=torch.int32, device=dev)
    weights = torch.empty(n_slots, dtype=wdt, device=dev)
    max_scores = torch.empty(V, dtype=torch.float32, device=dev)
    max_abs = torch.empty(V, dtype=torch.float32, device=dev)
    ws = torch.empty(L.gs_index_fill_workspace(nnz, V), dtype=torch.uint8, device=dev)
    if ev:
        ev[2].record()
    _lib.check(L.gs_index_fill(_lib.ptr(indptr_d), _lib.ptr(indices_d) if nnz else None,
                               _lib.ptr(data_d) if nnz else None, _lib.WTYPE_OF_DTYPE[wdt], n_docs, nnz, V,
                               _lib.ptr(offsets), _lib.ptr(lengths), _lib.ptr(padded), n_slots,
                               _lib.ptr(doc_ids) if n_slots else None, _lib.ptr(weights) if n_slots else None,
                               _lib.ptr(max_scores), _lib.ptr(max_abs), _lib.ptr(ws), ws.numel(), s),
               "gs_index_fill")
    if ev:
        ev[3].record()
        timing["count"] = (ev[0], ev[1])
        timing["fill"] = (ev[2], ev[3])
    del ws
    idx = GPUInvertedIndex(doc_ids=doc_ids, scores=weights, offsets=offsets, lengths=lengths,
                           padded_lengths=padded, max_scores=max_scores, num_docs=n_docs, vocab_size=V,
                           device=dev)
    idx.aux()["max_abs"] = max_abs
    idx.aux()["csr_nnz"] = nnz
    check_lists(idx)
    if wdt != torch.uint8 and nnz > 0 and n_docs > 0:
        # Float indexes are rescored from a doc-major copy.  When every CSR row is
        # sorted by term, the uploaded CSR is that copy (the same rows, a repeated
        # term's entries in CSR order, weights already in the storage type).
        unsorted = torch.empty(1, dtype=torch.int32, device=dev)
        _lib.check(L.gs_rows_sorted(_lib.ptr(indptr_d), _lib.ptr(indices_d), n_docs, _lib.ptr(unsorted), s),
                   "gs_rows_sorted")
        if int(unsorted.item()) == 0:
            idx.aux()["fwd"] = (indptr_d, indices_d, data_d)
    return idx


# ------------------------------------------------------------------ reference builders


def build_index(doc_csr, device, *, weight_dtype=torch.float32) -> GPUInvertedIndex:
    """Drop-in for build_index (lsr_benchmark_engine/gpusparse_retrieval.py:81-115):
    vocabulary = number of CSR columns; weights stored as float32 like the
    reference (:98) unless ``weight_dtype`` opts into torch.float16 or torch.uint8
    (uint8 data must already hold the quantized impacts)."""
    return build_from_csr(doc_csr, device, weight_dtype=weight_dtype)


def build_gpu_index_from_csr(csr_mat, device, *, weight_dtype=torch.float32) -> GPUInvertedIndex:
    """Drop-in for build_gpu_index_from_csr (src/run_correctness_verification.py:32-84):
    the vocabulary is fixed at 30522, larger term ids raise IndexError, weights
    are stored as float32 (:41) unless ``weight_dtype`` says otherwise."""
    return build_from_csr(csr_mat, device, vocab_size=VOCAB_SIZE, weight_dtype=weight_dtype, index_error=True)


def build_gpu_inverted_index(doc_term_ids: list, doc_term_scores: list, vocab_size: int,
                             device=torch.device("cuda:0")) -> GPUInvertedIndex:
    """Drop-in for build_gpu_inverted_index (src/gpu_inverted_index.py:38-113): one
    list of term ids and one of scores per document."""
    if len(doc_term_ids) != len(doc_term_scores):
        raise ValueError("doc_term_ids and doc_term_scores differ in length")
    lens = np.fromiter((len(t) for t in doc_term_ids), dtype=np.int64, count=len(doc_term_ids))
    for t, s in zip(doc_term_ids, doc_term_scores):
        if len(t) != len(s):
            raise ValueError("a document has different numbers of term ids and scores")
    indptr = np.zeros(len(doc_term_ids) + 1, dtype=np.int64)
    np.cumsum(lens, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = np.fromiter((int(x) for t in doc_term_ids for x in t), dtype=np.int64, count=nnz)
    if nnz and (indices.min() < 0 or indices.max() >= vocab_size):
        raise IndexError(f"term id outside [0, {vocab_size})")
    data = np.fromiter((float(x) for s in doc_term_scores for x in s), dtype=np.float32, count=nnz)
    csr = CSR(indptr, indices.astype(np.int32), data, (len(doc_term_ids), int(vocab_size)))
    return build_from_csr(csr, device)


def build_gpu_inverted_index_from_sparse(sparse_matrix, device=torch.device("cuda:0")) -> GPUInvertedIndex:
    """Drop-in for build_gpu_inverted_index_from_sparse (src/gpu_inverted_index.py:116-134),
    without densifying: a torch sparse (COO/CSR) or dense [num_docs, vocab] matrix;
    explicit zeros are dropped as np.nonzero does there."""
    m = sparse_matrix
    n_docs, V = (int(x) for x in m.shape)
    if m.layout == torch.sparse_coo:
        m = m.coalesce()
        ij = m.indices().cpu().numpy()
        vals = m.values().cpu().numpy()
        rows, cols = ij[0], ij[1]
    elif m.layout == torch.sparse_csr:
        crow = m.crow_indices().cpu().numpy().astype(np.int64)
        cols = m.col_indices().cpu().numpy()
        vals = m.values().cpu().numpy()
        rows = np.repeat(np.arange(n_docs), np.diff(crow))
        order = np.lexsort((cols, rows))
        rows, cols, vals = rows[order], cols[order], vals[order]
    else:
        dense = m.cpu().numpy()
        rows, cols = np.nonzero(dense)
        vals = dense[rows, cols]
    keep = vals != 0
    rows, cols, vals = rows[keep], cols[keep], vals[keep]
    indptr = np.zeros(n_docs + 1, dtype=np.int64)
    np.cumsum(np.bincount(rows, minlength=n_docs), out=indptr[1:])
    csr = CSR(indptr, cols.astype(np.int32), vals.astype(np.float32), (n_docs, V))
    return build_from_csr(csr, device)


# ------------------------------------------------------------------ checks and bounds


def check_lists(index) -> tuple[int, int]:
    """(non-ascending lists, non-empty lists); caches the per-list duplicate counts."""
    dev = _device_of(index)
    L = _lib.lib()
    V = int(index.vocab_size)
    bad = torch.empty(V, dtype=torch.int32, device=dev)
    dup = torch.empty(V, dtype=torch.int32, device=dev)
    info = torch.zeros(2, dtype=torch.int64, device=dev)
    _lib.check(L.gs_check_lists(_lib.ptr(index.doc_ids), _lib.ptr(index.offsets), _lib.ptr(index.lengths), V,
                                _lib.ptr(bad), _lib.ptr(dup), _lib.ptr(info), _lib.stream_ptr(dev)),
               "gs_check_lists")
    n_bad, n_nonempty = (int(x) for x in info.cpu())
    a = index.aux() if isinstance(index, GPUInvertedIndex) else {}
    a["n_bad_lists"] = n_bad
    a["n_nonempty"] = n_nonempty
    if n_bad == 0:
        a["dup"] = dup
    return n_bad, n_nonempty


def require_ascending(index) -> None:
    """Raises the reference's ValueError for non-ascending lists
    (src/triton_kernel_chunked.py:99-108)."""
    n_bad, n_nonempty = check_lists(index)
    if n_bad:
        raise ValueError(
            f"{n_bad} of {n_nonempty} posting lists are not ascending in "
            f"doc_id. Chunked scoring requires ascending lists (build the index with "
            f"np.argsort(..., kind='stable')); otherwise results are silently wrong.")


def build_forward(index):
    """Doc-major copy of the index (row pointers, term ids, weights) built on the
    GPU by gs_forward_fill; the exact rescoring of float indexes reads it."""
    dev = _device_of(index)
    L = _lib.lib()
    V = int(index.vocab_size)
    N = int(index.num_docs)
    nnz = int(index.lengths.sum().item())
    row_ptr = torch.empty(N + 1, dtype=torch.int64, device=dev)
    terms = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)
    w = torch.empty(max(nnz, 1), dtype=index.scores.dtype, device=dev)
    ws = torch.empty(int(L.gs_forward_fill_workspace(nnz, V)), dtype=torch.uint8, device=dev)
    _lib.check(L.gs_forward_fill(_lib.ptr(index.doc_ids), _lib.ptr(index.scores), index.wtype,
                                 _lib.ptr(index.offsets), _lib.ptr(index.lengths), V, N, nnz, _lib.ptr(row_ptr),
                                 _lib.ptr(terms), _lib.ptr(w), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev)),
               "gs_forward_fill")
    del ws
    return row_ptr, terms, w


def list_max_abs(index) -> torch.Tensor:
    """max |w| per posting list (gs_list_max), cached with the index."""
    a = index.aux()
    if "max_abs" not in a:
        dev = _device_of(index)
        V = int(index.vocab_size)
        ms = torch.empty(V, dtype=torch.float32, device=dev)
        ma = torch.empty(V, dtype=torch.float32, device=dev)
        ws = torch.empty(8 * V, dtype=torch.uint8, device=dev)
        _lib.check(_lib.lib().gs_list_max(_lib.ptr(index.scores), index.wtype, _lib.ptr(index.offsets),
                                          _lib.ptr(index.lengths), V, _lib.ptr(ms), _lib.ptr(ma), _lib.ptr(ws),
                                          ws.numel(), _lib.stream_ptr(dev)), "gs_list_max")
        a["max_abs"] = ma
    return a["max_abs"]


def heavy_terms(index) -> torch.Tensor:
    """The index's heavy lists, its _lib.heavy_term_count() (64) longest posting
    lists (gs_heavy_terms), int32 term ids by (length desc, term asc), -1 past the
    non-empty lists; gs_search groups the queries of a batch by which of the first
    64 they hold, and the hybrid search scores all of them as matrix products."""
    dev = _device_of(index)
    out = torch.empty(_lib.heavy_term_count(), dtype=torch.int32, device=dev)
    _lib.check(_lib.lib().gs_heavy_terms(_lib.ptr(index.lengths), int(index.vocab_size), _lib.ptr(out),
                                         _lib.stream_ptr(dev)), "gs_heavy_terms")
    return out


def hybrid_eligible(index) -> bool:
    """Whether the hybrid search can serve the index: float weights with a packed
    copy (finite weights), and heavy lists that hold each doc at most once.
    Reads the heavy lists' duplicate counts once (one host sync)."""
    a = index.aux()
    if "hybrid_ok" not in a:
        ok = index.wtype != _lib.GS_W_U8 and int(index.num_docs) > 0
        if ok:
            if "dup" not in a:
                require_ascending(index)
            if "heavy" not in a:
                a["heavy"] = heavy_terms(index)
            # small host copies (the heavy ids, the [vocab] counts): no device
            # reduction on the way to the first search
            h = a["heavy"].cpu().numpy()
            h = h[h >= 0]
            ok = h.size > 0 and int(a["dup"].cpu().numpy()[h].max()) == 0 and pack_shift(index) is not None
        a["hybrid_ok"] = bool(ok)
    return a["hybrid_ok"]


def build_head(index):
    """Dense copy of the heavy terms' packed integer weights (gs_head_fill): int8
    [num_docs rounded up to 512][2][heavy terms] limbs, and the [vocab] int16 heavy
    rank of each term (-1 for the others)."""
    a = index.aux()
    dev = _device_of(index)
    N, V = int(index.num_docs), int(index.vocab_size)
    n_rows = (N + _lib.HEAD_BLOCK - 1) // _lib.HEAD_BLOCK * _lib.HEAD_BLOCK
    head = torch.empty((n_rows, 2, _lib.heavy_term_count()), dtype=torch.int8, device=dev)
    rank = torch.empty(V, dtype=torch.int16, device=dev)
    _lib.check(_lib.lib().gs_head_fill(_lib.ptr(index.doc_ids), _lib.ptr(index.scores), index.wtype,
                                       _lib.ptr(index.offsets), _lib.ptr(index.lengths), V, _lib.ptr(a["heavy"]),
                                       pack_shift(index), N, n_rows, _lib.ptr(head), _lib.ptr(rank),
                                       _lib.stream_ptr(dev)), "gs_head_fill")
    return head, rank


def ensure_search_state(index, tile_log2: int | None = None, forward: bool = True, hybrid: bool = False) -> dict:
    """Derived arrays gs_search needs: max |w|, duplicate counts, the most frequent
    terms (query grouping), tile bounds, the
    packed scoring copy for this tile size (skipped when the GPU has no room for it
    or a weight is not finite: the scorer then reads the index arrays, with the
    same results), and for
    float weights the doc-major copy used by the exact rescoring (skipped when
    `forward` is false or the GPU has no room for it: the rescoring then searches
    the term lists, with the same results).  With `hybrid` also the heavy terms'
    dense copy (skipped when it does not fit: the search then adds every term in
    LDS, with the same results)."""
    if tile_log2 is None:
        tile_log2 = default_tile_log2(index)
    a = index.aux()
    dev = _device_of(index)
    L = _lib.lib()
    V = int(index.vocab_size)
    keys_before = set(a)
    if "dup" not in a:
        require_ascending(index)
    list_max_abs(index)
    if "heavy" not in a:
        a["heavy"] = heavy_terms(index)
    key = ("tile_bounds", tile_log2)
    if key not in a:
        N = int(index.num_docs)
        n_tiles = (N + (1 << tile_log2) - 1) >> tile_log2
        tb = torch.empty((V, n_tiles + 1), dtype=torch.int32, device=dev)
        _lib.check(L.gs_tile_bounds(_lib.ptr(index.doc_ids), _lib.ptr(index.offsets), _lib.ptr(index.lengths), V,
                                    N, tile_log2, _lib.ptr(tb), _lib.stream_ptr(dev)), "gs_tile_bounds")
        a[key] = tb
    key = ("packed", tile_log2)
    if key not in a and int(index.doc_ids.numel()) > 0:
        # One word per posting (4 of 8, 6 or 5 bytes).  One packed copy per index:
        # the one for the tile size last searched.
        for old in [k for k in a if isinstance(k, tuple) and k[0] == "packed"]:
            del a[old]
        try:
            a[key] = build_packed(index, tile_log2)
        except torch.cuda.OutOfMemoryError:
            a[key] = None
    if hybrid and "head" not in a and a.get(("packed", tile_log2)) is not None:
        try:
            a["head"] = build_head(index)
        except torch.cuda.OutOfMemoryError:
            a["head"] = None
    if forward and "fwd" not in a and index.wtype != _lib.GS_W_U8 and int(index.num_docs) > 0:
        try:
            a["fwd"] = build_forward(index)
        except torch.cuda.OutOfMemoryError:
            a["fwd"] = None
    if set(a) != keys_before:
        # built on the current stream: complete before a search on another
        # stream (search_async) reads it
        torch.cuda.current_stream(dev).synchronize()
    return a


def pack_shift(index) -> int | None:
    """Weight scale 2^shift of the packed copy (gs_pack_shift of the largest |w|
    of the index; 0 for uint8), or None when a weight is not finite."""
    if index.wtype == _lib.GS_W_U8:
        return 0
    a = index.aux()
    if "max_abs_all" not in a:
        a["max_abs_all"] = float(np.max(list_max_abs(index).cpu().numpy()))  # NaN when a weight is NaN
    m = a["max_abs_all"]
    if not math.isfinite(m):
        return None
    sh = C.c_int32(0)
    _lib.check(_lib.lib().gs_pack_shift(C.c_float(m), C.byref(sh)), "gs_pack_shift")
    return int(sh.value)


class Packed(NamedTuple):
    words: torch.Tensor   # int32 [n_slots]
    shift: int


def build_packed(index, tile_log2: int, arrange: bool = True) -> Packed | None:
    """Packed scoring copy of the postings for one tile size (gs_pack_postings):
    per slot the byte offset of its doc in a tile slice (bits 0-15) and the weight
    (bits 16-31): the uint8 weight, or int16 rint(w * 2^shift) for float weights.
    With `arrange` each (term, tile) sub-range of more than 64 postings is
    reordered so that every 64-posting group spreads its docs over the residues
    mod 64 (the LDS banks the scorer adds into); the sums do not depend on the
    order.  None when a weight is not finite."""
    shift = pack_shift(index)
    if shift is None:
        return None
    dev = _device_of(index)
    n = int(index.doc_ids.numel())
    N, V = int(index.num_docs), int(index.vocab_size)
    tb = None
    if arrange:
        tb = index.aux().get(("tile_bounds", tile_log2))
        if tb is None:
            n_tiles = (N + (1 << tile_log2) - 1) >> tile_log2
            tb = torch.empty((V, n_tiles + 1), dtype=torch.int32, device=dev)
            _lib.check(_lib.lib().gs_tile_bounds(_lib.ptr(index.doc_ids), _lib.ptr(index.offsets),
                                                 _lib.ptr(index.lengths), V, N, tile_log2, _lib.ptr(tb),
                                                 _lib.stream_ptr(dev)), "gs_tile_bounds")
    out = torch.empty(n, dtype=torch.int32, device=dev)
    _lib.check(_lib.lib().gs_pack_postings(_lib.ptr(index.doc_ids), _lib.ptr(index.scores), index.wtype, n,
                                           _lib.ptr(index.offsets), _lib.ptr(tb), V, N,
                                           tile_log2, shift, _lib.ptr(out), _lib.stream_ptr(dev)), "gs_pack_postings")
    return Packed(out, shift)


def gs_index_struct(index, tile_log2: int | None = None, hybrid: bool = False) -> _lib.GsIndex:
    """The C view of the index for tile_log2; with `hybrid` it carries the heavy
    terms' dense copy as well."""
    if tile_log2 is None:
        tile_log2 = default_tile_log2(index)
    a = ensure_search_state(index, tile_log2, hybrid=hybrid)
    N = int(index.num_docs)
    s = _lib.GsIndex()
    s.doc_ids_d = index.doc_ids.data_ptr()
    s.weights_d = index.scores.data_ptr()
    s.offsets_d = index.offsets.data_ptr()
    s.lengths_d = index.lengths.data_ptr()
    s.max_abs_d = a["max_abs"].data_ptr()
    s.dup_d = a["dup"].data_ptr()
    s.tile_bounds_d = a[("tile_bounds", tile_log2)].data_ptr()
    s.n_slots = int(index.doc_ids.numel())
    s.n_docs = N
    s.vocab = int(index.vocab_size)
    s.wtype = index.wtype
    s.tile_log2 = tile_log2
    s.n_tiles = (N + (1 << tile_log2) - 1) >> tile_log2
    fwd = a.get("fwd")
    if fwd is not None:
        s.fwd_ptr_d, s.fwd_terms_d, s.fwd_weights_d = (t.data_ptr() for t in fwd)
    s.heavy_d = a["heavy"].data_ptr()
    pk = a.get(("packed", tile_log2))
    if pk is not None:
        s.packed_d, s.packed_tile_log2, s.packed_shift = pk.words.data_ptr(), tile_log2, pk.shift
    hd = a.get("head") if hybrid else None
    if hd is not None:
        s.head_d, s.head_rank_d = hd[0].data_ptr(), hd[1].data_ptr()
    return s


def index_memory_stats(index) -> dict:
    """Same report as src/gpu_inverted_index.py:177-196."""
    doc_ids_bytes = index.doc_ids.nelement() * index.doc_ids.element_size()
    scores_bytes = index.scores.nelement() * index.scores.element_size()
    meta = [index.offsets, index.lengths, index.padded_lengths, index.max_scores]
    meta_bytes = sum(t.nelement() * t.element_size() for t in meta)
    n_post = int(index.lengths.sum().item())
    n_pad = int(index.padded_lengths.sum().item())
    return {
        "doc_ids_MB": doc_ids_bytes / 1e6,
        "scores_MB": scores_bytes / 1e6,
        "metadata_MB": meta_bytes / 1e6,
        "total_MB": (doc_ids_bytes + scores_bytes + meta_bytes) / 1e6,
        "num_postings": n_post,
        "num_padded": n_pad,
        "padding_overhead": 1.0 - n_post / max(1, n_pad),
    }


def to_host(index) -> dict[str, Any]:
    """numpy copies of the reference fields (for checks and for the CPU baseline)."""
    out = {k: getattr(index, k).cpu().numpy() for k in
           ("doc_ids", "scores", "offsets", "lengths", "padded_lengths", "max_scores")
           if getattr(index, k, None) is not None}
    out["num_docs"] = int(index.num_docs)
    out["vocab_size"] = int(index.vocab_size)
    return out
