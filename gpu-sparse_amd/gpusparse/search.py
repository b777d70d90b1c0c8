"""Batched exact search and the reference's scoring entry points.

``search(index, query_batch, k)`` is the batched retrieval call: scores and doc
ids of the k best documents per query, ordered by score descending, ties by doc
id ascending.  ``triton_fused_score`` (src/triton_kernel.py:159-200) keeps the
reference's name and signature.  Both run the fused pipeline of ``gs_search``
(for float indexes whose heavy lists hold each doc once, the hybrid search: the
heavy terms as int8 matrix products, the others added in LDS score tiles; else
every term added in LDS) and finish the rare rows it flags with the dense path
(``gs_search_dense``), or run the dense path directly when the full
``[B, num_docs]`` score rows are small.

Float indexes return float32 scores equal to the fp64 scatter-add rounded to
float32; uint8 indexes return the exact uint32 sums as int32.
"""
from __future__ import annotations

from collections import OrderedDict

import numpy as np
import torch

from . import _lib
from .index import DEFAULT_TILE_LOG2_HYBRID, default_tile_log2, gs_index_struct, hybrid_eligible, _device_of

MAX_K = 8192  # largest k of the fused path and of compacted_topk; search answers larger k densely
MAX_T = 8192  # widest query batch of the fused path (terms per query); search answers wider ones densely
DEFAULT_DENSE_BUDGET = 1 << 30   # bytes of [B, N] score rows below which the dense path is used


def _check_pow2(block_pl: int) -> None:
    # same check as src/triton_kernel.py:175-176
    assert block_pl > 0 and (block_pl & (block_pl - 1)) == 0, \
        f"block_pl must be a positive power of 2, got {block_pl}"


_U8_WEIGHTS_MSG = "a uint8 index takes uint8 query weights: float weights must be integers in [0, 255]"


def query_tensors(index, query_batch, defer_check: bool = False):
    """(term ids int32 [B, T], weights [B, T]) on the index device, from a tuple of
    tensors/arrays or from a query CSR (no truncation, as to_query_tensors; a
    uint8 CSR stays uint8).

    A uint8 index takes float query weights (the reference's query tensors are
    float32, gpusparse_retrieval.py:124) when every one is an integer in
    [0, 255]: the uint8 impacts they carry.  Weights in host memory are checked
    on the host before the upload.  Weights already on the GPU are checked there;
    reading that check waits for the GPU, so with `defer_check` it is returned
    instead, as a third item (a device bool, True when a weight fails; None when
    nothing was checked on the GPU), for the caller to read with its results."""
    dev = _device_of(index)
    if isinstance(query_batch, tuple) and len(query_batch) in (2, 3) and not hasattr(query_batch, "indptr"):
        qt, qw = query_batch[0], query_batch[1]
    else:
        from .engine import to_query_tensors
        qt, qw, _ = to_query_tensors(query_batch, dev, weight_dtype=None)
    qt = torch.as_tensor(qt)
    qw = torch.as_tensor(qw)
    if qt.dim() != 2 or qw.shape != qt.shape:
        raise ValueError(f"query term ids {tuple(qt.shape)} and weights {tuple(qw.shape)} must be the same [B, T]")
    want = torch.uint8 if index.scores.dtype == torch.uint8 else torch.float32
    bad = None
    if qw.dtype != want and want == torch.uint8:
        if not (qw.dtype.is_floating_point or qw.dtype in (torch.int16, torch.int32, torch.int64)):
            raise ValueError(f"a uint8 index takes uint8 query weights, got {qw.dtype}")
        if qw.numel():
            if qw.device.type == "cpu":
                h = qw.double().numpy()
                if not bool(np.all((h >= 0) & (h <= 255) & (h == np.round(h)))):
                    raise ValueError(_U8_WEIGHTS_MSG)
            else:
                qd = qw.to(dev)
                bad = ~((qd >= 0) & (qd <= 255) & (qd == torch.round(qd.double()))).all()
                if not defer_check:
                    if bool(bad):
                        raise ValueError(_U8_WEIGHTS_MSG)
                    bad = None
    qt = qt.to(dev)
    qw = qw.to(dev)
    if qt.dtype != torch.int32:
        qt = qt.to(torch.int32)
    if qw.dtype != want:
        qw = qw.to(want)
    if defer_check:
        return qt.contiguous(), qw.contiguous(), bad
    return qt.contiguous(), qw.contiguous()


HYBRID_DEFAULT = True  # whether searches that name no scorer take the hybrid one


U8_HYBRID_MAX_T = 258  # widest uint8 batch the float16 copy serves: 258 * 255 * 255 < 2^24


def u8_float_copy(index):
    """For a uint8 index: the same postings with the weights as float16 (exact
    for 0..255), which the hybrid search runs on; built once, kept in aux()
    (2 bytes per slot more HBM, plus that copy's own search state).  Its answers
    are the exact integer sums: the fp64 rescoring sums integer products, and
    the fp32 result of a sum below 2^24 is that sum."""
    from .index import GPUInvertedIndex
    a = index.aux()
    f = a.get("f16_copy")
    if f is None:
        f = GPUInvertedIndex(doc_ids=index.doc_ids, scores=index.scores.to(torch.float16), offsets=index.offsets,
                             lengths=index.lengths, padded_lengths=index.padded_lengths,
                             max_scores=index.max_scores, num_docs=index.num_docs, vocab_size=index.vocab_size,
                             device=_device_of(index))
        a["f16_copy"] = f
    return f


def u8_hybrid_ok(index, T: int | None = None) -> bool:
    """Whether a uint8 index can take the hybrid search through its float16 copy
    for batches T terms wide: no list repeats a doc (so a doc's sum holds at
    most T products of at most 255 * 255, below 2^24 for T <= 258, exact in
    fp32) and the copy is eligible.  Reads the lists' duplicate counts once."""
    if index.wtype != _lib.GS_W_U8 or int(index.num_docs) == 0:
        return False
    if T is not None and int(T) > U8_HYBRID_MAX_T:
        return False
    a = index.aux()
    if "u8_hybrid_ok" not in a:
        if "dup" not in a:
            from .index import require_ascending
            require_ascending(index)
        a["u8_hybrid_ok"] = int(a["dup"].cpu().numpy().max()) == 0 and hybrid_eligible(u8_float_copy(index))
    return a["u8_hybrid_ok"]


def search_index(index, hybrid: bool):
    """The index a search with this scorer runs on: a uint8 index's float16 copy
    for the hybrid search, else the index itself."""
    return u8_float_copy(index) if hybrid and index.wtype == _lib.GS_W_U8 else index


def scorer_choice(index, tile_log2: int | None = None, hybrid: bool | None = None,
                  T: int | None = None) -> tuple[int, bool]:
    """(tile_log2, hybrid) of a search.  hybrid: whether the index's heavy (64 longest)
    lists are scored as int8 matrix products (the hybrid search) instead of LDS
    adds; None takes HYBRID_DEFAULT when the index allows it.  hybrid=True
    requires an eligible index (float weights, heavy lists without repeated
    docs).  tile_log2 defaults to DEFAULT_TILE_LOG2_HYBRID (16384 docs, one query
    per workgroup) for the hybrid search and to index.default_tile_log2 (8192
    docs, two queries) otherwise: the terms left to the LDS adds of the hybrid
    search are rarely shared by the queries of a group, while longer runs per
    (term, tile) halve the per-run work (C3 scoring 5.68 vs 6.24 ms).  A uint8
    index takes the hybrid search through its float16 copy (u8_hybrid_ok; T =
    the batch width, when known)."""
    ok = u8_hybrid_ok(index, T) if index.wtype == _lib.GS_W_U8 else hybrid_eligible(index)
    if hybrid is None:
        hybrid = HYBRID_DEFAULT and ok
    if hybrid and not ok:
        raise ValueError("the hybrid search needs finite weights, heavy lists without repeated docs, and for "
                         f"uint8 weights no repeated docs at all and batches of at most {U8_HYBRID_MAX_T} terms")
    if tile_log2 is None:
        tile_log2 = DEFAULT_TILE_LOG2_HYBRID if hybrid else default_tile_log2(index)
    return int(tile_log2), bool(hybrid)


def _opts(sample_tiles=0, cand_cap=0, unroll=0, waves=0, tiles_per_wg=0, batch_order=False, hybrid=False):
    o = _lib.GsSearchOpts(sample_tiles, cand_cap, unroll, waves, None, None, tiles_per_wg)
    o.batch_order = int(bool(batch_order))
    o.no_hybrid = 0 if hybrid else 1
    return o


WORKSPACE_STREAMS = 4  # streams whose fused-search workspaces an index keeps


def _workspace(index, nbytes: int, stream_key: int = 0) -> torch.Tensor:
    """The index's fused-search workspace for one stream (searches in flight on
    different streams must not share one; on one stream they run in order).  The
    index keeps those of its WORKSPACE_STREAMS most recently used streams (a
    dropped one is freed once the searches queued with it are done: the
    allocator orders its reuse on its stream).  The one last handed out is also
    aux()["workspace"], which search_counts reads."""
    a = index.aux()
    pool = a.setdefault("workspaces", OrderedDict())
    ws = pool.get(stream_key)
    if ws is None or ws.numel() < nbytes:
        pool.pop(stream_key, None)  # a smaller one is replaced, not kept beside it
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=_device_of(index))
        pool[stream_key] = ws
    pool.move_to_end(stream_key)
    while len(pool) > WORKSPACE_STREAMS:
        pool.popitem(last=False)
    a["workspace"] = ws
    return ws


def _dense_rows(index, gidx, qt, qw, k, rows, out_s, out_i, dense_budget):
    """Runs gs_search_dense for `rows` (int32 device tensor or None = all)."""
    L = _lib.lib()
    dev = _device_of(index)
    B, T = qt.shape
    R = B if rows is None else int(rows.numel())
    if R == 0:
        return
    one = _lib.C.c_size_t()
    _lib.check(L.gs_search_dense_workspace(_lib.C.byref(gidx), 1, _lib.C.byref(one)), "gs_search_dense_workspace")
    per_row = max(int(one.value), 1)
    rows_per_pass = max(1, min(R, dense_budget // per_row))
    ws = torch.empty(rows_per_pass * per_row, dtype=torch.uint8, device=dev)
    _lib.check(L.gs_search_dense(_lib.C.byref(gidx), _lib.ptr(qt), _lib.ptr(qw), B, T, k, _lib.ptr(rows), R,
                                 _lib.ptr(out_s), _lib.ptr(out_i), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev)),
               "gs_search_dense")


class PendingSearch:
    """A search whose kernels are queued on a stream (`search_async`).

    `result()` waits for the fused pipeline's per-row status (one event, no
    device-wide synchronisation), finishes the rows it flagged with the dense
    path on the same stream and returns ``(scores [B, k], ids [B, k] int64)``.
    The returned tensors are ordered on the search's stream: the stream current
    at the `result()` call is made to wait for it."""

    __slots__ = ("_out", "_stream", "_event", "_status_h", "_finish", "_post")

    def __init__(self, out, stream=None, event=None, status_h=None, finish=None, post=None):
        self._out = out
        self._stream = stream
        self._event = event
        self._status_h = status_h
        self._finish = finish
        self._post = post  # applied to the results once, on the stream current at result()

    def done(self) -> bool:
        """True when result() would not wait for the GPU."""
        return self._finish is None or self._event.query()

    def result(self):
        if self._finish is not None:
            self._event.synchronize()
            bad = np.nonzero(self._status_h.numpy() != _lib.GS_ROW_DONE)[0]
            finish, self._finish = self._finish, None
            self._status_h = None
            finish(bad)
        if self._stream is not None:
            cur = torch.cuda.current_stream(self._stream.device)
            if cur != self._stream:
                cur.wait_stream(self._stream)
                for t in self._out:
                    t.record_stream(cur)  # freed only after the current stream's uses
        if self._post is not None:
            post, self._post = self._post, None
            self._out = post(self._out)
        return self._out


def search(index, query_batch, k: int = 10, *, tile_log2: int | None = None, path: str = "auto",
           sample_tiles: int = 0, cand_cap: int = 0, unroll: int = 0, waves: int = 0,
           tiles_per_wg: int = 0, dense_budget: int = DEFAULT_DENSE_BUDGET, timing: dict | None = None,
           batch_order: bool = False, hybrid: bool | None = None):
    """Exact top-k of a query batch.  Returns ``(scores [B, k], ids [B, k] int64)``.

    tile_log2: doc-tile size of the scorer (default: index.default_tile_log2).
    hybrid: the index's heavy (64 longest) lists as int8 matrix products, the other terms
    as LDS adds (scorer_choice; a uint8 index through its float16 copy); results
    are the same either way.
    path: "auto" (dense when the [B, N] rows fit `dense_budget`), "fused" or "dense";
    k above MAX_K (8192) or queries wider than MAX_T (8192 terms) always take the
    dense path (any k up to the doc count, any width).
    timing: optional dict; receives event pairs on the launch stream bracketing the
    fused scoring kernel ("score_kernel") and the whole gs_search call ("search"),
    the GS_SEARCH_PHASES events of each call ("phases": start, query prep,
    heavy-term sums, threshold seed, scoring, candidate selection, fp64
    rescoring, final sort) and
    the number of rows finished by the dense path ("dense_rows").  Events come
    from timing["event_pool"] while it lasts (see `timing_dict`).
    batch_order: score queries in groups of consecutive queries instead of groups of
    queries sharing frequent terms (same results; for comparisons)."""
    return search_async(index, query_batch, k, tile_log2=tile_log2, path=path, sample_tiles=sample_tiles,
                        cand_cap=cand_cap, unroll=unroll, waves=waves, tiles_per_wg=tiles_per_wg,
                        dense_budget=dense_budget, timing=timing, batch_order=batch_order,
                        hybrid=hybrid).result()


def search_async(index, query_batch, k: int = 10, *, tile_log2: int | None = None, path: str = "auto",
                 sample_tiles: int = 0, cand_cap: int = 0, unroll: int = 0, waves: int = 0,
                 tiles_per_wg: int = 0, dense_budget: int = DEFAULT_DENSE_BUDGET, timing: dict | None = None,
                 batch_order: bool = False, hybrid: bool | None = None) -> PendingSearch:
    """`search` without waiting: queues the batch on the current stream and
    returns a `PendingSearch` (same arguments and results as `search`).  The host
    can queue the next batch, or post-process the previous one, while this one
    runs; batches in flight on one stream run in order and share the index's
    workspace, batches on different streams get one workspace per stream."""
    dev = _lib.require_gpu(_device_of(index))
    N = int(index.num_docs)
    kk = min(int(k), N)
    if kk < 1:
        raise ValueError(f"k must be >= 1, got {k}")
    qt, qw, bad_w = query_tensors(index, query_batch, defer_check=True)
    B, T = qt.shape
    out_dtype = torch.int32 if index.scores.dtype == torch.uint8 else torch.float32
    out_s = torch.empty((B, kk), dtype=out_dtype, device=dev)
    out_i = torch.empty((B, kk), dtype=torch.int64, device=dev)
    if B == 0:
        return PendingSearch((out_s, out_i))
    if T == 0:
        qt = torch.full((B, 1), -1, dtype=torch.int32, device=dev)
        qw = torch.zeros((B, 1), dtype=qw.dtype, device=dev)
        T = 1
    tile_log2, hyb = scorer_choice(index, tile_log2, hybrid, T)
    if hyb and index.wtype == _lib.GS_W_U8:
        # the float16 copy's hybrid search; its fp32 scores are the exact sums.
        # The weights' check (device weights) is copied out ahead of the search,
        # so it has landed when result() has the search's status.
        bad_h = None
        if bad_w is not None:
            bad_h = torch.empty((), dtype=torch.bool, pin_memory=True)
            bad_h.copy_(bad_w, non_blocking=True)
        inner = search_async(u8_float_copy(index), (qt, qw.to(torch.float32)), k, tile_log2=tile_log2, path=path,
                             sample_tiles=sample_tiles, cand_cap=cand_cap, unroll=unroll, waves=waves,
                             tiles_per_wg=tiles_per_wg, dense_budget=dense_budget, timing=timing,
                             batch_order=batch_order, hybrid=True)

        def to_int(out):
            if bad_h is not None and bool(bad_h):
                raise ValueError(_U8_WEIGHTS_MSG)
            return out[0].to(torch.int32), out[1]

        inner._post = to_int
        return inner
    gidx = gs_index_struct(index, tile_log2, hyb)
    L = _lib.lib()
    acc_bytes = 4 if index.scores.dtype == torch.uint8 else 8
    dense_bytes = B * gidx.n_tiles * (1 << tile_log2) * acc_bytes
    if path not in ("auto", "fused", "dense"):
        raise ValueError(f"unknown path {path!r}")
    stream = torch.cuda.current_stream(dev)
    # k above MAX_K or queries wider than MAX_T terms: the dense path, whose
    # selection takes any k (rounds of MAX_K) and whose scorer any width
    use_dense = path == "dense" or kk > MAX_K or T > MAX_T or (path == "auto" and dense_bytes <= dense_budget)
    if use_dense:
        if bad_w is not None and bool(bad_w):
            raise ValueError(_U8_WEIGHTS_MSG)
        _dense_rows(index, gidx, qt, qw, kk, None, out_s, out_i, max(dense_budget, 1))
        return PendingSearch((out_s, out_i), stream)
    opts = _opts(sample_tiles, cand_cap, unroll, waves, tiles_per_wg, batch_order, hyb)
    need = _lib.C.c_size_t()
    _lib.check(L.gs_search_workspace(_lib.C.byref(gidx), B, T, kk, _lib.C.byref(opts), _lib.C.byref(need)),
               "gs_search_workspace")
    ws = _workspace(index, int(need.value), stream.cuda_stream)
    status = torch.empty(B, dtype=torch.int32, device=dev)
    s = _lib.stream_ptr(dev)
    if timing is not None:
        # events recorded by gs_search itself around the fused scoring kernel and at
        # its phase boundaries, and around the whole gs_search call, on the launch stream
        pool = timing.get("event_pool")
        evs, ph, ph_ptr = pool.pop() if pool else _call_events()
        opts.ev_score_begin, opts.ev_score_end = evs[0].cuda_event, evs[1].cuda_event
        opts.ev_phases = ph_ptr
        evs[2].record()
    _lib.check(L.gs_search(_lib.C.byref(gidx), _lib.ptr(qt), _lib.ptr(qw), B, T, kk, _lib.C.byref(opts),
                           _lib.ptr(out_s), _lib.ptr(out_i), _lib.ptr(status), _lib.ptr(ws), ws.numel(), s),
               "gs_search")
    if timing is not None:
        evs[3].record()
        timing.setdefault("score_kernel", []).append((evs[0], evs[1]))
        timing.setdefault("search", []).append((evs[2], evs[3]))
        if ph:
            timing.setdefault("phases", []).append(ph)
    status_h = torch.empty(B, dtype=torch.int32, pin_memory=True)
    status_h.copy_(status, non_blocking=True)
    bad_h = None
    if bad_w is not None:  # the weights' check, read with the status
        bad_h = torch.empty((), dtype=torch.bool, pin_memory=True)
        bad_h.copy_(bad_w, non_blocking=True)
    done = torch.cuda.Event()
    done.record(stream)

    def finish(bad):
        if bad_h is not None and bool(bad_h):
            raise ValueError(_U8_WEIGHTS_MSG)
        if timing is not None:
            timing["dense_rows"] = timing.get("dense_rows", 0) + int(bad.size)
        if bad.size:
            with torch.cuda.stream(stream):
                rows = torch.from_numpy(bad.astype(np.int32)).to(dev)
                _dense_rows(index, gidx, qt, qw, kk, rows, out_s, out_i, max(dense_budget, 1))

    return PendingSearch((out_s, out_i), stream, done, status_h, finish)


def _call_events(phases: bool = True):
    """The events of one timed `search` call: 4 bracketing ones, one per phase
    (unless `phases` is false) and the C array of the phase events.  Each is
    recorded once here, which creates its HIP event."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ph = [torch.cuda.Event(enable_timing=True) for _ in range(_lib.GS_SEARCH_PHASES)] if phases else []
    for e in evs + ph:
        e.record()
    ph_ptr = None
    if ph:
        arr = (_lib.C.c_void_p * len(ph))(*[e.cuda_event for e in ph])
        ph_ptr = _lib.C.cast(arr, _lib.C.POINTER(_lib.C.c_void_p))
        ph_ptr._keep = arr
    return evs, ph, ph_ptr


def timing_dict(n_calls: int, phases: bool = True) -> dict:
    """A `timing` dict for `search` holding the events of `n_calls` calls, created
    up front: the timed calls then only record them (creating them inside a call
    costs ~0.1 ms of host time, which the GPU waits out after the call's status
    read).  phases=False leaves out the per-phase events (and "phases")."""
    return {"event_pool": [_call_events(phases) for _ in range(int(n_calls))]}


def search_plan(index, B: int, T: int, k: int, *, tile_log2: int | None = None, sample_tiles: int = 0,
                cand_cap: int = 0, unroll: int = 0, tiles_per_wg: int = 0, batch_order: bool = False,
                hybrid: bool | None = None) -> dict:
    """How the fused path of `search` runs a batch of B queries of width T
    (gs_search_plan): seed tiles, queries per group, postings per lane per chunk,
    tiles per scoring workgroup, whether the packed copy is read and whether the
    hybrid scorer runs."""
    tile_log2, hyb = scorer_choice(index, tile_log2, hybrid, T)
    index = search_index(index, hyb)
    gidx = gs_index_struct(index, tile_log2, hyb)
    opts = _opts(sample_tiles, cand_cap, unroll, 0, tiles_per_wg, batch_order, hyb)
    info = _lib.GsSearchPlanInfo()
    _lib.check(_lib.lib().gs_search_plan(_lib.C.byref(gidx), int(B), int(T), min(int(k), int(index.num_docs)),
                                         _lib.C.byref(opts), _lib.C.byref(info)), "gs_search_plan")
    return {"tile_log2": tile_log2, "seed_tiles": info.seed_tiles, "group_size": info.group_size,
            "unroll": info.unroll, "tiles_per_wg": info.tiles_per_wg, "packed": bool(info.packed),
            "hybrid": bool(info.hybrid), "cand_cap": info.cand_cap}


def search_counts(index, B: int, T: int, k: int, *, tile_log2: int | None = None, sample_tiles: int = 0,
                  cand_cap: int = 0, unroll: int = 0, tiles_per_wg: int = 0, batch_order: bool = False,
                  hybrid: bool | None = None):
    """Per scoring slot of the fused search that last ran with these arguments:
    (docs the scorer emitted as candidates, candidates rescored in fp64), two
    numpy uint32 [B] arrays (gs_search_counts on the index's cached workspace)."""
    tile_log2, hyb = scorer_choice(index, tile_log2, hybrid, T)
    index = search_index(index, hyb)
    ws = index.aux().get("workspace")
    if ws is None:
        raise ValueError("no fused search has run on this index")
    dev = _device_of(index)
    gidx = gs_index_struct(index, tile_log2, hyb)
    opts = _opts(sample_tiles, cand_cap, unroll, 0, tiles_per_wg, batch_order, hyb)
    cand = torch.empty(B, dtype=torch.int32, device=dev)
    resc = torch.empty(B, dtype=torch.int32, device=dev)
    _lib.check(_lib.lib().gs_search_counts(_lib.C.byref(gidx), int(B), int(T), min(int(k), int(index.num_docs)),
                                           _lib.C.byref(opts), _lib.ptr(ws), ws.numel(), _lib.ptr(cand),
                                           _lib.ptr(resc), _lib.stream_ptr(dev)), "gs_search_counts")
    return cand.cpu().numpy().view(np.uint32), resc.cpu().numpy().view(np.uint32)


def triton_fused_score(index, query_term_ids: torch.Tensor, query_term_scores: torch.Tensor, top_k: int = 10,
                       block_pl: int = 128):
    """Drop-in for triton_fused_score (src/triton_kernel.py:159-200): exact top-k,
    (scores [B, k] desc, ids [B, k] int64).  block_pl is validated as the
    reference does; the LDS-tile scorer uses its own tuned posting chunk."""
    _check_pow2(block_pl)
    return search(index, (query_term_ids, query_term_scores), top_k)


def compacted_topk(scores: torch.Tensor, tau: torch.Tensor, k: int, max_cand: int = 8192, block: int = 1024):
    """Drop-in for compacted_topk (src/fused_topk.py:71-103): top-k of `scores`
    [B, L] among entries >= tau[B]; (values [B, kk], chunk-local indices [B, kk]),
    missing slots (-inf, 0).  Rows with more than max_cand candidates are selected
    from the full row.  `block` is accepted for signature compatibility."""
    if scores.dim() != 2:
        raise ValueError("scores must be [B, L]")
    dev = _lib.require_gpu(scores.device)
    B, Lc = scores.shape
    kk = min(int(k), Lc)
    if kk > MAX_K:
        raise ValueError(f"k={kk} exceeds the supported maximum {MAX_K}")
    max_cand = max(int(max_cand), kk)
    if scores.dtype != torch.float32 or scores.stride(1) != 1:
        scores = scores.float().contiguous()
    tau_d = None
    if tau is not None:
        tau_d = torch.as_tensor(tau, dtype=torch.float32, device=dev).contiguous()
    out_v = torch.empty((B, kk), dtype=torch.float32, device=dev)
    out_i = torch.empty((B, kk), dtype=torch.int64, device=dev)
    if B == 0:
        return out_v, out_i
    counts = torch.empty(B, dtype=torch.int32, device=dev)
    L = _lib.lib()
    ws = torch.empty(L.gs_compacted_topk_workspace(B, max_cand), dtype=torch.uint8, device=dev)
    _lib.check(L.gs_compacted_topk(_lib.ptr(scores), scores.stride(0), B, Lc, _lib.ptr(tau_d), kk, max_cand,
                                   _lib.ptr(out_v), _lib.ptr(out_i), _lib.ptr(counts), _lib.ptr(ws), ws.numel(),
                                   _lib.stream_ptr(dev)), "gs_compacted_topk")
    return out_v, out_i


def topk_rows(scores: torch.Tensor, k: int):
    """Exact top-k of each row (torch.topk semantics on [B, L]; ties: lower column first)."""
    return compacted_topk(scores, None, k, max_cand=max(k, 1))


def scatter_add(index, query_term_ids, query_term_scores, out: torch.Tensor, lo=None, hi=None, chunk_start: int = 0,
                chunk_len: int | None = None, block_pl: int = 128) -> torch.Tensor:
    """The reference kernel on this GPU: per (query, term) program, global atomic
    adds of q*w into `out` (pre-zeroed, [B, >= chunk_len], row stride out.stride(0)).
    lo/hi: int64 [V] posting bounds of one chunk (_chunked_scatter_add_kernel,
    src/triton_kernel_chunked.py:34-80) or None for whole lists
    (_fast_scatter_add_kernel, src/triton_kernel.py:93-156)."""
    _check_pow2(block_pl)
    dev = _lib.require_gpu(_device_of(index))
    qt, qw = query_tensors(index, (query_term_ids, query_term_scores))
    B, T = qt.shape
    clen = int(index.num_docs) if chunk_len is None else int(chunk_len)
    gidx = _lib.GsIndex()
    gidx.doc_ids_d = index.doc_ids.data_ptr()
    gidx.weights_d = index.scores.data_ptr()
    gidx.offsets_d = index.offsets.data_ptr()
    gidx.lengths_d = index.lengths.data_ptr()
    gidx.n_docs = int(index.num_docs)
    gidx.vocab = int(index.vocab_size)
    gidx.wtype = index.wtype
    want = torch.int32 if index.scores.dtype == torch.uint8 else torch.float32
    if out.dtype != want or out.dim() != 2 or out.stride(1) != 1 or out.device != dev:
        raise ValueError(f"out must be a row-contiguous [B, L] {want} tensor on {dev}")
    if out.shape[0] < B or out.shape[1] < clen:
        raise ValueError(f"out {tuple(out.shape)} is smaller than [{B}, {clen}]")
    V = int(index.vocab_size)
    for b in (lo, hi):
        if b is not None and (b.dtype != torch.int64 or b.numel() != V or b.device != dev):
            raise ValueError(f"chunk bounds must be int64 [{V}] tensors on {dev}")
    if (lo is None) != (hi is None):
        raise ValueError("lo and hi must both be given or both be None")
    if B == 0 or T == 0:
        return out
    lo = None if lo is None else lo.contiguous()
    hi = None if hi is None else hi.contiguous()
    _lib.check(_lib.lib().gs_scatter_add(_lib.C.byref(gidx), _lib.ptr(lo), _lib.ptr(hi), _lib.ptr(qt), _lib.ptr(qw),
                                         B, T, _lib.ptr(out), int(chunk_start), clen, out.stride(0), block_pl,
                                         _lib.stream_ptr(dev)), "gs_scatter_add")
    return out


def atomic_fused_score(index, query_term_ids, query_term_scores, top_k: int = 10, block_pl: int = 128):
    """The reference's monolithic algorithm on this GPU (zeroed [B, N] fp32
    accumulator, global-atomic scatter-add, exact row top-k): the baseline the
    LDS-tile path is compared against.  Scores are fp32 sums in atomic order."""
    dev = _lib.require_gpu(_device_of(index))
    qt, qw = query_tensors(index, (query_term_ids, query_term_scores))
    B = qt.shape[0]
    N = int(index.num_docs)
    dt = torch.int32 if index.scores.dtype == torch.uint8 else torch.float32
    out = torch.zeros((B, N), dtype=dt, device=dev)
    scatter_add(index, qt, qw, out, block_pl=block_pl)
    if dt == torch.int32:
        # uint8 sums stay below 2^24 for queries of <= 258 terms, where fp32 is exact
        v, i = topk_rows(out.to(torch.float32), top_k)
        return v.to(torch.int32), i
    return topk_rows(out, top_k)
