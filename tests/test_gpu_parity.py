"""GPU parity: the HIP path against the CPU oracle on the same seeded inputs.

Bar: index arrays, chunk bounds and uint8 results bit-exact; float results with
identical ids and scores equal to the oracle's fp64 scatter-add rounded to fp32
(bit-exact, which is stricter than the |diff| <= 1e-5 tolerance of the task)."""
import numpy as np
import pytest
import torch

import gpusparse as gs
from gpusparse import synth
from gpusparse.search import HYBRID_DEFAULT
from gpusparse.index import CSR, GPUInvertedIndex
from helpers import random_csr, random_queries
from oracle import oracle as O

pytestmark = pytest.mark.gpu

FIELDS = ("doc_ids", "scores", "offsets", "lengths", "padded_lengths", "max_scores")


def oracle_index(csr: CSR, vocab=None):
    return O.build_index(csr.indptr, csr.indices, csr.data, csr.shape[0], csr.shape[1] if vocab is None else vocab)


def assert_index_equal(ix, ref):
    for f in FIELDS:
        got = getattr(ix, f).cpu().numpy()
        want = ref[f]
        assert got.dtype == want.dtype, f
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f
    assert ix.num_docs == ref["num_docs"] and ix.vocab_size == ref["vocab_size"]


def assert_search_equal(ix, ref, ti, tw, k, **opts):
    s, i = gs.search(ix, (torch.from_numpy(ti), torch.from_numpy(tw)), k, **opts)
    vs, s64, vi = O.c_search(ref, ti, tw, k, threads=8)
    s, i = s.cpu().numpy(), i.cpu().numpy()
    assert np.array_equal(i, vi)
    assert s.dtype == vs.dtype and np.array_equal(s, vs)
    if s.dtype == np.float32:
        assert np.max(np.abs(s.astype(np.float64) - s64), initial=0.0) <= 1e-5
    return s, i


# ------------------------------------------------------------------ index build


@pytest.mark.parametrize("seed,n_docs,vocab,dtype,dup", [
    (0, 500, 300, np.float32, 0.0), (1, 2000, 9, np.float32, 0.2), (2, 300, 1, np.float32, 0.0),
    (3, 1000, 700, np.float16, 0.05), (4, 700, 250, np.uint8, 0.0), (5, 1, 3, np.float32, 0.0),
    (6, 400, 70000, np.float32, 0.0)])
def test_build_matches_oracle(device, seed, n_docs, vocab, dtype, dup):
    print(f"build case seed={seed} n_docs={n_docs} vocab={vocab} dtype={dtype.__name__}", flush=True)
    csr = random_csr(np.random.default_rng(seed), n_docs, vocab, dtype=dtype, dup_rate=dup)
    ix = gs.build_from_csr(csr, device)
    assert_index_equal(ix, oracle_index(csr))


@pytest.mark.parametrize("seed,n_docs,vocab,dtype,dup", [
    (0, 500, 300, np.float32, 0.0), (1, 2000, 9, np.float32, 0.2), (3, 1000, 700, np.float16, 0.05),
    (4, 700, 250, np.uint8, 0.0), (5, 1, 3, np.float32, 0.0), (6, 400, 70000, np.float16, 0.1)])
def test_forward_index_matches_oracle(device, seed, n_docs, vocab, dtype, dup):
    from gpusparse.index import build_forward
    print(f"forward case seed={seed} n_docs={n_docs} vocab={vocab} dtype={dtype.__name__}", flush=True)
    csr = random_csr(np.random.default_rng(seed), n_docs, vocab, dtype=dtype, dup_rate=dup)
    ix = gs.build_from_csr(csr, device)
    row_ptr, terms, w = build_forward(ix)
    want = O.forward_index(oracle_index(csr))
    nnz = int(want[0][-1])
    assert np.array_equal(row_ptr.cpu().numpy(), want[0])
    assert np.array_equal(terms.cpu().numpy()[:nnz], want[1])
    assert w.cpu().numpy()[:nnz].tobytes() == want[2].tobytes()


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_forward_copy_taken_from_sorted_csr(device, dtype):
    """A CSR whose rows are sorted by term (a repeated term's entries in CSR order)
    is kept as the doc-major copy at build time; it equals the copy gs_forward_fill
    builds from the index and the oracle's.  Unsorted rows leave the copy to the
    first search."""
    from gpusparse.index import build_forward
    rng = np.random.default_rng(21)
    csr = random_csr(rng, 3000, 400, dtype=dtype, dup_rate=0.1)
    idx, dat = csr.indices.copy(), csr.data.copy()
    for r in range(csr.shape[0]):
        a, b = csr.indptr[r], csr.indptr[r + 1]
        o = np.argsort(idx[a:b], kind="stable")
        idx[a:b], dat[a:b] = idx[a:b][o], dat[a:b][o]
    srt = CSR(csr.indptr, idx, dat, csr.shape)
    ix = gs.build_from_csr(srt, device)
    fwd = ix.aux().get("fwd")
    assert fwd is not None
    built = build_forward(ix)
    want = O.forward_index(oracle_index(srt))
    nnz = int(want[0][-1])
    assert np.array_equal(fwd[0].cpu().numpy(), want[0]) and np.array_equal(built[0].cpu().numpy(), want[0])
    for got, b, w in ((fwd[1], built[1], want[1]), (fwd[2], built[2], want[2])):
        assert got.cpu().numpy()[:nnz].tobytes() == w.tobytes() == b.cpu().numpy()[:nnz].tobytes()
    ti, tw = random_queries(rng, 16, 400, max_len=12)
    assert_search_equal(ix, oracle_index(srt), ti, tw, 50, path="fused")
    unsorted = gs.build_from_csr(csr, device)
    assert "fwd" not in unsorted.aux()


@pytest.mark.parametrize("seed,dtype,tile_log2,vocab", [(0, np.float32, 12, 300), (1, np.float16, 13, 300),
                                                       (2, np.uint8, 8, 300), (3, np.float16, 10, 300),
                                                       (4, np.float32, 14, 300), (5, np.float16, 13, 9),
                                                       (6, np.uint8, 12, 20), (7, np.float32, 6, 3)])
def test_packed_copy_matches_oracle(device, seed, dtype, tile_log2, vocab):
    """Bit for bit, including the bank-aware order inside (term, tile) sub-ranges
    of more than 64 postings (vocab 9 / 20 / 3: sub-ranges of up to a whole tile,
    with repeated doc ids)."""
    from gpusparse.index import build_packed
    print(f"packed copy seed={seed} {dtype.__name__} tile_log2={tile_log2} vocab={vocab}", flush=True)
    csr = random_csr(np.random.default_rng(seed), 20000, vocab, dtype=dtype, dup_rate=0.05)
    if dtype != np.uint8:  # signed weights and ties at half units of the scale
        csr.data[::5] *= -1
        csr.data[3::13] = ((np.arange(len(csr.data[3::13])) % 7) + 0.5).astype(dtype) / 2
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    pk = build_packed(ix, tile_log2)
    want_shift = 0 if dtype == np.uint8 else O.pack_shift(float(np.abs(csr.data.astype(np.float64)).max()))
    assert pk.shift == want_shift
    assert np.array_equal(pk.words.cpu().numpy(), O.pack_postings(ref, tile_log2))


@pytest.mark.parametrize("tile_log2", [12, 14])
def test_packed_copy_block_boundaries(device, tile_log2):
    """Bit for bit against the oracle, with (term, tile) sub-ranges sized around
    the 1024-posting blocks of the bank-aware order: tails of 1, 63, 64 and 65
    postings after whole blocks, single blocks just above 64 postings, and
    sub-ranges filling a whole tile (docs at random, one term per size, two
    tiles)."""
    from gpusparse.index import build_packed
    T = 1 << tile_log2
    sizes = [65, 127, 1024, 1025, 1087, 1088, 1089, 2047, 2113, T - 1, T]
    print(f"packed copy block boundaries tile_log2={tile_log2} sizes={sizes}", flush=True)
    rng = np.random.default_rng(tile_log2)
    rows, cols = [], []
    for t, n in enumerate(sizes):
        for j, m in enumerate((n, sizes[-1 - t])):  # tile 0 gets n postings, tile 1 another size
            d = j * T + rng.choice(T, size=m, replace=False)
            rows.append(d)
            cols.append(np.full(m, t))
    import scipy.sparse as sp
    r, c = np.concatenate(rows), np.concatenate(cols)
    w = rng.lognormal(-0.5, 0.8, size=len(r)).astype(np.float32)
    m = sp.csr_matrix((w, (r, c)), shape=(2 * T, len(sizes)))
    m.sort_indices()
    csr = CSR(m.indptr.astype(np.int64), m.indices.astype(np.int32), m.data.astype(np.float16), m.shape)
    ix = gs.build_from_csr(csr, device)
    pk = build_packed(ix, tile_log2)
    assert np.array_equal(pk.words.cpu().numpy(), O.pack_postings(oracle_index(csr), tile_log2))


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.uint8])
def test_search_without_packed_copy(device, dtype):
    """The scorer reads the index arrays when the packed copy is absent (no room
    for it, a non-finite weight, or another tile size) and gives the same,
    oracle, answer."""
    from gpusparse.index import default_tile_log2, ensure_search_state
    rng = np.random.default_rng(5)
    csr = random_csr(rng, 30000, 60, max_len=12, dtype=dtype, dup_rate=0.02)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = random_queries(rng, 24, 60, max_len=9, dtype=np.uint8 if dtype == np.uint8 else np.float32)
    print(f"packed vs plain scorer {dtype.__name__}", flush=True)
    assert_search_equal(ix, ref, ti, tw, 300, path="fused", hybrid=False)
    tl = default_tile_log2(ix)
    a = ensure_search_state(ix, tl)
    assert a[("packed", tl)] is not None
    a[("packed", tl)] = None
    assert_search_equal(ix, ref, ti, tw, 300, path="fused", hybrid=False)
    assert_search_equal(ix, ref, ti, tw, 300, path="fused", unroll=8, hybrid=False)


def test_rescoring_without_forward_copy(c1):
    """The rescoring that searches the term lists (used when the doc-major copy is
    absent) gives the same answer."""
    ix, ref, ti, tw = c1
    a = ix.aux()
    saved = a.get("fwd")
    a["fwd"] = None
    try:
        assert_search_equal(ix, ref, ti[:32], tw[:32], 100, path="fused")
    finally:
        a["fwd"] = saved


def test_search_with_packed_copy_in_slot_order(c1):
    """A packed copy left in slot order (gs_pack_postings without tile bounds)
    scores the same as the bank-aware one: the order inside a (term, tile)
    sub-range does not change the integer sums."""
    from gpusparse.index import build_packed, default_tile_log2, ensure_search_state
    ix, ref, ti, tw = c1
    tl = default_tile_log2(ix)
    a = ensure_search_state(ix, tl)
    saved = a[("packed", tl)]
    a[("packed", tl)] = build_packed(ix, tl, arrange=False)
    try:
        assert not torch.equal(a[("packed", tl)].words, saved.words)
        assert torch.equal(torch.sort(a[("packed", tl)].words).values, torch.sort(saved.words).values)
        assert_search_equal(ix, ref, ti[:64], tw[:64], 100, path="fused", hybrid=False)
    finally:
        a[("packed", tl)] = saved


def test_search_counts_cover_the_answers(c1):
    """gs_search_counts after a search: per scoring slot, the candidates emitted
    and the candidates rescored in fp64.  Slots hold the queries in group order,
    so the checks hold for every slot: each query's positive answers were all
    emitted (at least min(k, positives) candidates) and rescored, and the rescored
    set lies inside the candidates."""
    ix, ref, ti, tw = c1
    k, B = 100, 64
    timing = {}
    s, i = gs.search(ix, (torch.from_numpy(ti[:B]), torch.from_numpy(tw[:B])), k, timing=timing, path="fused")
    assert timing["dense_rows"] == 0  # a row finished by the dense path reports 0 rescored
    cand, resc = gs.search_counts(ix, B, ti.shape[1], k)
    pos = (s.cpu().numpy() > 0).sum(axis=1)
    assert cand.shape == (B,) and resc.shape == (B,)
    assert np.all(np.sort(cand) >= np.sort(pos))
    assert np.all(np.sort(resc) >= np.sort(pos))
    assert np.all(resc <= cand)
    with pytest.raises(ValueError):
        gs.search_counts(gs.build_from_csr(random_csr(np.random.default_rng(1), 50, 20), ix.doc_ids.device),
                         B, ti.shape[1], k)


def test_timing_dict_events(c1):
    """Searches timed with a pre-built `timing_dict` use its events (one call's
    set each), time every phase and return what an untimed search returns."""
    ix, ref, ti, tw = c1
    q = (torch.from_numpy(ti[:32]), torch.from_numpy(tw[:32]))
    s0, i0 = gs.search(ix, q, 50, path="fused")
    timing = gs.timing_dict(2)
    pool = [ev for pair in timing["event_pool"] for ev in pair[0] + pair[1]]
    for _ in range(2):
        s, i = gs.search(ix, q, 50, path="fused", timing=timing)
        assert torch.equal(s, s0) and torch.equal(i, i0)
    torch.cuda.synchronize()
    assert timing["event_pool"] == [] and len(timing["search"]) == 2 and len(timing["phases"]) == 2
    used = [e for pair in timing["search"] + timing["score_kernel"] for e in pair] + \
        [e for ph in timing["phases"] for e in ph]
    assert {id(e) for e in used} == {id(e) for e in pool}
    for e0, e1 in timing["search"]:
        assert e0.elapsed_time(e1) > 0
    for ph in timing["phases"]:
        assert all(ph[j].elapsed_time(ph[j + 1]) >= 0 for j in range(len(ph) - 1))
    # the pool exhausted, further calls create their own events
    gs.search(ix, q, 50, path="fused", timing=timing)
    assert len(timing["search"]) == 3
    # without phase events: the bracketing ones only
    t2 = gs.timing_dict(1, phases=False)
    s, i = gs.search(ix, q, 50, path="fused", timing=t2)
    torch.cuda.synchronize()
    assert torch.equal(s, s0) and torch.equal(i, i0)
    assert "phases" not in t2 and len(t2["score_kernel"]) == 1
    assert t2["score_kernel"][0][0].elapsed_time(t2["score_kernel"][0][1]) > 0


def test_build_generated_c1(device):
    docs, _ = synth.generate("C1")
    ix = gs.build_from_csr(docs, device)
    assert_index_equal(ix, oracle_index(docs))


def test_build_harness_vocab_and_range_check(device):
    csr = random_csr(np.random.default_rng(8), 300, 500)
    ix = gs.build_gpu_index_from_csr(csr, device)
    assert ix.vocab_size == 30522
    assert_index_equal(ix, oracle_index(csr, vocab=30522))
    big = CSR(csr.indptr, csr.indices + 30100, csr.data, (300, 31000))
    with pytest.raises(IndexError):
        gs.build_gpu_index_from_csr(big, device)


def test_build_from_lists_and_torch_sparse(device):
    rng = np.random.default_rng(9)
    csr = random_csr(rng, 200, 60, dup_rate=0.1)
    terms = [csr.indices[csr.indptr[d]:csr.indptr[d + 1]].tolist() for d in range(200)]
    ws = [csr.data[csr.indptr[d]:csr.indptr[d + 1]].tolist() for d in range(200)]
    ix = gs.build_gpu_inverted_index(terms, ws, 60, device)
    assert_index_equal(ix, oracle_index(csr))
    # torch sparse COO: duplicates coalesce (summed) and zeros drop, as the dense
    # round trip of gpu_inverted_index.py:121-132 does
    canon = random_csr(rng, 150, 40, sort_rows=True)
    rows = np.repeat(np.arange(150), np.diff(canon.indptr))
    coo = torch.sparse_coo_tensor(np.stack([rows, canon.indices]), canon.data, (150, 40))
    ix2 = gs.build_gpu_inverted_index_from_sparse(coo, device)
    assert_index_equal(ix2, oracle_index(canon))
    ix3 = gs.build_gpu_inverted_index_from_sparse(coo.to_dense(), device)
    assert_index_equal(ix3, oracle_index(canon))


def test_chunk_bounds_and_ascending_check(device):
    csr = random_csr(np.random.default_rng(10), 3000, 120, dup_rate=0.02)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    for chunk in (1, 100, 1024, 2999, 5000):
        b = gs.build_chunk_boundaries(ix, chunk).cpu().numpy()
        assert np.array_equal(b, O.chunk_bounds(ref["doc_ids"], ref["offsets"], ref["lengths"], 120, 3000, chunk))
    # a plug-in style index (built through __new__, no cached checks) with one list
    # made non-ascending must be rejected with the reference's message
    bad = GPUInvertedIndex.__new__(GPUInvertedIndex)
    doc = ix.doc_ids.clone()
    t = int(torch.argmax(ix.lengths).item())
    o = int(ix.offsets[t].item())
    doc[o], doc[o + 1] = ix.doc_ids[o + 1], ix.doc_ids[o]
    bad.doc_ids, bad.scores, bad.offsets, bad.lengths = doc, ix.scores, ix.offsets, ix.lengths
    bad.num_docs, bad.vocab_size, bad.device = ix.num_docs, ix.vocab_size, ix.device
    n_nonempty = int((ref["lengths"] > 0).sum())
    with pytest.raises(ValueError, match=f"1 of {n_nonempty} posting lists are not ascending"):
        gs.build_chunk_boundaries(bad, 1000)
    with pytest.raises(ValueError):
        gs.search(bad, (torch.zeros((1, 1), dtype=torch.int32), torch.ones((1, 1))), 5)


# ------------------------------------------------------------------ search


@pytest.fixture(scope="module")
def c1(device):
    docs, queries = synth.generate("C1")
    ix = gs.build_from_csr(docs, device)
    ti, tw, _ = O.to_query_tensors(queries.indptr, queries.indices, queries.data)
    return ix, oracle_index(docs), ti, tw


@pytest.mark.parametrize("path,hybrid", [("fused", True), ("fused", False), ("dense", None)])
@pytest.mark.parametrize("k", [10, 1000])
def test_search_c1(c1, path, hybrid, k):
    """The whole C1 batch: the hybrid scorer, the LDS-add scorer for every term,
    and the dense path."""
    ix, ref, ti, tw = c1
    print(f"search C1 path={path} hybrid={hybrid} k={k}", flush=True)
    if path == "fused":
        assert gs.search_plan(ix, len(ti), ti.shape[1], k, hybrid=hybrid)["hybrid"] == hybrid
    assert_search_equal(ix, ref, ti, tw, k, path=path, hybrid=hybrid)


@pytest.mark.parametrize("tile_log2", [8, 10, 13, 14])
def test_search_c1_tile_sizes(c1, tile_log2):
    ix, ref, ti, tw = c1
    print(f"search C1 tile_log2={tile_log2}", flush=True)
    assert_search_equal(ix, ref, ti[:64], tw[:64], 100, path="fused", tile_log2=tile_log2)


@pytest.mark.parametrize("hybrid", [True, False])
@pytest.mark.parametrize("unroll,waves,tiles_per_wg", [(1, 0, 1), (2, 4, 3), (16, 2, 64), (8, 0, 5)])
def test_search_c1_launch_shapes(c1, unroll, waves, tiles_per_wg, hybrid):
    ix, ref, ti, tw = c1
    print(f"C1 unroll={unroll} waves={waves} tiles_per_wg={tiles_per_wg} hybrid={hybrid}", flush=True)
    assert_search_equal(ix, ref, ti[:32], tw[:32], 50, path="fused", unroll=unroll, waves=waves,
                        tiles_per_wg=tiles_per_wg, hybrid=hybrid)


def test_search_dense_fallback_rows(c1):
    """A candidate cap far below what the rows emit sends them to the dense path;
    the answer must not change (the reference's overflow rule, fused_topk.py:96-102)."""
    ix, ref, ti, tw = c1
    timing = {}
    s, i = gs.search(ix, (torch.from_numpy(ti[:40]), torch.from_numpy(tw[:40])), 200, path="fused",
                     cand_cap=400, timing=timing)
    assert timing["dense_rows"] > 0
    vs, _, vi = O.c_search(ref, ti[:40], tw[:40], 200, threads=8)
    assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)


def test_search_async_batches_in_flight(c1):
    """Batches queued with search_async before any result is read, on one stream
    and round-robin over two and three streams, every other one with a candidate
    cap that sends rows to the dense path (finished at result()): each returns
    what the oracle returns for it."""
    ix, ref, ti, tw = c1
    dev = ix.doc_ids.device
    batches = [(0, 40), (40, 96), (96, 100), (100, 164)]
    want = {}
    for b0, b1 in batches:
        vs, _, vi = O.c_search(ref, ti[b0:b1], tw[b0:b1], 200, threads=8)
        want[(b0, b1)] = (vs, vi)
    qt, qw = torch.from_numpy(ti).to(dev), torch.from_numpy(tw).to(dev)
    for n_streams in (1, 2, 3):
        print(f"search_async streams={n_streams}", flush=True)
        streams = [torch.cuda.current_stream(dev)] + [torch.cuda.Stream(dev) for _ in range(n_streams - 1)]
        for st in streams[1:]:
            st.wait_stream(streams[0])
        pend = []
        for j, key in enumerate(batches * 2):
            b0, b1 = key
            timing = {}
            with torch.cuda.stream(streams[j % n_streams]):
                p = gs.search_async(ix, (qt[b0:b1], qw[b0:b1]), 200, path="fused", cand_cap=400 if j % 2 else 0,
                                    timing=timing)
            pend.append((key, timing, p))
        n_dense = 0
        for key, timing, p in pend:
            s, i = p.result()
            n_dense += timing["dense_rows"]
            vs, vi = want[key]
            assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs), (n_streams, key)
        assert n_dense > 0
        torch.cuda.synchronize(dev)


@pytest.mark.parametrize("streams", [1, 3])
def test_retrieve_streams(device, streams):
    """retrieve's batches in flight on `streams` streams: the reference's rankings
    (checked against the oracle's), for the plain and the chunked entry point."""
    rng = np.random.default_rng(43)
    csr = random_csr(rng, 2500, 300, max_len=16, sort_rows=True)
    ti, tw = random_queries(rng, 23, 300, max_len=8)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    vs, _, vi = O.c_search(ref, ti, tw, 15, threads=4)
    q_ids = [f"Q{q}" for q in range(23)]
    doc_ids = [f"D{d}" for d in range(2500)]
    want = O.rankings(q_ids, vs, vi, doc_ids, 15)
    qt, qw = torch.from_numpy(ti).to(device), torch.from_numpy(tw).to(device)
    for doc_chunk in (131072, 1000):
        print(f"retrieve streams={streams} doc_chunk={doc_chunk}", flush=True)
        got = gs.retrieve(ix, q_ids, qt, qw, doc_ids, 15, batch_size=5, doc_chunk=doc_chunk, streams=streams)
        assert got == want


def test_search_small_sample_and_single_tile(c1):
    ix, ref, ti, tw = c1
    assert_search_equal(ix, ref, ti[:16], tw[:16], 30, path="fused", sample_tiles=1)


@pytest.mark.parametrize("n_docs,tile_log2", [(3000, 12), (700, 8), (9000, 12), (9000, 13), (20000, 13)])
def test_search_few_tiles_with_dirty_workspace(device, n_docs, tile_log2):
    """Collections of 1-3 tiles (all of them in the tau = 0 seed launch) give the
    oracle's answer whatever the workspace held before the call."""
    rng = np.random.default_rng(n_docs)
    csr = random_csr(rng, n_docs, 90, dup_rate=0.05)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = random_queries(rng, 20, 90, max_len=8)
    assert_search_equal(ix, ref, ti, tw, 7, path="fused", tile_log2=tile_log2)
    ix.aux()["workspace"].fill_(0xAB)
    print(f"few tiles n_docs={n_docs} tile_log2={tile_log2}, dirty workspace", flush=True)
    for k in (7, min(300, n_docs)):
        assert_search_equal(ix, ref, ti, tw, k, path="fused", tile_log2=tile_log2)


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.uint8])
def test_search_edge_cases(device, dtype):
    """Empty queries, invalid term ids, duplicate list entries, k = N (zero-score
    documents fill the list by ascending id) and k > N (clamped)."""
    rng = np.random.default_rng(21)
    csr = random_csr(rng, 700, 50, dtype=dtype, dup_rate=0.05, empty_rate=0.3, max_len=4)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    qdt = np.uint8 if dtype == np.uint8 else np.float32
    ti, tw = random_queries(rng, 12, 50, dtype=qdt, invalid_rate=0.3, max_len=5)
    ti[0, :] = -1
    for k in (1, 17, 700):
        for path in ("fused", "dense"):
            print(f"edge dtype={dtype.__name__} k={k} path={path}", flush=True)
            assert_search_equal(ix, ref, ti, tw, k, path=path, tile_log2=8)
    s, i = gs.search(ix, (torch.from_numpy(ti), torch.from_numpy(tw)), 10_000, tile_log2=8)
    assert s.shape == (12, 700)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_rescoring_stops_at_last_valid_term(device, dtype):
    """Padded query rows whose valid terms start past the first 64 columns or sit
    only in the last column: the fp64 rescoring reads each row up to its last
    valid term (in query order) and returns the oracle's scores bit for bit."""
    rng = np.random.default_rng(33)
    csr = random_csr(rng, 20000, 300, max_len=20, dtype=dtype)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    B, T = 24, 150
    ti = np.full((B, T), -1, np.int32)
    tw = np.zeros((B, T), np.float32)
    for q in range(B):
        cols = {0: [T - 1], 1: [70, 149], 2: [64, 65, 127, 128]}.get(q % 6, sorted(rng.choice(np.arange(64, T), 12,
                                                                                           replace=False)))
        ti[q, cols] = rng.choice(300, len(cols), replace=False)
        tw[q, cols] = rng.uniform(0.1, 3.0, len(cols)).astype(np.float32)
        if q % 6 == 4:
            ti[q, rng.choice(cols, 2, replace=False)] = 300 + q  # invalid ids among the valid ones
    assert_search_equal(ix, ref, ti, tw, 120, path="fused")


@pytest.mark.parametrize("hybrid", [True, False])
def test_search_f16_config_reduced(device, hybrid):
    cfg = synth.scaled(synth.CONFIGS["C3"], n_docs=300_000, n_queries=64)
    docs, queries = synth.generate(cfg)
    ix = gs.build_from_csr(docs, device)
    assert ix.scores.dtype == torch.float16
    ref = oracle_index(docs)
    ti, tw, _ = O.to_query_tensors(queries.indptr, queries.indices, queries.data)
    for k in (10, 1000):
        print(f"C3 reduced k={k} hybrid={hybrid}", flush=True)
        assert_search_equal(ix, ref, ti, tw, k, path="fused", hybrid=hybrid)


@pytest.fixture(scope="module")
def c3_small(device):
    cfg = synth.scaled(synth.CONFIGS["C3"], n_docs=120_000, n_queries=24)
    docs, queries = synth.generate(cfg)
    ix = gs.build_from_csr(docs, device)
    ti, tw, _ = O.to_query_tensors(queries.indptr, queries.indices, queries.data)
    return ix, oracle_index(docs), ti, tw


@pytest.mark.parametrize("unroll,tile_log2,tiles_per_wg", [(1, 12, 1), (2, 10, 3), (4, 13, 2), (8, 12, 2),
                                                           (16, 12, 1), (16, 9, 4), (16, 13, 0)])
def test_search_packed_launch_shapes(c3_small, unroll, tile_log2, tiles_per_wg):
    """fp16 postings read from the packed scoring copy, for every chunk length and
    several tile sizes and tiles per workgroup."""
    from gpusparse.index import ensure_search_state
    ix, ref, ti, tw = c3_small
    print(f"packed unroll={unroll} tile_log2={tile_log2} tiles_per_wg={tiles_per_wg}", flush=True)
    assert_search_equal(ix, ref, ti, tw, 100, path="fused", unroll=unroll, tile_log2=tile_log2,
                        tiles_per_wg=tiles_per_wg)
    assert ensure_search_state(ix, tile_log2)[("packed", tile_log2)] is not None


def test_search_plan_reports_defaults(c1, c3_small):
    """The plan of the fused search: the packed copy, 16 postings per lane per
    chunk, 64 KiB of LDS slices: 8192-doc tiles and 2 queries per group for the
    LDS-only search, 16384-doc tiles and one query for the hybrid one (heavy terms
    as matrix products)."""
    ix32, _, ti, _ = c1
    h = gs.search_plan(ix32, 32, ti.shape[1], 100, hybrid=True)
    assert h["hybrid"] and h["tile_log2"] == 14 and h["packed"] and h["group_size"] == 1
    assert gs.search_plan(ix32, 32, ti.shape[1], 100)["hybrid"] == HYBRID_DEFAULT
    p32 = gs.search_plan(ix32, 32, ti.shape[1], 100, hybrid=False)
    assert not p32["hybrid"]
    assert p32["tile_log2"] == 13 and p32["packed"] and p32["unroll"] == 16 and p32["group_size"] == 2
    assert p32["seed_tiles"] >= 1 and p32["tiles_per_wg"] in (1, 2, 3)
    p12 = gs.search_plan(ix32, 32, ti.shape[1], 100, tile_log2=12)
    assert p12["group_size"] == 4 and p12["hybrid"] == HYBRID_DEFAULT
    ix16, _, ti16, _ = c3_small
    p16 = gs.search_plan(ix16, 24, ti16.shape[1], 1000, hybrid=False)
    assert p16["tile_log2"] == 13 and p16["packed"] and p16["unroll"] == 16 and p16["group_size"] == 2
    assert gs.search_plan(ix16, 24, ti16.shape[1], 1000, sample_tiles=3, unroll=4)["seed_tiles"] == 3


@pytest.mark.parametrize("vocab,seed", [(20, 0), (65, 1), (129, 4), (200, 5), (3000, 2), (30522, 3)])
def test_heavy_terms_matches_oracle(device, vocab, seed):
    from gpusparse.index import heavy_terms
    rng = np.random.default_rng(seed)
    print(f"heavy terms vocab={vocab}", flush=True)
    csr = random_csr(rng, 4000, vocab, max_len=12, dtype=np.float32)
    ix = gs.build_from_csr(csr, device)
    from gpusparse import _lib
    assert np.array_equal(heavy_terms(ix).cpu().numpy(), O.heavy_terms(ix.lengths.cpu().numpy(),
                                                                        _lib.heavy_term_count()))


@pytest.mark.parametrize("B,k", [(24, 1000), (7, 10)])
def test_grouped_queries_equal_batch_order(c3_small, B, k):
    """Scoring groups of queries that share frequent terms (the default) and of
    consecutive queries give the same, oracle, answer."""
    ix, ref, ti, tw = c3_small
    ti, tw = ti[:B], tw[:B]
    print(f"grouped vs batch order B={B} k={k}", flush=True)
    s0, i0 = assert_search_equal(ix, ref, ti, tw, k, path="fused", hybrid=False)
    s1, i1 = assert_search_equal(ix, ref, ti, tw, k, path="fused", batch_order=True, hybrid=False)
    assert np.array_equal(i0, i1) and np.array_equal(s0, s1)


def test_grouped_queries_many_blocks(device):
    """More queries than one ordering block (1024 at G = 2), an odd batch (not a
    multiple of the group size), and queries repeating terms."""
    rng = np.random.default_rng(7)
    csr = random_csr(rng, 6000, 200, max_len=20, dtype=np.float16, dup_rate=0.02)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = random_queries(rng, 1503, 200, max_len=10)
    ti[::11, 1] = ti[::11, 0]
    print("grouped queries, 1503 queries", flush=True)
    assert gs.search_plan(ix, 1503, ti.shape[1], 20, hybrid=False)["group_size"] == 2
    assert_search_equal(ix, ref, ti, tw, 20, path="fused", hybrid=False)


@pytest.mark.parametrize("hybrid", [True, False])
@pytest.mark.parametrize("dtype,pattern", [(np.float32, "fine"), (np.float16, "coarse"), (np.float32, "coarse")])
def test_packed_scores_exact_under_near_ties(device, dtype, pattern, hybrid):
    """The packed copy holds rounded weights, so many docs share one fixed-point
    score while their fp64 scores differ: 'fine' weights 1 + j 2^-20 all round to
    a few values of the 2^-12 grid; 'coarse' puts one weight of 600 in the index,
    so the others (in [0.01, 1)) round to multiples of 1/8.  The margin must send every doc that
    can reach the top k to the fp64 rescoring, and the answer must equal the
    oracle's, ties by doc id included (equal-weight docs are planted too)."""
    rng = np.random.default_rng(11)
    n_docs, vocab = 6000, 8
    rows = []
    for d in range(n_docs):
        terms = np.sort(rng.choice(6, size=rng.integers(2, 6), replace=False))
        if pattern == "fine":
            w = 1.0 + rng.integers(0, 2000, size=len(terms)) * 2.0 ** -20
        else:
            w = rng.uniform(0.01, 1.0, size=len(terms))
            if dtype == np.float32:
                w *= np.where(rng.random(len(terms)) < 0.2, -1.0, 1.0)
        if d % 97 == 0 and d:  # exact duplicates of an earlier doc: ties broken by doc id
            terms, w = rows[d - 1]
        rows.append((terms, w))
    rows[4321] = (np.array([6, 7]), np.array([600.0, 1.0]) if pattern == "coarse" else np.array([1.5, 1.0]))
    indptr = np.cumsum([0] + [len(t) for t, _ in rows]).astype(np.int64)
    csr = CSR(indptr, np.concatenate([t for t, _ in rows]).astype(np.int32),
              np.concatenate([w for _, w in rows]).astype(dtype), (n_docs, vocab))
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti = np.array([[0, 1, 2, 3, 4, 5], [2, 3, 5, -1, -1, -1], [0, 0, 1, 4, -1, -1], [5, 4, 3, 2, 1, 0]], np.int32)
    tw = np.array([[0.7, 1.3, 0.9, 2.1, 0.4, 1.0], [1.0, 1.0, 1.0, 0, 0, 0], [0.5, 0.25, 3.0, 1.0, 0, 0],
                   [1e-3, 2.0, 0.3, 0.3, 7.0, 0.11]], np.float32)
    print(f"near ties {dtype.__name__} {pattern} hybrid={hybrid}", flush=True)
    plan = gs.search_plan(ix, 4, ti.shape[1], 200, hybrid=hybrid)
    assert plan["packed"] and plan["hybrid"] == hybrid
    for k in (1, 50, 200):
        assert_search_equal(ix, ref, ti, tw, k, path="fused", hybrid=hybrid)


@pytest.mark.parametrize("hybrid", [None, True, False])
def test_search_u8_config_reduced(device, hybrid):
    """uint8 impacts: exact uint32 sums (int32 scores), by the hybrid search on
    the index's float16 copy (the default) or by LDS adds of every term."""
    cfg = synth.scaled(synth.CONFIGS["C5"], n_docs=300_000, n_queries=64)
    docs, queries = synth.generate(cfg)
    ix = gs.build_from_csr(docs, device)
    assert ix.scores.dtype == torch.uint8
    ref = oracle_index(docs)
    assert_index_equal(ix, ref)
    ti, tw, _ = O.to_query_tensors(queries.indptr, queries.indices, queries.data)
    assert tw.dtype == np.uint8
    want = HYBRID_DEFAULT if hybrid is None else hybrid
    assert gs.search_plan(ix, len(ti), ti.shape[1], 1000, hybrid=hybrid)["hybrid"] == want
    s, _ = assert_search_equal(ix, ref, ti, tw, 1000, path="fused", hybrid=hybrid)
    assert s.dtype == np.int32


@pytest.mark.parametrize("tile_log2", [10, 12, 13])
def test_search_queries_repeating_terms(device, tile_log2):
    """Queries that repeat a term: every occurrence adds its own product, as in
    the reference's scatter-add, so a term can have more (slot, weight) entries
    than its query group has queries (groups of 16, 4 and 2 queries here)."""
    rng = np.random.default_rng(31)
    csr = random_csr(rng, 30000, 40, max_len=12)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = random_queries(rng, 24, 40, max_len=6)
    # column 0 three times, columns 1 and 2 twice, with other weights
    ti = np.ascontiguousarray(np.concatenate([ti, ti[:, :3], ti[:, :1]], axis=1))
    tw = np.ascontiguousarray(np.concatenate([tw, tw[:, :3] * 0.5, tw[:, :1] * 2.0], axis=1).astype(np.float32))
    print(f"repeated query terms tile_log2={tile_log2} T={ti.shape[1]}", flush=True)
    for k in (10, 300):
        assert_search_equal(ix, ref, ti, tw, k, path="fused", tile_log2=tile_log2)


@pytest.mark.parametrize("packed", [True, False])
@pytest.mark.parametrize("unroll", [1, 4, 16])
def test_search_terms_held_by_more_than_64_slots(device, packed, unroll):
    """256-doc tiles put 32 queries in a group; every query holds one term three
    times, so that term has more than 64 (slot, weight) entries in each group (the
    scorer's per-entry loop for such terms).  Lists repeat docs, so with one
    posting per lane a chunk can be full; otherwise chunks end inside the tile."""
    from gpusparse.index import ensure_search_state
    rng = np.random.default_rng(47)
    csr = random_csr(rng, 20000, 30, max_len=10, dup_rate=0.05)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = random_queries(rng, 40, 30, max_len=5)
    ti = np.ascontiguousarray(np.concatenate([ti, np.full((40, 3), 3, np.int32)], axis=1))
    tw = np.ascontiguousarray(np.concatenate([tw, np.tile(np.float32([0.5, 1.25, 2.0]), (40, 1))], axis=1))
    a = ensure_search_state(ix, 8)
    if not packed:
        a[("packed", 8)] = None
    plan = gs.search_plan(ix, 40, ti.shape[1], 200, tile_log2=8, unroll=unroll)
    assert plan["group_size"] == 32 and plan["packed"] == packed
    print(f"term in >64 slots packed={packed} unroll={unroll}", flush=True)
    for k in (10, 200):
        assert_search_equal(ix, ref, ti, tw, k, path="fused", tile_log2=8, unroll=unroll)


@pytest.mark.parametrize("tile_log2,tiles_per_wg", [(8, 0), (10, 0), (12, 0), (13, 0), (10, 4), (13, 2)])
def test_search_head_heavy_reduced(device, tile_log2, tiles_per_wg):
    """Wide head-heavy queries: group unions above one LDS batch of terms."""
    cfg = synth.scaled(synth.CONFIGS["C4"], n_docs=200_000, n_queries=32)
    docs, queries = synth.generate(cfg)
    ix = gs.build_from_csr(docs, device)
    ref = oracle_index(docs)
    ti, tw, _ = O.to_query_tensors(queries.indptr, queries.indices, queries.data)
    print(f"C4 reduced tile_log2={tile_log2} tiles_per_wg={tiles_per_wg} T={ti.shape[1]}", flush=True)
    assert_search_equal(ix, ref, ti, tw, 1000, path="fused", tile_log2=tile_log2, tiles_per_wg=tiles_per_wg)


# ------------------------------------------------------------------ selection and scatter


def test_compacted_topk_matches_oracle(device):
    rng = np.random.default_rng(31)
    s = rng.normal(size=(9, 5000)).astype(np.float32)
    s[3, :] = 1.0                               # one row of ties
    tau = np.array([0.5, 2.0, -np.inf, 1.0, 3.5, 0.0, 1.2, 9.0, -1.0], np.float32)
    st = torch.from_numpy(s).to(device)
    for k, max_cand in ((10, 8192), (300, 8192), (300, 300), (1000, 1000)):
        v, i = gs.compacted_topk(st, torch.from_numpy(tau).to(device), k, max_cand=max_cand)
        ov, oi = O.compacted_topk(s, tau, k)
        assert np.array_equal(i.cpu().numpy(), oi) and np.array_equal(v.cpu().numpy(), ov)
    v, i = gs.topk_rows(st[:, :4000], 77)
    ov, oi = O.compacted_topk(s[:, :4000], None, 77)
    assert np.array_equal(i.cpu().numpy(), oi) and np.array_equal(v.cpu().numpy(), ov)
    # a strided [B, chunk] view, as the reference's final short chunk (triton_kernel_chunked.py:147-151)
    v, i = gs.compacted_topk(st[:, :1234], torch.from_numpy(tau).to(device), 50)
    ov, oi = O.compacted_topk(s[:, :1234], tau, 50)
    assert np.array_equal(i.cpu().numpy(), oi) and np.array_equal(v.cpu().numpy(), ov)


@pytest.mark.parametrize("dtype", [np.float32, np.uint8])
def test_scatter_add_matches_oracle(device, dtype):
    rng = np.random.default_rng(32)
    csr = random_csr(rng, 4000, 200, dtype=dtype)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    qdt = np.uint8 if dtype == np.uint8 else np.float32
    ti, tw = random_queries(rng, 10, 200, dtype=qdt, invalid_rate=0.1)
    odt = torch.int32 if dtype == np.uint8 else torch.float32
    out = torch.zeros((10, 4000), dtype=odt, device=device)
    gs.scatter_add(ix, torch.from_numpy(ti), torch.from_numpy(tw), out, block_pl=512)
    if dtype == np.uint8:
        assert np.array_equal(out.cpu().numpy().astype(np.uint32), O.scores_u32(ref, ti, tw))
    else:
        np.testing.assert_allclose(out.cpu().numpy(), O.scores_f64(ref, ti, tw), rtol=2e-6, atol=1e-6)
    # one chunk through per-term bounds (the chunked kernel)
    b = gs.build_chunk_boundaries(ix, 1500)
    out2 = torch.zeros((10, 1500), dtype=odt, device=device)
    gs.scatter_add(ix, torch.from_numpy(ti), torch.from_numpy(tw), out2, lo=b[1], hi=b[2], chunk_start=1500,
                   chunk_len=1500)
    assert np.array_equal(out2.cpu().numpy(), out.cpu().numpy()[:, 1500:3000]) or dtype != np.uint8
    if dtype != np.uint8:
        np.testing.assert_allclose(out2.cpu().numpy(), out.cpu().numpy()[:, 1500:3000], rtol=2e-6, atol=1e-6)


def test_atomic_path_agrees(c1):
    ix, ref, ti, tw = c1
    s, i = gs.atomic_fused_score(ix, torch.from_numpy(ti[:32]), torch.from_numpy(tw[:32]), 10)
    vs, s64, vi = O.c_search(ref, ti[:32], tw[:32], 10, threads=8)
    assert np.max(np.abs(s.cpu().numpy() - s64)) <= 1e-5


# ------------------------------------------------------------------ drop-in surface


def test_reference_entry_points(c1):
    ix, ref, ti, tw = c1
    qt, qw = torch.from_numpy(ti[:50]).to(ix.device), torch.from_numpy(tw[:50]).to(ix.device)
    vs, _, vi = O.c_search(ref, ti[:50], tw[:50], 100, threads=8)
    for fn in (lambda: gs.triton_fused_score(ix, qt, qw, top_k=100),
               lambda: gs.triton_fused_score(ix, qt, qw, top_k=100, block_pl=512),
               lambda: gs.triton_chunked_score(ix, qt, qw, top_k=100, doc_chunk=30000),
               lambda: gs.triton_chunked_score_fused(ix, qt, qw, top_k=100, doc_chunk=30000,
                                                     chunk_bounds=gs.build_chunk_boundaries(ix, 30000))):
        s, i = fn()
        assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
    with pytest.raises(AssertionError, match="power of 2"):
        gs.triton_fused_score(ix, qt, qw, block_pl=100)


def test_chunked_entry_points_ignore_bound_contents_and_block_pl(c1):
    """Contract of this build: triton_chunked_score(_fused) check chunk_bounds for
    shape (and the lists for ascending order) but schedule by their own tile
    bounds, so the contents of a well-shaped table do not change the answer;
    block_pl is validated (power of two) and has no effect."""
    ix, ref, ti, tw = c1
    qt, qw = torch.from_numpy(ti[:24]).cuda(), torch.from_numpy(tw[:24]).cuda()
    vs, _, vi = O.c_search(ref, ti[:24], tw[:24], 50, threads=8)
    good = gs.build_chunk_boundaries(ix, 30000)
    junk = torch.zeros_like(good)
    for bounds in (good, junk):
        for block_pl in (32, 128, 1024):
            for fn in (gs.triton_chunked_score, gs.triton_chunked_score_fused):
                s, i = fn(ix, qt, qw, top_k=50, doc_chunk=30000, block_pl=block_pl, chunk_bounds=bounds)
                assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
    with pytest.raises(ValueError, match="shape"):
        gs.triton_chunked_score_fused(ix, qt, qw, top_k=50, doc_chunk=30000, chunk_bounds=good[:-1])


def test_k_above_8192_and_width_limit(c1):
    """k above 8192 (the LDS selection's capacity) is answered by the dense path
    in rounds of 8192 and equals the oracle bit for bit, up to k = num_docs, for
    any path argument; so are queries wider than 8192 terms (repeated terms
    included); compacted_topk raises ValueError above its capacity."""
    ix, ref, ti, tw = c1
    assert gs.MAX_K == 8192
    q = (torch.from_numpy(ti[:3]), torch.from_numpy(tw[:3]))
    for k, path in ((8192, "fused"), (8193, "fused"), (20000, "auto"), (24577, "dense")):
        print(f"large k={k} path={path}", flush=True)
        s, i = gs.search(ix, q, k, path=path)
        vs, _, vi = O.c_search(ref, ti[:3], tw[:3], k, threads=8)
        assert s.shape == (3, k)
        assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
    s, i = gs.triton_fused_score(ix, q[0], q[1], top_k=9000)
    vs, _, vi = O.c_search(ref, ti[:3], tw[:3], 9000, threads=8)
    assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
    assert gs.MAX_T == 8192
    rng = np.random.default_rng(12)
    wt = rng.integers(-1, 4000, size=(2, 9000)).astype(np.int32)  # -1: padding
    ww = rng.random((2, 9000), dtype=np.float32)
    for path in ("fused", "auto"):
        print(f"width 9000 path={path}", flush=True)
        s, i = gs.search(ix, (torch.from_numpy(wt), torch.from_numpy(ww)), 100, path=path)
        vs, _, vi = O.c_search(ref, wt, ww, 100, threads=8)
        assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
    rows = torch.rand((2, 20000), device=ix.doc_ids.device)
    with pytest.raises(ValueError, match="8192"):
        gs.compacted_topk(rows, torch.zeros(2, device=rows.device), 9000, max_cand=9000)


@pytest.mark.parametrize("dtype", [np.float16, np.uint8])
def test_k_up_to_num_docs(device, dtype):
    """k = num_docs and k just above a multiple of 8192 on a small index: every
    doc ranked, zero-score docs by ascending id, bit for bit against the oracle
    (uint8: int32 sums)."""
    rng = np.random.default_rng(9)
    csr = random_csr(rng, 17000, 40, max_len=6, dtype=dtype, empty_rate=0.3)
    ix = gs.build_from_csr(csr, device, weight_dtype=None)
    ref = oracle_index(csr)
    ti, tw = random_queries(rng, 4, 40, max_len=5, dtype=np.uint8 if dtype == np.uint8 else np.float32)
    for k in (16385, 17000):
        print(f"k={k} of 17000 {dtype.__name__}", flush=True)
        assert_search_equal(ix, ref, ti, tw, k)


@pytest.mark.parametrize("width,n_q", [(3000, 6), (8192, 2)])
def test_search_very_wide_queries(c1, width, n_q):
    """Queries of thousands of terms (up to the 8192-term limit, some repeated):
    a group's union then spans many batches of union terms and the group size
    shrinks to fit the LDS sort of its entries; answers equal the oracle's."""
    ix, ref, _, _ = c1
    rng = np.random.default_rng(width)
    V = int(ref["vocab_size"])
    ti = np.stack([rng.choice(V, width, replace=False) for _ in range(n_q)]).astype(np.int32)
    ti[:, -5:] = ti[:, :5]  # repeated terms
    tw = rng.uniform(0.01, 1.0, ti.shape).astype(np.float32)
    print(f"wide queries T={width}", flush=True)
    assert_search_equal(ix, ref, ti, tw, 100, path="fused")


@pytest.mark.parametrize("dtype", [np.float16, np.uint8])
def test_reference_builders_store_float32(device, dtype):
    """build_index / build_gpu_index_from_csr store float32 weights whatever the
    CSR holds, as the reference does (gpusparse_retrieval.py:98), and answer
    float32 queries; weight_dtype opts into the native types."""
    rng = np.random.default_rng(3)
    csr = random_csr(rng, 3000, 200, dtype=dtype, max_len=10)
    ti, tw = random_queries(rng, 16, 200, max_len=6, dtype=np.float32)
    if dtype == np.uint8:
        tw = np.rint(tw * 40).clip(1, 255).astype(np.float32)
    f32 = CSR(csr.indptr, csr.indices, csr.data.astype(np.float32), csr.shape)
    ref = oracle_index(f32)
    for build in (gs.build_index, gs.build_gpu_index_from_csr):
        ix = build(csr, device)
        assert ix.scores.dtype == torch.float32
        assert np.array_equal(ix.scores.cpu().numpy(), ref["scores"])
        s, i = gs.triton_fused_score(ix, torch.from_numpy(ti).cuda(), torch.from_numpy(tw).cuda(), top_k=20)
        vs, _, vi = O.c_search(ref, ti, tw, 20, threads=8)
        assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
    native = gs.build_index(csr, device, weight_dtype=torch.float16 if dtype == np.float16 else torch.uint8)
    assert native.scores.dtype == (torch.float16 if dtype == np.float16 else torch.uint8)
    if dtype == np.uint8:
        # float query weights that are integers in [0, 255] are the uint8 impacts
        nref = oracle_index(csr)
        s, i = gs.search(native, (torch.from_numpy(ti), torch.from_numpy(tw)), 20)
        vs, _, vi = O.c_search(nref, ti, tw.astype(np.uint8), 20, threads=8)
        assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
        with pytest.raises(ValueError, match="integers"):
            gs.search(native, (torch.from_numpy(ti), torch.from_numpy(tw + 0.5)), 20)
        # weights already on the GPU: the same answer, and the same error, which
        # search_async defers to result() (its launches do not wait for the check)
        s2, i2 = gs.search(native, (torch.from_numpy(ti).cuda(), torch.from_numpy(tw).cuda()), 20, path="fused")
        assert np.array_equal(i2.cpu().numpy(), vi) and np.array_equal(s2.cpu().numpy(), vs)
        pend = gs.search_async(native, (torch.from_numpy(ti).cuda(), torch.from_numpy(tw + 0.5).cuda()), 20,
                               path="fused")
        with pytest.raises(ValueError, match="integers"):
            pend.result()
        with pytest.raises(ValueError, match="integers"):
            gs.search(native, (torch.from_numpy(ti).cuda(), torch.from_numpy(tw - 300).cuda()), 20, path="dense")


def test_retrieve_and_run_engine(device, tmp_path):
    rng = np.random.default_rng(41)
    csr = random_csr(rng, 3000, 400, max_len=20, sort_rows=True)
    ti, tw = random_queries(rng, 30, 400, max_len=8)
    docs = [(f"D{d}", csr.indices[csr.indptr[d]:csr.indptr[d + 1]].tolist(),
             csr.data[csr.indptr[d]:csr.indptr[d + 1]].tolist()) for d in range(3000)]
    qs = [(f"Q{q}", [int(t) for t in ti[q] if t >= 0], [float(w) for t, w in zip(ti[q], tw[q]) if t >= 0])
          for q in range(30)]
    res = gs.run_engine(docs, qs, str(tmp_path), 20, doc_chunk=1000, batch_size=7)
    dim = gs.determine_dimension(docs, qs)
    ref = oracle_index(CSR(csr.indptr, csr.indices, csr.data, (3000, dim)))
    q_ids, qcsr = gs.to_csr(qs, dim)
    oti, otw, _ = O.to_query_tensors(qcsr.indptr, qcsr.indices, qcsr.data)
    vs, _, vi = O.c_search(ref, oti, otw, 20, threads=4)
    want = O.rankings(q_ids, vs, vi, [d[0] for d in docs], 20)
    assert res == want
    assert (tmp_path / "run.txt.gz").exists()
