"""GPU parity of the hybrid search: the index's heavy lists (its 64 longest) as
int8 matrix products (MFMA, k_head_scores), whose coarse sums start the LDS slices of the
other terms' adds, against the CPU oracle.

Same bar as the other search tests: ids and scores bit-identical to the oracle
(the fp64 scatter-add rounded to fp32).  The cases aim at what the hybrid adds:
the dense head copy, the query limbs and shift (negative and repeated weights,
limbs that do not fit), the coarse start and its margin, batches that are not a
multiple of 16, blocks past the last doc, vocabularies with fewer terms than
the heavy set, every tile size."""
import numpy as np
import pytest
import torch

import gpusparse as gs
from gpusparse import _lib, synth
from gpusparse.index import CSR, ensure_search_state
from helpers import random_csr, random_queries
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def oracle_index(csr: CSR):
    return O.build_index(csr.indptr, csr.indices, csr.data, csr.shape[0], csr.shape[1])


def check(ix, ref, ti, tw, k, **opts):
    """Hybrid search (asserted to run hybrid) equals the oracle bit for bit."""
    B, T = ti.shape
    opts = dict(opts, hybrid=True)
    assert gs.search_plan(ix, B, T, k, **opts)["hybrid"]
    timing = {}
    s, i = gs.search(ix, (torch.from_numpy(ti), torch.from_numpy(tw)), k, path="fused", timing=timing, **opts)
    vs, s64, vi = O.c_search(ref, ti, tw, min(k, ix.num_docs), threads=8)
    s, i = s.cpu().numpy(), i.cpu().numpy()
    assert np.array_equal(i, vi)
    assert s.dtype == vs.dtype and np.array_equal(s, vs)
    if s.dtype == np.float32:
        # 1e-5, or half an fp32 unit for scores above 2^7 (the scores equal the
        # fp64 sums rounded to fp32, checked above)
        tol = np.maximum(1e-5, np.abs(s64) * 2.0 ** -24)
        assert np.all(np.abs(s.astype(np.float64) - s64) <= tol)
    return timing


def zipf_csr(rng, n_docs, vocab, dtype, max_len=30, s=1.1):
    """Docs whose term ids follow a Zipf law (a few terms in most docs, like the
    synthetic configurations), no repeated (doc, term) pairs."""
    p = 1.0 / np.arange(1, vocab + 1) ** s
    p /= p.sum()
    indptr, idx, val = [0], [], []
    for _ in range(n_docs):
        n = int(rng.integers(1, max_len + 1))
        t = rng.choice(vocab, size=min(n, vocab), replace=False, p=p)
        idx.extend(t.tolist())
        indptr.append(len(idx))
        if dtype == np.uint8:
            val.extend(rng.integers(1, 256, size=len(t)).tolist())
        else:
            val.extend(rng.lognormal(-0.5, 0.8, size=len(t)).tolist())
    return CSR(np.asarray(indptr, np.int64), np.asarray(idx, np.int32), np.asarray(val).astype(dtype),
               (n_docs, vocab))


def zipf_queries(rng, n, vocab, dtype, max_len=25, s=1.1):
    p = 1.0 / np.arange(1, vocab + 1) ** s
    p /= p.sum()
    T = max_len
    ti = np.full((n, T), -1, np.int32)
    tw = np.zeros((n, T), dtype)
    for q in range(n):
        L = int(rng.integers(1, max_len + 1))
        ti[q, :L] = rng.choice(vocab, size=L, replace=False, p=p)
        tw[q, :L] = rng.integers(1, 256, size=L) if dtype == np.uint8 else rng.lognormal(-0.5, 0.8, size=L)
    return ti, tw


# ------------------------------------------------------------------ the dense head copy


@pytest.mark.parametrize("dtype,n_docs", [(np.float32, 5000), (np.float16, 1537), (np.uint8, 700), (np.float16, 1500),
                                         (np.float32, 300)])
def test_head_copy_matches_oracle(device, dtype, n_docs):
    """gs_head_fill against oracle.head_limbs, byte for byte, rows up to the
    last 512-doc block (zero past the docs), and the heavy-rank table.  A
    workgroup takes four 256-doc blocks: 1500 and 300 docs end their rows half
    way through the last workgroup's blocks, 1537 and 700 leave a block without
    docs."""
    from gpusparse.index import build_head
    rng = np.random.default_rng(n_docs)
    csr = zipf_csr(rng, n_docs, 400, dtype)
    if dtype != np.uint8:
        csr.data[::4] *= -1
    ix = gs.build_from_csr(csr, device)
    ensure_search_state(ix)
    head, rank = build_head(ix)
    ref = oracle_index(csr)
    heavy = O.heavy_terms(ref["lengths"], _lib.heavy_term_count())
    n_rows = ((n_docs + 511) // 512) * 512
    assert head.shape == (n_rows, 2, _lib.heavy_term_count()) and len(heavy) == _lib.heavy_term_count()
    assert np.array_equal(head.cpu().numpy(), O.head_limbs(ref, heavy, n_rows))
    want_rank = np.full(400, -1, np.int16)
    want_rank[heavy[heavy >= 0]] = np.arange((heavy >= 0).sum())
    assert np.array_equal(rank.cpu().numpy(), want_rank)


# ------------------------------------------------------------------ search


@pytest.mark.parametrize("cfg,n_docs", [("C1", 100_000), ("C3", 120_000), ("C4", 100_000), ("C2", 60_001)])
@pytest.mark.parametrize("B,k", [(1, 10), (16, 1000), (17, 100), (40, 1000)])
def test_hybrid_synthetic_configs(device, cfg, n_docs, B, k):
    """The float configurations' generators at reduced sizes: batches of 1, 16,
    17 and 40 queries (the products run on blocks of 16 queries, rows past the
    batch zero), k from 10 to 1000."""
    c = synth.scaled(synth.CONFIGS[cfg], n_docs=n_docs, n_queries=B)
    docs, queries = synth.generate(c)
    ix = gs.build_from_csr(docs, device)
    ref = oracle_index(docs)
    ti, tw, _ = O.to_query_tensors(queries.indptr, queries.indices, queries.data)
    print(f"hybrid {cfg} n_docs={n_docs} B={B} k={k}", flush=True)
    check(ix, ref, ti, tw, k)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_hybrid_negative_and_repeated_weights(device, dtype):
    """Negative doc and query weights (negative limbs), heavy terms repeated in
    a query with different weights (their rounded weights summed into one
    limb pair), invalid term ids, an empty query and ties planted by copying docs."""
    rng = np.random.default_rng(3)
    csr = zipf_csr(rng, 20000, 500, dtype)
    csr.data[::3] *= -1
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = zipf_queries(rng, 37, 500, np.float32, max_len=12)
    tw[::2, :4] *= -1
    heavy = O.heavy_terms(ref["lengths"], _lib.heavy_term_count())
    ti = np.ascontiguousarray(np.concatenate([ti, np.tile(heavy[:3], (37, 1)), np.tile(heavy[:2], (37, 1))], axis=1))
    tw = np.ascontiguousarray(np.concatenate([tw, rng.uniform(-1, 2, (37, 5)).astype(np.float32)], axis=1))
    ti[5, :] = -1
    ti[7, 3] = 500 + 7
    ti[8, 2] = -9
    for k in (1, 25, 400):
        print(f"negative/repeated {dtype.__name__} k={k}", flush=True)
        check(ix, ref, ti, tw, k)


def test_hybrid_large_repeated_heavy_weights(device):
    """A heavy term repeated 40 times in some queries, one occurrence weighing
    3000: the summed limb pair only fits with a large shift r (the heavy terms'
    weights rounded to a coarse grid, the margin widened to match), and the
    answers still equal the oracle's."""
    rng = np.random.default_rng(4)
    csr = zipf_csr(rng, 9000, 300, np.float32)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = zipf_queries(rng, 20, 300, np.float32, max_len=10)
    h0 = int(O.heavy_terms(ref["lengths"], _lib.heavy_term_count())[0])
    extra_t = np.full((20, 40), -1, np.int32)
    extra_w = np.zeros((20, 40), np.float32)
    extra_t[::5] = h0
    extra_w[::5] = rng.uniform(1e-3, 3.0, (4, 40)).astype(np.float32)
    extra_w[::5, 0] = 3000.0
    ti = np.ascontiguousarray(np.concatenate([ti, extra_t], axis=1))
    tw = np.ascontiguousarray(np.concatenate([tw, extra_w], axis=1))
    check(ix, ref, ti, tw, 50)


def test_hybrid_uint8_through_float16_copy(device):
    """A uint8 index takes the hybrid search on its float16 copy: int32 scores
    equal to the exact uint32 sums, for uint8 and for integer float query
    weights, equal to the LDS-only search's.  Batches wider than 258 terms (sums
    could pass 2^24) and indexes whose lists repeat a doc fall back to LDS adds
    (hybrid=True raises there); weights that are not integers in [0, 255] raise,
    from device memory too."""
    from gpusparse.search import U8_HYBRID_MAX_T
    rng = np.random.default_rng(14)
    csr = zipf_csr(rng, 6000, 300, np.uint8)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = zipf_queries(rng, 21, 300, np.uint8)
    print("uint8 hybrid", flush=True)
    for k in (1, 100, 6000):
        check(ix, ref, ti, tw, k)
        s, i = gs.search(ix, (torch.from_numpy(ti), torch.from_numpy(tw)), k, hybrid=False)
        s2, i2 = gs.search(ix, (torch.from_numpy(ti).cuda(), torch.from_numpy(tw.astype(np.float32)).cuda()), k)
        assert s.dtype == s2.dtype == torch.int32
        assert torch.equal(s, s2) and torch.equal(i, i2)
    with pytest.raises(ValueError, match="integers"):
        gs.search(ix, (torch.from_numpy(ti).cuda(), torch.from_numpy(tw.astype(np.float32) + 0.5).cuda()), 10)
    wide = np.full((3, U8_HYBRID_MAX_T + 1), -1, np.int32)
    wide[:, :20] = ti[:3, :20]
    ww = np.zeros(wide.shape, np.uint8)
    ww[:, :20] = tw[:3, :20]
    assert not gs.search_plan(ix, 3, wide.shape[1], 50)["hybrid"]
    with pytest.raises(ValueError, match="258"):
        gs.search_plan(ix, 3, wide.shape[1], 50, hybrid=True)
    vs, _, vi = O.c_search(ref, wide, ww, 50, threads=8)
    s, i = gs.search(ix, (torch.from_numpy(wide), torch.from_numpy(ww)), 50)
    assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
    dup = random_csr(rng, 2000, 50, dtype=np.uint8, dup_rate=0.2)
    ixd = gs.build_from_csr(dup, device)
    assert not gs.search_plan(ixd, 4, 6, 20)["hybrid"]


@pytest.mark.parametrize("vocab", [20, 64, 70, 128, 134])
def test_hybrid_small_vocabularies(device, vocab):
    """Vocabularies of at most as many terms as the heavy set (64): every term is
    heavy (no tail term at all; unused heavy slots hold -1); larger ones have
    tail terms."""
    rng = np.random.default_rng(vocab)
    csr = zipf_csr(rng, 7000, vocab, np.float32, max_len=min(12, vocab))
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = zipf_queries(rng, 33, vocab, np.float32, max_len=min(9, vocab))
    for k in (5, 300):
        print(f"small vocab {vocab} k={k}", flush=True)
        check(ix, ref, ti, tw, k)


def test_hybrid_many_tail_terms_and_large_entry_lists(device):
    """150 distinct tail terms per query (a group's union spans several LDS
    batches of terms) and one tail term repeated 30 times in every query."""
    rng = np.random.default_rng(6)
    V = 3000
    csr = zipf_csr(rng, 30000, V, np.float32, max_len=60, s=0.9)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    heavy = set(O.heavy_terms(ref["lengths"], _lib.heavy_term_count()).tolist())
    tail = np.array([t for t in range(V) if t not in heavy], np.int32)
    B = 40
    ti = np.stack([rng.choice(tail, 150, replace=False) for _ in range(B)]).astype(np.int32)
    rep = int(tail[rng.integers(len(tail))])
    ti = np.ascontiguousarray(np.concatenate([ti, np.full((B, 30), rep, np.int32)], axis=1))
    tw = rng.uniform(0.05, 2.0, ti.shape).astype(np.float32)
    print("many tail terms", flush=True)
    check(ix, ref, ti, tw, 200)


@pytest.mark.parametrize("tile_log2", [None, 8, 9, 13])
@pytest.mark.parametrize("n_docs", [300, 512, 513, 1100, 2600])
def test_hybrid_tiles_past_the_docs(device, n_docs, tile_log2):
    """Collections of less than one 512-doc block to a few: blocks past the head
    rows write zero sums and the tile's docs past the collection never become
    candidates.  With 256-doc tiles an odd tile count ends half way through a
    512-doc block, whose sums must still be computed (a workspace filled with
    garbage before the call shows sums that were not)."""
    rng = np.random.default_rng(n_docs)
    csr = zipf_csr(rng, n_docs, 200, np.float16, max_len=15)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = zipf_queries(rng, 18, 200, np.float32, max_len=8)
    print(f"tiles past the docs: n_docs={n_docs} tile_log2={tile_log2}", flush=True)
    for k in (1, min(100, n_docs), n_docs):
        check(ix, ref, ti, tw, k, tile_log2=tile_log2)
        ix.aux()["workspace"].fill_(0xCD)


@pytest.mark.parametrize("tile_log2,tiles_per_wg,sample_tiles", [(14, 3, 0), (14, 1, 2), (13, 1, 0), (12, 2, 1),
                                                                  (10, 7, 3), (8, 64, 0), (9, 0, 0)])
def test_hybrid_launch_shapes_and_dirty_workspace(device, tile_log2, tiles_per_wg, sample_tiles):
    """Every tile size (groups of 2 to 32 queries), several tiles per workgroup,
    seed launches of 1 and 3 tiles, and a workspace filled with garbage before
    the call."""
    rng = np.random.default_rng(tiles_per_wg)
    csr = zipf_csr(rng, 25000, 800, np.float32)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = zipf_queries(rng, 48, 800, np.float32)
    kw = dict(tile_log2=tile_log2, tiles_per_wg=tiles_per_wg, sample_tiles=sample_tiles)
    check(ix, ref, ti, tw, 60, **kw)
    ix.aux()["workspace"].fill_(0xCD)
    check(ix, ref, ti, tw, 60, **kw)


def test_hybrid_not_used_when_heavy_lists_repeat_docs(device):
    """An index whose heavy lists repeat a doc cannot hold a single dense cell
    per (doc, heavy term): hybrid=True raises and the default search runs the
    LDS-add scorer (same answers)."""
    rng = np.random.default_rng(8)
    csr = random_csr(rng, 3000, 30, dup_rate=0.2)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti, tw = random_queries(rng, 10, 30, max_len=6)
    assert not gs.search_plan(ix, 10, ti.shape[1], 20)["hybrid"]
    s, i = gs.search(ix, (torch.from_numpy(ti), torch.from_numpy(tw)), 20, path="fused")
    vs, _, vi = O.c_search(ref, ti, tw, 20, threads=8)
    assert np.array_equal(i.cpu().numpy(), vi) and np.array_equal(s.cpu().numpy(), vs)
    with pytest.raises(ValueError, match="hybrid"):
        gs.search(ix, (torch.from_numpy(ti), torch.from_numpy(tw)), 20, hybrid=True)


def test_hybrid_wide_queries(device):
    """300-term queries: every heavy term of the collection in most queries,
    many tail terms."""
    rng = np.random.default_rng(9)
    csr = zipf_csr(rng, 8000, 2000, np.float32, max_len=40)
    ix = gs.build_from_csr(csr, device)
    ref = oracle_index(csr)
    ti = np.stack([rng.choice(2000, 300, replace=False) for _ in range(24)]).astype(np.int32)
    tw = rng.uniform(0.01, 1.0, ti.shape).astype(np.float32)
    check(ix, ref, ti, tw, 100)
