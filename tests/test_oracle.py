"""Pins the CPU oracle (oracle/oracle.py, oracle/oracle_score.c) against
independent computations.  The reference holds no golden vectors for this path,
so each oracle function is checked against a different algorithm: brute-force
Python lists, dense matrix products, full sorts and closed forms."""
import numpy as np
import pytest

from helpers import dense_docs, dense_queries, random_csr, random_queries
from oracle import oracle as O


def brute_index(csr, vocab):
    """Dict-of-lists builder in the manner of src/gpu_inverted_index.py:59-99."""
    lists = [[] for _ in range(vocab)]
    for d in range(csr.shape[0]):
        for p in range(csr.indptr[d], csr.indptr[d + 1]):
            lists[int(csr.indices[p])].append((d, csr.data[p]))
    docs, scores, offsets, lengths, padded, maxs = [], [], [], [], [], []
    pos = 0
    for t in range(vocab):
        pl = sorted(lists[t], key=lambda x: x[0])  # Python's sort is stable
        n = len(pl)
        pn = (n + 31) // 32 * 32
        offsets.append(pos)
        lengths.append(n)
        padded.append(pn)
        maxs.append(max(float(s) for _, s in pl) if pl else 0.0)
        docs.extend([d for d, _ in pl] + [-1] * (pn - n))
        scores.extend([s for _, s in pl] + [0] * (pn - n))
        pos += pn
    return docs, scores, offsets, lengths, padded, maxs


@pytest.mark.parametrize("seed,n_docs,vocab,dtype,dup", [
    (0, 50, 40, np.float32, 0.0), (1, 200, 7, np.float32, 0.3), (2, 64, 1, np.float32, 0.0),
    (3, 100, 300, np.float16, 0.1), (4, 80, 60, np.uint8, 0.0), (5, 0, 10, np.float32, 0.0)])
def test_build_index_matches_brute_force(seed, n_docs, vocab, dtype, dup):
    rng = np.random.default_rng(seed)
    csr = random_csr(rng, n_docs, vocab, dtype=dtype, dup_rate=dup)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, n_docs, vocab)
    docs, scores, offsets, lengths, padded, maxs = brute_index(csr, vocab)
    assert ix["doc_ids"].tolist() == docs
    assert ix["scores"].astype(np.float64).tolist() == [float(s) for s in scores]
    assert ix["scores"].dtype == csr.data.dtype
    assert ix["offsets"].tolist() == offsets
    assert ix["lengths"].tolist() == lengths
    assert ix["padded_lengths"].tolist() == padded
    assert np.array_equal(ix["max_scores"], np.asarray(maxs, np.float32))


def test_build_index_invariants():
    rng = np.random.default_rng(7)
    csr = random_csr(rng, 500, 90, dup_rate=0.05)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 500, 90)
    assert int(ix["lengths"].sum()) == csr.nnz
    assert np.all(ix["offsets"] % 32 == 0) and np.all(ix["padded_lengths"] % 32 == 0)
    pairs = []
    for t in range(90):
        o, L, P = ix["offsets"][t], ix["lengths"][t], ix["padded_lengths"][t]
        seg = ix["doc_ids"][o:o + L]
        assert np.all(np.diff(seg) >= 0)
        assert np.all(ix["doc_ids"][o + L:o + P] == -1) and np.all(ix["scores"][o + L:o + P] == 0)
        pairs.extend((int(d), t) for d in seg)
    rows = np.repeat(np.arange(500), np.diff(csr.indptr))
    assert sorted(pairs) == sorted(zip(rows.tolist(), csr.indices.tolist()))


def test_build_index_rejects_out_of_range_terms():
    csr = random_csr(np.random.default_rng(0), 10, 5)
    with pytest.raises(IndexError):
        O.build_index(csr.indptr, csr.indices, csr.data, 10, int(csr.indices.max()))


@pytest.mark.parametrize("seed,dtype,dup", [(0, np.float32, 0.0), (1, np.float16, 0.3), (2, np.uint8, 0.1)])
def test_forward_index_is_the_csr_sorted_by_column(seed, dtype, dup):
    """Transposing the term-major index back gives each CSR row with its columns
    sorted stably: a (doc, term) pair repeated in a row keeps its row order, which
    is also its list order in the inverted index."""
    rng = np.random.default_rng(seed)
    csr = random_csr(rng, 300, 40, dtype=dtype, dup_rate=dup)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 300, 40)
    row_ptr, terms, w = O.forward_index(ix)
    assert np.array_equal(row_ptr, csr.indptr)
    for d in range(300):
        b, e = csr.indptr[d], csr.indptr[d + 1]
        order = sorted(range(b, e), key=lambda i: (csr.indices[i], i))
        assert terms[b:e].tolist() == [int(csr.indices[i]) for i in order]
        assert w[b:e].tobytes() == csr.data[order].tobytes()


@pytest.mark.parametrize("tile_log2", [4, 8, 11])
def test_tile_bounds_match_linear_scan(tile_log2):
    rng = np.random.default_rng(tile_log2)
    csr = random_csr(rng, 2500, 20, dup_rate=0.1)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 2500, 20)
    tb = O.tile_bounds(ix, tile_log2)
    n_tiles = (2500 + (1 << tile_log2) - 1) >> tile_log2
    assert tb.shape == (20, n_tiles + 1)
    for t in range(20):
        o, n = int(ix["offsets"][t]), int(ix["lengths"][t])
        seg = ix["doc_ids"][o:o + n].tolist()
        for j in range(n_tiles + 1):
            edge = j << tile_log2
            assert tb[t, j] == next((i for i, d in enumerate(seg) if d >= edge), n)


@pytest.mark.parametrize("n", [64, 128])
@pytest.mark.parametrize("vocab,seed", [(20, 0), (64, 1), (65, 2), (128, 5), (129, 6), (3000, 3), (30522, 4)])
def test_heavy_terms_matches_sorted(vocab, seed, n):
    """Ties of equal length (lengths drawn from a few values) and empty lists."""
    rng = np.random.default_rng(seed)
    lengths = rng.choice([0, 0, 1, 2, 3, 7, 7, 50], size=vocab).astype(np.int32)
    if vocab > 100:
        lengths[rng.choice(vocab, 90, replace=False)] = rng.integers(100, 130, 90)
    want = [t for t in sorted(range(vocab), key=lambda t: (-int(lengths[t]), t)) if lengths[t] > 0][:n]
    got = O.heavy_terms(lengths, n)
    assert got.tolist() == want + [-1] * (n - len(want))


@pytest.mark.parametrize("max_abs,want", [(1.0, 12), (3.0, 11), (8191.0, 0), (8192.0, -1), (0.5, 13),
                                          (1e-3, 22), (0.0, 0), (float(np.finfo(np.float32).max), -116),
                                          (float(np.float32(2.0 ** -149)), 161), (4095.75, 0), (4095.5, 1),
                                          (4096.0, 0)])
def test_pack_shift_closed_forms(max_abs, want):
    """Largest s with max_abs * 2^s <= 8191: at powers of two 8191 / 2^s falls
    between consecutive powers, so s = 12 - log2(max_abs); checked by hand for the
    others (1e-3 * 2^22 = 4194.3, * 2^23 = 8388.6; 4095.75 * 2 = 8191.5, 4095.5 * 2 = 8191; FLT_MAX =
    (2 - 2^-23) 2^127, so FLT_MAX * 2^-115 = 8192 - 2^-11 > 8191)."""
    assert O.pack_shift(max_abs) == want
    with pytest.raises(ValueError):
        O.pack_shift(-1.0)
    with pytest.raises(ValueError):
        O.pack_shift(float("inf"))


def test_head_limbs_hand_made():
    """Two heavy lists: term 1 with weights giving packed values 300, -5, 8191
    (shift 0 after scaling by hand), term 0 with one posting; limbs by hand:
    300 = 2 * 128 + 44, -5 = -1 * 128 + 123, 8191 = 63 * 128 + 127."""
    indptr = np.array([0, 1, 2, 4], np.int64)
    indices = np.array([1, 1, 1, 0], np.int32)
    data = np.array([300.0, -5.0, 8191.0, 7.0], np.float32)
    ix = O.build_index(indptr, indices, data, 3, 4)
    heavy = O.heavy_terms(ix["lengths"], 4)
    assert heavy.tolist() == [1, 0, -1, -1]
    got = O.head_limbs(ix, heavy, 4)
    assert O.pack_shift(8191.0) == 0
    want = np.zeros((4, 2, 4), np.int8)
    want[0, :, 0] = (44, 2)
    want[1, :, 0] = (123, -1)
    want[2, :, 0] = (127, 63)
    want[2, :, 1] = (7, 0)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.uint8])
def test_head_limbs_recombine_to_packed_weights(dtype):
    """Random lists: for every heavy posting 128 * high + low equals the packed
    weight rint(w 2^shift) (computed here from the weights, not from
    pack_postings), low in [0, 127]; cells of docs lacking a heavy term are zero."""
    rng = np.random.default_rng(5)
    csr = random_csr(rng, 3000, 90, dtype=dtype)
    if dtype != np.uint8:
        csr.data[::3] *= -1
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 3000, 90)
    heavy = O.heavy_terms(ix["lengths"])
    got = O.head_limbs(ix, heavy, 3072)
    lo, hi = got[:, 0, :].astype(np.int64), got[:, 1, :].astype(np.int64)
    assert lo.min() >= 0 and lo.max() <= 127
    rec = 128 * hi + lo
    w64 = csr.data.astype(np.float64)
    shift = 0 if dtype == np.uint8 else O.pack_shift(float(np.abs(w64).max()))
    want = np.zeros((3072, len(heavy)), np.int64)
    rows = np.repeat(np.arange(3000), np.diff(csr.indptr))
    col_of = {int(t): h for h, t in enumerate(heavy) if t >= 0}
    for r, t, w in zip(rows, csr.indices, w64):
        if int(t) in col_of:
            want[r, col_of[int(t)]] = int(w) if dtype == np.uint8 else int(np.rint(np.ldexp(w, shift)))
    assert np.array_equal(rec, want)


@pytest.mark.parametrize("tile_log2,dtype", [(12, np.float16), (8, np.uint8), (13, np.float32), (14, np.float16)])
def test_pack_postings_decodes_and_matches_scalar_loop(tile_log2, dtype):
    from fractions import Fraction
    rng = np.random.default_rng(tile_log2)
    csr = random_csr(rng, 40000, 50, dtype=dtype, dup_rate=0.05)
    if dtype != np.uint8:  # signed weights and exact ties at half units
        csr.data[::7] *= -1
        csr.data[5::11] = (np.arange(len(csr.data[5::11])) % 9 + 0.5).astype(dtype) / 4
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 40000, 50)
    pk = O.pack_postings(ix, tile_log2, arrange=False)
    doc, w = ix["doc_ids"], ix["scores"]
    mask = (1 << tile_log2) - 1
    u = pk.view(np.uint32)
    off, wb = u & 0xFFFF, u >> 16
    assert np.array_equal(off[doc >= 0] >> 2, doc[doc >= 0] & mask) and not np.any(off[doc >= 0] & 3)
    assert not np.any(pk[doc < 0])
    if dtype == np.uint8:
        assert np.array_equal(wb[doc >= 0], w[doc >= 0].astype(np.uint32))
        shift = 0
    else:
        shift = O.pack_shift(float(np.abs(w[doc >= 0].astype(np.float64)).max()))
        q = wb.astype(np.uint16).view(np.int16).astype(np.int64)
        assert np.abs(q).max() <= 8191
        err = np.abs(q[doc >= 0] - np.ldexp(w[doc >= 0].astype(np.float64), shift))
        assert err.max() <= 0.5
    # scalar loop with exact rational rounding (Python's round: half to even)
    for i in range(0, len(doc), 97):
        d = int(doc[i])
        if d < 0:
            assert int(pk[i]) == 0
            continue
        o = (d % (1 << tile_log2)) * 4
        if dtype == np.uint8:
            b = int(w[i])
        else:
            b = round(Fraction(float(w[i])) * Fraction(2) ** shift) & 0xFFFF
        assert int(pk[i]) & 0xFFFFFFFF == o + (b << 16)


def deal_by_enumeration(docs):
    """arrange_order restated as a literal deal: the cells (group, position) are
    listed position by position, groups in order, skipping positions the last
    (partial) group does not have; the postings sorted by (doc mod 64, doc) fill
    them in that order."""
    n = len(docs)
    G = (n + 63) // 64
    cap = [64] * (G - 1) + [n - 64 * (G - 1)]
    cells = [(g, p) for p in range(64) for g in range(G) if p < cap[g]]
    srt = sorted(range(n), key=lambda i: (int(docs[i]) % 64, int(docs[i]), i))
    order = [None] * n
    for (g, p), i in zip(cells, srt):
        order[g * 64 + p] = i
    return np.array(order)


@pytest.mark.parametrize("n,seed", [(65, 0), (128, 1), (130, 2), (191, 3), (1000, 4), (4096, 5), (8191, 6)])
def test_arrange_order_is_the_deal(n, seed):
    rng = np.random.default_rng(seed)
    docs = np.sort(rng.choice(8192 if n < 8000 else 16384, size=n, replace=False)).astype(np.int64)
    if seed % 2:  # repeated doc ids (a term twice in one doc) keep their order
        docs = np.sort(np.concatenate([docs[: n - n // 8], docs[: n // 8]]))
    order = O.arrange_order(docs)
    assert np.array_equal(order, deal_by_enumeration(docs))
    assert np.array_equal(np.sort(order), np.arange(n))
    G = (n + 63) // 64
    res = docs[order] & 63
    counts = np.bincount(docs & 63, minlength=64)
    for g in range(G):
        per = np.bincount(res[g * 64:(g + 1) * 64], minlength=64)
        assert np.all(per <= -(-counts // max(G - 1, 1)))


def test_arrange_order_known_answers():
    # consecutive docs: every group already holds 64 distinct residues -> identity
    for n in (65, 130, 1000):
        d = np.arange(n, dtype=np.int64) + 4096
        assert np.array_equal(O.arrange_order(d), np.arange(n))
    # docs 0, 2, 4, ...: 32 even residues, each 4 times among 128 postings (G = 2):
    # residue r's docs r, r + 64, r + 128, r + 192 go to groups 0, 1, 0, 1
    d = np.arange(0, 256, 2, dtype=np.int64)
    got = d[O.arrange_order(d)]
    assert list(got[:4]) == [0, 128, 2, 130] and list(got[64:68]) == [64, 192, 66, 194]


def test_pack_arrangement_permutes_blocks_only():
    """Each (term, tile) sub-range is rearranged in blocks of ARRANGE_BLOCK postings
    from its start: a block of more than 64 postings is a permutation of itself in
    the deal order of its own docs, a shorter one (a sub-range's tail) and every
    short sub-range stay in slot order.  vocab 12 and 4096-doc tiles give
    sub-ranges of about 1800 postings: two blocks each, the second one partial."""
    rng = np.random.default_rng(11)
    csr = random_csr(rng, 30000, 12, dtype=np.float16, dup_rate=0.05)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 30000, 12)
    tl = 12
    plain, arr = O.pack_postings(ix, tl, arrange=False), O.pack_postings(ix, tl)
    moved, blocks, tails = 0, 0, 0
    edges = np.arange(((30000 + (1 << tl) - 1) >> tl) + 1, dtype=np.int64) << tl
    covered = np.zeros(len(plain), dtype=bool)
    for t in range(12):
        o, L = int(ix["offsets"][t]), int(ix["lengths"][t])
        docs = ix["doc_ids"][o:o + L].astype(np.int64)
        b = np.searchsorted(docs, edges)
        for lo, hi in zip(b[:-1], b[1:]):
            a, z = o + lo, o + hi
            assert np.array_equal(np.sort(arr[a:z]), np.sort(plain[a:z]))
            for c in range(int(lo), int(hi), O.ARRANGE_BLOCK):
                e = min(c + O.ARRANGE_BLOCK, int(hi))
                if e - c > 64:
                    want = plain[o + c:o + e][O.arrange_order(docs[c:e])]
                    assert np.array_equal(arr[o + c:o + e], want)
                    covered[o + c:o + e] = True
                    moved += int(np.count_nonzero(arr[o + c:o + e] != plain[o + c:o + e]))
                    blocks += 1
                    tails += e - c < O.ARRANGE_BLOCK
    assert np.array_equal(arr[~covered], plain[~covered]) and moved > 0
    assert blocks > tails > 0


@pytest.mark.parametrize("chunk", [1, 3, 17, 64, 1000])
def test_chunk_bounds_match_linear_scan(chunk):
    rng = np.random.default_rng(chunk)
    csr = random_csr(rng, 150, 30, dup_rate=0.1)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 150, 30)
    b = O.chunk_bounds(ix["doc_ids"], ix["offsets"], ix["lengths"], 30, 150, chunk)
    n_chunks = (150 + chunk - 1) // chunk
    assert b.shape == (n_chunks + 1, 30)
    for t in range(30):
        o, L = int(ix["offsets"][t]), int(ix["lengths"][t])
        seg = ix["doc_ids"][o:o + L].tolist()
        for c in range(n_chunks + 1):
            edge = c * chunk if c < n_chunks else 150
            first = next((i for i, d in enumerate(seg) if d >= edge), L)
            assert b[c, t] == o + first
        # the chunk sub-ranges partition the list
        assert b[0, t] == o and b[-1, t] == o + L
        assert np.all(np.diff(b[:, t]) >= 0)


def test_chunk_bounds_reject_non_ascending():
    csr = random_csr(np.random.default_rng(3), 100, 8, empty_rate=0.0)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 100, 8)
    t = int(np.argmax(ix["lengths"]))
    o = ix["offsets"][t]
    ix["doc_ids"][o], ix["doc_ids"][o + 1] = ix["doc_ids"][o + 1], ix["doc_ids"][o]
    with pytest.raises(ValueError, match="1 of .* posting lists are not ascending"):
        O.chunk_bounds(ix["doc_ids"], ix["offsets"], ix["lengths"], 8, 100, 16)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_scores_f64_equal_dense_product(dtype):
    rng = np.random.default_rng(11)
    csr = random_csr(rng, 120, 50, dtype=dtype, dup_rate=0.1)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 120, 50)
    ti, tw = random_queries(rng, 9, 50, invalid_rate=0.2)
    got = O.scores_f64(ix, ti, tw)
    want = dense_queries(ti, tw, 50) @ dense_docs(csr).T
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)


def test_scores_u32_equal_integer_product():
    rng = np.random.default_rng(12)
    csr = random_csr(rng, 120, 50, dtype=np.uint8, dup_rate=0.1)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 120, 50)
    ti, tw = random_queries(rng, 9, 50, dtype=np.uint8, invalid_rate=0.2)
    got = O.scores_u32(ix, ti, tw)
    want = dense_queries(ti, tw, 50, dtype=np.int64) @ dense_docs(csr, dtype=np.int64).T
    assert np.array_equal(got.astype(np.int64), want)


def test_scores_f32_sequential_is_the_reference_cpu_accumulation():
    """Scalar float32 loop of src/gpu_scoring.py:246-251 (product rounded to fp32,
    added to the fp32 accumulator) on a tiny input."""
    rng = np.random.default_rng(13)
    csr = random_csr(rng, 40, 20)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 40, 20)
    ti, tw = random_queries(rng, 5, 20)
    got = O.scores_f32_sequential(ix, ti, tw)
    for q in range(5):
        acc = [np.float32(0)] * 40
        for t, wq in zip(ti[q], tw[q]):
            if t < 0:
                continue
            for d in range(40):
                for p in range(csr.indptr[d], csr.indptr[d + 1]):
                    if csr.indices[p] == t:
                        acc[d] = np.float32(acc[d] + np.float32(float(wq) * float(csr.data[p])))
        assert np.array_equal(got[q], np.asarray(acc, np.float32))


def test_topk_tie_rule_matches_full_sort():
    rng = np.random.default_rng(14)
    s = rng.integers(0, 6, size=(7, 50)).astype(np.float64)  # many ties
    v, i = O.topk(s, 13)
    for q in range(7):
        want = sorted(range(50), key=lambda d: (-s[q, d], d))[:13]
        assert i[q].tolist() == want
        assert v[q].tolist() == [s[q, d] for d in want]
    vu, iu = O.topk(s.astype(np.uint32), 50)
    assert np.array_equal(iu, np.stack([sorted(range(50), key=lambda d: (-s[q, d], d)) for q in range(7)]))


def test_search_matches_brute_force_including_zero_fill():
    rng = np.random.default_rng(15)
    csr = random_csr(rng, 60, 30, empty_rate=0.3)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 60, 30)
    ti, tw = random_queries(rng, 6, 30, max_len=3)
    v, i = O.search(ix, ti, tw, 60)   # k = N: zero-score docs fill by ascending id
    S = dense_queries(ti, tw, 30) @ dense_docs(csr).T
    for q in range(6):
        want = sorted(range(60), key=lambda d: (-S[q, d], d))
        assert i[q].tolist() == want
        np.testing.assert_allclose(v[q], S[q, want].astype(np.float32), rtol=1e-6)


def test_compacted_topk_semantics():
    rng = np.random.default_rng(16)
    s = rng.normal(size=(5, 40)).astype(np.float32)
    tau = np.array([0.0, 1.5, -np.inf, 3.0, 0.5], np.float32)
    v, i = O.compacted_topk(s, tau, 12)
    for b in range(5):
        cand = [c for c in range(40) if s[b, c] >= tau[b]]
        want = sorted(cand, key=lambda c: (-s[b, c], c))[:12]
        assert i[b, :len(want)].tolist() == want
        assert np.all(np.isneginf(v[b, len(want):])) and np.all(i[b, len(want):] == 0)
    v2, i2 = O.compacted_topk(s, None, 40)
    assert np.array_equal(i2, np.stack([sorted(range(40), key=lambda c: (-s[b, c], c)) for b in range(5)]))


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.uint8])
def test_c_oracle_equals_numpy_oracle(dtype):
    rng = np.random.default_rng(17)
    csr = random_csr(rng, 300, 80, dtype=dtype, dup_rate=0.05)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 300, 80)
    qdt = np.uint8 if dtype == np.uint8 else np.float32
    ti, tw = random_queries(rng, 11, 80, dtype=qdt, invalid_rate=0.1)
    for k in (1, 7, 300):
        v, s64, i = O.c_search(ix, ti, tw, k, threads=2)
        vn, inn = O.search(ix, ti, tw, k)
        assert np.array_equal(i, inn)
        assert np.array_equal(v, vn)          # identical summation order -> identical bits


def test_c_cpu_sequential_equals_reference_cpu_path():
    rng = np.random.default_rng(18)
    n_docs, vocab = 80, 25
    doc_terms = [list(rng.choice(vocab, size=int(rng.integers(1, 8)), replace=False)) for _ in range(n_docs)]
    doc_w = [list(np.float32(rng.lognormal(-0.5, 0.8, size=len(t)))) for t in doc_terms]
    qt = [list(rng.choice(vocab, size=5, replace=False)) for _ in range(4)]
    qw = [list(np.float32(rng.lognormal(-0.5, 0.8, size=5))) for _ in range(4)]
    ref_s, ref_i = O.cpu_sequential_score(doc_terms, doc_w, qt, qw, n_docs, top_k=6)
    indptr = np.cumsum([0] + [len(t) for t in doc_terms])
    ix = O.build_index(indptr, np.concatenate(doc_terms), np.concatenate(doc_w).astype(np.float32), n_docs, vocab)
    v, i = O.c_cpu_sequential(ix, np.asarray(qt, np.int32), np.asarray(qw, np.float32), 6)
    for q in range(4):
        assert np.array_equal(np.asarray(ref_s[q], np.float32), v[q])
        assert set(ref_i[q]) == set(i[q].tolist()) or len(set(ref_s[q])) < 6


def test_to_query_tensors_oracle():
    indptr = np.array([0, 3, 3, 5]); indices = np.array([4, 1, 9, 2, 2]); data = np.array([.5, .25, 1., 2., 3.])
    ti, ts, T = O.to_query_tensors(indptr, indices, data)
    assert T == 3
    assert ti.tolist() == [[4, 1, 9], [-1, -1, -1], [2, 2, -1]]
    assert ts.tolist() == [[.5, .25, 1.], [0, 0, 0], [2., 3., 0]]


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.uint8])
def test_posting_checksum_detects_planted_changes(dtype):
    """The full-size index check: CSR and index checksums agree on an index and
    its CSR, and each planted mistake (in the oracle's index, on the CPU) changes
    the checksum or the layout count."""
    rng = np.random.default_rng(5)
    csr = random_csr(rng, 400, 60, dtype=dtype, max_len=15)
    ix = O.build_index(csr.indptr, csr.indices, csr.data, 400, 60)
    want = O.checksum_csr(csr.indptr, csr.indices, csr.data)
    assert O.checksum_index(ix) == (want, 0)
    t = int(np.argmax(ix["lengths"]))
    o, n = int(ix["offsets"][t]), int(ix["lengths"][t])

    def planted(fn):
        j = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in ix.items()}
        fn(j)
        return O.checksum_index(j)

    def move(j):   # a posting filed under the wrong doc
        j["doc_ids"][o] = (j["doc_ids"][o] + 1) % 400

    def alter(j):  # one weight bit flipped
        j["scores"].view(np.uint8)[o * j["scores"].itemsize] ^= 1

    def drop(j):   # last posting lost (list shortened, slot padded)
        j["lengths"][t] -= 1
        j["doc_ids"][o + n - 1] = -1
        j["scores"][o + n - 1] = 0

    def swap_terms(j):  # two postings exchanged between lists
        t2 = int(np.argsort(j["lengths"])[-2])
        o2 = int(j["offsets"][t2])
        j["doc_ids"][o], j["doc_ids"][o2] = j["doc_ids"][o2], j["doc_ids"][o]

    for fn in (move, alter, drop, swap_terms):
        assert planted(fn)[0] != want, fn.__name__

    def dirty_pad(j):
        j["doc_ids"][o + n] = 3 if j["padded_lengths"][t] > n else j["doc_ids"][o + n]

    if ix["padded_lengths"][t] > n:
        assert planted(dirty_pad)[1] == 1
