"""Synthetic workload generator (csrc/synth.c): determinism, laws, codes."""
import numpy as np
import pytest

from gpusparse import synth


def test_rows_are_deterministic_and_thread_independent():
    spec = synth.RowSpec(n_rows=3000, nnz_mean=40.0, nnz_max=200)
    a = synth.generate_rows(spec, 5, synth.STREAM_DOCS, threads=1)
    b = synth.generate_rows(spec, 5, synth.STREAM_DOCS, threads=7)
    for x, y in zip(a[:3], b[:3]):
        assert np.array_equal(x, y)
    c = synth.generate_rows(spec, 6, synth.STREAM_DOCS, threads=3)
    assert not np.array_equal(a.indices[:500], c.indices[:500])


def test_row_laws():
    spec = synth.RowSpec(n_rows=20000)
    m = synth.generate_rows(spec, 1, synth.STREAM_DOCS)
    lens = np.diff(m.indptr)
    assert lens.min() >= 16 and lens.max() <= 512
    assert abs(lens.mean() - 120.0) < 2.0            # lognormal mean 120, sigma 0.5, light clipping
    for r in range(0, 20000, 997):                     # ascending, distinct term ids per row
        row = m.indices[m.indptr[r]:m.indptr[r + 1]]
        assert np.all(np.diff(row) > 0) and row.min() >= 0 and row.max() < synth.VOCAB
    w = m.data
    assert w.dtype == np.float32 and w.min() > 0 and w.max() <= 3.0
    # lognormal(-0.5, 0.8) median exp(-0.5)
    assert abs(np.median(w) - np.exp(-0.5)) < 0.01


def test_zipf_head_frequency():
    """P(rank 1 in a row) under successive sampling is 1 - P(never drawn); for the
    most frequent rank it is close to 1 - (1 - p1)^draws; check the ordering of
    document frequencies follows the ranks and the top rank is near-universal."""
    m = synth.generate_rows(synth.RowSpec(n_rows=20000), 2, synth.STREAM_DOCS)
    df = np.bincount(m.indices, minlength=synth.VOCAB)
    assert df[0] > 0.97 * 20000
    assert df[0] >= df[10] >= df[100] >= df[1000] >= df[10000]
    h = np.sum(np.arange(1, synth.VOCAB + 1, dtype=np.float64) ** -1.1)
    assert abs(df[1000] / 20000 - (1 - (1 - 1001 ** -1.1 / h) ** 260)) < 0.05


def test_forced_head_terms():
    spec = synth.RowSpec(n_rows=2000, nnz_mean=80.0, nnz_min=16, nnz_max=256, n_head_forced=8, head_pool=50,
                         zipf_s=1.3)
    m = synth.generate_rows(spec, 3, synth.STREAM_QUERIES)
    for r in range(0, 2000, 101):
        row = m.indices[m.indptr[r]:m.indptr[r + 1]]
        assert np.sum(row < 50) >= 8


def test_f16_codes_match_numpy_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.lognormal(-0.5, 3.0, 200000).astype(np.float32),
                        -rng.lognormal(-8, 4.0, 20000).astype(np.float32),
                        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                                  np.inf, -np.inf], np.float32)])
    got = synth.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_and_u8_configs():
    spec = synth.RowSpec(n_rows=500, weights="f32")
    f32 = synth.generate_rows(spec, 9, synth.STREAM_DOCS)
    f16 = synth.generate_rows(synth.RowSpec(n_rows=500, weights="f16"), 9, synth.STREAM_DOCS)
    u8 = synth.generate_rows(synth.RowSpec(n_rows=500, weights="u8"), 9, synth.STREAM_DOCS)
    assert np.array_equal(f32.indices, f16.indices)
    assert np.array_equal(f16.data, f32.data.astype(np.float16))
    q = synth.quantize_u8(f32)
    assert np.array_equal(u8.indptr, q.indptr) and np.array_equal(u8.indices, q.indices)
    assert np.array_equal(u8.data, q.data)


def test_u8_code_closed_form():
    from gpusparse.index import CSR
    w = np.array([3.0, 1.5, 0.0058, 0.00589, 0.006, 1.0], np.float32)
    c = CSR(np.array([0, 6]), np.arange(6, dtype=np.int32), w, (1, 6))
    q = synth.quantize_u8(c)
    # 3 -> 255; 1.5 -> 127.5 -> 128 (half to even); 0.0058*85 = 0.493 -> dropped;
    # 0.00589*85 = 0.50065 -> 1; 0.006*85 = 0.51 -> 1; 1.0 -> 85
    assert q.indices.tolist() == [0, 1, 3, 4, 5]
    assert q.data.tolist() == [255, 128, 1, 1, 85]


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_config_manifest(name):
    m = synth.manifest(name)
    assert m["name"] == name and m["docs"]["vocab"] == 30522


def test_c4_is_head_heavy():
    """C4's defining property at its full size (1M docs): each of the 50 most
    frequent terms holds more than 200K postings, and every query holds at least
    8 of those 50 terms (its forced head terms) within at most 256 terms."""
    cfg = synth.CONFIGS["C4"]
    docs = synth.generate_rows(cfg.docs, cfg.seed, synth.STREAM_DOCS)
    assert docs.shape[0] == 1_000_000
    df = np.bincount(docs.indices, minlength=synth.VOCAB)
    top50 = np.argsort(-df, kind="stable")[:50]
    assert df[top50].min() > 200_000
    assert set(top50.tolist()) == set(range(50))  # term id = Zipf rank - 1
    queries = synth.generate_rows(cfg.queries, cfg.seed, synth.STREAM_QUERIES)
    lens = np.diff(queries.indptr)
    assert lens.max() <= 256 and lens.min() >= 16
    rows = np.repeat(np.arange(queries.shape[0]), lens)
    held = np.bincount(rows[queries.indices < 50], minlength=queries.shape[0])
    assert held.min() >= 8
