"""GPU parity at the configurations' full sizes (C2: 1M docs, B=1024; C4: 1M docs
with Zipf(1.3) terms, B=512; C3 and C5: 8.8M docs, ~1.06e9 postings, B=512),
after src/remeasure_2026_09.py:155-235.

At these sizes the oracle does not rebuild the index on the host.  Instead:
- the GPU-built index is checked against its CSR by size-independent
  properties: lengths equal the CSR's column counts, padding to 32, exclusive
  offsets, every list ascending (gs_check_lists), and the same multiset of
  (doc, term, weight) postings (the oracle's order-independent checksum);
- the oracle then scores the host copy of that index (as bench.py does), and
  the GPU answers to every query of the batch must equal its exact top-k bit
  for bit: ids, and scores equal
  to the fp64 scatter-add rounded to fp32 (|diff| <= 1e-5 follows) or the
  exact uint32 sums.
One configuration is held at a time (the previous one is freed first)."""
import gc

import numpy as np
import pytest
import torch

import gpusparse as gs
from gpusparse import synth
from gpusparse.index import to_host
from oracle import oracle as O

pytestmark = pytest.mark.gpu

_held = {}


def full(name, device):
    """(config, index, host index, query terms, query weights, CSR checksum) of
    one configuration at full size, built once."""
    if name not in _held:
        _held.clear()
        gc.collect()
        torch.cuda.empty_cache()
        cfg = synth.CONFIGS[name]
        print(f"generating {name} at full size ({cfg.docs.n_rows} docs)", flush=True)
        docs, queries = synth.generate(cfg)
        want = O.checksum_csr(docs.indptr, docs.indices, docs.data, threads=16)
        counts = np.bincount(docs.indices, minlength=docs.shape[1]).astype(np.int32)
        ix = gs.build_from_csr(docs, device)
        nnz = docs.nnz
        del docs
        qt, qw, _ = gs.to_query_tensors(queries, device, weight_dtype=None)
        _held[name] = (cfg, ix, to_host(ix), qt, qw, want, counts, nnz)
    return _held[name]


def check_index(name, device):
    cfg, ix, h, qt, qw, want, counts, nnz = full(name, device)
    print(f"{name}: index invariants over {nnz} postings", flush=True)
    assert np.array_equal(h["lengths"], counts)
    assert int(h["lengths"].astype(np.int64).sum()) == nnz
    assert np.array_equal(h["padded_lengths"], (counts + 31) // 32 * 32)
    off = np.zeros_like(h["offsets"])
    np.cumsum(h["padded_lengths"][:-1].astype(np.int64), out=off[1:])
    assert np.array_equal(h["offsets"], off)
    assert ix.doc_ids.numel() == int(off[-1]) + int(h["padded_lengths"][-1])
    n_bad, n_nonempty = gs.check_lists(ix)
    assert n_bad == 0 and n_nonempty == int(np.count_nonzero(counts))
    assert O.checksum_index(h, threads=16) == (want, 0)


def check_search(name, device, k, rows=None, batch=None, **opts):
    """The GPU's top-k of the whole batch (or of its first `batch` queries); `rows`
    of it (all by default) checked against the oracle."""
    cfg, ix, h, qt, qw, *_ = full(name, device)
    if batch is not None:
        qt, qw = qt[:batch].contiguous(), qw[:batch].contiguous()
    if rows is None:
        rows = np.arange(qt.shape[0])
    print(f"{name}: search B={qt.shape[0]} k={k} {opts}, {len(rows)} rows checked", flush=True)
    timing = {}
    s, i = gs.search(ix, (qt, qw), k, timing=timing, path="fused", **opts)
    assert s.shape == (qt.shape[0], k)
    ti, tw = qt.cpu().numpy()[rows], qw.cpu().numpy()[rows]
    vs, s64, vi = O.c_search(h, ti, tw, k, threads=16)
    got_s, got_i = s.cpu().numpy()[rows], i.cpu().numpy()[rows]
    assert np.array_equal(got_i, vi)
    assert got_s.dtype == vs.dtype and np.array_equal(got_s, vs)
    if got_s.dtype == np.float32:
        assert np.max(np.abs(got_s.astype(np.float64) - s64)) <= 1e-5
    return timing


def test_c2_full_index(device):
    check_index("C2", device)


def test_c2_full_search_whole_batch(device):
    """1M docs, B=1024 (the groups of a whole 1024-query ordering block), fp32,
    k=1000: every query of the batch checked."""
    check_search("C2", device, 1000)


def test_c4_full_index(device):
    check_index("C4", device)


@pytest.mark.parametrize("tile_log2,hybrid", [(None, None), (None, False), (8, True), (8, False), (10, None),
                                              (12, None), (13, True)])
def test_c4_full_search(device, tile_log2, hybrid):
    """1M docs whose top-50 terms each hold > 200K postings (dense in every tile):
    the head-heavy case of the scorer, every row of the 512-query batch, over the
    tile sweep (256, 1K, 4K, 8K docs and the defaults: 16K for the hybrid search,
    8K for the LDS-only one); at 256-doc tiles 32 queries share a workgroup, with
    and without the heavy terms as matrix products."""
    check_search("C4", device, 1000, tile_log2=tile_log2, hybrid=hybrid)


def test_c3_full_index(device):
    check_index("C3", device)


@pytest.mark.parametrize("k,hybrid", [(1000, None), (1000, False), (10, None)])
def test_c3_full_search(device, k, hybrid):
    """Every row of the 512-query batch, by the default search (the hybrid one
    for these fp16 weights) and by the LDS-only one."""
    timing = check_search("C3", device, k, hybrid=hybrid)
    assert timing["dense_rows"] == 0


@pytest.mark.parametrize("B", [1, 8, 16, 64])
def test_c3_full_small_batches(device, B):
    """Few query groups score all their tiles at once, so tau rises little after
    the seed; the seed widened for them and the default candidate cap spread over
    the batch keep every row on the fused path, exact."""
    timing = check_search("C3", device, 1000, batch=B)
    assert timing["dense_rows"] == 0


def test_c5_full_index(device):
    check_index("C5", device)


@pytest.mark.parametrize("hybrid", [None, False])
def test_c5_full_search_bit_exact(device, hybrid):
    """The integer configuration: uint8 x uint8 products summed in uint32,
    bit-exact with the CPU integer reference, ties by ascending doc id; by the
    hybrid search on the index's float16 copy (the default) and by LDS adds."""
    check_search("C5", device, 1000, hybrid=hybrid)


def test_zz_release_full_size(device):
    _held.clear()
    gc.collect()
    torch.cuda.empty_cache()
