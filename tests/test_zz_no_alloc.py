"""gs_search_noalloc (the allocation-free search; no counterpart in the
reference) against gs_search with a caller workspace, through the C ABI: two
calls in a row, the second with a smaller batch, must give identical ids,
scores and row status; a search too large for the scratch array is refused."""
import ctypes as C

import numpy as np
import pytest
import torch

import gpusparse as gs
from gpusparse import _lib, synth
from gpusparse.index import gs_index_struct
from gpusparse.search import scorer_choice

pytestmark = pytest.mark.gpu


def run_both(ix, qt, qw, k, cand_cap=0, hybrid=False):
    L = _lib.lib()
    dev = qt.device
    B, T = qt.shape
    tile, hyb = scorer_choice(ix, None, hybrid)
    assert hyb == hybrid
    gidx = gs_index_struct(ix, tile, hybrid=hyb)
    opts = _lib.GsSearchOpts(0, cand_cap, 0, 0, None, None, 0)
    sdt = torch.int32 if ix.scores.dtype == torch.uint8 else torch.float32
    s = _lib.stream_ptr(dev)
    need = C.c_size_t()
    _lib.check(L.gs_search_workspace(C.byref(gidx), B, T, k, C.byref(opts), C.byref(need)), "gs_search_workspace")
    ws = torch.empty(int(need.value), dtype=torch.uint8, device=dev)
    outs = []
    for noalloc in (False, True):
        os_ = torch.full((B, k), -7, dtype=sdt, device=dev)
        oi = torch.full((B, k), -7, dtype=torch.int64, device=dev)
        st = torch.full((B,), -7, dtype=torch.int32, device=dev)
        if noalloc:
            rc = L.gs_search_noalloc(C.byref(gidx), qt.data_ptr(), qw.data_ptr(), B, T, k, C.byref(opts),
                                     os_.data_ptr(), oi.data_ptr(), st.data_ptr(), s)
        else:
            rc = L.gs_search(C.byref(gidx), qt.data_ptr(), qw.data_ptr(), B, T, k, C.byref(opts), os_.data_ptr(),
                             oi.data_ptr(), st.data_ptr(), ws.data_ptr(), ws.numel(), s)
        _lib.check(rc, "gs_search_noalloc" if noalloc else "gs_search")
        torch.cuda.synchronize(dev)
        outs.append((os_.cpu().numpy(), oi.cpu().numpy(), st.cpu().numpy()))
    (s0, i0, st0), (s1, i1, st1) = outs
    assert np.array_equal(st0, st1)
    assert np.array_equal(i0, i1)
    assert s0.dtype == s1.dtype and np.array_equal(s0.view(np.uint8), s1.view(np.uint8))
    return st0


@pytest.mark.parametrize("name,hybrid", [("C1", True), ("C1", False), ("C5", False)])
def test_noalloc_matches_gs_search(device, name, hybrid):
    cfg = synth.scaled(synth.CONFIGS[name], n_docs=150_000, n_queries=192)
    docs, queries = synth.generate(cfg)
    ix = gs.build_from_csr(docs, device)
    qt, qw, _ = gs.to_query_tensors(queries, device, weight_dtype=None)
    print(f"noalloc {name} hybrid={hybrid}: B=192 k=1000, then B=37 k=100", flush=True)
    st = run_both(ix, qt, qw, 1000, hybrid=hybrid)
    assert (st == _lib.GS_ROW_DONE).all()
    st = run_both(ix, qt[:37].contiguous(), qw[:37].contiguous(), 100, hybrid=hybrid)
    assert (st == _lib.GS_ROW_DONE).all()
    # rows the capped candidate buffer cannot hold are flagged alike
    st = run_both(ix, qt[:20].contiguous(), qw[:20].contiguous(), 50, cand_cap=100, hybrid=hybrid)
    assert (st == _lib.GS_ROW_DENSE).any()


def test_noalloc_refuses_searches_beyond_its_scratch(device):
    cfg = synth.scaled(synth.CONFIGS["C1"], n_docs=20_000, n_queries=4)
    docs, queries = synth.generate(cfg)
    ix = gs.build_from_csr(docs, device)
    gidx = gs_index_struct(ix)
    B, T, k = 600, 8, 1000  # 600 queries x (64K candidates + 16K rescored) exceed 256 MiB
    opts = _lib.GsSearchOpts()
    opts.cand_cap = 65536  # the default would be held to the 20K docs
    need = C.c_size_t()
    L = _lib.lib()
    _lib.check(L.gs_search_workspace(C.byref(gidx), B, T, k, C.byref(opts), C.byref(need)), "gs_search_workspace")
    assert need.value > _lib.NOALLOC_SCRATCH_BYTES
    qt = torch.full((B, T), -1, dtype=torch.int32, device=device)
    qw = torch.zeros((B, T), dtype=torch.float32, device=device)
    os_ = torch.empty((B, k), dtype=torch.float32, device=device)
    oi = torch.empty((B, k), dtype=torch.int64, device=device)
    st = torch.empty(B, dtype=torch.int32, device=device)
    rc = L.gs_search_noalloc(C.byref(gidx), qt.data_ptr(), qw.data_ptr(), B, T, k, C.byref(opts), os_.data_ptr(),
                             oi.data_ptr(), st.data_ptr(), _lib.stream_ptr(device))
    assert rc == _lib.GS_ENOSPC
    assert b"allocation-free" in L.gs_last_error()
