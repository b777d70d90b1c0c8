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


def test_noalloc_replays_from_a_hip_graph(device):
    """After one eager call on the device (which looks up the scratch array's
    address), a gs_search_noalloc call captured into a HIP graph replays to
    gs_search's answer, replay after replay, with eager searches (one of them
    allocation-free, sharing the scratch) and synchronisations in between."""
    cfg = synth.scaled(synth.CONFIGS["C1"], n_docs=150_000, n_queries=48)
    docs, queries = synth.generate(cfg)
    ix = gs.build_from_csr(docs, device)
    qt, qw, _ = gs.to_query_tensors(queries, device, weight_dtype=None)
    B, T = qt.shape
    k = 100
    L = _lib.lib()
    tile, hyb = scorer_choice(ix, None, None)
    gidx = gs_index_struct(ix, tile, hybrid=hyb)
    opts = _lib.GsSearchOpts()
    print(f"graph replay: B={B} k={k} hybrid={hyb}", flush=True)
    need = C.c_size_t()
    _lib.check(L.gs_search_workspace(C.byref(gidx), B, T, k, C.byref(opts), C.byref(need)), "gs_search_workspace")
    ws = torch.empty(int(need.value), dtype=torch.uint8, device=device)
    rs = torch.empty((B, k), dtype=torch.float32, device=device)
    ri = torch.empty((B, k), dtype=torch.int64, device=device)
    rst = torch.empty(B, dtype=torch.int32, device=device)
    _lib.check(L.gs_search(C.byref(gidx), qt.data_ptr(), qw.data_ptr(), B, T, k, C.byref(opts), rs.data_ptr(),
                           ri.data_ptr(), rst.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_ptr(device)),
               "gs_search")
    torch.cuda.synchronize(device)
    want = (rs.cpu().numpy(), ri.cpu().numpy(), rst.cpu().numpy())
    assert (want[2] == _lib.GS_ROW_DONE).all()
    os_ = torch.empty((B, k), dtype=torch.float32, device=device)
    oi = torch.empty((B, k), dtype=torch.int64, device=device)
    st = torch.empty(B, dtype=torch.int32, device=device)

    def call(stream_ptr, b=B):
        return L.gs_search_noalloc(C.byref(gidx), qt.data_ptr(), qw.data_ptr(), b, T, k, C.byref(opts),
                                   os_.data_ptr(), oi.data_ptr(), st.data_ptr(), stream_ptr)

    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        _lib.check(call(side.cuda_stream), "gs_search_noalloc")  # eager: scratch address looked up here
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side, capture_error_mode="relaxed"):
        rc = call(torch.cuda.current_stream(device).cuda_stream)
    _lib.check(rc, "gs_search_noalloc under capture")
    for rep in range(3):
        os_.fill_(-7.0)
        oi.fill_(-7)
        st.fill_(-7)
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        got = (os_.cpu().numpy(), oi.cpu().numpy(), st.cpu().numpy())
        assert np.array_equal(got[2], want[2]), rep
        assert np.array_equal(got[1], want[1]), rep
        assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32)), rep
        # eager work between the replays: a smaller allocation-free search (same
        # scratch, same outputs' first rows) and a regular one
        _lib.check(call(_lib.stream_ptr(device), b=B // 3), "gs_search_noalloc")
        gs.search(ix, (qt[:7], qw[:7]), 20)
        torch.cuda.synchronize(device)
