"""Host logic and the C ABI boundary, without a GPU."""
import ctypes
import gzip
import os
import re

import numpy as np
import pytest

import gpusparse
from gpusparse import _lib, engine
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "gpusparse.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gs_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 15
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with include/gpusparse.h"
    assert _lib.lib().gs_query_version() == _lib.ABI_VERSION


def test_argument_errors_map_to_python_exceptions():
    L = _lib.lib()
    rc = L.gs_index_count(None, 0, 0, None, None, None, None, None)
    assert rc == _lib.GS_EINVAL
    with pytest.raises(ValueError, match="vocab must be positive"):
        _lib.check(rc, "gs_index_count")
    rc = L.gs_compacted_topk(None, 4, 2, 4, None, 9, 16, None, None, None, None, 0, None)
    with pytest.raises(ValueError, match="k=9 outside"):
        _lib.check(rc, "gs_compacted_topk")
    idx = _lib.GsIndex()
    rc = L.gs_search(ctypes.byref(idx), None, None, 1, 1, 1, None, None, None, None, None, 0, None)
    with pytest.raises(ValueError):
        _lib.check(rc, "gs_search")
    # the heavy-term rows must cover the last doc's whole GS_HEAD_BLOCK block,
    # which the search reads; rejected before any pointer is used
    n_docs = _lib.HEAD_BLOCK + 1
    rc = L.gs_head_fill(None, None, 1, None, None, 8, None, 0, n_docs, n_docs + 15, None, None, None)
    with pytest.raises(ValueError, match="rounded up to GS_HEAD_BLOCK"):
        _lib.check(rc, "gs_head_fill")


def test_pack_shift_matches_oracle():
    """gs_pack_shift is host code: the C ABI and the oracle agree on random,
    power-of-two and extreme magnitudes, and reject negative / non-finite input."""
    L = _lib.lib()
    rng = np.random.default_rng(3)
    vals = list(np.float32(rng.lognormal(0.0, 6.0, 300))) + [np.float32(2.0) ** e for e in range(-149, 128, 7)]
    vals += [np.float32(0.0), np.finfo(np.float32).max, np.float32(8191.0), np.float32(8191.5), np.float32(4095.75)]
    for v in vals:
        sh = ctypes.c_int32(99)
        assert L.gs_pack_shift(ctypes.c_float(float(v)), ctypes.byref(sh)) == _lib.GS_OK
        assert sh.value == O.pack_shift(float(v)), float(v)
    for bad in (-1.0, float("inf"), float("nan")):
        assert L.gs_pack_shift(ctypes.c_float(bad), ctypes.byref(ctypes.c_int32())) == _lib.GS_EINVAL


def test_no_gpu_raises_runtime_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU visible")
    with pytest.raises(RuntimeError, match="requires a GPU"):
        _lib.require_gpu()
    with pytest.raises(RuntimeError):
        gpusparse.build_index(gpusparse.CSR(np.array([0, 1]), np.array([0], np.int32),
                                            np.array([1.0], np.float32), (1, 1)), "cuda:0")


def test_to_csr_and_dimension():
    emb = [("d0", [3, 1], [0.5, 1.0]), ("d1", [], []), ("d2", [7], [2.0])]
    q = [("q0", [9], [1.0])]
    assert engine.determine_dimension(emb, q) == 11
    ids, c = engine.to_csr(emb, 11)
    assert ids == ["d0", "d1", "d2"]
    assert c.indptr.tolist() == [0, 2, 2, 3] and c.indices.tolist() == [3, 1, 7]
    assert c.data.dtype == np.float32 and c.shape == (3, 11)


def test_to_query_tensors_matches_oracle():
    rng = np.random.default_rng(0)
    lens = rng.integers(0, 9, size=40)
    indptr = np.concatenate([[0], np.cumsum(lens)])
    indices = rng.integers(0, 100, size=indptr[-1]).astype(np.int32)
    data = rng.random(indptr[-1]).astype(np.float32)
    ti, ts, T = engine.to_query_tensors(gpusparse.CSR(indptr, indices, data, (40, 100)), "cpu")
    ot, os_, oT = O.to_query_tensors(indptr, indices, data)
    assert T == oT and np.array_equal(ti.numpy(), ot) and np.array_equal(ts.numpy(), os_)


def test_run_file_format(tmp_path):
    res = [[("q1", 2.5, "dA"), ("q1", 1.0, "dB")], [], [("q3", 0.25, "dC")]]
    p = tmp_path / "run.txt.gz"
    engine.write_run(res, p)
    lines = gzip.open(p, "rt").read().splitlines()
    assert lines == ["q1 Q0 dA 1 2.5 gpusparse", "q1 Q0 dB 2 1.0 gpusparse", "q3 Q0 dC 1 0.25 gpusparse"]


def test_main_without_harness_raises():
    try:
        import lsr_benchmark  # noqa: F401
        pytest.skip("harness installed")
    except ImportError:
        pass
    with pytest.raises(ImportError):
        engine.main("ds", "emb", "out", 10)


def test_dropin_modules_import():
    import importlib
    import sys
    d = os.path.join(ROOT, "gpu-sparse_amd", "dropin")
    sys.path.insert(0, d)
    try:
        for m in ("triton_kernel", "triton_kernel_chunked", "fused_topk", "gpu_inverted_index",
                  "run_correctness_verification"):
            mod = importlib.import_module(m)
            assert mod.__file__.startswith(d)
        assert importlib.import_module("triton_kernel").triton_fused_score is gpusparse.triton_fused_score
    finally:
        sys.path.remove(d)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 ends with status 2 and a message,
    before anything touches a device."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and r.stdout == ""
