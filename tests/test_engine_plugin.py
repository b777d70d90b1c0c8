"""The plug-in entry point end to end (lsr_benchmark_engine/gpusparse_retrieval.py:
175-222) on offline stand-ins for the TIRA harness (tests/harness_stubs/).

Golden: tests/golden/engine_run.txt, the TREC run of tests/golden/
engine_embeddings.npz at k = 10, written by tests/golden/make_golden.py from a
brute-force ranking that uses neither the oracle nor the library."""
import gzip
import importlib
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
STUBS = os.path.join(HERE, "harness_stubs")
FIXTURE = os.path.join(HERE, "golden", "engine_embeddings.npz")
K = 10
STUB_MODULES = ("lsr_benchmark", "lsr_benchmark.click", "lsr_benchmark.irds", "tirex_tracker")


def golden_lines():
    with open(os.path.join(HERE, "golden", "engine_run.txt")) as f:
        return f.read().splitlines()


def fixture_embeddings():
    sys.path.insert(0, STUBS)
    try:
        irds = importlib.import_module("lsr_benchmark.irds")
        return irds.embeddings(FIXTURE, "stub", "doc"), irds.embeddings(FIXTURE, "stub", "query")
    finally:
        sys.path.remove(STUBS)
        for m in STUB_MODULES:
            sys.modules.pop(m, None)


@pytest.fixture
def harness():
    """gpusparse.engine re-imported with the stand-ins importable, so that its
    `main` is bound through lsr_benchmark.click.retrieve_command as in the
    reference; afterwards the stand-ins are removed and engine re-imported."""
    import gpusparse.engine as engine
    sys.path.insert(0, STUBS)
    try:
        eng = importlib.reload(engine)
        yield eng
    finally:
        sys.path.remove(STUBS)
        for m in STUB_MODULES:
            sys.modules.pop(m, None)
        importlib.reload(engine)


def test_main_binds_to_the_harness_command(harness):
    assert harness.main.__wrapped__ is harness._main


def test_main_without_gpu_raises_runtime_error(harness, tmp_path):
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU visible")
    with pytest.raises(RuntimeError, match="requires a GPU"):
        harness.main(FIXTURE, "stub", str(tmp_path / "out"), K)


def test_oracle_rankings_reproduce_golden_run():
    """Pins oracle.rankings (and the host formatting functions) against the
    independent brute-force run."""
    from gpusparse import engine
    docs, queries = fixture_embeddings()
    dim = engine.determine_dimension(docs, queries)
    doc_ids, dcsr = engine.to_csr(docs, dim)
    q_ids, qcsr = engine.to_csr(queries, dim)
    ix = O.build_index(dcsr.indptr, dcsr.indices, dcsr.data, dcsr.shape[0], dim)
    ti, tw, _ = O.to_query_tensors(qcsr.indptr, qcsr.indices, qcsr.data)
    vs, _, vi = O.c_search(ix, ti, tw, K, threads=2)
    ranked = O.rankings(q_ids, vs, vi, doc_ids, K)
    lines = [f"{qid} Q0 {docno} {r} {score} gpusparse"
             for rk in ranked for r, (qid, score, docno) in enumerate(rk, start=1)]
    assert lines == golden_lines()


@pytest.mark.gpu
def test_main_writes_the_golden_run(harness, device, tmp_path):
    out = tmp_path / "out"
    print("plug-in main on the engine fixture, k=10", flush=True)
    harness.main(FIXTURE, "stub-splade", str(out), K)
    with gzip.open(out / "run.txt.gz", "rt") as f:
        lines = f.read().splitlines()
    assert lines == golden_lines()
    assert (out / "index-metadata.yml").exists() and (out / "retrieval-metadata.yml").exists()
    import lsr_benchmark
    import tirex_tracker
    assert lsr_benchmark.REGISTERED[-1] == FIXTURE
    assert tirex_tracker.METADATA[-1]["tag"] == f"gpusparse-stub-splade-{K}"


@pytest.mark.gpu
@pytest.mark.parametrize("doc_chunk,batch_size", [(131072, 200), (64, 7)])
def test_retrieve_reproduces_golden_run(device, tmp_path, doc_chunk, batch_size):
    """retrieve on both of its paths: monolithic (collection within one chunk)
    and chunked with chunk bounds (triton_chunked_score_fused)."""
    from gpusparse import engine
    print(f"retrieve doc_chunk={doc_chunk} batch_size={batch_size}", flush=True)
    docs, queries = fixture_embeddings()
    dim = engine.determine_dimension(docs, queries)
    doc_ids, dcsr = engine.to_csr(docs, dim)
    index = engine.build_index(dcsr, device)
    assert index.scores.dtype.is_floating_point and index.scores.element_size() == 4
    q_ids, qcsr = engine.to_csr(queries, dim)
    q_ti, q_ts, _ = engine.to_query_tensors(qcsr, device)
    res = engine.retrieve(index, q_ids, q_ti, q_ts, doc_ids, K, batch_size=batch_size, doc_chunk=doc_chunk)
    engine.write_run(res, tmp_path / "run.txt.gz")
    with gzip.open(tmp_path / "run.txt.gz", "rt") as f:
        assert f.read().splitlines() == golden_lines()
    assert np.sum([len(r) for r in res]) == len(golden_lines())
