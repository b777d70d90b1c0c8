"""Committed golden vectors (tests/golden/golden.npz, written by
tests/golden/make_golden.py): the generator, the oracle and -- on a GPU -- the
HIP path must reproduce them exactly."""
import os

import numpy as np
import pytest
import torch

from gpusparse import synth
from gpusparse.index import CSR
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False)
VARIANTS = ("f32", "f16", "u8")
FIELDS = ("doc_ids", "scores", "offsets", "lengths", "padded_lengths", "max_scores")


def arr(v, name):
    return G[f"{v}/{name}"]


def same(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("v", VARIANTS)
def test_generator_reproduces_inputs(v):
    import make_golden as M  # noqa: E402  (tests/golden on sys.path below)
    docs = synth.generate_rows(M.replace(M.DOCS, weights=v), M.SEED, synth.STREAM_DOCS)
    assert same(docs.indptr, arr(v, "doc_indptr")) and same(docs.indices, arr(v, "doc_indices"))
    assert same(docs.data, arr(v, "doc_data"))


@pytest.mark.parametrize("v", VARIANTS)
def test_oracle_reproduces_outputs(v):
    ix = O.build_index(arr(v, "doc_indptr"), arr(v, "doc_indices"), arr(v, "doc_data"), 400, 1500)
    for f in FIELDS:
        assert same(ix[f], arr(v, "ix_" + f)), f
    cb = O.chunk_bounds(ix["doc_ids"], ix["offsets"], ix["lengths"], 1500, 400, 128)
    assert same(cb, arr(v, "chunk_bounds"))
    for k in (10, 400):
        s, i = O.search(ix, arr(v, "q_terms"), arr(v, "q_weights"), k)
        assert same(s, arr(v, f"top{k}_scores")) and same(i, arr(v, f"top{k}_ids"))
        cs, _, ci = O.c_search(ix, arr(v, "q_terms"), arr(v, "q_weights"), k, threads=2)
        assert same(cs, arr(v, f"top{k}_scores")) and same(ci, arr(v, f"top{k}_ids"))


@pytest.mark.gpu
@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("path", ["fused", "dense"])
def test_gpu_reproduces_outputs(device, v, path):
    import gpusparse as gs
    csr = CSR(arr(v, "doc_indptr"), arr(v, "doc_indices"), arr(v, "doc_data"), (400, 1500))
    ix = gs.build_from_csr(csr, device)
    for f in FIELDS:
        assert same(getattr(ix, f).cpu().numpy(), arr(v, "ix_" + f)), f
    assert same(gs.build_chunk_boundaries(ix, 128).cpu().numpy(), arr(v, "chunk_bounds"))
    q = (torch.from_numpy(arr(v, "q_terms")), torch.from_numpy(arr(v, "q_weights")))
    for k in (10, 400):
        s, i = gs.search(ix, q, k, path=path, tile_log2=8)
        assert same(s.cpu().numpy(), arr(v, f"top{k}_scores")) and same(i.cpu().numpy(), arr(v, f"top{k}_ids"))
