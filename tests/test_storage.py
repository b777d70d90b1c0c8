"""On-disk index format: round trips and rejection of damaged files (CPU), and a
GPU round trip that searches the loaded index."""
import os

import numpy as np
import pytest
import torch

import gpusparse as gs
from gpusparse import storage
from gpusparse.index import GPUInvertedIndex
from helpers import random_csr
from oracle import oracle as O


def cpu_index(seed=0, n_docs=300, vocab=50, dtype=np.float32):
    csr = random_csr(np.random.default_rng(seed), n_docs, vocab, dtype=dtype, dup_rate=0.1)
    ref = O.build_index(csr.indptr, csr.indices, csr.data, n_docs, vocab)
    t = {k: torch.from_numpy(np.ascontiguousarray(ref[k])) for k in
         ("doc_ids", "scores", "offsets", "lengths", "padded_lengths", "max_scores")}
    return GPUInvertedIndex(num_docs=n_docs, vocab_size=vocab, device=torch.device("cpu"), **t), ref


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.uint8])
def test_round_trip_is_bit_exact(tmp_path, dtype):
    ix, ref = cpu_index(dtype=dtype)
    p = str(tmp_path / "ix.gsp")
    meta = gs.save_index(ix, p)
    assert meta["weights"] == np.dtype(dtype).name
    for e in meta["arrays"]:
        assert e["offset"] % storage.ALIGN == 0
    back = gs.load_index(p, "cpu", verify=True)
    assert back.num_docs == ix.num_docs and back.vocab_size == ix.vocab_size
    for f in ("doc_ids", "scores", "offsets", "lengths", "padded_lengths", "max_scores"):
        a, b = getattr(ix, f), getattr(back, f)
        assert a.dtype == b.dtype and a.numpy().tobytes() == b.numpy().tobytes(), f


def test_rejects_damaged_files(tmp_path):
    ix, _ = cpu_index()
    p = str(tmp_path / "ix.gsp")
    gs.save_index(ix, p)
    raw = open(p, "rb").read()
    bad = str(tmp_path / "bad.gsp")
    open(bad, "wb").write(b"XXXXXXXX" + raw[8:])
    with pytest.raises(ValueError, match="bad magic"):
        gs.load_index(bad, "cpu")
    open(bad, "wb").write(raw[: len(raw) - 4096])
    with pytest.raises(ValueError, match="outside the file"):
        gs.load_index(bad, "cpu")
    # flip one byte of the doc ids: caught by the CRC-32 check
    meta = storage.read_header(p)
    off = meta["arrays"][0]["offset"]
    flipped = bytearray(raw)
    flipped[off] ^= 0x40
    open(bad, "wb").write(bytes(flipped))
    with pytest.raises(ValueError, match="CRC-32"):
        gs.load_index(bad, "cpu", verify=True)
    # a list pointing past the slot arrays is refused before any device copy
    arrs = {e["name"]: e for e in meta["arrays"]}
    o = arrs["offsets"]["offset"]
    broken = bytearray(raw)
    broken[o:o + 8] = np.int64(1 << 40).tobytes()
    open(bad, "wb").write(bytes(broken))
    with pytest.raises(ValueError, match="outside the slot arrays"):
        gs.load_index(bad, "cpu")


@pytest.mark.gpu
def test_gpu_round_trip_searches_identically(device, tmp_path):
    from gpusparse import synth
    cfg = synth.scaled(synth.CONFIGS["C1"], n_docs=60_000, n_queries=16)
    docs, queries = synth.generate(cfg)
    ix = gs.build_from_csr(docs, device)
    p = str(tmp_path / "c1.gsp")
    gs.save_index(ix, p, forward=True)
    back = gs.load_index(p, device, verify=True)
    assert "fwd" in back.aux()
    ti, tw, _ = O.to_query_tensors(queries.indptr, queries.indices, queries.data)
    q = (torch.from_numpy(ti), torch.from_numpy(tw))
    s1, i1 = gs.search(ix, q, 100, path="fused")
    s2, i2 = gs.search(back, q, 100, path="fused")
    assert torch.equal(i1, i2) and torch.equal(s1, s2)
    fwd = [t.cpu().numpy() for t in ix.aux()["fwd"]]
    nnz = int(fwd[0][-1])
    got = [t.cpu().numpy() for t in back.aux()["fwd"]]
    assert np.array_equal(fwd[0], got[0]) and np.array_equal(fwd[1][:nnz], got[1])
    assert fwd[2][:nnz].tobytes() == got[2].tobytes()
    os.remove(p)
