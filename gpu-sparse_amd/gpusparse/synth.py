"""Seeded synthetic SPLADE-like collections and query batches (csrc/synth.c).

The five configurations measured by this project (C1..C5).  Parameters the
workload description leaves open are fixed here and recorded in ``manifest``:
the lognormal sigma of row lengths (0.5, with mu chosen so the unclipped mean is
the stated mean), the C4 query length law and its forced head terms.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import asdict, dataclass, replace

import numpy as np

from . import _lib
from .index import CSR

VOCAB = 30522
W_MU, W_SIGMA, W_MAX = -0.5, 0.8, 3.0
WMODE = {"f32": 0, "f16": 1, "u8": 2}
STREAM_DOCS = 0x444F43
STREAM_QUERIES = 0x515259


@dataclass(frozen=True)
class RowSpec:
    n_rows: int
    zipf_s: float = 1.1
    nnz_mean: float = 120.0
    nnz_sigma: float = 0.5
    nnz_min: int = 16
    nnz_max: int = 512
    n_head_forced: int = 0
    head_pool: int = 0
    vocab: int = VOCAB
    weights: str = "f32"


@dataclass(frozen=True)
class Config:
    name: str
    docs: RowSpec
    queries: RowSpec
    k: int
    seed: int
    description: str


def _docs(n, s=1.1, w="f32"):
    return RowSpec(n_rows=n, zipf_s=s, weights=w)


def _queries(n, s=1.1, w="f32", mean=30.0, lo=4, hi=107, forced=0, pool=0):
    return RowSpec(n_rows=n, zipf_s=s, nnz_mean=mean, nnz_min=lo, nnz_max=hi, n_head_forced=forced,
                   head_pool=pool, weights=w)


CONFIGS = {
    "C1": Config("C1", _docs(100_000), _queries(256), 10, 101,
                 "CPU-runnable plumbing: 100K docs, 256 queries, fp32, top-10"),
    "C2": Config("C2", _docs(1_000_000), _queries(1024), 1000, 102,
                 "1M docs, 1024 queries, fp32 postings and accumulators, k=1000"),
    "C3": Config("C3", _docs(8_800_000, w="f16"), _queries(512), 1000, 103,
                 "8.8M docs, fp16 posting weights, fp32 accumulation, 512 queries, k=1000 (and k=10)"),
    "C4": Config("C4", _docs(1_000_000, s=1.3), _queries(512, s=1.3, mean=80.0, lo=16, hi=256, forced=8, pool=50),
                 1000, 104, "1M docs Zipf(1.3) head-heavy, 512 queries up to 256 terms with 8 of the top-50 "
                            "terms forced in, fp32, k=1000, tile sweep"),
    "C5": Config("C5", _docs(8_800_000, w="u8"), _queries(512, w="u8"), 1000, 105,
                 "8.8M docs, uint8 impacts round(w*255/3) (zeros dropped), uint8 query weights, uint32 sums, "
                 "512 queries, k=1000"),
}


def scaled(cfg: Config, n_docs: int | None = None, n_queries: int | None = None) -> Config:
    """The same generators at another size (parity tests use reduced sizes)."""
    d = cfg.docs if n_docs is None else replace(cfg.docs, n_rows=int(n_docs))
    q = cfg.queries if n_queries is None else replace(cfg.queries, n_rows=int(n_queries))
    return replace(cfg, docs=d, queries=q)


def _threads(n=None) -> int:
    if n:
        return int(n)
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(16, os.cpu_count() or 1))


def generate_rows(spec: RowSpec, seed: int, stream: int, threads: int | None = None) -> CSR:
    """CSR [n_rows, vocab] with ascending term ids per row."""
    L = _lib.synth_lib()
    sp = _lib.GsSynthSpec()
    sp.n_rows = spec.n_rows
    sp.vocab = spec.vocab
    sp.wmode = WMODE[spec.weights]
    sp.zipf_s = spec.zipf_s
    sp.nnz_mean = spec.nnz_mean
    sp.nnz_sigma = spec.nnz_sigma
    sp.nnz_min = spec.nnz_min
    sp.nnz_max = spec.nnz_max
    sp.w_mu, sp.w_sigma, sp.w_max = W_MU, W_SIGMA, W_MAX
    sp.n_head_forced = spec.n_head_forced
    sp.head_pool = spec.head_pool
    sp.seed = seed
    sp.stream = stream
    nt = _threads(threads)
    row_nnz = np.empty(spec.n_rows, dtype=np.int64)
    total = L.gs_synth_count(C.byref(sp), row_nnz.ctypes.data, nt)
    if total < 0:
        raise ValueError(f"bad synthetic spec {spec}")
    indptr = np.zeros(spec.n_rows + 1, dtype=np.int64)
    np.cumsum(row_nnz, out=indptr[1:])
    indices = np.empty(total, dtype=np.int32)
    dt = {"f32": np.float32, "f16": np.float16, "u8": np.uint8}[spec.weights]
    data = np.empty(total, dtype=dt)
    rc = L.gs_synth_fill(C.byref(sp), indptr.ctypes.data, indices.ctypes.data, data.ctypes.data, nt)
    if rc != 0:
        raise RuntimeError("synthetic generator failed")
    return CSR(indptr, indices, data, (spec.n_rows, spec.vocab))


def generate(cfg: Config | str, threads: int | None = None):
    """(doc CSR, query CSR) of a configuration."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    docs = generate_rows(cfg.docs, cfg.seed, STREAM_DOCS, threads)
    queries = generate_rows(cfg.queries, cfg.seed, STREAM_QUERIES, threads)
    return docs, queries


def manifest(cfg: Config | str) -> dict:
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    m = asdict(cfg)
    m["weights_law"] = f"min(lognormal(mu={W_MU}, sigma={W_SIGMA}), {W_MAX}) rounded to fp32"
    m["u8_code"] = "rint(float64(w_fp32) * 255 / 3), zero codes dropped"
    m["f16_code"] = "IEEE binary16 round-to-nearest-even of the fp32 weight"
    m["row_length_law"] = "clip(rint(exp(mu + sigma z)), min, max), mu = ln(mean) - sigma^2 / 2"
    m["term_law"] = "Zipf(s) ranks without replacement (i.i.d. draws, repeats rejected); term id = rank - 1"
    return m


def f32_to_f16_bits(x: np.ndarray, threads: int | None = None) -> np.ndarray:
    """Binary16 bits of fp32 values by the generator's converter (round to nearest even)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    _lib.synth_lib().gs_f32_to_f16_array(x.ctypes.data, out.ctypes.data, x.size, _threads(threads))
    return out


def quantize_u8(csr: CSR, w_max: float = W_MAX) -> CSR:
    """uint8 impacts rint(w * 255 / w_max) (half to even) with zero codes dropped."""
    q = np.rint(csr.data.astype(np.float64) * 255.0 / w_max)
    q = np.clip(q, 0, 255).astype(np.uint8)
    keep = q != 0
    rows = np.repeat(np.arange(csr.shape[0]), np.diff(csr.indptr))[keep]
    indptr = np.zeros(csr.shape[0] + 1, dtype=np.int64)
    np.cumsum(np.bincount(rows, minlength=csr.shape[0]), out=indptr[1:])
    return CSR(indptr, csr.indices[keep].astype(np.int32), q[keep], csr.shape)
