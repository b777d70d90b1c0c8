"""Timed CPU baseline: the reference CPU path on C pinned cores.  TEST / BENCH
INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg runs it; no product path).

The reference CPU path is cpu_sequential_score (src/gpu_scoring.py:221-259): per
query a float32 accumulator over all docs, `acc[doc] += w_q * w` over every
posting of every query term, then a top-k.  It runs here as the C restatement
orc_cpu_sequential (oracle/oracle_score.c), OpenMP over queries.

bench.py starts this file as a fresh child process that never touches a GPU:

    taskset -c <cpus> python3 oracle/cpu_baseline.py --dir D --cores C --k K --queries Q

with OMP/MKL/OPENBLAS/NUMEXPR/RAYON_NUM_THREADS = C in its environment before
the interpreter starts (the thread pinning the reference's CPU baselines use,
baselines/seismic_k_calibration.py:50-53,99-117).  D holds the host copy of the
index and the query batch as .npy files.  It prints one JSON line: wall
seconds, CPU seconds of the whole process (getrusage: every thread), their
ratio and queries/s, over the timed call only (loading is outside it).
"""
from __future__ import annotations

import argparse
import json
import os
import resource
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
if sys.path and os.path.abspath(sys.path[0] or ".") == HERE:  # run as a script: `oracle` is the package
    sys.path.pop(0)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import oracle as O  # noqa: E402

FILES = ("doc_ids", "scores", "offsets", "lengths", "q_terms", "q_weights")


def save_inputs(d: str, index_h: dict, q_terms: np.ndarray, q_weights: np.ndarray) -> None:
    """Writes what the child reads: the index's host arrays and the queries."""
    os.makedirs(d, exist_ok=True)
    arrays = {k: index_h[k] for k in FILES[:4]}
    arrays["q_terms"] = q_terms
    arrays["q_weights"] = q_weights
    for k, a in arrays.items():
        np.save(os.path.join(d, k + ".npy"), np.ascontiguousarray(a), allow_pickle=False)
    with open(os.path.join(d, "meta.json"), "w") as f:
        json.dump({"num_docs": int(index_h["num_docs"]), "vocab_size": int(index_h["vocab_size"])}, f)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--dir", required=True)
    ap.add_argument("--cores", type=int, required=True)
    ap.add_argument("--k", type=int, required=True)
    ap.add_argument("--queries", type=int, required=True)
    a = ap.parse_args()
    with open(os.path.join(a.dir, "meta.json")) as f:
        meta = json.load(f)
    ix = {k: np.load(os.path.join(a.dir, k + ".npy"), allow_pickle=False) for k in FILES}
    ix.update(meta)
    nq = min(a.queries, ix["q_terms"].shape[0])
    qt, qw = ix["q_terms"][:nq], ix["q_weights"][:nq]
    O.clib()
    r0 = resource.getrusage(resource.RUSAGE_SELF)
    t0 = time.perf_counter()
    O.c_cpu_sequential(ix, qt, qw, a.k, threads=a.cores)
    wall = time.perf_counter() - t0
    r1 = resource.getrusage(resource.RUSAGE_SELF)
    cpu_s = (r1.ru_utime - r0.ru_utime) + (r1.ru_stime - r0.ru_stime)
    print(json.dumps({"cores": a.cores, "queries": nq, "wall_s": round(wall, 3), "cpu_s": round(cpu_s, 3),
                      "cpu_wall_ratio": round(cpu_s / wall, 3) if wall > 0 else 0.0,
                      "qps": round(nq / wall, 3) if wall > 0 else 0.0,
                      "affinity": sorted(os.sched_getaffinity(0)),
                      "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}), flush=True)


if __name__ == "__main__":
    main()
