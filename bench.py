"""Benchmark of the exact SPLADE search path on one MI355X.

Default workload (the headline metric): config C3 -- 8.8M synthetic docs
(~1.06e9 postings, fp16 posting weights, fp32 accumulation), batches of 512
queries, k = 1000.  A step is one ``search`` of one 512-query batch: the heavy
terms' coarse sums (int8 matrix products), LDS-tile scoring of the other terms
with threshold selection, candidate selection, fp64 rescoring and the status
check.  Inputs (index and query batch) are resident in HBM before the timed
region.

Prints one JSON line.  ``value`` is queries/s with the results left in HBM (as
the reference's benchmarks time it); ``queries_per_s_incl_d2h`` adds the
hand-over of each batch's [B, k] scores and ids to host memory.  ``roofline`` is
for the dominant kernel (the fused tile scoring kernel), timed with HIP events
on its launch stream.  Its unit of work is one scored posting of a term added in
LDS (a (query, posting) pair), which is one LDS atomic add, and its bound is the
LDS atomic rate measured on the same GPU type (profiles/lds_atomic_rates.json).
Beside it: the physical HBM bytes per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE,
calibrated by a copy kernel; profiles/traffic_k_score_union_[hybrid_]<config>.json) as a
fraction of 8 TB/s, and the reference kernel's stream (4 B doc id + weight bytes
per scored posting) as a labelled equivalent.  With the hybrid search (the 64
heaviest terms as int8 matrix products) ``heavy_terms_kernel`` gives that
kernel's HBM and MFMA fractions.  ``selection`` and ``index_build`` give bytes
moved over time for candidate selection + fp64 rescoring + final sort, and for
the device index build.  ``cpu_baseline`` times the reference CPU path
(cpu_sequential_score, restated in C) on a bounded sample of the same batch in
fresh child processes pinned with taskset and the thread-pool variables.
``workloads`` holds, from the same run, C3 at B = 16, 64, 256 and 1024, C3 at
k = 10, and C5 (uint8) at B = 512 (measured by a child bench.py process); with
the CPU leg the whole batch of the headline, of k = 10 and of C5 is checked
against the C oracle.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "gpu-sparse_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "queries/s @8.8M docs k=1000 batch 512; scoring HBM GB/s as % of peak"
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=15)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C3")
    ap.add_argument("--n-docs", type=int, default=None, help="override the config's collection size")
    ap.add_argument("--batch", type=int, default=0, help="queries per batch (0: the config's)")
    ap.add_argument("--k", type=int, default=0, help="top-k (0: the config's)")
    ap.add_argument("--tile-log2", type=int, default=0, help="doc tile size, log2 (0: the library default)")
    ap.add_argument("--unroll", type=int, default=0, help="postings per lane per chunk (0: library default)")
    ap.add_argument("--waves", type=int, default=0)
    ap.add_argument("--tiles-per-wg", type=int, default=0, help="tiles walked by one scoring workgroup (0: default)")
    ap.add_argument("--sample-tiles", type=int, default=0, help="tiles scored with tau = 0 first (0: default)")
    ap.add_argument("--cpu-queries-1", type=int, default=96, help="queries timed on one core")
    ap.add_argument("--cpu-queries-all", type=int, default=512, help="queries timed on all cores")
    ap.add_argument("--cpu-cores", type=int, default=16,
                    help="cap on the cores of the all-core row, which takes every core of the process's "
                         "affinity up to this cap (the GPU boxes give a process 16 CPUs, one GPU's share of "
                         "the host; the JSON records the affinity beside the cores used)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--parity-queries", type=int, default=None,
                    help="queries of the batch checked against the C oracle (default: the whole batch when the "
                         "CPU leg runs, else 4)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the extra workloads (batch curve, k = 10, C5) after the headline")
    ap.add_argument("--path", default="fused", choices=["fused", "dense", "atomic"])
    ap.add_argument("--scorer", default="auto", choices=["auto", "hybrid", "lds"],
                    help="fused scorer: hybrid (heavy terms as int8 MFMA products, 16384-doc tiles), lds (LDS adds "
                         "for every term) or auto (hybrid when the index allows it and no tile size is named)")
    ap.add_argument("--inflight", type=int, default=2,
                    help="batches in flight: batch i is queued before batch i - D's status is read (1: one at a time)")
    ap.add_argument("--streams", type=int, default=1,
                    help="streams the batches in flight take in turn (at most --inflight; 1: all on one stream, "
                         "so their kernels run one after another)")
    ap.add_argument("--summarize-traffic", default=None, metavar="DIR",
                    help="write profiles/traffic_k_score_union_[hybrid_]<config>.json from rocprofv3 --pmc "
                         "runs under DIR")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run a plain device-to-device copy of this many bytes (PMC counter calibration)")
    return ap.parse_args()


def lds_peak():
    """Measured LDS atomic rate of the MI355X (profiles/lds_atomic_rates.json,
    written by gpu-sparse_amd/csrc/microbench/lds_atomic_rate.hip): ds_add_u32 on
    random addresses of a 64 KiB workgroup allocation, in lane-adds/s over the
    whole GPU.  None when the file is missing."""
    path = os.path.join(ROOT, "profiles", "lds_atomic_rates.json")
    try:
        with open(path) as f:
            r = json.load(f)
    except (OSError, ValueError):
        return None
    return {"peak": float(r["ds_add_u32_random"]["lane_ops_per_s"]),
            "conflict_free": float(r["ds_add_u32_conflict_free"]["lane_ops_per_s"]),
            "source": os.path.relpath(path, ROOT) + ": ds_add_u32, random addresses"}


def traffic_file(cfg_name, hybrid=False):
    """The committed traffic measurement of one configuration and scorer."""
    return os.path.join(ROOT, "profiles", f"traffic_k_score_union_{'hybrid_' if hybrid else ''}{cfg_name}.json")


def measured_traffic(cfg_name, n_docs, tile_log2, hybrid, batch, k):
    """The committed rocprofv3 PMC measurement of this workload (HBM bytes per
    launch of the fused scorer and, for the hybrid search, of the heavy-term
    kernel: FETCH_SIZE + WRITE_SIZE scaled by a copy kernel of known size), when
    it was taken on this workload (collection, tile size, batch size, k) and
    scorer; None otherwise."""
    try:
        with open(traffic_file(cfg_name, hybrid)) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("config") != cfg_name or t.get("n_docs") != n_docs or t.get("tile_log2") != tile_log2 or \
            bool(t.get("hybrid", False)) != bool(hybrid) or t.get("batch") != batch or t.get("k") != k:
        return None
    return t


def summarize_traffic(d, cfg_name, n_docs, tile_log2, copy_bytes):
    """Writes the traffic file from four rocprofv3 --pmc runs under `d`: f/ and w/
    (FETCH_SIZE, WRITE_SIZE of this benchmark), cf/ and cw/ (the same counters over
    ``--copy-bytes`` copies).  Each counter is scaled by bytes copied / counter
    value of the last copy dispatch; values are KiB per dispatch, summed over
    the counter's instances, last dispatch of the kernel."""
    import csv
    import glob

    def last(sub, name, required=True):
        rows = {}
        for path in glob.glob(os.path.join(d, sub, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                if name in r["Kernel_Name"]:
                    did = int(r["Dispatch_Id"])
                    rows[did] = rows.get(did, 0.0) + float(r["Counter_Value"])
        if not rows:
            if not required:
                return None
            raise SystemExit(f"no {name} dispatch under {os.path.join(d, sub)}")
        return rows[max(rows)]

    def dispatches(sub, names):
        rows = {}
        for path in glob.glob(os.path.join(d, sub, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                if any(n in r["Kernel_Name"] for n in names):
                    did = int(r["Dispatch_Id"])
                    name = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
                    rows.setdefault(did, [name, 0.0])[1] += float(r["Counter_Value"])
        return [rows[k] for k in sorted(rows)]

    f, w = last("f", "k_score_union"), last("w", "k_score_union")
    cf, cw = last("cf", "copyBuffer"), last("cw", "copyBuffer")
    fs, ws = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)
    # the hybrid search's heavy-term kernel, when the profiled run took it (then
    # at the hybrid search's default tile, unless one was named)
    hf, hw = last("f", "k_head_scores", False), last("w", "k_head_scores", False)
    hybrid = hf is not None and hw is not None
    if tile_log2 is None:
        from gpusparse.index import DEFAULT_TILE_LOG2_HYBRID, DEFAULT_TILE_LOG2_PACKED
        tile_log2 = DEFAULT_TILE_LOG2_HYBRID if hybrid else DEFAULT_TILE_LOG2_PACKED
    # the radix passes of the index build (term keys) and of the doc-major copy
    # (doc-id keys), in launch order: a histogram, then a scatter, per pass
    rf, rw = dispatches("f", ("k_rs_hist", "k_rs_scatter")), dispatches("w", ("k_rs_hist", "k_rs_scatter"))
    radix = [{"kernel": a[0], "fetch_bytes": round(a[1] * 1024 * fs), "write_bytes": round(b[1] * 1024 * ws)}
             for a, b in zip(rf, rw) if a[0] == b[0]]
    from gpusparse import synth
    out = {"config": cfg_name, "n_docs": n_docs, "tile_log2": tile_log2, "kernel": "k_score_union",
           "hybrid": hybrid, "batch": synth.CONFIGS[cfg_name].queries.n_rows, "k": synth.CONFIGS[cfg_name].k,
           "fetch_kib_per_launch": f, "write_kib_per_launch": w, "copy_bytes": copy_bytes,
           "copy_fetch_kib": cf, "copy_write_kib": cw, "fetch_scale": fs, "write_scale": ws,
           "fetch_bytes_per_launch": f * 1024 * fs, "write_bytes_per_launch": w * 1024 * ws,
           "traffic_bytes_per_launch": f * 1024 * fs + w * 1024 * ws,
           "head_kernel": "k_head_scores" if hybrid else None,
           "head_fetch_bytes_per_launch": hf * 1024 * fs if hybrid else None,
           "head_write_bytes_per_launch": hw * 1024 * ws if hybrid else None,
           "head_traffic_bytes_per_launch": hf * 1024 * fs + hw * 1024 * ws if hybrid else None,
           "radix_dispatches": radix,
           "commands": [
               f"rocprofv3 --pmc FETCH_SIZE -d <out>/f -o f --output-format csv -- python3 bench.py --config {cfg_name} "
               "--no-cpu --no-extra --parity-queries 0 --steps 1 --warmup 1",
               f"rocprofv3 --pmc WRITE_SIZE -d <out>/w -o w --output-format csv -- python3 bench.py --config {cfg_name} "
               "--no-cpu --no-extra --parity-queries 0 --steps 1 --warmup 1",
               f"rocprofv3 --pmc FETCH_SIZE -d <out>/cf -o cf --output-format csv -- python3 bench.py --copy-bytes {copy_bytes}",
               f"rocprofv3 --pmc WRITE_SIZE -d <out>/cw -o cw --output-format csv -- python3 bench.py --copy-bytes {copy_bytes}",
               f"python3 bench.py --config {cfg_name} --summarize-traffic <out>"]}
    with open(traffic_file(cfg_name, hybrid), "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out), flush=True)


def copy_only(nbytes):
    """A plain copy kernel of known size: the calibration of FETCH_SIZE / WRITE_SIZE."""
    import torch
    n = nbytes // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n * 4, "launches": 3}), flush=True)


THREAD_VARS = ("OMP_NUM_THREADS", "MKL_NUM_THREADS", "OPENBLAS_NUM_THREADS", "NUMEXPR_NUM_THREADS",
               "RAYON_NUM_THREADS")


def cpu_rows(index_h, ti, tw, k, n1, n_all, cap):
    """Reference CPU path (cpu_sequential_score restated in C) on one core and on
    min(cores in this process's affinity, cap) cores.  Each row is a fresh child
    process, ``taskset -c <cpus> python3 oracle/cpu_baseline.py``, with the
    thread-pool variables set in its environment before it starts; it never
    touches the GPU.  The index and queries reach it as .npy files in a
    temporary directory (/dev/shm when it has room)."""
    import shutil
    import subprocess
    import tempfile

    from oracle.cpu_baseline import save_inputs
    allowed = sorted(os.sched_getaffinity(0))
    need = sum(index_h[f].nbytes for f in ("doc_ids", "scores", "offsets", "lengths")) + ti.nbytes + tw.nbytes
    parent = "/dev/shm" if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > 2 * need else None
    d = tempfile.mkdtemp(prefix="gs_cpu_", dir=parent)
    rows = []
    try:
        save_inputs(d, index_h, ti, tw)
        for cores, nq in ((1, n1), (min(cap, len(allowed)), n_all)):
            if nq <= 0:
                continue
            cpus = ",".join(str(c) for c in allowed[:cores])
            env = dict(os.environ)
            env.update({v: str(cores) for v in THREAD_VARS})
            cmd = ["taskset", "-c", cpus, sys.executable, os.path.join(ROOT, "oracle", "cpu_baseline.py"),
                   "--dir", d, "--cores", str(cores), "--k", str(k), "--queries", str(nq)]
            r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
            if r.returncode != 0:
                raise RuntimeError(f"CPU baseline child failed ({r.returncode}): {r.stderr[-2000:]}")
            row = json.loads(r.stdout.strip().splitlines()[-1])
            row["pinned_cpus"] = row.pop("affinity")
            row["pinning_clean"] = bool(row["cpu_wall_ratio"] < 1.35 * cores and len(row["pinned_cpus"]) == cores)
            row["command"] = f"{' '.join(f'{v}={cores}' for v in THREAD_VARS)} taskset -c {cpus} " \
                             f"python3 oracle/cpu_baseline.py --cores {cores} --k {k} --queries {row['queries']}"
            rows.append(row)
            log(f"cpu baseline cores={cores} queries={row['queries']} wall={row['wall_s']:.2f}s "
                f"cpu/wall={row['cpu_wall_ratio']:.2f} q/s={row['qps']:.2f}")
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return rows, len(allowed)




# Published fused-path latencies of the reference at 8.84M docs, k = 1000, on one
# H100 (final_results/corrected_2026_08/fused_topk_8m.json:3-32): context for the
# batch curve only (other hardware, other data)
REFERENCE_FUSED_MS = {16: 26.67, 64: 37.07, 256: 131.82}
CURVE_BATCHES = (16, 64, 256, 1024)
HEAD_BLOCK = 512       # docs per block of the heavy-term kernel (GS_HEAD_BLOCK)
PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, TOP/s


def phase_matrix(timing):
    """[calls, phases] milliseconds of the library's per-phase events."""
    import numpy as np
    return np.array([[ev[i].elapsed_time(ev[i + 1]) for i in range(len(ev) - 1)] for ev in timing["phases"]])


def time_search(a, index, qt, qw, k, hyb, depth, n_streams):
    """Times a.steps searches of one batch resident in HBM, with `depth` batches
    in flight over n_streams streams, after a.warmup untimed ones; then the same
    batches one at a time (a batch's own latency), and the hand-over of one
    batch's [B, k] scores and ids to pinned host memory (what retrieve does after
    each batch, gpusparse_retrieval.py:166-167), timed on its own."""
    import torch

    import gpusparse as gs

    def step_async(timing=None):
        if a.path == "atomic":
            return gs.PendingSearch(gs.atomic_fused_score(index, qt, qw, k))
        return gs.search_async(index, (qt, qw), k, tile_log2=a.tile_log2, path=a.path, unroll=a.unroll,
                               waves=a.waves, tiles_per_wg=a.tiles_per_wg, sample_tiles=a.sample_tiles,
                               timing=timing, hybrid=hyb)

    # Batch i is queued on stream i mod S once batch i - D has finished (its
    # status read and any flagged rows completed), so up to D batches are in
    # flight.  D = 1 runs them one at a time; with S = 1 the batches in flight
    # share one stream, so only the host's work (the next batch's launches, the
    # previous one's status read) overlaps the GPU's.
    streams = [torch.cuda.current_stream()] + [torch.cuda.Stream() for _ in range(max(1, n_streams) - 1)]
    for st in streams[1:]:
        st.wait_stream(streams[0])

    def run_steps(n, timing=None):
        pend, out = [], None
        for i in range(n):
            if len(pend) == depth:
                out = pend.pop(0).result()
            with torch.cuda.stream(streams[i % len(streams)]):
                pend.append(step_async(timing))
        for p in pend:
            out = p.result()
        return out

    run_steps(max(a.warmup, depth))
    # Events are created before the timed region.  Kernel and phase times come
    # from kernels that do not overlap: from the timed steps on one stream, else
    # from the second pass with one batch at a time.
    timing = gs.timing_dict(a.steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = run_steps(a.steps, timing if len(streams) == 1 else None)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    one_ms = None
    if depth > 1:
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(a.steps):
            step_async(timing if len(streams) > 1 else None).result()
        torch.cuda.synchronize()
        one_ms = 1000.0 * (time.perf_counter() - t1) / a.steps
    hs = torch.empty(out[0].shape, dtype=out[0].dtype, pin_memory=True)
    hi = torch.empty(out[1].shape, dtype=out[1].dtype, pin_memory=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(a.steps):
        hs.copy_(out[0], non_blocking=True)
        hi.copy_(out[1], non_blocking=True)
        torch.cuda.synchronize()
    d2h_ms = 1000.0 * (time.perf_counter() - t1) / a.steps
    B = qt.shape[0]
    return {"B": B, "k": k, "ms_per_step": 1000.0 * wall / a.steps, "qps": B * a.steps / wall, "one_ms": one_ms,
            "d2h_ms": d2h_ms, "timing": timing, "out": out, "depth": depth, "streams": len(streams)}


def scorer_roofline(a, index, qt, T, k, hyb, timing, cfg_name):
    """(roofline of the fused LDS scoring kernel, plan, roofline of the heavy-term
    kernel or None).

    LDS-only search: the scorer's unit of work is one LDS atomic add, one scored
    posting (a (query, posting) pair of a valid query term), so the LDS-atomic
    issue rate bounds it, not HBM (each posting is fetched once per doc tile and
    query group and added to every query of the group holding its term).
    Hybrid search: the heavy terms' part of every (query, doc) sum arrives as a
    12-bit coarse sum, and the other ("tail") terms are added in LDS, about a
    tenth of the scored postings.  The scorer then streams its inputs: per
    launch it reads the coarse sums of its tiles (1.5 B per (query, doc)) and, per
    query group and tile, the packed words of the group's tail terms (4 B per
    posting and group holding the term); those algorithmic bytes over its time,
    against the HBM peak, are its roofline, with the LDS-atomic rate of its adds
    beside it.  The heavy-term kernel reads the heavy terms' int8 doc rows (128 B
    per doc) once and writes one 12-bit coarse sum per (query slot, doc):
    HBM-bound; its int8 MFMA work (4 limb products of the heavy terms per (slot,
    doc)) is given beside it."""
    import numpy as np

    import gpusparse as gs
    from gpusparse import _lib
    from gpusparse.search import search_index
    B = qt.shape[0]
    kern_ms = [e0.elapsed_time(e1) for e0, e1 in timing["score_kernel"]]
    call_ms = [e0.elapsed_time(e1) for e0, e1 in timing["search"]]
    N = int(index.num_docs)
    n_tiles = (N + (1 << a.tile_log2) - 1) >> a.tile_log2
    # the main launch scores the tiles after the seed tiles
    plan = gs.search_plan(index, B, T, k, tile_log2=a.tile_log2, sample_tiles=a.sample_tiles, unroll=a.unroll,
                          tiles_per_wg=a.tiles_per_wg, hybrid=hyb)
    S = min(plan["seed_tiles"], n_tiles)
    sidx = search_index(index, plan["hybrid"])  # a uint8 index's hybrid search runs on its float16 copy
    tb = sidx.aux()[("tile_bounds", a.tile_log2)]
    cols = tb[:, [S, n_tiles]].cpu().numpy().astype(np.int64)
    per_term = cols[:, 1] - cols[:, 0]
    all_term = index.lengths.cpu().numpy().astype(np.int64)
    qt_h = qt.cpu().numpy()
    valid = (qt_h >= 0) & (qt_h < index.vocab_size)
    tq = np.where(valid, qt_h, 0)
    heavy = np.zeros(int(index.vocab_size), dtype=bool)
    if plan["hybrid"]:
        heavy[sidx.aux()["heavy"].cpu().numpy()] = True
    in_lds = valid & ~heavy[tq]
    post_launch = int((per_term[tq] * in_lds).sum())
    post_tiles = int((per_term[tq] * valid).sum())
    post_all = int((all_term[tq] * valid).sum())
    wbytes = index.scores.element_size()
    per_post = 4 + wbytes
    avg_ms = float(np.mean(kern_ms))
    adds_per_s = post_launch / (avg_ms * 1e-3)
    lds = lds_peak()
    tr = measured_traffic(cfg_name, N, a.tile_log2, plan["hybrid"], int(qt.shape[0]), k)
    phys = None if tr is None else tr.get("traffic_bytes_per_launch")
    # the hybrid scorer's algorithmic bytes: coarse sums of the main launch's
    # tiles, and the tail words once per (group of consecutive queries, term)
    docs_main = max(0, min(N, n_tiles << a.tile_log2) - (S << a.tile_log2))
    G = plan["group_size"]
    word_reads = 0
    for g0 in range(0, B, G):
        t = qt_h[g0:g0 + G][in_lds[g0:g0 + G]]
        word_reads += int(per_term[np.unique(t)].sum())
    coarse_bytes = 3 * B * docs_main // 2  # 12 bits per (query, doc)
    hd_bytes = coarse_bytes + 4 * word_reads
    head = None
    head_ms = 0.0
    if plan["hybrid"] and timing.get("phases"):
        head_ms = float(np.median(phase_matrix(timing)[:, 1]))  # the heavy_terms phase: k_head_scores alone
        Bpad = (B + 15) // 16 * 16
        rows = (N + HEAD_BLOCK - 1) // HEAD_BLOCK * HEAD_BLOCK
        cols_h = ((n_tiles << a.tile_log2) + HEAD_BLOCK - 1) // HEAD_BLOCK * HEAD_BLOCK
        n_heavy = _lib.heavy_term_count()  # lists taken as int8 matrix products
        hbytes = rows * 2 * n_heavy + Bpad * cols_h * 3 // 2 + Bpad * 2 * n_heavy + B * 4
        ops = 4 * 2 * n_heavy * Bpad * rows
        hphys = None if tr is None else tr.get("head_traffic_bytes_per_launch")
        head = {"kernel": f"k_head_scores (the {n_heavy} heavy terms as int8 MFMA limb products; 12-bit coarse sums "
                          "written block-major, the LDS slices' start)",
                "bound": "hbm", "achieved": round(hbytes / (head_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(hbytes / (head_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                "bytes_per_launch": hbytes, "traffic": hphys,
                "bytes_note": "algorithmic: heavy int8 doc rows read once (128 B per doc) + one 12-bit coarse sum "
                              "(1.5 B) written per (query slot, doc) + query limbs",
                "ms": round(head_ms, 3),
                "mfma_int8": {"ops_per_launch": ops, "achieved": round(ops / (head_ms * 1e-3) / 1e12, 1),
                              "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                              "frac": round(ops / (head_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)}}
    ref_bytes = post_tiles * per_post
    ref_ms = avg_ms + head_ms
    lds_roof = {"bound": "lds_atomic", "achieved": round(adds_per_s / 1e9, 1),
                "peak": None if lds is None else round(lds["peak"] / 1e9, 1),
                "unit": "G LDS atomic adds/s (one per scored posting of a term added in LDS)",
                "frac": None if lds is None else round(adds_per_s / lds["peak"], 4),
                "peak_source": None if lds is None else lds["source"],
                # the packed copy's bank-aware order brings the adds close to the
                # conflict-free rate, the higher ceiling
                "frac_of_conflict_free_rate": None if lds is None else round(adds_per_s / lds["conflict_free"], 4)}
    if plan["hybrid"]:
        roof = {"bound": "hbm", "achieved": round(hd_bytes / (avg_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(hd_bytes / (avg_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                "traffic": phys, "bytes_per_launch": hd_bytes,
                "bytes_note": "algorithmic: 12-bit coarse heavy-term sum (1.5 B) per (query, doc) of the launch's "
                              f"tiles ({coarse_bytes} B) + 4 B packed word per tail posting and group holding its "
                              f"term ({4 * word_reads} B)",
                "lds_atomic": lds_roof}
    else:
        roof = dict(lds_roof, traffic=phys)
    roof.update({
            "hbm_physical": None if phys is None else {
                "achieved": round(phys / (avg_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(phys / (avg_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                "source": os.path.relpath(traffic_file(cfg_name, plan["hybrid"]), ROOT)},
            "reference_stream_equiv": {
                "bytes_per_launch": ref_bytes, "bytes_per_posting": per_post,
                "GBs": round(ref_bytes / (ref_ms * 1e-3) / 1e9, 1),
                "x_hbm_peak": round(ref_bytes / (ref_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 3),
                "note": "the reference kernel's stream (each posting of the main launch's tiles read once per "
                        "(query, term): doc id + weight) over the scoring kernels' time (LDS scorer + heavy-term "
                        "kernel); here each posting is read once per (doc tile, query group), so this is not a "
                        "fraction of any hardware peak"},
            "kernel": "k_score_union (fused group-tile LDS scoring + threshold emission"
                      + (", slices started from the heavy-term sums)" if plan["hybrid"] else ")"),
            "kernel_ms_avg": round(avg_ms, 3), "kernel_ms_median": round(float(np.median(kern_ms)), 3),
            "kernel_ms_min": round(float(np.min(kern_ms)), 3),
            "scored_postings_per_launch": post_launch, "postings_in_launch_tiles": post_tiles,
            "search_call_ms_avg": round(float(np.mean(call_ms)), 3),
            "batch_scored_postings": post_all})
    return roof, plan, head


def components_of(timing):
    """Median per-phase milliseconds of gs_search (HIP events the library records
    on its launch stream) over the timed steps."""
    import numpy as np

    from gpusparse import _lib
    per = phase_matrix(timing)
    comp = {name: round(float(np.median(per[:, i])), 3) for i, name in enumerate(_lib.PHASE_NAMES)}
    comp["total_gs_search"] = round(float(np.median(per.sum(axis=1))), 3)
    return comp


def check_parity(index_h, qt, qw, out, k, rows):
    """The GPU's answers for `rows` queries of the batch against the C oracle's
    exact top-k (ids, and scores bit for bit)."""
    import numpy as np

    from oracle import oracle as O
    t0 = time.perf_counter()
    ti, tw = qt.cpu().numpy()[:rows], qw.cpu().numpy()[:rows]
    vs, s64, vi = O.c_search(index_h, ti, tw, k, threads=min(16, os.cpu_count() or 1))
    got_s, got_i = out[0][:rows].cpu().numpy(), out[1][:rows].cpu().numpy()
    diff = np.abs(got_s.astype(np.float64) - s64) if s64 is not None else np.zeros(1)
    return {"queries_checked": rows, "ids_equal": bool(np.array_equal(got_i, vi)),
            "scores_equal": bool(got_s.dtype == vs.dtype and np.array_equal(got_s, vs)),
            "max_abs_diff_vs_fp64": float(np.max(diff, initial=0.0)), "s": round(time.perf_counter() - t0, 1)}


def workload_entry(a, index, qt, qw, k, hyb, cfg_name, index_h=None):
    """One extra workload under the same clock: q/s with two batches in flight on
    one stream, one batch's latency, the scorer's and heavy-term kernel's times
    and roofline fractions, the phases, and with index_h the whole batch's parity."""
    m = time_search(a, index, qt, qw, k, hyb, 2, 1)
    B, T = qt.shape
    e = {"B": B, "k": k, "queries_per_s": round(m["qps"], 1), "ms_per_batch": round(m["ms_per_step"], 3),
         "ms_per_batch_one_in_flight": None if m["one_ms"] is None else round(m["one_ms"], 3),
         "d2h_ms": round(m["d2h_ms"], 3), "dense_rows": m["timing"].get("dense_rows", 0)}
    if a.path == "fused" and m["timing"].get("score_kernel"):
        roof, plan, head = scorer_roofline(a, index, qt, T, k, hyb, m["timing"], cfg_name)
        e.update({"hybrid": plan["hybrid"], "scorer_ms": roof["kernel_ms_avg"], "scorer_bound": roof["bound"],
                  "scorer_frac": roof["frac"], "scorer_lds_frac": roof.get("lds_atomic", roof)["frac"],
                  "scorer_hbm_frac": None if roof["hbm_physical"] is None else roof["hbm_physical"]["frac"],
                  "heavy_terms_ms": None if head is None else head["ms"],
                  "heavy_terms_hbm_frac": None if head is None else head["frac"],
                  "phases_ms": components_of(m["timing"]) if m["timing"].get("phases") else None})
    if index_h is not None:
        e["parity"] = check_parity(index_h, qt, qw, m["out"], k, B)
    ref = REFERENCE_FUSED_MS.get(B) if (cfg_name == "C3" and k == 1000) else None
    if ref is not None:
        e["reference_published_ms_h100"] = ref
    log(f"{cfg_name} B={B} k={k}: {e['ms_per_batch']:.2f} ms/batch, {e['queries_per_s']:.0f} q/s"
        + (f", scorer {e['scorer_ms']:.2f} ms" if e.get("scorer_ms") is not None else "")
        + (f", parity {e['parity']['ids_equal'] and e['parity']['scores_equal']}" if "parity" in e else ""))
    return e


def child_workload(a, cfg_name):
    """A configuration measured by a fresh bench.py process (its own GPU context
    and allocations: the same C5 search measured after the C3 workloads in this
    process, whose buffers have come and gone, ran ~10% slower), with the same
    steps, and the whole batch's parity when the CPU leg runs."""
    import subprocess
    cmd = [sys.executable, os.path.join(ROOT, "bench.py"), "--config", cfg_name, "--no-extra", "--no-cpu",
           "--steps", str(a.steps), "--warmup", str(a.warmup), "--parity-queries", "0" if a.no_cpu else "100000"]
    t0 = time.perf_counter()
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"{cfg_name} child bench failed ({r.returncode}): {r.stderr[-2000:]}")
    c = json.loads(r.stdout.strip().splitlines()[-1])
    roof = c.get("roofline") or {}
    head = c.get("heavy_terms_kernel")
    e = {"B": c["config"]["global_batch"], "k": c["config"]["k"], "queries_per_s": c["value"],
         "ms_per_batch": c["ms_per_step"], "ms_per_batch_one_in_flight": c["ms_per_batch_one_in_flight"],
         "d2h_ms": c["d2h_ms_per_batch"], "dense_rows": c["dense_rows"],
         "hybrid": (c["config"].get("scorer") or {}).get("hybrid"), "scorer_ms": roof.get("kernel_ms_avg"),
         "scorer_bound": roof.get("bound"), "scorer_frac": roof.get("frac"),
         "scorer_lds_frac": (roof.get("lds_atomic") or roof).get("frac"),
         "scorer_hbm_frac": (roof.get("hbm_physical") or {}).get("frac"),
         "heavy_terms_ms": None if head is None else head["ms"],
         "heavy_terms_hbm_frac": None if head is None else head["frac"],
         "phases_ms": c.get("components_ms"), "parity": c.get("parity"),
         "first_search_state_ms": (c.get("index_build") or {}).get("first_search_state_ms"),
         "measured_in": "a child bench.py process: " + " ".join(["python3", "bench.py"] + cmd[2:]),
         "child_wall_s": round(time.perf_counter() - t0, 1)}
    log(f"{cfg_name} B={e['B']} k={e['k']}: {e['ms_per_batch']:.2f} ms/batch, {e['queries_per_s']:.0f} q/s"
        + (f", scorer {e['scorer_ms']:.2f} ms" if e["scorer_ms"] is not None else "")
        + ("" if not e["parity"] else f", parity {e['parity']['ids_equal'] and e['parity']['scores_equal']}"))
    return e


def main():
    a = parse()
    if a.summarize_traffic:
        from gpusparse import synth
        cfg = synth.CONFIGS[a.config]
        n_docs = a.n_docs or cfg.docs.n_rows
        summarize_traffic(a.summarize_traffic, cfg.name, n_docs, a.tile_log2 or None, a.copy_bytes or (1 << 30))
        return
    if a.copy_bytes:
        copy_only(a.copy_bytes)
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {a.gpus}); "
              "the index would shard by doc range, one shard per GPU, with the per-GPU top-k merged.",
              file=sys.stderr)
        sys.exit(2)
    import gc
    from dataclasses import replace

    import numpy as np
    import torch

    import gpusparse as gs
    from gpusparse import synth
    from gpusparse.index import ensure_search_state
    from gpusparse.search import scorer_choice, search_index

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    cfg = synth.CONFIGS[a.config]
    full_size = not a.n_docs and not a.batch
    if a.n_docs:
        cfg = synth.scaled(cfg, n_docs=a.n_docs)
    if a.batch:
        cfg = synth.scaled(cfg, n_queries=a.batch)

    t0 = time.perf_counter()
    docs, queries = synth.generate(cfg)
    t_gen = time.perf_counter() - t0
    log(f"generated {cfg.name}: {docs.shape[0]} docs, {docs.nnz} postings, {queries.shape[0]} queries "
        f"in {t_gen:.1f}s")

    def build(docs):
        """The index (gs_index_count + gs_index_fill) and its search state."""
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev = {}
        ix = gs.build_from_csr(docs, dev, timing=ev)
        torch.cuda.synchronize()
        t_build = time.perf_counter() - t0
        t0 = time.perf_counter()
        tile, hyb = scorer_choice(ix, a.tile_log2 or None, want_hybrid)
        ensure_search_state(search_index(ix, hyb), tile, hybrid=hyb)
        torch.cuda.synchronize()
        return ix, ev, t_build, time.perf_counter() - t0, tile, hyb

    want_hybrid = {"auto": None, "hybrid": True, "lds": False}[a.scorer]
    index, build_ev, t_build, t_state, a.tile_log2, hyb = build(docs)
    log(f"index built in {t_build:.2f}s (incl. H2D of the CSR); first-search state (tile bounds, packed copy, "
        f"doc-major copy{', heavy-term rows' if hyb else ''}) {t_state:.3f}s")
    qt, qw, T = gs.to_query_tensors(queries, dev, weight_dtype=None)
    B = qt.shape[0]
    k = min(a.k or cfg.k, docs.shape[0])
    del docs

    m = time_search(a, index, qt, qw, k, hyb, max(1, a.inflight, a.streams), a.streams)
    timing, out = m["timing"], m["out"]
    ms_per_step, qps, one_ms = m["ms_per_step"], m["qps"], m["one_ms"]
    if one_ms is not None:
        log(f"one batch in flight: {one_ms:.2f} ms/batch")
    log(f"{a.steps} steps: {ms_per_step:.2f} ms/step, {qps:.1f} queries/s (results resident in HBM), "
        f"dense rows {timing.get('dense_rows', 0)}; [B, k] hand-over to host {m['d2h_ms']:.3f} ms")

    d2h_ms, dense_rows = m["d2h_ms"], timing.get("dense_rows", 0)
    wbytes = index.scores.element_size()
    roof = plan = head = None
    if a.path == "fused" and timing.get("score_kernel"):
        roof, plan, head = scorer_roofline(a, index, qt, T, k, hyb, timing, cfg.name)
        lr = roof.get("lds_atomic", roof)
        log(f"scoring kernel {roof['kernel_ms_avg']:.2f} ms avg"
            + (f": {roof['achieved']:.0f} GB/s algorithmic ({100 * roof['frac']:.1f}% of HBM)"
               if roof["bound"] == "hbm" else "")
            + f", {lr['achieved']:.0f} G LDS adds/s"
            + ("" if lr["frac"] is None else f" ({100 * lr['frac']:.1f}% of the measured LDS atomic rate)")
            + ("" if roof["hbm_physical"] is None else f", HBM {roof['hbm_physical']['achieved']:.0f} GB/s physical"))
        if head is not None:
            log(f"heavy-term kernel {head['ms']:.3f} ms: {head['achieved']:.0f} GB/s algorithmic "
                f"({100 * head['frac']:.1f}% of HBM), int8 MFMA {head['mfma_int8']['achieved']:.0f} TOP/s")

    # ---- selection after scoring: candidate selection, fp64 rescoring of the
    # candidates near the k-th score (doc-major rows), final sort.  Bytes are those
    # these kernels move: candidate (doc, key) pairs read, rescoring set written,
    # each rescored doc's row (row pointers + term ids + weights, at the mean row
    # length) read, fp64 keys written and read back, the [B, k] results written.
    selection = None
    if a.path == "fused" and timing.get("phases"):
        cand, resc = gs.search_counts(index, B, T, k, tile_log2=a.tile_log2, sample_tiles=a.sample_tiles,
                                      unroll=a.unroll, tiles_per_wg=a.tiles_per_wg, hybrid=hyb)
        per = phase_matrix(timing)
        sel_ms = float(np.median(per[:, 4:7].sum(axis=1)))
        n_cand = int(np.minimum(cand.astype(np.int64), plan["cand_cap"] if plan else 65536).sum())
        n_resc = int(resc.astype(np.int64).sum())
        row_bytes = 16 + (int(index.lengths.sum().item()) / max(1, int(index.num_docs))) * (4 + wbytes)
        sel_bytes = n_cand * 8 + n_resc * 4 + int(n_resc * row_bytes) + n_resc * 8 + n_resc * 12 + B * k * 12
        selection = {"kernels": "k_select_cands + k_rescore_fwd + k_select_final", "ms": round(sel_ms, 3),
                     "bytes": sel_bytes, "achieved": round(sel_bytes / (sel_ms * 1e-3) / 1e9, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(sel_bytes / (sel_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "candidates_per_query": round(n_cand / B, 1), "rescored_per_query": round(n_resc / B, 1),
                     "reference_selection_bytes": B * int(index.num_docs) * 4 + B * k * 8,
                     "note": "latency-bound (a few thousand candidates per query); the reference's torch.topk "
                             "reads the whole [B, N] fp32 score matrix instead"}
        log(f"selection {sel_ms:.3f} ms: {n_cand / B:.0f} candidates, {n_resc / B:.0f} rescored per query")

    # ---- index build on the device (gs_index_count + gs_index_fill; the CSR is in
    # HBM): algorithmic bytes = CSR term ids + weights + row pointers read, padded
    # doc ids + weights written, per-term arrays written
    index_build = None
    if build_ev:
        b_ms = build_ev["count"][0].elapsed_time(build_ev["count"][1]) + \
            build_ev["fill"][0].elapsed_time(build_ev["fill"][1])
        nnz_b = int(index.lengths.sum().item())
        n_slots = int(index.doc_ids.numel())
        b_bytes = nnz_b * (4 + wbytes) + (int(index.num_docs) + 1) * 8 + n_slots * (4 + wbytes) + \
            int(index.vocab_size) * 24
        index_build = {"kernels": "gs_index_count + gs_index_fill (stable radix transpose)", "ms": round(b_ms, 3),
                       "postings": nnz_b, "bytes": b_bytes,
                       "achieved": round(b_bytes / (b_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                       "frac": round(b_bytes / (b_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                       "first_search_state_ms": round(1000.0 * t_state, 3),
                       "first_search_state": "host wall time of ensure_search_state: tile bounds, packed copy "
                                             "(pack + bank-aware arrange), list checks, doc-major copy"
                                             + (", heavy-term rows" if hyb else "")}
        log(f"index build on device {b_ms:.2f} ms for {nnz_b} postings ({index_build['achieved']} GB/s algorithmic)")

    components = None
    if a.path == "fused" and timing.get("phases"):
        components = components_of(timing)
        log(f"phases (median ms): {components}")

    # ---- parity at full size (the whole batch when the CPU leg runs), and the CPU baseline
    parity = None
    cpu = None
    n_parity = a.parity_queries if a.parity_queries is not None else (4 if a.no_cpu else B)
    index_h = None
    if n_parity > 0 or not a.no_cpu:
        from gpusparse.index import to_host
        index_h = to_host(index)
        if n_parity > 0:
            parity = check_parity(index_h, qt, qw, out, k, min(n_parity, B))
            log(f"parity vs CPU oracle on {parity['queries_checked']} queries: {parity}")
        if not a.no_cpu:
            rows, n_aff = cpu_rows(index_h, qt.cpu().numpy(), qw.cpu().numpy(), k, a.cpu_queries_1,
                                   a.cpu_queries_all, a.cpu_cores)
            best = rows[-1]
            cpu = {"value": best["qps"], "unit": "queries/s", "cores": best["cores"], "kind": "port",
                   "sample": f"first {best['queries']} queries of the batch over the full index "
                             f"(reference CPU path cpu_sequential_score restated in C, fp32 accumulator)",
                   "cpu_wall_ratio": best["cpu_wall_ratio"], "affinity_cores": n_aff,
                   "core_cap": a.cpu_cores, "rows": rows,
                   "noise": "the one-core C3 rate has varied by about +-20% between boxes of this pool"}

    n_docs = int(index.num_docs)
    postings = int(index.lengths.sum().item())
    weights = str(index.scores.dtype).replace("torch.", "")

    # ---- the other workloads under the same clock: the batch curve and k = 10 on
    # this index, then C5 (uint8) at B = 512
    extra = None
    if not a.no_extra and cfg.name == "C3" and full_size and a.path == "fused":
        extra = {}
        qbig = synth.generate_rows(replace(cfg.queries, n_rows=max(CURVE_BATCHES)), cfg.seed,
                                   synth.STREAM_QUERIES)
        qt_c, qw_c, _ = gs.to_query_tensors(qbig, dev, weight_dtype=None)
        for Bc in CURVE_BATCHES:
            extra[f"C3_B{Bc}_k1000"] = workload_entry(a, index, qt_c[:Bc].contiguous(), qw_c[:Bc].contiguous(),
                                                      1000, hyb, "C3")
        del qt_c, qw_c
        extra["C3_B512_k10"] = workload_entry(a, index, qt, qw, 10, hyb, "C3", index_h if not a.no_cpu else None)
        del index, index_h, out, m, timing
        gc.collect()
        torch.cuda.empty_cache()
        extra["C5_B512_k1000"] = child_workload(a, "C5")

    res = {
        "metric": METRIC if (cfg.name == "C3" and k == 1000 and B == 512)
        else f"queries/s @{n_docs} docs k={k} batch {B} ({cfg.name})", "value": round(qps, 2), "unit": "queries/s",
        "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_per_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32" if wbytes != 1 else "u32", "data": "synthetic",
        "results": "device-resident: a step ends with the [B, k] scores and ids in HBM (as the reference's "
                   "benchmarks time it); queries_per_s_incl_d2h adds one batch's hand-over to pinned host memory "
                   "per step, serially",
        "queries_per_s_incl_d2h": round(B / ((ms_per_step + d2h_ms) * 1e-3), 2),
        "d2h_ms_per_batch": round(d2h_ms, 3),
        "config": {"workload": f"{cfg.name}: {cfg.description}", "n_docs": n_docs,
                   "postings": postings, "global_batch": B, "k": k, "max_query_terms": T,
                   "weights": weights, "tile_docs": 1 << a.tile_log2,
                   "path": a.path, "inflight": max(1, a.inflight, a.streams), "streams": a.streams,
                   "scorer": None if plan is None else {key: plan[key] for key in
                                                        ("group_size", "unroll", "tiles_per_wg", "seed_tiles", "packed",
                                                         "hybrid")}},
        "ms_per_batch_one_in_flight": None if one_ms is None else round(one_ms, 3),
        "roofline": roof, "heavy_terms_kernel": head, "selection": selection, "index_build": index_build,
        "cpu_baseline": cpu, "parity": parity, "components_ms": components,
        "index_build_s": round(t_build, 3), "search_state_s": round(t_state, 3), "generate_s": round(t_gen, 1),
        "dense_rows": dense_rows,
        "workloads": extra,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
