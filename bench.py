"""Benchmark of the exact SPLADE search path on one MI355X.

Default workload (BASELINE.json's metric): config C3 -- 8.8M synthetic docs
(~1.06e9 postings, fp16 posting weights, fp32 accumulation), batches of 512
queries, k = 1000.  A step is one ``search`` of one 512-query batch: fused
LDS-tile scoring with threshold selection, candidate selection, fp64 rescoring
and the status check.  Inputs (index and query batch) are resident in HBM before
the timed region.

Prints one JSON line.  ``roofline`` is for the dominant kernel (the fused tile
scoring kernel), timed with HIP events on its launch stream: algorithmic bytes =
sum over queries and valid terms of the postings that launch streams x (4 B doc
id + weight bytes).  ``cpu_baseline`` times the reference CPU path
(cpu_sequential_score, restated in C) on a bounded sample of the same batch,
pinned to C cores.
"""
from __future__ import annotations

import argparse
import json
import os
import resource
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
    ap.add_argument("--cpu-cores", type=int, default=16, help="cap on the cores of the all-core row")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--parity-queries", type=int, default=4)
    ap.add_argument("--path", default="fused", choices=["fused", "dense", "atomic"])
    ap.add_argument("--summarize-traffic", default=None, metavar="DIR",
                    help="write profiles/traffic_k_score_union_<config>.json from rocprofv3 --pmc runs under DIR")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run a plain device-to-device copy of this many bytes (PMC counter calibration)")
    return ap.parse_args()


def traffic_file(cfg_name):
    return os.path.join(ROOT, "profiles", f"traffic_k_score_union_{cfg_name}.json")


def measured_traffic(cfg_name, n_docs, tile_log2):
    """HBM bytes per launch of the fused scorer from the committed rocprofv3 PMC
    measurement (FETCH_SIZE + WRITE_SIZE scaled by a copy kernel of known size),
    when it was taken on this workload; None otherwise."""
    try:
        with open(traffic_file(cfg_name)) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("config") != cfg_name or t.get("n_docs") != n_docs or t.get("tile_log2") != tile_log2:
        return None
    return t.get("traffic_bytes_per_launch")


def summarize_traffic(d, cfg_name, n_docs, tile_log2, copy_bytes):
    """Writes the traffic file from four rocprofv3 --pmc runs under `d`: f/ and w/
    (FETCH_SIZE, WRITE_SIZE of this benchmark), cf/ and cw/ (the same counters over
    ``--copy-bytes`` copies).  Each counter is scaled by bytes copied / counter
    value of the last copy dispatch; values are KiB per dispatch, summed over
    the counter's instances, last dispatch of the kernel."""
    import csv
    import glob

    def last(sub, name):
        rows = {}
        for path in glob.glob(os.path.join(d, sub, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                if name in r["Kernel_Name"]:
                    did = int(r["Dispatch_Id"])
                    rows[did] = rows.get(did, 0.0) + float(r["Counter_Value"])
        if not rows:
            raise SystemExit(f"no {name} dispatch under {os.path.join(d, sub)}")
        return rows[max(rows)]

    f, w = last("f", "k_score_union"), last("w", "k_score_union")
    cf, cw = last("cf", "copyBuffer"), last("cw", "copyBuffer")
    fs, ws = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)
    out = {"config": cfg_name, "n_docs": n_docs, "tile_log2": tile_log2, "kernel": "k_score_union",
           "fetch_kib_per_launch": f, "write_kib_per_launch": w, "copy_bytes": copy_bytes,
           "copy_fetch_kib": cf, "copy_write_kib": cw, "fetch_scale": fs, "write_scale": ws,
           "fetch_bytes_per_launch": f * 1024 * fs, "write_bytes_per_launch": w * 1024 * ws,
           "traffic_bytes_per_launch": f * 1024 * fs + w * 1024 * ws,
           "commands": [
               f"rocprofv3 --pmc FETCH_SIZE -d <out>/f -o f --output-format csv -- python3 bench.py --config {cfg_name} "
               "--no-cpu --parity-queries 0 --steps 1 --warmup 1",
               f"rocprofv3 --pmc WRITE_SIZE -d <out>/w -o w --output-format csv -- python3 bench.py --config {cfg_name} "
               "--no-cpu --parity-queries 0 --steps 1 --warmup 1",
               f"rocprofv3 --pmc FETCH_SIZE -d <out>/cf -o cf --output-format csv -- python3 bench.py --copy-bytes {copy_bytes}",
               f"rocprofv3 --pmc WRITE_SIZE -d <out>/cw -o cw --output-format csv -- python3 bench.py --copy-bytes {copy_bytes}",
               f"python3 bench.py --config {cfg_name} --summarize-traffic <out>"]}
    with open(traffic_file(cfg_name), "w") as fh:
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


def cpu_rows(index_h, ti, tw, k, n1, n_all, cap):
    """Reference CPU path on one core and on `cap` cores: wall, CPU seconds,
    CPU/wall and queries/s per row.  Pinned with sched_setaffinity (taskset's
    syscall) and the thread-pool variables."""
    from oracle import oracle as O
    allowed = sorted(os.sched_getaffinity(0))
    rows = []
    for cores, nq in ((1, n1), (min(cap, len(allowed)), n_all)):
        if nq <= 0:
            continue
        nq = min(nq, ti.shape[0])
        pin = set(allowed[:cores])
        for v in ("OMP_NUM_THREADS", "MKL_NUM_THREADS", "OPENBLAS_NUM_THREADS", "NUMEXPR_NUM_THREADS",
                  "RAYON_NUM_THREADS"):
            os.environ[v] = str(cores)
        os.sched_setaffinity(0, pin)
        try:
            r0 = resource.getrusage(resource.RUSAGE_SELF)
            t0 = time.perf_counter()
            O.c_cpu_sequential(index_h, ti[:nq], tw[:nq], k, threads=cores)
            wall = time.perf_counter() - t0
            r1 = resource.getrusage(resource.RUSAGE_SELF)
        finally:
            os.sched_setaffinity(0, set(allowed))
        cpu_s = (r1.ru_utime - r0.ru_utime) + (r1.ru_stime - r0.ru_stime)
        ratio = cpu_s / wall if wall > 0 else 0.0
        rows.append({"cores": cores, "queries": nq, "wall_s": round(wall, 3), "cpu_s": round(cpu_s, 3),
                     "cpu_wall_ratio": round(ratio, 3), "qps": round(nq / wall, 3),
                     "pinning_clean": bool(ratio < 1.35 * cores)})
        log(f"cpu baseline cores={cores} queries={nq} wall={wall:.2f}s cpu/wall={ratio:.2f} "
            f"q/s={nq / wall:.2f}")
    return rows


def main():
    a = parse()
    if a.summarize_traffic:
        from gpusparse import synth
        cfg = synth.CONFIGS[a.config]
        n_docs = a.n_docs or cfg.docs.n_rows
        from gpusparse.index import DEFAULT_TILE_LOG2_PACKED
        tile = a.tile_log2 or DEFAULT_TILE_LOG2_PACKED
        summarize_traffic(a.summarize_traffic, cfg.name, n_docs, tile, a.copy_bytes or (1 << 30))
        return
    if a.copy_bytes:
        copy_only(a.copy_bytes)
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {a.gpus}); "
              "see DESIGN.md for how the index would shard.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import gpusparse as gs
    from gpusparse import synth
    from gpusparse.index import default_tile_log2, ensure_search_state

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    cfg = synth.CONFIGS[a.config]
    if a.n_docs:
        cfg = synth.scaled(cfg, n_docs=a.n_docs)
    if a.batch:
        cfg = synth.scaled(cfg, n_queries=a.batch)

    t0 = time.perf_counter()
    docs, queries = synth.generate(cfg)
    t_gen = time.perf_counter() - t0
    log(f"generated {cfg.name}: {docs.shape[0]} docs, {docs.nnz} postings, {queries.shape[0]} queries "
        f"in {t_gen:.1f}s")

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    index = gs.build_index(docs, dev)
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t0
    t0 = time.perf_counter()
    if not a.tile_log2:
        a.tile_log2 = default_tile_log2(index)
    ensure_search_state(index, a.tile_log2)
    torch.cuda.synchronize()
    t_bounds = time.perf_counter() - t0
    log(f"index built in {t_build:.2f}s (incl. H2D of the CSR); search state (tile bounds, doc-major copy) "
        f"{t_bounds:.3f}s")
    qt, qw, T = gs.to_query_tensors(queries, dev)
    B = qt.shape[0]
    k = min(a.k or cfg.k, docs.shape[0])
    del docs

    def step(timing=None):
        if a.path == "atomic":
            return gs.atomic_fused_score(index, qt, qw, k)
        return gs.search(index, (qt, qw), k, tile_log2=a.tile_log2, path=a.path, unroll=a.unroll,
                         waves=a.waves, tiles_per_wg=a.tiles_per_wg, sample_tiles=a.sample_tiles, timing=timing)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    timing = {}
    t0 = time.perf_counter()
    for _ in range(a.steps):
        out = step(timing)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = 1000.0 * wall / a.steps
    qps = B * a.steps / wall
    log(f"{a.steps} steps: {ms_per_step:.2f} ms/step, {qps:.1f} queries/s, "
        f"dense rows {timing.get('dense_rows', 0)}")

    # ---- roofline of the fused tile-scoring kernel
    wbytes = index.scores.element_size()
    S = 0
    roof = None
    plan = None
    if a.path == "fused" and timing.get("score_kernel"):
        kern_ms = [e0.elapsed_time(e1) for e0, e1 in timing["score_kernel"]]
        call_ms = [e0.elapsed_time(e1) for e0, e1 in timing["search"]]
        n_tiles = (index.num_docs + (1 << a.tile_log2) - 1) >> a.tile_log2
        # the main launch scores the tiles after the seed tiles
        plan = gs.search_plan(index, B, T, k, tile_log2=a.tile_log2, sample_tiles=a.sample_tiles, unroll=a.unroll,
                              tiles_per_wg=a.tiles_per_wg)
        S = min(plan["seed_tiles"], n_tiles)
        tb = index.aux()[("tile_bounds", a.tile_log2)]
        cols = tb[:, [S, n_tiles]].cpu().numpy().astype(np.int64)
        per_term = cols[:, 1] - cols[:, 0]
        all_term = index.lengths.cpu().numpy().astype(np.int64)
        qt_h = qt.cpu().numpy()
        valid = (qt_h >= 0) & (qt_h < index.vocab_size)
        tq = np.where(valid, qt_h, 0)
        post_launch = int((per_term[tq] * valid).sum())
        post_all = int((all_term[tq] * valid).sum())
        per_post = 4 + wbytes
        bytes_launch = post_launch * per_post
        avg_ms = float(np.mean(kern_ms))
        achieved = bytes_launch / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": measured_traffic(cfg.name, int(index.num_docs), a.tile_log2),
                "kernel": "k_score_union (fused group-tile LDS scoring + threshold emission)",
                "kernel_ms_avg": round(avg_ms, 3), "kernel_ms_median": round(float(np.median(kern_ms)), 3),
                "kernel_ms_min": round(float(np.min(kern_ms)), 3),
                "scored_postings_per_launch": post_launch, "bytes_per_posting": per_post,
                "algorithmic_bytes_per_launch": bytes_launch,
                "search_call_ms_avg": round(float(np.mean(call_ms)), 3),
                "batch_scored_postings": post_all,
                "batch_gbs_algorithmic": round(post_all * per_post / (ms_per_step * 1e-3) / 1e9, 1)}
        log(f"scoring kernel {avg_ms:.2f} ms avg: {achieved:.0f} GB/s algorithmic "
            f"({100 * achieved / PEAK_HBM_GBS:.1f}% of {PEAK_HBM_GBS:.0f} GB/s); "
            f"batch scored postings {post_all:.3e}")

    # ---- per-phase times of gs_search (HIP events recorded by the library on
    # its launch stream), medians over the timed steps
    components = None
    if a.path == "fused" and timing.get("phases"):
        from gpusparse import _lib
        per = np.array([[ev[i].elapsed_time(ev[i + 1]) for i in range(len(ev) - 1)] for ev in timing["phases"]])
        components = {name: round(float(np.median(per[:, i])), 3) for i, name in enumerate(_lib.PHASE_NAMES)}
        components["total_gs_search"] = round(float(np.median(per.sum(axis=1))), 3)
        log(f"phases (median ms): {components}")

    # ---- parity sample at full size, and the CPU baseline
    parity = None
    cpu = None
    need_host = a.parity_queries > 0 or not a.no_cpu
    if need_host:
        from gpusparse.index import to_host
        from oracle import oracle as O
        index_h = to_host(index)
        ti_h, tw_h = qt.cpu().numpy(), qw.cpu().numpy()
        if a.parity_queries > 0:
            nq = min(a.parity_queries, B)
            t0 = time.perf_counter()
            vs, s64, vi = O.c_search(index_h, ti_h[:nq], tw_h[:nq], k, threads=min(16, os.cpu_count() or 1))
            got_s, got_i = out[0][:nq].cpu().numpy(), out[1][:nq].cpu().numpy()
            parity = {"queries_checked": nq, "ids_equal": bool(np.array_equal(got_i, vi)),
                      "scores_equal": bool(np.array_equal(got_s, vs)),
                      "max_abs_diff_vs_fp64": float(np.max(np.abs(got_s.astype(np.float64) - s64)))}
            log(f"parity vs CPU oracle on {nq} queries: {parity} ({time.perf_counter() - t0:.1f}s)")
        if not a.no_cpu:
            rows = cpu_rows(index_h, ti_h, tw_h, k, a.cpu_queries_1, a.cpu_queries_all, a.cpu_cores)
            best = rows[-1]
            cpu = {"value": best["qps"], "unit": "queries/s", "cores": best["cores"], "kind": "port",
                   "sample": f"first {best['queries']} queries of the batch over the full index "
                             f"(reference CPU path cpu_sequential_score restated in C, fp32 accumulator)",
                   "cpu_wall_ratio": best["cpu_wall_ratio"], "rows": rows}

    n_docs = int(index.num_docs)
    res = {
        "metric": METRIC if (cfg.name == "C3" and k == 1000 and B == 512)
        else f"queries/s @{n_docs} docs k={k} batch {B} ({cfg.name})", "value": round(qps, 2), "unit": "queries/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_per_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32" if wbytes != 1 else "u32", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.description}", "n_docs": n_docs,
                   "postings": int(index.lengths.sum().item()), "global_batch": B, "k": k, "max_query_terms": T,
                   "weights": str(index.scores.dtype).replace("torch.", ""), "tile_docs": 1 << a.tile_log2,
                   "path": a.path,
                   "scorer": None if plan is None else {key: plan[key] for key in
                                                        ("group_size", "unroll", "tiles_per_wg", "seed_tiles", "packed")}},
        "roofline": roof, "cpu_baseline": cpu, "parity": parity, "components_ms": components,
        "index_build_s": round(t_build, 3), "search_state_s": round(t_bounds, 3), "generate_s": round(t_gen, 1),
        "dense_rows": timing.get("dense_rows", 0),
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
