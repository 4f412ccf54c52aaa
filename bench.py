"""Headline benchmark: batched IVF-PQ search, 1M x 128, nlist 4096, M 16,
ksub 256, nprobe 32, k 100, batch 10,000 queries, on one MI355X.

A step is one search_batch over the whole 10k-query batch with the queries
already resident in HBM.  The dominant kernel is the ADC scan; its duration
comes from hipEvents recorded on the engine's stream around that kernel in
every timed step, and its algorithmic bytes are (code bytes + 4) per scanned
list entry, counted by the kernel itself.  The CPU baseline is the oracle
(the C restatement of the reference search) on the host cores, over a
bounded sample of the same queries and index arrays.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "IVF-PQ QPS @ fixed nprobe, 1M×d128 batch 10k; ADC-scan HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def traffic_from_profile():
    """HBM bytes per scan launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (calibrated against a copy kernel), or None."""
    path = os.path.join(ROOT, "profiles", "scan8_fast_ivfpq_1m_d128_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch"):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


def cpu_baseline(art, queries, k, nprobe, budget_s=15.0):
    """Oracle search (python.rs batch shape over a thread pool) on a bounded
    query sample; returns (qps, threads, sample_size, ids, dists)."""
    from oracle import oracle as orc

    orc.build()
    oix = orc.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                    art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"],
                    art["rotation"])
    threads = min(os.cpu_count() or 1, 16)
    probe = 200
    t0 = time.perf_counter()
    oix.search_batch(queries[:probe], k, nprobe, threads=threads)
    per_q = (time.perf_counter() - t0) / probe
    n = int(min(len(queries), max(probe, budget_s / max(per_q, 1e-9))))
    t0 = time.perf_counter()
    ids, dists = oix.search_batch(queries[:n], k, nprobe, threads=threads)
    dt = time.perf_counter() - t0
    return n / dt, threads, n, ids, dists


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", default="fast", choices=["fast", "exact"])
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--train-sample", type=int, default=262_144)
    ap.add_argument("--kmeans-iters", type=int, default=25)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--opq", action="store_true",
                    help="build with use_opq (OPQ rotation, EXACT-mode scan of rotated residual "
                         "tables) instead of the headline product quantizer")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only run three 256 MiB device-to-device copies (the reference "
                         "kernel for calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.calib_copy:
        import torch

        a = torch.ones(64 << 20, device="cuda:0")  # 256 MiB of float32
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"three copies of {a.numel() * 4} bytes")
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the index and the "
              "query batch fit one MI355X; multi-GPU query/list sharding is not built.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import vicinity_amd as v
    from vicinity_amd import datagen

    if not v.device_available():
        raise RuntimeError("no gfx950 device visible")
    t0 = time.perf_counter()
    w = datagen.ivfpq_1m(n=args.n)
    p = w.params
    log(f"data {w.base.shape} in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    ix = v.IVFPQIndex(128, num_clusters=p["num_clusters"], num_codebooks=p["num_codebooks"],
                      codebook_size=p["codebook_size"], nprobe=p["nprobe"], use_opq=args.opq,
                      seed=42)
    ix.add_items(w.base)
    ix.build(training_sample_size=args.train_sample, kmeans_max_iter=args.kmeans_iters)
    log(f"build in {time.perf_counter() - t0:.1f}s")
    ix.set_mode(args.mode)
    # Timed steps carry only the two hipEvents around the scan kernel (the
    # roofline's launch duration); the per-phase breakdown comes from a
    # separate, untimed pass with every-phase events.
    ix.set_profiling(2)
    k, nprobe = p["k"], p["nprobe"]
    nq = w.queries.shape[0]
    q = torch.from_numpy(w.queries).to("cuda:0")
    out_ids = torch.empty((nq, k), dtype=torch.int64, device="cuda:0")
    out_d = torch.empty((nq, k), dtype=torch.float32, device="cuda:0")
    for _ in range(args.warmup):
        ix.search_batch_device(q, k, nprobe, out_ids=out_ids, out_dists=out_d)
    torch.cuda.synchronize()
    stats = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ix.search_batch_device(q, k, nprobe, out_ids=out_ids, out_dists=out_d)
        stats.append(ix.last_stats())
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_step = dt * 1e3 / args.steps
    qps = nq * args.steps / dt
    scan_ms = float(np.mean([s["ms_scan"] for s in stats]))
    scan_bytes = float(np.mean([s["scan_bytes"] for s in stats]))
    cands = float(np.mean([s["candidates"] for s in stats]))
    achieved = scan_bytes / (scan_ms * 1e-3) / 1e9
    ix.set_profiling(1)
    pstats = []
    for _ in range(max(3, min(args.steps, 10))):
        ix.search_batch_device(q, k, nprobe, out_ids=out_ids, out_dists=out_d)
        pstats.append(ix.last_stats())
    ix.set_profiling(0)
    phases = {key: round(float(np.mean([s[key] for s in pstats])), 4)
              for key in ("ms_normalize", "ms_coarse", "ms_select", "ms_scan", "ms_fallback",
                          "ms_rerank", "ms_total")}
    fallbacks = int(max(s["fallback_queries"] for s in stats))
    scan_diag = {"flushes_per_query": round(stats[-1]["fast_flushes"] / nq, 3),
                 "appends_per_query": round(stats[-1]["fast_appends"] / nq, 1),
                 "candidates_per_query": round(stats[-1]["candidates"] / nq, 1),
                 "fallback_ties": int(stats[-1]["fallback_ties"]),
                 "second_passes": int(stats[-1]["fast_retries"]),
                 "coarse_fallbacks": int(stats[-1]["coarse_overflow"])}
    log(f"{qps:.0f} QPS, {ms_step:.3f} ms/batch, scan {scan_ms:.3f} ms, {achieved:.0f} GB/s, "
        f"phases {phases}, fallback queries {fallbacks}, scan {scan_diag}")

    gpu_ids = out_ids.cpu().numpy()
    gpu_d = out_d.cpu().numpy()
    cpu = None
    parity = None
    if not args.no_cpu:
        art = ix.export()
        cqps, threads, n_s, cids, cd = cpu_baseline(art, w.queries, k, nprobe)
        parity = {"queries_checked": n_s,
                  "ids_equal": bool(np.array_equal(gpu_ids[:n_s], cids)),
                  "dists_bitexact": bool(gpu_d[:n_s].tobytes() == cd.tobytes())}
        cpu = {"value": round(cqps, 1), "unit": "queries/s", "cores": threads, "kind": "port",
               "sample": f"first {n_s} of the 10k queries, same index arrays, k={k}, "
                         f"nprobe={nprobe}, oracle C restatement, {threads} threads"}
        log(f"cpu baseline {cqps:.0f} QPS on {threads} threads ({n_s} queries); parity {parity}")

    line = {
        "metric": METRIC,
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Gaussian mixture, vicinity_amd/datagen.py)",
        "config": {"workload": w.name + ("_opq" if args.opq else ""), "n": args.n, "d": 128, "nlist": p["num_clusters"],
                   "M": p["num_codebooks"], "ksub": p["codebook_size"], "nprobe": nprobe, "k": k,
                   "batch": nq, "mode": "exact" if args.opq else args.mode,
                   "use_opq": args.opq, "train_sample": args.train_sample,
                   "kmeans_iters": args.kmeans_iters},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (traffic_from_profile()
                                 if args.n == 1_000_000 and not args.opq and args.mode == "fast"
                                 else None),
                     "kernel": ("scan8_exact_kernel<16,256>" if args.opq or args.mode == "exact"
                                else "scan8_fast_kernel<16,256,8,1>"),
                     "kernel_ms": round(scan_ms, 4),
                     "algorithmic_bytes_per_launch": int(scan_bytes),
                     "candidates_per_launch": int(cands)},
        "phases_ms": phases,
        "fallback_queries": fallbacks,
        "scan_diagnostics": scan_diag,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
