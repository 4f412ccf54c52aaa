"""Benchmark of batched IVF-PQ search on one MI355X.

Default (the headline): 1M x 128, nlist 4096, M 16, ksub 256, nprobe 32,
k 100, batch 10,000 queries.  --workload picks another of the five seeded
configurations (vicinity_amd/datagen.py): ivfpq_small (20k x 32),
flat (100k x 96 exact L2), ivfpq_1m, ivfpq_10m (10M x 96 angular, nlist
16384, M 48, nprobe 64, k 10), ivfpq_4bit (1M x 100 FastScan, nprobe 64,
rerank pool 100, k 10).

A step is one search over the whole 10k-query batch with the queries
already resident in HBM.  The dominant kernel is the ADC scan (the flat
GEMM for `flat`); its duration comes from hipEvents recorded on the search's
stream around that kernel in every timed step, and its algorithmic bytes are
(code bytes + 4) per scanned list entry, counted by the kernel itself.  The
CPU baseline is the oracle (the C restatement of the reference search) on the
host cores, over a bounded sample of the same queries and index arrays.
Recall@k is measured against exact cosine ground truth (the flat GPU path on
the normalised vectors, the reference's own ground truth).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
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
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def traffic_from_profile(name):
    """HBM bytes per scan launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary profiles/<kernel>_<workload>_traffic.md or
    profiles/<kernel>_<workload>.md (calibrated against a copy kernel), or None."""
    for fname in (f"{name}_traffic.md", f"{name}.md"):
        try:
            for line in open(os.path.join(ROOT, "profiles", fname)):
                if line.startswith("traffic_bytes_per_launch"):
                    return int(line.split("=")[1])
        except OSError:
            pass
    return None


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _cgroup_cpu_quota():
    """Cores this job may use by its cgroup's CPU quota (cpu.max), or None."""
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            return max(1, int(round(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    return None


def _timed_oracle(oix, queries, k, nprobe, pool, threads, budget_s, probe=64):
    """QPS of the oracle's batch search on `threads` threads over the first
    queries, sized to about budget_s seconds; returns (qps, n, ids, dists)."""
    t0 = time.perf_counter()
    oix.search_batch(queries[:probe], k, nprobe, rerank_pool=pool, threads=threads)
    per_q = (time.perf_counter() - t0) / probe
    n = int(min(len(queries), max(probe, budget_s / max(per_q, 1e-9))))
    t0 = time.perf_counter()
    ids, dists = oix.search_batch(queries[:n], k, nprobe, rerank_pool=pool, threads=threads)
    return n / (time.perf_counter() - t0), n, ids, dists


def _baseline_threads():
    """Every core this process may run on: its CPU affinity, capped by a
    cgroup CPU quota when one is set."""
    affinity = len(os.sched_getaffinity(0))
    quota = _cgroup_cpu_quota()
    return min(affinity, quota) if quota else affinity


def cpu_baseline(art, queries, k, nprobe, pool=0, budget_s=15.0):
    """The oracle (C restatement of the reference search, built -march=native
    -ffp-contract=off on this host) over a thread pool shaped like the
    reference's rayon par_iter over queries, on every core this process may
    run on (its CPU affinity, capped by a cgroup CPU quota when one is set),
    plus a one-thread figure.  Returns the JSON object and the multi-thread
    run's ids and distances for the parity check."""
    from oracle import oracle as orc

    orc.use_native()
    oix = orc.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                    art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"],
                    art["rotation"])
    affinity = len(os.sched_getaffinity(0))
    quota = _cgroup_cpu_quota()
    threads = _baseline_threads()
    qps1, n1, _, _ = _timed_oracle(oix, queries, k, nprobe, pool, 1, budget_s / 2)
    qps, n, ids, dists = _timed_oracle(oix, queries, k, nprobe, pool, threads, budget_s)
    out = {"value": round(qps, 1), "unit": "queries/s", "cores": threads, "kind": "port",
           "sample": f"first {n} of the {len(queries)} queries, same index arrays, k={k}, "
                     f"nprobe={nprobe}, rerank pool {pool}; "
                     f"oracle C restatement built -march=native -ffp-contract=off, {threads} "
                     f"threads over queries",
           "qps_1thread": round(qps1, 1), "sample_1thread": n1,
           "host_cpus": os.cpu_count(), "affinity_cpus": affinity, "cgroup_cpu_quota": quota,
           "cpu_model": _cpu_model()}
    return out, n, ids, dists


IVFPQ_RUNS = {  # workload -> (training sample or None for every vector, k-means iterations)
    "ivfpq_small": (None, 10),
    "ivfpq_1m": (262_144, 25),
    "ivfpq_10m": (262_144, 10),
    "ivfpq_4bit": (262_144, 10),
}


def recall_at_k(ids, truth):
    """Mean over queries of |result ids ∩ true top-k| / k."""
    k = truth.shape[1]
    hits = sum(len(set(a[a >= 0].tolist()) & set(t.tolist())) for a, t in zip(ids, truth))
    return hits / (k * len(truth))


def cosine_truth(vectors, queries, k):
    """Exact top-k of 1 - q.x over the normalised vectors (the flat GPU path)."""
    from vicinity_amd import FlatIndex

    qn = queries / np.maximum(np.linalg.norm(queries, axis=1, keepdims=True), 1e-30)
    fx = FlatIndex(vectors.shape[1], "cosine")
    fx.add(vectors)
    ids, _ = fx.search(qn.astype(np.float32), k)
    return ids


def base_line(args, metric, value, unit, ms_step, dtype, config):
    return {"metric": metric, "value": round(value, 1), "unit": unit, "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
            "data": "synthetic (seeded Gaussian mixture, vicinity_amd/datagen.py)",
            "config": config}


def run_ivfpq(args, w):
    import torch

    import vicinity_amd as v

    p = w.params
    d = w.base.shape[1]
    sample, iters = IVFPQ_RUNS[args.workload]
    if args.train_sample is not None:
        sample = args.train_sample
    if args.kmeans_iters is not None:
        iters = args.kmeans_iters
    t0 = time.perf_counter()
    ix = v.IVFPQIndex(d, num_clusters=p["num_clusters"], num_codebooks=p["num_codebooks"],
                      codebook_size=p["codebook_size"], nprobe=p["nprobe"], use_opq=args.opq,
                      seed=42)
    ix.add_items(w.base)
    ix.build(training_sample_size=sample, kmeans_max_iter=iters)
    log(f"build in {time.perf_counter() - t0:.1f}s")
    ix.set_mode(args.mode)
    # Timed steps carry only the two hipEvents around the scan kernel (the
    # roofline's launch duration); the per-phase breakdown comes from a
    # separate, untimed pass with every-phase events.
    ix.set_profiling(2)
    k, nprobe, pool = p["k"], args.nprobe or p["nprobe"], p.get("rerank_pool")
    nq = w.queries.shape[0]
    q = torch.from_numpy(w.queries).to("cuda:0")
    out_ids = torch.empty((nq, k), dtype=torch.int64, device="cuda:0")
    out_d = torch.empty((nq, k), dtype=torch.float32, device="cuda:0")
    search = lambda: ix.search_batch_device(q, k, nprobe, rerank_pool=pool, out_ids=out_ids,
                                            out_dists=out_d)
    for _ in range(args.warmup):
        search()
    torch.cuda.synchronize()
    stats = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        search()
        stats.append(ix.last_stats())
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_step = dt * 1e3 / args.steps
    qps = nq * args.steps / dt
    scan_ms = float(np.mean([s["ms_scan"] for s in stats]))
    table_ms = float(np.mean([s["ms_table"] for s in stats]))
    scan_bytes = float(np.mean([s["scan_bytes"] for s in stats]))
    cands = float(np.mean([s["candidates"] for s in stats]))
    achieved = scan_bytes / (scan_ms * 1e-3) / 1e9
    ix.set_profiling(1)
    pstats = []
    for _ in range(max(3, min(args.steps, 10))):
        search()
        pstats.append(ix.last_stats())
    ix.set_profiling(0)
    phases = {key: round(float(np.mean([s[key] for s in pstats])), 4)
              for key in ("ms_normalize", "ms_coarse", "ms_select", "ms_table", "ms_scan",
                          "ms_fallback", "ms_rerank", "ms_total")}
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
    art = ix.export()
    recall = None
    if not args.no_recall:
        t0 = time.perf_counter()
        truth = cosine_truth(art["vectors"], w.queries, k)
        recall = round(recall_at_k(gpu_ids, truth), 4)
        log(f"recall@{k} {recall} (ground truth in {time.perf_counter() - t0:.1f}s)")
    cpu = None
    parity = None
    if not args.no_cpu:
        cpu, n_s, cids, cd = cpu_baseline(art, w.queries, k, nprobe, pool or 0)
        parity = {"queries_checked": n_s,
                  "ids_equal": bool(np.array_equal(gpu_ids[:n_s], cids)),
                  "dists_bitexact": bool(gpu_d[:n_s].tobytes() == cd.tobytes())}
        log(f"cpu baseline {cpu['value']:.0f} QPS on {cpu['cores']} threads, "
            f"{cpu['qps_1thread']:.0f} QPS on one ({cpu['cpu_model']}); parity {parity}")

    K, M = p["codebook_size"], p["num_codebooks"]
    exact = args.opq or args.mode == "exact"
    if K == 16:
        kernel, kname = "fastscan_kernel", "fastscan"
    elif exact:
        kernel, kname = f"scan8_exact_kernel<{M},{K}>", "scan8_exact"
    else:
        # 16 codebooks on transposed blocks read their tables from the MFMA
        # pre-pass (t2_table_kernel): the scan's fifth template argument is 1
        pre = ",1" if M == 16 and K == 256 and d // M in (2, 4, 8) else ""
        kernel, kname = f"scan8_fast_kernel<{M},{K},{d // M},1{pre}>", "scan8_fast"
    wl = w.name + ("_opq" if args.opq else "")
    config = {"workload": wl, "n": w.base.shape[0], "d": d, "nlist": p["num_clusters"],
              "M": M, "ksub": K, "nprobe": nprobe, "k": k, "rerank_pool": pool, "batch": nq,
              "mode": "exact" if exact else args.mode, "use_opq": args.opq,
              "train_sample": sample, "kmeans_iters": iters}
    metric = METRIC if args.workload == "ivfpq_1m" else (
        f"IVF-PQ QPS @ fixed nprobe, {w.name} batch {nq // 1000}k; ADC-scan HBM GB/s vs peak")
    line = base_line(args, metric, qps, "queries/s", ms_step, "f32", config)
    line.update({
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None if exact or args.n else traffic_from_profile(f"{kname}_{w.name}"),
                     "kernel": kernel, "kernel_ms": round(scan_ms, 4),
                     "table_prepass_ms": round(table_ms, 4),
                     "algorithmic_bytes_per_launch": int(scan_bytes),
                     "candidates_per_launch": int(cands)},
        "recall_at_k": recall,
        "phases_ms": phases,
        "fallback_queries": fallbacks,
        "scan_diagnostics": scan_diag,
        "cpu_baseline": cpu,
        "parity": parity,
    })
    return line


def run_flat(args, w):
    """Exact top-k (the ground-truth path): squared L2 over the raw vectors,
    one launch sequence per 10k batch.  Roofline: fp32 MFMA on the ranking
    GEMM, 2 n d flops per query."""
    import torch

    from vicinity_amd import FlatIndex

    k = w.params["k"]
    n, d = w.base.shape
    nq = w.queries.shape[0]
    fx = FlatIndex(d, "l2")
    fx.add(w.base)
    q = torch.from_numpy(w.queries).to("cuda:0")
    out_ids = torch.empty((nq, k), dtype=torch.int64, device="cuda:0")
    out_d = torch.empty((nq, k), dtype=torch.float32, device="cuda:0")
    for _ in range(args.warmup):
        fx.search_device(q, k, out_ids, out_d)
    torch.cuda.synchronize()
    gemm = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        fx.search_device(q, k, out_ids, out_d)
        gemm.append(fx.last_ms()[0])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_step = dt * 1e3 / args.steps
    qps = nq * args.steps / dt
    gemm_ms = float(np.mean(gemm))
    tflops = 2.0 * n * d * nq / (gemm_ms * 1e-3) / 1e12
    fallbacks = fx.last_fallbacks()
    log(f"{qps:.0f} QPS, {ms_step:.3f} ms/batch, ranking {gemm_ms:.3f} ms = {tflops:.1f} TFLOP/s, "
        f"{fallbacks} exhaustive fallbacks")
    gpu_ids = out_ids.cpu().numpy()
    gpu_d = out_d.cpu().numpy()
    cpu = parity = None
    if not args.no_cpu:
        from oracle import oracle as orc

        orc.use_native()
        threads = _baseline_threads()
        probe = 16
        t0 = time.perf_counter()
        orc.flat_search(w.base, w.queries[:probe], k, 0, threads)
        per_q = (time.perf_counter() - t0) / probe
        ns = int(min(nq, max(probe, 15.0 / max(per_q, 1e-9))))
        t0 = time.perf_counter()
        cids, cd = orc.flat_search(w.base, w.queries[:ns], k, 0, threads)
        cqps = ns / (time.perf_counter() - t0)
        cpu = {"value": round(cqps, 1), "unit": "queries/s", "cores": threads, "kind": "port",
               "sample": f"first {ns} of the 10k queries, brute-force l2_distance_squared "
                         f"(oracle, -march=native -ffp-contract=off), {threads} threads",
               "host_cpus": os.cpu_count(), "cpu_model": _cpu_model()}
        parity = {"queries_checked": ns, "ids_equal": bool(np.array_equal(gpu_ids[:ns], cids)),
                  "dists_bitexact": bool(gpu_d[:ns].tobytes() == cd.tobytes())}
        log(f"cpu baseline {cqps:.0f} QPS on {threads} threads; parity {parity}")
    config = {"workload": w.name, "n": n, "d": d, "k": k, "batch": nq, "metric": "l2"}
    rank_bf16 = d <= 128 and k <= 32
    peak = BF16_PEAK_TFLOPS if rank_bf16 else FP32_PEAK_TFLOPS
    line = base_line(args, f"flat exact top-{k} QPS, {w.name} batch {nq // 1000}k; ranking GEMM "
                           f"TFLOP/s vs {'bf16' if rank_bf16 else 'fp32'} MFMA peak", qps, "queries/s",
                     ms_step, "f32", config)
    line.update({
        # achieved: the algorithmic product work 2 n d per query over the ranking
        # kernel's time, against the dense peak of the MFMA type that runs it:
        # bf16 for flat_rank_kernel, which computes each product as three bf16
        # MFMA products (bf16x3; its executed bf16 rate is mfma_bf16_frac of
        # that peak), fp32 for flat_partial_kernel
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(tflops / peak, 4),
                     "traffic": None,
                     "kernel": f"flat_rank_kernel<{(d + 31) // 32}>" if rank_bf16 else "flat_partial_kernel",
                     "kernel_ms": round(gemm_ms, 4),
                     "mfma_dtype": "bf16x3" if rank_bf16 else "f32",
                     "mfma_bf16_frac": round(3 * tflops / BF16_PEAK_TFLOPS, 4) if rank_bf16 else None,
                     "vs_fp32_matrix_peak": round(tflops / FP32_PEAK_TFLOPS, 4),
                     "algorithmic_flops_per_launch": int(2 * n * d * nq)},
        "exhaustive_fallbacks": fallbacks,
        "cpu_baseline": cpu,
        "parity": parity,
    })
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="ivfpq_1m",
                    choices=["ivfpq_1m", "ivfpq_small", "ivfpq_10m", "ivfpq_4bit", "flat"])
    ap.add_argument("--mode", default="fast", choices=["fast", "exact"])
    ap.add_argument("--n", type=int, default=None, help="base vectors (default: the workload's)")
    ap.add_argument("--train-sample", type=int, default=None)
    ap.add_argument("--kmeans-iters", type=int, default=None)
    ap.add_argument("--nprobe", type=int, default=None,
                    help="probed lists per query (default: the workload's; other values are profiling runs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-recall", action="store_true")
    ap.add_argument("--opq", action="store_true",
                    help="build with use_opq (OPQ rotation, EXACT-mode scan of rotated residual "
                         "tables) instead of the product quantizer")
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

    import vicinity_amd as v
    from vicinity_amd import datagen

    if not v.device_available():
        raise RuntimeError("no gfx950 device visible")
    t0 = time.perf_counter()
    gen = datagen.WORKLOADS[args.workload]
    w = gen(n=args.n) if args.n else gen()
    log(f"{w.name}: data {w.base.shape} in {time.perf_counter() - t0:.1f}s")
    line = run_flat(args, w) if args.workload == "flat" else run_ivfpq(args, w)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
