"""Full-size runs of the other benchmark configurations, each whole 10k-query
batch checked against the oracle (16 threads) and through size-independent
properties:

- 10M x 96 angular IVF-PQ (nlist 16384, M 48 x 2, ksub 256, nprobe 64, k 10);
- 1M x 100 4-bit FastScan IVF-PQ with rerank (nlist 2048, M 50 x 2, ksub 16,
  nprobe 64, pool 100, k 10);
- 100k x 96 flat L2 (k 10), 10k queries.

Base and query vectors are drawn on the GPU from a seeded torch generator with
the distributions of vicinity_amd/datagen.py (mixtures on the unit sphere,
std 0.1), because the numpy generator needs minutes at 10M rows.  The oracle
runs every query on the arrays the GPU build exports, and checks the build
itself: list assignment and PQ codes of sampled vectors recomputed by the
oracle from the exported centroids and codebooks (argmin, ties to the lowest
index)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


def _sphere_mixture(n, d, centres, std, seed):
    import torch

    g = torch.Generator(device="cuda:0").manual_seed(seed)
    c = torch.randn(centres, d, generator=g, device="cuda:0")
    c /= c.norm(dim=1, keepdim=True)
    out = np.empty((n, d), np.float32)
    step = 1 << 21
    for s in range(0, n, step):
        e = min(n, s + step)
        lab = torch.randint(0, centres, (e - s,), generator=g, device="cuda:0")
        x = c[lab] + std * torch.randn(e - s, d, generator=g, device="cuda:0")
        x /= x.norm(dim=1, keepdim=True)
        out[s:e] = x.cpu().numpy()
    return out


def _check_rows(ids, dists, k):
    """Every row ascending, ids unique within a row, no padding (each query has
    at least k candidates at these shapes)."""
    assert ids.shape[1] == k
    assert (ids >= 0).all()
    assert np.all(np.diff(dists, axis=1) >= 0)
    s = np.sort(ids, axis=1)
    assert (s[:, 1:] != s[:, :-1]).all()


def _check_build(oracle, art, vecs, sample):
    """Assignment and codes of sampled vectors equal the oracle's argmins on the
    exported centroids and codebooks (residual = x - c, search.rs:722-729)."""
    off = art["list_offsets"].astype(np.int64)
    pos_of = np.empty(len(art["list_ids"]), np.int64)
    pos_of[art["list_ids"]] = np.arange(len(art["list_ids"]))
    lst = np.searchsorted(off, pos_of[sample], side="right") - 1
    assign = oracle.assign_cosine(vecs[sample], art["centroids"])
    assert np.array_equal(lst, assign.astype(np.int64))
    M, K = art["M"], art["K"]
    d = art["centroids"].shape[1]
    resid = (vecs[sample] - art["centroids"][lst]).astype(np.float32)
    codes = oracle.pq_encode(art["codebooks"], M, K, d // M, resid)
    assert np.array_equal(codes.reshape(len(sample), M), art["codes"][sample])


def test_config_10m_d96_angular(oracle):
    from vicinity_amd import IVFPQIndex

    _print_case("10M x 96 angular: generate")
    base = _sphere_mixture(10_000_000, 96, 10_000, 0.1, 40)
    queries = _sphere_mixture(10_000, 96, 10_000, 0.1, 41)
    _print_case("10M x 96 angular: build")
    ix = IVFPQIndex(96, num_clusters=16384, num_codebooks=48, codebook_size=256, nprobe=64, seed=42)
    ix.add_items(base)
    ix.build(training_sample_size=262_144, kmeans_max_iter=10)
    ix.compact()  # no rerank here; keeps the export small
    _print_case("10M x 96 angular: search")
    ids, dists = ix.batch_search(queries, 10)
    _check_rows(ids, dists, 10)
    art = ix.export()
    rng = np.random.default_rng(7)
    _print_case("10M x 96 angular: oracle on all 10k queries")
    oix = oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                       art["codes"], art["doc_ids"], None, art["M"], art["K"])
    oids, odists = oix.search_batch(queries, 10, 64, threads=16)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()
    _check_build(oracle, art, oracle.normalize_rows(base), rng.choice(len(base), 4000, replace=False))
    # EXACT mode agrees with FAST on the whole batch (same reference arithmetic)
    _print_case("10M x 96 angular: exact mode")
    ix.set_mode("exact")
    eids, edists = ix.batch_search(queries[:2000], 10)
    assert np.array_equal(eids, ids[:2000])
    assert edists.tobytes() == dists[:2000].tobytes()


def test_config_1m_d100_fastscan_rerank(oracle):
    from vicinity_amd import IVFPQIndex

    _print_case("1M x 100 FastScan + rerank: generate")
    base = _sphere_mixture(1_000_000, 100, 500, 0.1, 50)
    queries = _sphere_mixture(10_000, 100, 500, 0.1, 51)
    _print_case("1M x 100 FastScan + rerank: build")
    ix = IVFPQIndex(100, num_clusters=2048, num_codebooks=50, codebook_size=16, nprobe=64, seed=42)
    ix.add_items(base)
    ix.build(training_sample_size=262_144, kmeans_max_iter=10)
    _print_case("1M x 100 FastScan + rerank: search")
    ids, dists = ix.batch_search(queries, 10, rerank_pool=100)
    _check_rows(ids, dists, 10)
    art = ix.export()
    rng = np.random.default_rng(8)
    _print_case("1M x 100 FastScan + rerank: oracle on all 10k queries")
    oix = oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                       art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"])
    oids, odists = oix.search_batch(queries, 10, 64, rerank_pool=100, threads=16)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()
    # without rerank (FastScan distances)
    _print_case("1M x 100 FastScan, no rerank: oracle on all 10k queries")
    pids, pdists = ix.batch_search(queries, 10)
    oids, odists = oix.search_batch(queries, 10, 64, threads=16)
    assert np.array_equal(pids, oids)
    assert pdists.tobytes() == odists.tobytes()
    _check_build(oracle, art, art["vectors"], rng.choice(len(base), 4000, replace=False))


def test_config_flat_100k_d96(oracle):
    from vicinity_amd import FlatIndex, datagen

    _print_case("flat 100k x 96 L2, 10k queries")
    w = datagen.flat_gaussian()
    fx = FlatIndex(96, "l2")
    fx.add(w.base)
    ids, dists = fx.search(w.queries, 10)
    _check_rows(ids, dists, 10)
    _print_case("flat 100k x 96 L2: oracle on all 10k queries")
    oids, odists = oracle.flat_search(w.base, w.queries, 10, metric=0, threads=16)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()


def test_config_1m_d128_headline(oracle):
    """The configuration the benchmark is quoted on, built exactly as
    bench.py builds it: 1M x 128 Gaussian mixture (datagen.ivfpq_1m), nlist
    4096, M 16 x 8, ksub 256, nprobe 32, k 100, training sample 262,144, 25
    k-means iterations.  The whole 10k batch equals the oracle on the exported
    arrays (ids, float32 bits); the build's assignments and codes are the
    oracle's argmins on 4,000 sampled vectors; EXACT mode equals FAST."""
    from vicinity_amd import IVFPQIndex, datagen

    _print_case("1M x 128 headline: generate")
    w = datagen.ivfpq_1m()
    p = w.params
    _print_case("1M x 128 headline: build")
    ix = IVFPQIndex(128, num_clusters=p["num_clusters"], num_codebooks=p["num_codebooks"],
                    codebook_size=p["codebook_size"], nprobe=p["nprobe"], seed=42)
    ix.add_items(w.base)
    ix.build(training_sample_size=262_144, kmeans_max_iter=25)
    k, nprobe = p["k"], p["nprobe"]
    _print_case("1M x 128 headline: search 10k")
    ids, dists = ix.batch_search(w.queries, k, nprobe=nprobe)
    st = ix.last_stats()
    _check_rows(ids, dists, k)
    art = ix.export()
    _print_case("1M x 128 headline: oracle on all 10k queries")
    oix = oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                       art["codes"], art["doc_ids"], None, art["M"], art["K"])
    oids, odists = oix.search_batch(w.queries, k, nprobe, threads=16)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()
    # the probe sets themselves (search.rs:1602-1617) on a sample
    rng = np.random.default_rng(10)
    qs = rng.choice(len(w.queries), 500, replace=False)
    probes = ix.probe(w.queries[qs], nprobe)
    for row, qi in zip(probes, qs):
        assert row.tolist() == oix.probe(w.queries[qi], nprobe)[0].tolist()
    _print_case("1M x 128 headline: build argmins")
    _check_build(oracle, art, art["vectors"], rng.choice(len(w.base), 4000, replace=False))
    _print_case("1M x 128 headline: exact mode")
    ix.set_mode("exact")
    eids, edists = ix.batch_search(w.queries[:2000], k, nprobe=nprobe)
    assert np.array_equal(eids, ids[:2000])
    assert edists.tobytes() == dists[:2000].tobytes()
    assert st["nq"] == len(w.queries) and st["candidates"] > 0
