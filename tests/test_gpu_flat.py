"""GPU parity of the flat exact search (src/distance.rs:78-109 brute force,
the reference's ground truth, src/ivf_pq/search.rs:3376-3392) against the
oracle: ids equal and float32 distances bit-identical, over the shapes of
the bf16x3 ranking kernel (d <= 128, k <= 32: one to four 32-dimension
steps, ragged d and n, several workgroups of queries and database slices)
and of the fp32 path it falls back to (k > 32, d > 128), with exact
duplicates (ties at the threshold) and zero vectors."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


def _check(ids, dists, oids, odists):
    assert ids.shape == oids.shape
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()


@pytest.mark.parametrize("n,d,nq,k", [
    (50, 7, 5, 3),          # four tiles, one of them partial
    (1000, 32, 129, 10),    # one 32-dim step, queries across two workgroups
    (3001, 33, 40, 32),     # two steps (d just past 32), k at the limit
    (20_000, 96, 300, 10),  # config-2 dims, several slices
    (9000, 100, 64, 1),     # ragged d, k = 1
    (17_000, 128, 260, 17), # four steps, three query workgroups
])
@pytest.mark.parametrize("metric", [0, 1])
def test_flat_rank_kernel_shapes(oracle, n, d, nq, k, metric):
    from vicinity_amd import FlatIndex

    _print_case(f"flat n={n} d={d} nq={nq} k={k} metric={metric}")
    rng = np.random.default_rng(n + d + k + metric)
    base = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    if metric == 1:
        base = oracle.normalize_rows(base)
        q = oracle.normalize_rows(q)
    fx = FlatIndex(d, "l2" if metric == 0 else "cosine")
    fx.add(base)
    ids, dists = fx.search(q, k)
    oids, odists = oracle.flat_search(base, q, k, metric=metric)
    _check(ids, dists, oids, odists)


@pytest.mark.parametrize("k", [5, 33, 100])
def test_flat_duplicates_zero_vectors_and_fallback_path(oracle, k):
    """200 exact copies of one vector around the queries (equal ranking keys at
    the threshold, so the gap test fails and the exhaustive exact scan runs),
    zero rows, and k above the ranking kernel's 32 (the fp32 path)."""
    from vicinity_amd import FlatIndex

    _print_case(f"flat duplicates k={k}")
    rng = np.random.default_rng(7 + k)
    base = rng.standard_normal((6000, 64)).astype(np.float32)
    base[1000:1200] = base[17]
    base[3000:3010] = 0.0
    q = np.concatenate([base[17:18] + 1e-3 * rng.standard_normal((3, 64)).astype(np.float32),
                        rng.standard_normal((20, 64)).astype(np.float32),
                        np.zeros((1, 64), np.float32)])
    fx = FlatIndex(64, "l2")
    fx.add(base)
    ids, dists = fx.search(q, k)
    oids, odists = oracle.flat_search(base, q, k, metric=0)
    _check(ids, dists, oids, odists)


def test_flat_wide_rows_take_the_fp32_path(oracle):
    from vicinity_amd import FlatIndex

    _print_case("flat d=160 (fp32 path)")
    rng = np.random.default_rng(3)
    base = rng.standard_normal((4000, 160)).astype(np.float32)
    q = rng.standard_normal((50, 160)).astype(np.float32)
    fx = FlatIndex(160, "l2")
    fx.add(base)
    ids, dists = fx.search(q, 10)
    oids, odists = oracle.flat_search(base, q, 10, metric=0)
    _check(ids, dists, oids, odists)


@pytest.mark.parametrize("metric,nnear", [(0, 4), (1, 4), (0, 300)])
def test_flat_fallback_rescans_crowded_lanes(oracle, metric, nnear):
    """Near-copies of one vector crowded into single ranking lanes (more than
    the four keys a lane keeps, so the merge cannot prove the result and the
    fallback rescans those lanes' columns) beside near-copies spread one per
    lane in another slice (kept keys, rescored) and exact duplicates (ties
    broken by index).  40000 rows make 32 slices of 80 tiles: vector
    16 (80 s + t) + c is slice s, lane c.  300 such queries pass the 256 the
    device-driven fallback takes, so the rest run after the final wait."""
    from vicinity_amd import FlatIndex

    _print_case(f"flat crowded lanes metric={metric} near queries={nnear}")
    rng = np.random.default_rng(71 + metric)
    n, d = 40_000, 64
    base = rng.standard_normal((n, d)).astype(np.float32)
    v = base[17].copy()
    near = lambda m, s: v + s * rng.standard_normal((m, d)).astype(np.float32)  # noqa: E731
    base[(160 + np.arange(12)) * 16 + 5] = near(12, 1e-4)      # slice 2, lane 5
    base[(560 + 3) * 16 + np.arange(6)] = near(6, 1e-4)       # slice 7, lanes 0-5
    base[(1600 + 2 * np.arange(5)) * 16 + 9] = v              # slice 20, lane 9
    q = np.concatenate([near(nnear, 1e-3), rng.standard_normal((20, d)).astype(np.float32)])
    if metric == 1:
        base = oracle.normalize_rows(base)
        q = oracle.normalize_rows(q)
    fx = FlatIndex(d, "l2" if metric == 0 else "cosine")
    fx.add(base)
    for k in (10, 32, 3):
        ids, dists = fx.search(q, k)
        oids, odists = oracle.flat_search(base, q, k, metric=metric)
        _check(ids, dists, oids, odists)
        assert fx.last_fallbacks() >= nnear, k
