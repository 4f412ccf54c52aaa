"""Non-finite queries on the device entry points.

vgpu_ivfpq_search_batch (host buffers) rejects a query holding a NaN or an
infinity before any device work.  The device entry point cannot look at the
queries on the host, so the normalisation kernels mark such a row, search it
as the zero vector, and the end of the call pads its result row with
(-1, +inf) and returns VGPU_ERR_INVALID_PARAMETER.  These tests check that:
the error, padding in exactly the offending rows, and every other row equal
to a search of the same batch without the offending rows.  Paths covered:
the fused coarse kernel (d <= 128, nprobe <= 64), the GEMM coarse path
(nprobe above 64), a reranked search (rows mapped by the finish kernel) and
nprobe 0 (no list probed)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ERR_INVALID_PARAMETER = 2


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def indexes():
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    _print_case("non-finite: build 20000 x 32 (nlist 64 and nlist 160)")
    w = v.datagen.ivfpq_small()
    a = v.IVFPQIndex(32, num_clusters=64, num_codebooks=8, codebook_size=256, nprobe=8, seed=3)
    a.add_items(w.base)
    a.build(kmeans_max_iter=8)
    b = v.IVFPQIndex(32, num_clusters=160, num_codebooks=8, codebook_size=256, nprobe=8, seed=4)
    b.add_items(w.base)
    b.build(kmeans_max_iter=8)
    return a, b, w.queries[:300].copy()


def _with_bad_rows(q):
    bad = q.copy()
    rows = [0, 17, 64, 65, 299]
    bad[0, 5] = np.nan
    bad[17, 0] = np.inf
    bad[64, 31] = -np.inf
    bad[65, :] = np.nan
    bad[299, 12] = np.float32(np.nan)
    return bad, rows


def _device(ix, q, k, nprobe, pool):
    import torch

    t = torch.from_numpy(q).to("cuda:0")
    ids = torch.full((q.shape[0], k), -7, dtype=torch.int64, device="cuda:0")
    dists = torch.full((q.shape[0], k), -7.0, dtype=torch.float32, device="cuda:0")
    err = None
    try:
        ix.search_batch_device(t, k, nprobe, rerank_pool=pool, out_ids=ids, out_dists=dists)
    except ValueError as e:
        err = e
    torch.cuda.synchronize()
    return err, ids.cpu().numpy(), dists.cpu().numpy()


def _noalloc(ix, q, k, nprobe, pool):
    import torch

    from vicinity_amd import _lib

    t = torch.from_numpy(q).to("cuda:0")
    ids = torch.full((q.shape[0], k), -7, dtype=torch.int64, device="cuda:0")
    dists = torch.full((q.shape[0], k), -7.0, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    rc = _lib.load().vgpu_ivfpq_search_batch_device_noalloc(
        ix._h, t.data_ptr(), q.shape[0], q.shape[1], k, nprobe, pool, ids.data_ptr(),
        dists.data_ptr(), None)
    return rc, ids.cpu().numpy(), dists.cpu().numpy()


def _check_rows(q, bad_rows, ids, dists, want_ids, want_d):
    good = np.setdiff1d(np.arange(q.shape[0]), bad_rows)
    assert (ids[bad_rows] == -1).all()
    assert np.isposinf(dists[bad_rows]).all()
    assert np.array_equal(ids[good], want_ids[good])
    assert dists[good].tobytes() == want_d[good].tobytes()


@pytest.mark.parametrize("which,k,nprobe,pool", [
    ("fused", 10, 8, None),
    ("fused", 20, 64, 50),
    ("gemm", 10, 100, None),
    ("gemm", 7, 90, 30),
])
def test_device_entry_reports_and_pads_nonfinite_queries(indexes, which, k, nprobe, pool):
    a, b, q = indexes
    ix = a if which == "fused" else b
    _print_case(f"non-finite: search_batch_device {which} k {k} nprobe {nprobe} pool {pool}")
    bad, rows = _with_bad_rows(q)
    want_ids, want_d = ix.batch_search(q, k, nprobe=nprobe, rerank_pool=pool)
    err, ids, dists = _device(ix, bad, k, nprobe, pool)
    assert err is not None and err.code == ERR_INVALID_PARAMETER and "non-finite" in str(err)
    _check_rows(q, rows, ids, dists, want_ids, want_d)
    # the same handle then searches a clean batch normally
    err, ids, dists = _device(ix, q, k, nprobe, pool)
    assert err is None
    assert np.array_equal(ids, want_ids) and dists.tobytes() == want_d.tobytes()


def test_noalloc_entry_reports_and_pads_nonfinite_queries(indexes):
    a, _, q = indexes
    bad, rows = _with_bad_rows(q)
    for k, nprobe, pool in [(10, 8, 0), (15, 8, 40)]:
        _print_case(f"non-finite: no-alloc k {k} nprobe {nprobe} pool {pool}")
        want_ids, want_d = a.batch_search(q, k, nprobe=nprobe, rerank_pool=pool or None)
        rc, ids, dists = _noalloc(a, bad, k, nprobe, pool)
        assert rc == ERR_INVALID_PARAMETER
        _check_rows(q, rows, ids, dists, want_ids, want_d)
        rc, ids, dists = _noalloc(a, q, k, nprobe, pool)
        assert rc == 0
        assert np.array_equal(ids, want_ids) and dists.tobytes() == want_d.tobytes()


def test_nprobe_zero_still_checks_the_queries(indexes):
    a, _, q = indexes
    bad, _ = _with_bad_rows(q)
    _print_case("non-finite: index nprobe 0 (no list probed)")
    a.set_nprobe(0)
    try:
        err, ids, dists = _device(a, bad, 5, None, None)
        assert err is not None and err.code == ERR_INVALID_PARAMETER
        assert (ids == -1).all() and np.isposinf(dists).all()
        err, ids, dists = _device(a, q, 5, None, None)
        assert err is None and (ids == -1).all() and np.isposinf(dists).all()
        rc, ids, _ = _noalloc(a, bad, 5, 0, 0)
        assert rc == ERR_INVALID_PARAMETER and (ids == -1).all()
    finally:
        a.set_nprobe(8)


def test_large_finite_values_are_not_rejected(indexes):
    """Finite values whose squares overflow normalise to zeros, as in the
    reference (search.rs:55-62: x / inf); they are valid queries."""
    a, _, q = indexes
    big = q[:20].copy()
    big[3] = np.float32(3e38)
    _print_case("non-finite: finite rows with an overflowing norm")
    want_ids, want_d = a.batch_search(big, 10, nprobe=8)
    err, ids, dists = _device(a, big, 10, 8, None)
    assert err is None
    assert np.array_equal(ids, want_ids) and dists.tobytes() == want_d.tobytes()
