"""GPU parity: every kernel called through the C ABI against the oracle on the
same seeded inputs.  Integer/byte/index outputs and distances are compared
bit for bit (the engine is built to return the oracle's float32 values)."""

import numpy as np
import pytest

from tests.helpers import total_cmp_key

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vg():
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    return v


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


# ---- per-kernel ------------------------------------------------------------

def test_normalize_is_bitexact(vg, oracle):
    from vicinity_amd import _lib

    rng = np.random.default_rng(0)
    x = rng.standard_normal((300, 37)).astype(np.float32)
    x[5] = 0.0
    x[6] = 1e-12
    x[7] *= np.float32(1e20)
    out = np.empty_like(x)
    _lib.check(_lib.load().vgpu_test_normalize(_lib.ptr(x), 300, 37, _lib.ptr(out)))
    assert out.tobytes() == oracle.normalize_rows(x).tobytes()


@pytest.mark.parametrize("nq,L,d", [(70, 100, 36), (64, 64, 32), (1, 3, 128), (130, 257, 100)])
def test_coarse_mfma_dots(vg, nq, L, d):
    from vicinity_amd import _lib

    rng = np.random.default_rng(nq + L + d)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    c = rng.standard_normal((L, d)).astype(np.float32)
    out = np.empty((nq, L), np.float32)
    _lib.check(_lib.load().vgpu_test_coarse_dots(_lib.ptr(q), nq, _lib.ptr(c), L, d, _lib.ptr(out)))
    ref = q.astype(np.float64) @ c.astype(np.float64).T
    bound = (d + 2) * 2.0 ** -24 * (np.abs(q).astype(np.float64) @ np.abs(c).astype(np.float64).T)
    assert (np.abs(out - ref) <= bound + 1e-30).all()


@pytest.mark.parametrize("M,K,ds", [(2, 3, 1), (4, 256, 2), (3, 16, 8), (2, 7, 10)])
def test_adc_tables_are_bitexact(vg, oracle, M, K, ds):
    from vicinity_amd import _lib

    rng = np.random.default_rng(M * K * ds)
    cb = rng.standard_normal(M * K * ds).astype(np.float32)
    r = rng.standard_normal((9, M * ds)).astype(np.float32)
    out = np.empty((9, M * K), np.float32)
    _lib.check(_lib.load().vgpu_test_adc_tables(_lib.ptr(cb), M, K, ds, _lib.ptr(r), 9, _lib.ptr(out)))
    for t in range(9):
        assert out[t].tobytes() == oracle.adc_table(cb, M, K, ds, r[t]).tobytes()
    # pq.rs:335-350 known answer through the GPU
    cb1 = np.array([0.0, 1.0, 3.0, -1.0, 2.0, 4.0], np.float32)
    q1 = np.array([[2.0, 1.0]], np.float32)
    o1 = np.empty(6, np.float32)
    _lib.check(_lib.load().vgpu_test_adc_tables(_lib.ptr(cb1), 2, 3, 1, _lib.ptr(q1), 1, _lib.ptr(o1)))
    assert o1.tolist() == [4.0, 1.0, 1.0, 4.0, 1.0, 9.0]


@pytest.mark.parametrize("M,K,ds", [(8, 256, 4), (4, 16, 2), (3, 5, 10), (2, 256, 16)])
def test_pq_encode_is_bitexact(vg, oracle, M, K, ds):
    from vicinity_amd import _lib

    rng = np.random.default_rng(7 * M + K + ds)
    cb = rng.standard_normal(M * K * ds).astype(np.float32)
    x = rng.standard_normal((1000, M * ds)).astype(np.float32)
    x[3] = 0.0
    codes = np.empty((1000, M), np.uint8)
    _lib.check(_lib.load().vgpu_test_pq_encode(_lib.ptr(cb), M, K, ds, _lib.ptr(x), 1000, _lib.ptr(codes)))
    assert np.array_equal(codes, oracle.pq_encode(cb, M, K, ds, x))


@pytest.mark.parametrize("n,M", [(1, 1), (32, 8), (100, 8), (33, 5), (488, 50), (64, 257)])
def test_fastscan_is_bitexact(vg, oracle, n, M):
    from vicinity_amd import _lib

    rng = np.random.default_rng(n * 1000 + M)
    codes = rng.integers(0, 16, n * M, dtype=np.uint8)
    lut = (rng.random(M * 16) * 3).astype(np.float32)
    packed = oracle.pack4(codes, n, M)
    out = np.empty(n, np.float32)
    _lib.check(_lib.load().vgpu_test_fastscan(_lib.ptr(packed), n, M, _lib.ptr(lut), _lib.ptr(out)))
    assert out.tobytes() == oracle.fastscan_batch(packed, n, M, lut).tobytes()


def test_fastscan_refuses_u16_overflow(vg):
    from vicinity_amd import _lib

    M = 258
    packed = np.zeros(16 * M, np.uint8)
    lut = np.ones(M * 16, np.float32)
    out = np.empty(32, np.float32)
    with pytest.raises(ValueError, match="overflow"):
        _lib.check(_lib.load().vgpu_test_fastscan(_lib.ptr(packed), 32, M, _lib.ptr(lut), _lib.ptr(out)))


# ---- whole index -----------------------------------------------------------

def _oracle_index(oracle, art):
    return oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                        art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"])


def _assert_same_results(ids_a, d_a, ids_b, d_b):
    assert ids_a.shape == ids_b.shape
    assert d_a.tobytes() == d_b.tobytes()
    assert np.array_equal(ids_a, ids_b)


@pytest.fixture(scope="module")
def small(vg, oracle):
    """20k x 32 uniform, nlist 64, M 8, ksub 256: built on the GPU, then
    rebuilt by the oracle from the same normalised vectors."""
    from vicinity_amd import IVFPQIndex, datagen

    w = datagen.ivfpq_small()
    p = w.params
    _print_case("build ivfpq_small on GPU")
    ix = IVFPQIndex(32, num_clusters=p["num_clusters"], num_codebooks=p["num_codebooks"],
                    codebook_size=p["codebook_size"], nprobe=p["nprobe"], seed=42)
    ix.add_items(w.base)
    ix.build(kmeans_max_iter=p["kmeans_max_iter"])
    art = ix.export()
    return ix, art, w


def test_gpu_build_is_bitexact_with_oracle_build(small, oracle):
    ix, art, w = small
    vecs = oracle.normalize_rows(w.base)
    assert art["vectors"].tobytes() == vecs.tobytes()  # add_slice normalisation
    oix, assign = oracle.ivfpq_build(vecs, 64, 8, 256, 42, 0, 10)
    assert art["centroids"].tobytes() == oix.centroids.tobytes()
    assert art["codebooks"].tobytes() == oix.codebooks.tobytes()
    assert np.array_equal(art["list_offsets"], oix.list_offsets)
    assert np.array_equal(art["list_ids"], oix.list_ids)
    assert np.array_equal(art["codes"], oix.codes)


@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_small_search_is_bitexact(small, oracle, mode):
    ix, art, w = small
    _print_case(f"ivfpq_small search mode={mode}")
    ix.set_mode(mode)
    ids, dists = ix.batch_search(w.queries, 10, nprobe=8)
    oids, odists = _oracle_index(oracle, art).search_batch(w.queries, 10, 8)
    _assert_same_results(ids, dists, oids, odists)
    st = ix.last_stats()
    assert st["nq"] == 1000
    ix.set_mode("fast")


def test_small_probe_sets_are_bitexact(small, oracle):
    ix, art, w = small
    lists = ix.probe(w.queries[:200], 8)
    oix = _oracle_index(oracle, art)
    for i in range(200):
        assert lists[i].tolist() == oix.probe(w.queries[i], 8)[0].tolist()


@pytest.mark.parametrize("k,nprobe", [(1, 1), (100, 8), (37, 64), (250, 3)])
def test_small_search_shapes(small, oracle, k, nprobe):
    ix, art, w = small
    q = w.queries[:64]
    ids, dists = ix.batch_search(q, k, nprobe=nprobe)
    oids, odists = _oracle_index(oracle, art).search_batch(q, k, nprobe)
    _assert_same_results(ids, dists, oids, odists)


def test_small_rerank_is_bitexact(small, oracle):
    ix, art, w = small
    ids, dists = ix.batch_search(w.queries[:100], 10, nprobe=8, rerank_pool=50)
    oids, odists = _oracle_index(oracle, art).search_batch(w.queries[:100], 10, 8, rerank_pool=50)
    _assert_same_results(ids, dists, oids, odists)


def test_single_search_and_self_retrieval(small, oracle):
    ix, art, w = small
    ids, dists = ix.search(w.base[5], 5, nprobe=8, rerank_pool=64)
    assert ids[0] == 5 and abs(dists[0]) < 1e-4
    assert ids.dtype == np.int64 and dists.dtype == np.float32
    # scaled query gives the same ids (correctness_regression :109-131)
    a, _ = ix.search(w.queries[3], 10)
    b, _ = ix.search((w.queries[3] * np.float32(5.3)).astype(np.float32), 10)
    assert a.tolist() == b.tolist()


def test_edge_cases(small, oracle, vg):
    ix, art, w = small
    # k larger than every candidate -> padding (python.rs:778-785)
    ids, dists = ix.batch_search(w.queries[:3], 2000, nprobe=1)
    n1 = int(np.sum(ids[0] >= 0))
    assert (ids[0, n1:] == -1).all() and np.isinf(dists[0, n1:]).all()
    # zero query: every centroid ties (coarse overflow path), lower index wins
    z = np.zeros((1, 32), np.float32)
    ids, dists = ix.batch_search(z, 10, nprobe=8)
    oids, odists = _oracle_index(oracle, art).search_batch(z, 10, 8)
    _assert_same_results(ids, dists, oids, odists)
    # k = 0 -> empty rows
    ids, _ = ix.batch_search(w.queries[:2], 0)
    assert ids.shape == (2, 0)
    with pytest.raises(ValueError, match="dimension"):
        ix.batch_search(np.zeros((2, 31), np.float32), 5)
    bad = w.queries[:2].copy()
    bad[1, 3] = np.nan
    with pytest.raises(ValueError, match="non-finite"):
        ix.batch_search(bad, 5)


def test_not_built_and_empty_errors(vg):
    from vicinity_amd import IVFPQIndex

    ix = IVFPQIndex(8, num_clusters=4, num_codebooks=4, codebook_size=8)
    with pytest.raises(ValueError, match="before build"):
        ix.batch_search(np.zeros((1, 8), np.float32), 3)
    with pytest.raises(ValueError, match="empty"):
        ix.build()
    ix.add_items(np.eye(8, dtype=np.float32)[:4])
    with pytest.raises(ValueError, match="codebook_size"):
        ix.build()
    with pytest.raises(ValueError, match="duplicate doc_id"):
        ix.add_items(np.eye(8, dtype=np.float32)[:2], ids=np.array([11, 11]))
    assert len(ix) == 4


def test_batch_search_padding_with_rerank(vg):
    # test_python.py:555-563 through this engine
    from vicinity_amd import MISSING_DISTANCE, MISSING_LABEL, IVFPQIndex

    x = np.random.default_rng(0).standard_normal((16, 8), dtype=np.float32)
    ix = IVFPQIndex(8, num_clusters=8, num_codebooks=4, codebook_size=8, nprobe=8, seed=0)
    ix.add_items(x)
    ix.build(training_sample_size=16, kmeans_max_iter=5)
    ids, dists = ix.batch_search(x[:2], 20, nprobe=8, rerank_pool=16)
    assert ids.shape == (2, 20)
    assert np.all(ids[:, 16:] == MISSING_LABEL) and np.all(dists[:, 16:] == MISSING_DISTANCE)
    ids, dists = ix.search(x[0], 5, nprobe=8, rerank_pool=16)
    assert ids[0] == 0 and abs(float(dists[0])) < 1e-4


@pytest.mark.parametrize("d,M,K,L,n", [(96, 48, 256, 32, 6000), (50, 25, 64, 16, 3000),
                                       (100, 50, 16, 24, 8000), (16, 4, 16, 48, 256)])
def test_other_shapes_via_load_artifacts(vg, oracle, d, M, K, L, n):
    """Oracle-built indexes uploaded through vgpu_ivfpq_load: the M=48, generic
    M / ksub, and 4-bit FastScan (with exact small lists) kernels."""
    from vicinity_amd import IVFPQIndex

    _print_case(f"load_artifacts d={d} M={M} K={K} L={L} n={n}")
    rng = np.random.default_rng(d + M + K)
    vecs = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    oix, _ = oracle.ivfpq_build(vecs, L, M, K, 3, 0, 8)
    ix = IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=L // 2)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                      doc_ids=np.arange(n, dtype=np.uint32) * 3 + 7, vectors=vecs)
    oix.doc_ids = np.arange(n, dtype=np.uint32) * 3 + 7
    oix.__post_init__()
    q = oracle.normalize_rows(rng.standard_normal((50, d)).astype(np.float32))
    for mode in ["fast", "exact"]:
        ix.set_mode(mode)
        ids, dists = ix.batch_search(q, 10, nprobe=L // 2)
        oids, odists = oix.search_batch(q, 10, L // 2)
        _assert_same_results(ids, dists, oids, odists)
    ids, dists = ix.batch_search(q, 10, nprobe=L // 2, rerank_pool=60)
    oids, odists = oix.search_batch(q, 10, L // 2, rerank_pool=60)
    _assert_same_results(ids, dists, oids, odists)


def test_duplicate_vectors_tie_by_insertion_index(vg, oracle):
    from vicinity_amd import IVFPQIndex

    rng = np.random.default_rng(11)
    base = rng.standard_normal((400, 16)).astype(np.float32)
    x = np.concatenate([base, base, base])  # every vector three times
    vecs = oracle.normalize_rows(x)
    oix, _ = oracle.ivfpq_build(vecs, 8, 4, 16, 5, 0, 10)
    ix = IVFPQIndex(16, num_clusters=8, num_codebooks=4, codebook_size=16, nprobe=4)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                      vectors=vecs)
    ids, dists = ix.batch_search(base[:20], 9, nprobe=4)
    oids, odists = oix.search_batch(base[:20], 9, 4)
    _assert_same_results(ids, dists, oids, odists)
    k = total_cmp_key(dists[0])
    assert (np.diff(k.astype(np.int64)) >= 0).all()


def test_flat_search_is_bitexact(vg, oracle):
    from vicinity_amd import FlatIndex, datagen

    w = datagen.flat_gaussian(n=20_000, nq=300)
    fx = FlatIndex(96, "l2")
    fx.add(w.base)
    ids, dists = fx.search(w.queries, 10)
    oids, odists = oracle.flat_search(w.base, w.queries, 10, metric=0)
    _assert_same_results(ids, dists, oids, odists)
    fc = FlatIndex(96, "cosine")
    xb = oracle.normalize_rows(w.base[:5000])
    xq = oracle.normalize_rows(w.queries[:100])
    fc.add(xb)
    ids, dists = fc.search(xq, 7)
    oids, odists = oracle.flat_search(xb, xq, 7, metric=1)
    _assert_same_results(ids, dists, oids, odists)


@pytest.mark.parametrize("copies,k", [(40, 9), (700, 5), (700, 100)])
def test_fast_scan_ties_and_fallback_match_oracle(vg, oracle, copies, k):
    """Byte codes with heavy exact duplicates: equal approximate distances at
    the buffer threshold (ties kept), and with 700 copies more ties than the
    buffer holds, which sends the query to the EXACT kernel.  Both must return
    the oracle's rows (ties ordered by insertion index)."""
    from vicinity_amd import IVFPQIndex

    _print_case(f"fast ties copies={copies} k={k}")
    rng = np.random.default_rng(copies + k)
    distinct = rng.standard_normal((60, 16)).astype(np.float32)
    x = np.concatenate([np.repeat(distinct[:1], copies, axis=0), np.repeat(distinct[1:], 20, axis=0)])
    vecs = oracle.normalize_rows(x)
    oix, _ = oracle.ivfpq_build(vecs, 4, 4, 256, 9, 0, 10)
    ix = IVFPQIndex(16, num_clusters=4, num_codebooks=4, codebook_size=256, nprobe=4)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                      vectors=vecs)
    q = np.concatenate([distinct[:3], rng.standard_normal((5, 16)).astype(np.float32)])
    for mode in ["fast", "exact"]:
        ix.set_mode(mode)
        ids, dists = ix.batch_search(q, k, nprobe=4)
        oids, odists = oix.search_batch(q, k, 4)
        _assert_same_results(ids, dists, oids, odists)


@pytest.mark.parametrize("copies,expect", [(200, "second_pass"), (900, "exact_rerun")])
def test_fast_second_pass_and_exact_rerun(vg, oracle, copies, expect):
    """Near-duplicates (copies of one vector with 1e-6 noise) put hundreds of
    approximate distances inside the proof window A_k + 2 tau.  With 200 copies
    the FAST kernel's second pass collects them all (its buffer holds 256 past
    a flush for k = 5); with 900 they overflow it and the query is rerun by
    the EXACT kernel.  Both must return the oracle's rows, and the statistics
    must show which path ran."""
    from vicinity_amd import IVFPQIndex

    _print_case(f"fast second pass copies={copies}")
    rng = np.random.default_rng(copies)
    v0 = rng.standard_normal(16).astype(np.float32)
    near = (v0 + rng.standard_normal((copies, 16)).astype(np.float32) * np.float32(1e-6))
    x = np.concatenate([near.astype(np.float32), rng.standard_normal((1100, 16)).astype(np.float32)])
    vecs = oracle.normalize_rows(x)
    oix, _ = oracle.ivfpq_build(vecs, 4, 4, 256, 13, 0, 10)
    ix = IVFPQIndex(16, num_clusters=4, num_codebooks=4, codebook_size=256, nprobe=4)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                      vectors=vecs)
    q = v0[None, :].copy()
    ix.set_mode("fast")
    ids, dists = ix.batch_search(q, 5, nprobe=4)
    st = ix.last_stats()
    oids, odists = oix.search_batch(q, 5, 4)
    _assert_same_results(ids, dists, oids, odists)
    if expect == "second_pass":
        assert st["fast_retries"] == 1 and st["fallback_queries"] == 0, st
    else:
        assert st["fallback_queries"] == 1, st


@pytest.mark.parametrize("d,L,P", [(24, 37, 8), (16, 300, 20), (32, 2000, 40), (16, 13, 13)])
def test_probe_selection_paths(vg, oracle, d, L, P):
    """Probe lists for L not a multiple of the 16-list tile or the 64-list
    stage, L < 16 and P = L (every list probed), P above 32 (the 16-key lane
    lists), and zero queries (all scores tie).  Lists must equal the oracle's,
    ties by lower list index."""
    from vicinity_amd import IVFPQIndex

    _print_case(f"probe paths d={d} L={L} P={P}")
    rng = np.random.default_rng(d * L + P)
    cent = oracle.normalize_rows(rng.standard_normal((L, d)).astype(np.float32))
    n = 4 * L
    M, K = 4, 4
    ds = d // M
    cb = rng.standard_normal(M * K * ds).astype(np.float32)
    assign = np.arange(n) % L
    off, ids = oracle.build_lists(assign.astype(np.uint32), L)
    codes = rng.integers(0, K, (n, M), dtype=np.uint8)
    ix = IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=P)
    ix.load_artifacts(cent, cb, off, ids, codes)
    q = rng.standard_normal((40, d)).astype(np.float32)
    q[3] = 0.0
    q[17] = 0.0
    lists = ix.probe(q, P)
    oix = oracle.Index(cent, cb, off, ids, codes, np.arange(n, dtype=np.uint32), None, M, K)
    for i in range(len(q)):
        assert lists[i].tolist() == oix.probe(q[i], P)[0].tolist(), i


@pytest.mark.parametrize("nq,L,d", [(70, 100, 36), (64, 64, 32), (1, 3, 128), (130, 257, 100),
                                    (200, 4096, 128)])
def test_coarse_bf16x3_dots_within_bound(vg, nq, L, d):
    """Split-bfloat16 MFMA dot products (the search path's coarse kernel)
    against float64, within the bound its proof window uses:
    (3.01 * 2^-16 + 7 d u) sum|q_j c_j|.  A wrong operand or output lane layout
    fails by orders of magnitude."""
    from vicinity_amd import _lib

    rng = np.random.default_rng(nq * 7 + L + d)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    c = rng.standard_normal((L, d)).astype(np.float32)
    out = np.empty((nq, L), np.float32)
    _lib.check(_lib.load().vgpu_test_coarse_dots_bf16x3(_lib.ptr(q), nq, _lib.ptr(c), L, d, _lib.ptr(out)))
    ref = q.astype(np.float64) @ c.astype(np.float64).T
    absdot = np.abs(q).astype(np.float64) @ np.abs(c).astype(np.float64).T
    bound = (3.01 * 2.0 ** -16 + 7 * d * 2.0 ** -24) * absdot
    err = np.abs(out - ref)
    assert (err <= bound + 1e-30).all(), float((err / (absdot + 1e-30)).max())


@pytest.mark.parametrize("step,copies,P", [(16, 12, 8), (1, 12, 8), (16, 20, 40), (3, 30, 32)])
def test_probe_ties_through_the_exact_fallback(vg, oracle, step, copies, P):
    """Copies of one centroid at lists 5, 5 + step, ...: with step 16 they all
    share one lane's column class and overflow its key list, so the query
    takes the exact fallback; with other steps the tie window spans lanes.
    Either way the P lists are the copies in index order (oracle ties by
    lower index), then the next nearest."""
    from vicinity_amd import IVFPQIndex

    _print_case(f"probe ties step={step} copies={copies} P={P}")
    d, L = 32, 700
    rng = np.random.default_rng(step * 100 + copies + P)
    cent = oracle.normalize_rows(rng.standard_normal((L, d)).astype(np.float32))
    base = cent[1].copy()
    cent[5 + step * np.arange(copies)] = base
    n = 2 * L
    M, K = 4, 16
    cb = rng.standard_normal(M * K * (d // M)).astype(np.float32)
    off, ids = oracle.build_lists((np.arange(n) % L).astype(np.uint32), L)
    codes = rng.integers(0, K, (n, M), dtype=np.uint8)
    ix = IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=P)
    ix.load_artifacts(cent, cb, off, ids, codes)
    q = (base[None, :] + 0.01 * rng.standard_normal((6, d))).astype(np.float32)
    q[0] = base
    lists = ix.probe(q, P)
    oix = oracle.Index(cent, cb, off, ids, codes, np.arange(n, dtype=np.uint32), None, M, K)
    for i in range(len(q)):
        assert lists[i].tolist() == oix.probe(q[i], P)[0].tolist(), i


def test_many_flagged_probe_queries(vg, oracle):
    """More queries through the coarse exact fallback than its grid-wide
    path takes (64): 100 queries near a centroid copied 12 times in one lane's
    column class, among 60 ordinary queries, over 2000 lists (8 slices of
    256).  Probe lists equal the oracle's, in order."""
    from vicinity_amd import IVFPQIndex

    _print_case("probe ties: 100 flagged queries of 160, L 2000")
    d, L, P, copies = 32, 2000, 16, 12
    rng = np.random.default_rng(77)
    cent = oracle.normalize_rows(rng.standard_normal((L, d)).astype(np.float32))
    base = cent[1].copy()
    cent[5 + 16 * np.arange(copies)] = base
    n = 2 * L
    M, K = 4, 16
    cb = rng.standard_normal(M * K * (d // M)).astype(np.float32)
    off, ids = oracle.build_lists((np.arange(n) % L).astype(np.uint32), L)
    codes = rng.integers(0, K, (n, M), dtype=np.uint8)
    ix = IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=P)
    ix.load_artifacts(cent, cb, off, ids, codes)
    near = (base[None, :] + 0.01 * rng.standard_normal((100, d))).astype(np.float32)
    q = np.concatenate([near[:50], rng.standard_normal((60, d)).astype(np.float32), near[50:]])
    oix = oracle.Index(cent, cb, off, ids, codes, np.arange(n, dtype=np.uint32), None, M, K)
    for rep in range(2):  # the second call reuses the slice counters the first one reset
        lists = ix.probe(q, P)
        for i in range(len(q)):
            assert lists[i].tolist() == oix.probe(q[i], P)[0].tolist(), (rep, i)

@pytest.mark.parametrize("P", [48, 64])
def test_wide_candidate_window_probe_ties(vg, oracle, P):
    """Above 32 probes the coarse lists keep ten keys and a query may bring up
    to 320 candidates to the exact order: 300 exact copies of one centroid,
    spread over every column class (about five per kept list, so no list
    overflows), all tie for a query near them.  Probe lists equal the
    oracle's, ties in list order (find_nearest_centroids, search.rs:1602-1617)."""
    from vicinity_amd import IVFPQIndex

    _print_case(f"probe ties: 300 copies of a centroid, nprobe {P}, L 4096")
    d, L, copies = 32, 4096, 300
    rng = np.random.default_rng(5 + P)
    cent = oracle.normalize_rows(rng.standard_normal((L, d)).astype(np.float32))
    base = cent[7].copy()
    cent[(7 + 13 * np.arange(copies)) % L] = base
    n = 2 * L
    M, K = 4, 16
    cb = rng.standard_normal(M * K * (d // M)).astype(np.float32)
    off, ids = oracle.build_lists((np.arange(n) % L).astype(np.uint32), L)
    codes = rng.integers(0, K, (n, M), dtype=np.uint8)
    ix = IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=P)
    ix.load_artifacts(cent, cb, off, ids, codes)
    near = (base[None, :] + 0.001 * rng.standard_normal((40, d))).astype(np.float32)
    q = np.concatenate([near, rng.standard_normal((24, d)).astype(np.float32)])
    oix = oracle.Index(cent, cb, off, ids, codes, np.arange(n, dtype=np.uint32), None, M, K)
    lists = ix.probe(q, P)
    for i in range(len(q)):
        assert lists[i].tolist() == oix.probe(q[i], P)[0].tolist(), i
    # nearly all of the 40 tied windows went through the candidate order, not
    # the exact fallback (a window that also takes near-tied other lists may
    # still overflow a kept list)
    ix.batch_search(q, 10, nprobe=P)
    assert ix.last_stats()["coarse_overflow"] <= 4
