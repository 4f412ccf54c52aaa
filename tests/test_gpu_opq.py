"""OPQ on the GPU (src/ivf_pq/opq.rs; IVF-PQ build with use_opq,
search.rs:732-749): the GPU build's rotation, codebooks and codes equal the
oracle's OPQ build bit for bit, and searches through the C ABI (ranked,
reranked, FastScan ksub 16, filtered) return the oracle's ids and
bit-identical float32 distances on the rotated residual tables."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def vg():
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    return v


def _same(ids, dists, oids, odists):
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()


def _oracle_index(oracle, art):
    return oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                        art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"],
                        art["rotation"])


def _build(vg, n, d, L, M, K, seed, data_seed, sample=None, max_iter=10):
    rng = np.random.default_rng(data_seed)
    base = rng.standard_normal((n, d)).astype(np.float32)
    ix = vg.IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=4,
                       use_opq=True, seed=seed)
    ix.add_items(base)
    ix.build(training_sample_size=sample, kmeans_max_iter=max_iter)
    return ix, base, rng


@pytest.fixture(scope="module")
def k64(vg):
    _print_case("OPQ build 2000 x 32, nlist 16, M 8, ksub 64")
    return _build(vg, 2000, 32, 16, 8, 64, 7, 1)


@pytest.mark.parametrize("case", ["k64", "k16", "sampled"])
def test_opq_build_is_bitexact_with_oracle(vg, oracle, k64, case):
    if case == "k64":
        ix, base, _ = k64
        args = (16, 8, 64, 7, 0, 10)
    elif case == "k16":
        _print_case("OPQ build 1500 x 16, nlist 8, M 4, ksub 16")
        ix, base, _ = _build(vg, 1500, 16, 8, 4, 16, 3, 2)
        args = (8, 4, 16, 3, 0, 10)
    else:
        _print_case("OPQ build 3000 x 16 from a 1000-row sample, nlist 12, M 4, ksub 32")
        ix, base, _ = _build(vg, 3000, 16, 12, 4, 32, 11, 3, sample=1000)
        args = (12, 4, 32, 11, 1000, 10)
    art = ix.export()
    vecs = oracle.normalize_rows(base)
    oix, _ = oracle.ivfpq_build(vecs, *args, use_opq=True)
    assert art["rotation"] is not None
    assert art["rotation"].tobytes() == oix.rotation.tobytes()
    assert art["centroids"].tobytes() == oix.centroids.tobytes()
    assert art["codebooks"].tobytes() == oix.codebooks.tobytes()
    assert np.array_equal(art["list_ids"], oix.list_ids)
    assert np.array_equal(art["codes"], oix.codes)
    R = art["rotation"].astype(np.float64)
    assert np.allclose(R @ R.T, np.eye(R.shape[0]), atol=1e-5)


@pytest.mark.parametrize("mode", ["fast", "exact"])
@pytest.mark.parametrize("k,nprobe,pool", [(10, 4, 0), (1, 1, 0), (50, 16, 0), (10, 6, 40)])
def test_opq_search_is_bitexact(k64, oracle, mode, k, nprobe, pool):
    ix, _, rng = k64
    _print_case(f"OPQ search mode={mode} k={k} nprobe={nprobe} pool={pool}")
    ix.set_mode(mode)
    q = rng.standard_normal((300, 32)).astype(np.float32)
    ids, dists = ix.batch_search(q, k, nprobe=nprobe, rerank_pool=pool or None)
    oids, odists = _oracle_index(oracle, ix.export()).search_batch(q, k, nprobe, pool)
    _same(ids, dists, oids, odists)
    ix.set_mode("fast")


def test_opq_fastscan_ksub16_is_bitexact(vg, oracle):
    _print_case("OPQ ksub 16 search, 4000 x 32, nlist 8, M 8")
    ix, _, rng = _build(vg, 4000, 32, 8, 8, 16, 5, 4)
    q = rng.standard_normal((200, 32)).astype(np.float32)
    ids, dists = ix.batch_search(q, 20, nprobe=3)
    oids, odists = _oracle_index(oracle, ix.export()).search_batch(q, 20, 3)
    _same(ids, dists, oids, odists)


def test_given_rotation_through_load(vg, oracle):
    # an index built elsewhere with an arbitrary orthogonal rotation: only
    # the search side is exercised
    from vicinity_amd import IVFPQIndex

    _print_case("OPQ load_artifacts with a random rotation, 3000 x 64, M 16, ksub 256")
    rng = np.random.default_rng(9)
    vecs = oracle.normalize_rows(rng.standard_normal((3000, 64)).astype(np.float32))
    pix, _ = oracle.ivfpq_build(vecs, 24, 16, 256, 2, 0, 8)
    Q, r = np.linalg.qr(rng.standard_normal((64, 64)))
    R = (Q * np.sign(np.diag(r))).astype(np.float32)
    oix = oracle.Index(pix.centroids, pix.codebooks, pix.list_offsets, pix.list_ids, pix.codes,
                       pix.doc_ids, pix.vectors, 16, pix.K, R)
    ix = IVFPQIndex(64, num_clusters=24, num_codebooks=16, codebook_size=256, nprobe=5,
                    use_opq=True)
    ix.load_artifacts(pix.centroids, pix.codebooks, pix.list_offsets, pix.list_ids, pix.codes,
                      vectors=pix.vectors, rotation=R)
    assert ix.export()["rotation"].tobytes() == R.tobytes()
    q = rng.standard_normal((500, 64)).astype(np.float32)
    for k, pool in ((10, 0), (100, 0), (10, 64)):
        ids, dists = ix.batch_search(q, k, nprobe=5, rerank_pool=pool or None)
        oids, odists = oix.search_batch(q, k, 5, pool)
        _same(ids, dists, oids, odists)
    plain = IVFPQIndex(64, num_clusters=24, num_codebooks=16, codebook_size=256)
    with pytest.raises(ValueError, match="use_opq"):
        plain.load_artifacts(pix.centroids, pix.codebooks, pix.list_offsets, pix.list_ids,
                             pix.codes, rotation=R)


def test_opq_filtered_search_is_bitexact(vg, oracle):
    from vicinity_amd import IVFPQIndex, MetadataFilter

    _print_case("OPQ filtered search 1500 x 16, nlist 8, M 4, ksub 64")
    rng = np.random.default_rng(13)
    ix = IVFPQIndex.with_filtering(16, "g", num_clusters=8, num_codebooks=4, codebook_size=64,
                                   nprobe=2, use_opq=True, seed=17)
    ix.add_items(rng.standard_normal((1500, 16)).astype(np.float32),
                 (70_000 + np.arange(1500)).astype(np.int64))
    for i in range(1500):
        ix.add_metadata(70_000 + i, {"g": i % 5 if i > 2 else 9})
    ix.build(kmeans_max_iter=10)
    art = ix.export()
    oix = _oracle_index(oracle, art)
    cat = np.array([(d - 70_000) % 5 if d - 70_000 > 2 else 9 for d in art["doc_ids"]], np.int8)
    qs, gs = [], []
    for t in range(12):
        g = 9 if t % 4 == 0 else t % 5  # 9: three documents, the probe widens
        q = rng.standard_normal(16).astype(np.float32)
        ids, dists = ix.search_with_filter(q, 10, MetadataFilter.equals("g", g))
        oids, odists = oix.search_filtered(q, 10, 2, g, cat)
        assert ids.tolist() == oids.tolist() and dists.tobytes() == odists.tobytes()
        qs.append(q)
        gs.append(g)
    # A batch whose rotated residuals go in several passes: a query's slots
    # are the lists that carry its category (two or three here), 16 floats
    # each, and the bound holds seven slots, so a pass takes two or three
    # queries and the 12 queries take four to six passes.
    from vicinity_amd import _lib

    _print_case("OPQ filtered batch in several rotation passes")
    _lib.check(_lib.load().vgpu_test_set_rres_limit(ix._h, 7 * 16))
    ids, dists = ix.batch_search_with_filter(np.stack(qs), 10,
                                             [MetadataFilter.equals("g", g) for g in gs])
    for t in range(12):
        oids, odists = oix.search_filtered(qs[t], 10, 2, gs[t], cat)
        m = len(oids)
        assert ids[t, :m].tolist() == oids.tolist() and dists[t, :m].tobytes() == odists.tobytes()
        assert (ids[t, m:] == -1).all()


def test_opq_snapshot_round_trip(k64, tmp_path):
    from vicinity_amd import IVFPQIndex

    ix, _, rng = k64
    q = rng.standard_normal((100, 32)).astype(np.float32)
    before = ix.batch_search(q, 10, rerank_pool=30)
    ix.save(tmp_path)
    loaded = IVFPQIndex.load(tmp_path)
    assert loaded.use_opq
    assert loaded.export()["rotation"].tobytes() == ix.export()["rotation"].tobytes()
    after = loaded.batch_search(q, 10, rerank_pool=30)
    _same(before[0], before[1], after[0], after[1])


@pytest.mark.parametrize("d,M,K,L", [
    (18, 3, 32, 8),     # d % 4 != 0: the rotation's scalar path
    (200, 8, 100, 12),  # d > 128 and ksub 100: the table read from the codebooks per list
    (300, 10, 64, 10),  # d > 256: several rotation outputs per thread
])
def test_opq_shapes_build_and_search_bitexact(vg, oracle, d, M, K, L):
    _print_case(f"OPQ shape d={d} M={M} ksub={K} nlist={L}")
    ix, base, rng = _build(vg, 1200, d, L, M, K, 21, d)
    art = ix.export()
    oix, _ = oracle.ivfpq_build(oracle.normalize_rows(base), L, M, K, 21, 0, 10, use_opq=True)
    assert art["rotation"].tobytes() == oix.rotation.tobytes()
    assert art["codebooks"].tobytes() == oix.codebooks.tobytes()
    assert np.array_equal(art["codes"], oix.codes)
    q = rng.standard_normal((80, d)).astype(np.float32)
    for k, nprobe, pool in ((10, 4, 0), (25, L, 0), (5, 3, 20)):
        ids, dists = ix.batch_search(q, k, nprobe=nprobe, rerank_pool=pool or None)
        oids, odists = _oracle_index(oracle, art).search_batch(q, k, nprobe, pool)
        _same(ids, dists, oids, odists)
