"""GPU parity of search_with_filter (src/ivf_pq/search.rs:1407-1549) through
the C ABI against the oracle on the same index arrays and categories: ids
equal and float32 distances bit-identical."""

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


def _metadata(i):
    """Document i's metadata: a group for most, no group field for some, none for a few."""
    if i % 11 == 0:
        return {"label": f"doc-{i}"} if i % 2 == 0 else None
    return {"group": i % 7, "label": f"doc-{i}"}


def _build(vg, n, d, L, M, K, nprobe, data_seed, doc_base=10_000):
    rng = np.random.default_rng(data_seed)
    base = rng.standard_normal((n, d)).astype(np.float32)
    ix = vg.IVFPQIndex.with_filtering(d, "group", num_clusters=L, num_codebooks=M,
                                      codebook_size=K, nprobe=nprobe, seed=42)
    ids = (doc_base + np.arange(n)).astype(np.int64)
    ix.add_items(base, ids)
    for i in range(n):
        md = _metadata(i)
        if md is not None:
            ix.add_metadata(int(ids[i]), md)
    ix.build(kmeans_max_iter=10)
    return ix, rng


def _oracle_index(oracle, art):
    return oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                        art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"])


def _categories(art, cat_of_doc):
    return np.array([cat_of_doc(int(doc)) for doc in art["doc_ids"]], dtype=np.int8)


def _group_of(doc, doc_base=10_000):
    md = _metadata(doc - doc_base)
    return md["group"] if md is not None and "group" in md else -1


@pytest.fixture(scope="module")
def k256(vg, oracle):
    _print_case("build filtered index 6000 x 32, nlist 32, M 8, ksub 256")
    ix, rng = _build(vg, 6000, 32, 32, 8, 256, 3, 1)
    art = ix.export()
    return ix, art, _oracle_index(oracle, art), _categories(art, _group_of), rng


@pytest.mark.parametrize("k", [1, 10, 100, 700])
def test_filtered_search_is_bitexact(k256, k):
    from vicinity_amd import MetadataFilter

    ix, art, oix, cat, rng = k256
    _print_case(f"filtered search k={k}")
    for t in range(12):
        q = rng.standard_normal(32).astype(np.float32)
        g = t % 7
        ids, dists = ix.search_with_filter(q, k, MetadataFilter.equals("group", g))
        oids, odists = oix.search_filtered(q, k, 3, g, cat)
        assert ids.tolist() == oids.tolist(), (t, g)
        assert dists.tobytes() == odists.tobytes(), (t, g)
        assert all(cat[np.flatnonzero(art["doc_ids"] == i)[0]] == g for i in ids.tolist())


@pytest.mark.parametrize("d,M", [(64, 16), (64, 8), (32, 16), (96, 16)])
def test_filtered_widths_against_oracle(vg, oracle, d, M):
    """Subvector widths a half, a quarter or three quarters of the widest the
    kernels hold in registers (4, 8, 2 and 6 floats)."""
    from vicinity_amd import MetadataFilter

    _print_case(f"build filtered index 4000 x {d}, nlist 16, M {M}, ksub 256")
    ix, rng = _build(vg, 4000, d, 16, M, 256, 3, 3 + d + M)
    art = ix.export()
    oix, cat = _oracle_index(oracle, art), _categories(art, _group_of)
    for k in (10, 100):
        for t in range(6):
            q = rng.standard_normal(d).astype(np.float32)
            ids, dists = ix.search_with_filter(q, k, MetadataFilter.equals("group", t % 7))
            oids, odists = oix.search_filtered(q, k, 3, t % 7, cat)
            assert ids.tolist() == oids.tolist() and dists.tobytes() == odists.tobytes(), (k, t)


def test_ksub16_uses_the_table_arithmetic(vg, oracle):
    _print_case("build filtered index 3000 x 16, nlist 16, M 4, ksub 16")
    ix, rng = _build(vg, 3000, 16, 16, 4, 16, 2, 2)
    art = ix.export()
    oix, cat = _oracle_index(oracle, art), _categories(art, _group_of)
    from vicinity_amd import MetadataFilter

    for t in range(10):
        q = rng.standard_normal(16).astype(np.float32)
        ids, dists = ix.search_with_filter(q, 25, MetadataFilter.equals("group", t % 7))
        oids, odists = oix.search_filtered(q, 25, 2, t % 7, cat)
        assert ids.tolist() == oids.tolist() and dists.tobytes() == odists.tobytes()


def test_widens_past_nprobe(vg, oracle):
    # search.rs:2652-2688: three documents carry tag 0, the rest tag 1; with
    # nprobe 1 all three come back however their lists lie.
    from vicinity_amd import IVFPQIndex, MetadataFilter

    _print_case("widening case 240 x 16, nlist 8, nprobe 1")
    rng = np.random.default_rng(77)
    ix = IVFPQIndex.with_filtering(16, "tag", num_clusters=8, num_codebooks=4, codebook_size=16,
                                   nprobe=1, seed=919)
    ix.add_items(rng.random((240, 16), dtype=np.float32),
                 (50_000 + np.arange(240)).astype(np.int64))
    for i in range(240):
        ix.add_metadata(50_000 + i, {"tag": 0 if i < 3 else 1})
    ix.build(kmeans_max_iter=10)
    art = ix.export()
    oix = _oracle_index(oracle, art)
    cat = np.array([0 if d < 50_003 else 1 for d in art["doc_ids"]], np.int8)
    for t in range(10):
        q = rng.random(16, dtype=np.float32)
        ids, dists = ix.search_with_filter(q, 5, MetadataFilter.equals("tag", 0))
        assert sorted(ids.tolist()) == [50_000, 50_001, 50_002]
        oids, odists = oix.search_filtered(q, 5, 1, 0, cat)
        assert ids.tolist() == oids.tolist() and dists.tobytes() == odists.tobytes()


def test_metadata_after_build_keeps_the_build_time_bitmasks(k256, oracle):
    ix, art, oix, cat, rng = k256
    from vicinity_amd import MetadataFilter

    masks = oix.list_masks(cat)  # the lists as built
    moved = [10_001, 10_002, 10_100]
    for doc in moved:
        ix.add_metadata(doc, {"group": 5})
    new = cat.copy()
    for doc in moved:
        new[np.flatnonzero(art["doc_ids"] == doc)[0]] = 5
    q = rng.standard_normal(32).astype(np.float32)
    for g in (5, 1):
        ids, dists = ix.search_with_filter(q, 40, MetadataFilter.equals("group", g))
        oids, odists = oix.search_filtered(q, 40, 3, g, new, list_mask=masks)
        assert ids.tolist() == oids.tolist() and dists.tobytes() == odists.tobytes()
    for doc in moved:  # restore for the other tests
        ix.add_metadata(doc, _metadata(doc - 10_000))


def test_filter_errors(vg, k256):
    from vicinity_amd import IVFPQIndex, MetadataFilter
    from vicinity_amd import _lib

    ix, art, oix, cat, rng = k256
    q = rng.standard_normal(32).astype(np.float32)
    with pytest.raises(ValueError, match="non-equality"):
        ix.search_with_filter(q, 5, MetadataFilter.range("group", 1, 2))
    with pytest.raises(ValueError, match="doesn't match"):
        ix.search_with_filter(q, 5, MetadataFilter.equals("label", 1))
    with pytest.raises(ValueError, match="exceeds bitmask limit"):
        ix.search_with_filter(q, 5, MetadataFilter.equals("group", 64))
    with pytest.raises(ValueError, match="exceeds bitmask limit"):
        ix.add_metadata(10_000, {"group": 99})
    with pytest.raises(ValueError, match="dimension mismatch"):
        ix.search_with_filter(q[:16].copy(), 5, MetadataFilter.equals("group", 1))
    assert ix.search_with_filter(q, 0, MetadataFilter.equals("group", 1))[0].size == 0
    L = _lib.load()
    assert L.vgpu_ivfpq_enable_filtering(ix._h) == _lib.ERR_ALREADY_BUILT
    plain = IVFPQIndex(16, num_clusters=4, num_codebooks=4, codebook_size=16)
    with pytest.raises(ValueError, match="with_filtering"):
        plain.add_metadata(1, {"group": 1})
    assert L.vgpu_ivfpq_set_category(plain._h, 1, 1) == _lib.ERR_UNSUPPORTED
    plain.add_items(rng.random((64, 16), dtype=np.float32))
    plain.build(kmeans_max_iter=5)
    with pytest.raises(ValueError, match="doesn't match"):
        plain.search_with_filter(rng.random(16, dtype=np.float32), 5,
                                 MetadataFilter.equals("group", 1))


def test_nprobe_zero_widens_on_a_fresh_handle_and_after_a_search(vg, oracle):
    """set_nprobe(0) probes no list, so every list that carries the category
    is a widening candidate (search.rs:1486-1545).  The queries must still be
    normalised for the scan, on a handle that never searched and on one whose
    last search left other queries in its buffers."""
    from vicinity_amd import MetadataFilter, _lib

    _print_case("filtered search with nprobe 0 (fresh handle, then after a search)")
    ix, rng = _build(vg, 2000, 32, 16, 8, 256, 3, 5)
    art = ix.export()
    oix, cat = _oracle_index(oracle, art), _categories(art, _group_of)
    L = _lib.load()
    _lib.check(L.vgpu_ivfpq_set_nprobe(ix._h, 0))
    queries = rng.standard_normal((6, 32)).astype(np.float32)
    for t, q in enumerate(queries):
        if t == 3:  # a plain search in between refills the workspace with other queries
            ix.batch_search(rng.standard_normal((64, 32)).astype(np.float32), 10, nprobe=4)
        g = t % 7
        ids, dists = ix.search_with_filter(q, 20, MetadataFilter.equals("group", g))
        oids, odists = oix.search_filtered(q, 20, 0, g, cat)
        assert ids.tolist() == oids.tolist(), t
        assert dists.tobytes() == odists.tobytes(), t
        assert len(ids) == 20


def test_batched_filter_rows_equal_single_queries(k256):
    from vicinity_amd import MetadataFilter

    ix, art, oix, cat, rng = k256
    _print_case("batched filtered search vs one query at a time")
    qs = rng.standard_normal((40, 32)).astype(np.float32)
    filters = [MetadataFilter.equals("group", t % 7) for t in range(40)]
    for k in (1, 17, 700):
        ids, dists = ix.batch_search_with_filter(qs, k, filters)
        for t in range(40):
            sids, sd = ix.search_with_filter(qs[t], k, filters[t])
            m = len(sids)
            assert ids[t, :m].tolist() == sids.tolist() and dists[t, :m].tobytes() == sd.tobytes()
            assert (ids[t, m:] == -1).all() and np.isinf(dists[t, m:]).all()
