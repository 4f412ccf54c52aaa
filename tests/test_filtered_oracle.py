"""search_with_filter (src/ivf_pq/search.rs:1407-1549): the oracle's
restatement, pinned by the reference's own filtered-search test (the widening
case, search.rs:2652-2688), by full probe == an exhaustive float64 scan of the
category over the reconstructed vectors, by the build-time list bitmasks
(search.rs:626-648), and the metadata predicate semantics
(src/filtering/mod.rs:151-218) of the Python mirror."""

import math

import numpy as np
import pytest

from vicinity_amd.filtering import (MetadataFilter, filter_category, metadata_category,
                                    metadata_value)


def _index(oracle, n, d, L, M, K, seed, data_seed, doc_base=0):
    rng = np.random.default_rng(data_seed)
    base = rng.random((n, d), dtype=np.float32)
    vecs = oracle.normalize_rows(base)
    oix, assign = oracle.ivfpq_build(vecs, L, M, K, seed, 0, 25)
    oix = oracle.Index(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                       (doc_base + np.arange(n)).astype(np.uint32), oix.vectors, M, oix.K)
    return oix, assign, rng


def _reconstruct(oracle, oix, assign, v):
    ds = oix.d // oix.M
    return oix.centroids[assign[v]].astype(np.float64) + oracle.pq_reconstruct(
        oix.codebooks, oix.M, oix.K, ds, oix.codes[v]).astype(np.float64)


def test_widens_past_nprobe_to_the_only_tagged_documents(oracle):
    # search.rs:2652-2688: nprobe 1, three documents carry tag 0 and the rest
    # tag 1; k = 5 must return exactly the three, wherever their lists are.
    n, dim = 240, 16
    oix, assign, rng = _index(oracle, n, dim, 8, 4, 16, 919, 77, doc_base=50_000)
    cat = np.where(np.arange(n) < 3, 0, 1).astype(np.int8)
    widened = 0
    for t in range(20):
        q = rng.random(dim, dtype=np.float32)
        ids, dists = oracle.Index.search_filtered(oix, q, 5, 1, 0, cat)
        assert sorted(ids.tolist()) == [50_000, 50_001, 50_002]
        assert np.all(np.diff(dists) >= 0)
        probed = oix.probe(q, 1)[0].tolist()
        widened += any(int(assign[v]) not in probed for v in range(3))
    assert widened > 0, "no query needed the widening"


def test_full_probe_equals_exhaustive_scan_of_the_category(oracle):
    # search.rs:2589-2645 restricted to a category: with nprobe = nlist the
    # filtered result is the k nearest reconstructed vectors of the category.
    n, dim, L = 256, 16, 32
    oix, assign, rng = _index(oracle, n, dim, L, 4, 16, 7, 4242)
    cat = (np.arange(n) % 5).astype(np.int8)
    for c in range(5):
        q = oracle.normalize_rows(rng.random((1, dim), dtype=np.float32))[0]
        ids, dists = oix.search_filtered(q, 10, L, c, cat)
        members = [v for v in range(n) if cat[v] == c]
        exact = sorted((float(np.sum((q.astype(np.float64) - _reconstruct(oracle, oix, assign, v)) ** 2)),
                        v) for v in members)
        assert ids.tolist() == [v for _, v in exact[:10]]
        for (e, _), dd in zip(exact[:10], dists):
            assert math.isclose(e, float(dd), rel_tol=1e-4, abs_tol=1e-5)


def test_results_carry_the_category_and_short_categories_come_back_whole(oracle):
    n, dim = 600, 16
    oix, assign, rng = _index(oracle, n, dim, 16, 4, 256, 3, 5)
    cat = rng.integers(-1, 6, n).astype(np.int8)  # -1: no value for the field
    cat[rng.integers(0, n, 4)] = 7  # a rare category
    q = rng.random(dim, dtype=np.float32)
    for c in range(6):
        ids, _ = oix.search_filtered(q, 20, 2, c, cat)
        assert len(ids) == 20 and all(cat[v] == c for v in ids.tolist())
    ids, _ = oix.search_filtered(q, 50, 2, 7, cat)  # fewer than k anywhere: all of them
    assert sorted(ids.tolist()) == sorted(np.flatnonzero(cat == 7).tolist())
    ids, _ = oix.search_filtered(q, 5, 2, 9, cat)  # no such category
    assert ids.size == 0
    with pytest.raises(ValueError):
        oix.search_filtered(q, 5, 2, 64, cat)


def test_list_bitmasks_are_taken_at_build_time(oracle):
    # search.rs:626-648 vs :1504-1506: a document whose category changes after
    # the lists were built is skipped when its list never held that category.
    n, dim = 400, 16
    oix, assign, rng = _index(oracle, n, dim, 8, 4, 16, 11, 9)
    old = np.where(np.arange(n) % 2 == 0, 0, 1).astype(np.int8)
    masks = oix.list_masks(old)
    for l in range(8):
        members = oix.list_ids[oix.list_offsets[l]:oix.list_offsets[l + 1]]
        want = 0
        for v in members:
            want |= 1 << int(old[v])
        assert int(masks[l]) == want
    new = old.copy()
    new[5] = 2  # category 2 existed in no list at build time
    q = rng.random(dim, dtype=np.float32)
    ids, _ = oix.search_filtered(q, 5, 8, 2, new, list_mask=masks)
    assert ids.size == 0
    ids, _ = oix.search_filtered(q, 5, 8, 2, new)  # lists rebuilt with the new metadata
    assert ids.tolist() == [5]


# ---- metadata predicates (filtering/mod.rs) -----------------------------------

def test_metadata_values_are_typed():
    assert metadata_value(True) == ("bool", True)
    assert metadata_value(3) == ("int", 3)
    assert metadata_value(3.0) == ("float", 3.0)
    assert metadata_value("x") == ("str", "x")
    with pytest.raises(TypeError):
        metadata_value([1])
    with pytest.raises(ValueError):
        metadata_value(1 << 63)


def test_equality_and_range_semantics():
    eq = MetadataFilter.equals("g", 2)
    assert eq.matches({"g": 2}) and not eq.matches({"g": 2.0}) and not eq.matches({"g": True})
    assert not eq.matches({"h": 2})
    assert MetadataFilter.equals("b", True).matches({"b": True})
    r = MetadataFilter.range("x", 1.0, 2.0)
    assert r.matches({"x": 1.0}) and r.matches({"x": 2.0}) and r.matches({"x": 1.5})
    assert not r.matches({"x": 2.5}) and not r.matches({"x": 1}) and not r.matches({"x": float("nan")})
    assert MetadataFilter.range("x", min=3).matches({"x": 7})
    assert not MetadataFilter.range("s", "b", "d").matches({"s": "e"})
    both = MetadataFilter.and_([eq, MetadataFilter.range("x", max=0)])
    assert both.matches({"g": 2, "x": -1}) and not both.matches({"g": 2, "x": 1})
    either = MetadataFilter.or_([eq, MetadataFilter.equals("h", "a")])
    assert either.matches({"h": "a"}) and not either.matches({"h": "b"})


def test_filtered_search_accepts_only_an_integer_equality_on_the_field():
    # search.rs:1429-1457
    assert filter_category(MetadataFilter.equals("category", 5), "category") == 5
    with pytest.raises(ValueError, match="non-equality"):
        filter_category(MetadataFilter.range("category", 1, 2), "category")
    with pytest.raises(ValueError, match="doesn't match"):
        filter_category(MetadataFilter.equals("other", 1), "category")
    with pytest.raises(ValueError, match="doesn't match"):
        filter_category(MetadataFilter.equals("category", 1), None)
    with pytest.raises(ValueError, match="exceeds bitmask limit"):
        filter_category(MetadataFilter.equals("category", 64), "category")
    with pytest.raises(ValueError, match="must be an integer"):
        filter_category(MetadataFilter.equals("category", "a"), "category")


def test_add_metadata_checks_the_filter_field():
    # search.rs:445-465
    assert metadata_category({"category": 0}, "category") == 0
    assert metadata_category({"label": "x"}, "category") == -1
    with pytest.raises(ValueError, match="exceeds bitmask limit"):
        metadata_category({"category": 64}, "category")
    with pytest.raises(ValueError, match="exceeds bitmask limit"):
        metadata_category({"category": -1}, "category")
    with pytest.raises(ValueError, match="must be an integer"):
        metadata_category({"category": 1.0}, "category")
