"""Snapshots on the GPU: an index saved in the reference's directory format and
loaded back searches exactly as before (search.rs:2495-2588, :3027-3072),
and a snapshot's arrays searched by the oracle give the loaded index's results."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def built():
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    _print_case("build 4000 x 32, nlist 32, M 8, ksub 256 with filtering")
    rng = np.random.default_rng(21)
    ix = v.IVFPQIndex.with_filtering(32, "group", num_clusters=32, num_codebooks=8,
                                     codebook_size=256, nprobe=4, seed=5)
    ix.add_items(rng.standard_normal((4000, 32)).astype(np.float32),
                 (30_000 + np.arange(4000)).astype(np.int64))
    for i in range(4000):
        ix.add_metadata(30_000 + i, {"group": i % 4, "label": f"doc-{i}"})
    ix.build(kmeans_max_iter=10)
    return ix, rng.standard_normal((64, 32)).astype(np.float32)


def _results(ix, q):
    from vicinity_amd import MetadataFilter

    out = {"approx": ix.batch_search(q, 10), "rerank": ix.batch_search(q, 10, rerank_pool=50)}
    for g in range(4):
        out[f"filter{g}"] = ix.search_with_filter(q[g], 10, MetadataFilter.equals("group", g))
    return out


def _same(a, b):
    assert a.keys() == b.keys()
    for key in a:
        ia, da = a[key]
        ib, db = b[key]
        assert np.array_equal(ia, ib), key
        assert da.tobytes() == db.tobytes(), key


def test_save_load_round_trip(built, tmp_path):
    from vicinity_amd import IVFPQIndex

    ix, q = built
    before = _results(ix, q)
    ix.save(tmp_path)
    _print_case("load snapshot")
    loaded = IVFPQIndex.load(tmp_path)
    assert loaded.num_vectors == 4000 and loaded.nprobe == 4
    _same(before, _results(loaded, q))
    loaded.set_mode("exact")
    ix.set_mode("exact")
    _same(_results(ix, q), _results(loaded, q))
    ix.set_mode("fast")


def test_snapshot_arrays_through_the_oracle(built, tmp_path, oracle):
    from vicinity_amd import IVFPQIndex
    from vicinity_amd.snapshot import read_snapshot

    ix, q = built
    ix.save(tmp_path)
    s = read_snapshot(tmp_path)
    oix = oracle.Index(s["centroids"], s["codebooks"], s["list_offsets"], s["list_ids"],
                       s["codes"], s["doc_ids"], s["vectors"], s["M"], s["K"])
    loaded = IVFPQIndex.load(tmp_path)
    ids, dists = loaded.batch_search(q, 10)
    oids, odists = oix.search_batch(q, 10, 4)
    assert np.array_equal(ids, oids) and dists.tobytes() == odists.tobytes()


def test_build_time_bitmasks_survive_the_snapshot(built, tmp_path):
    from vicinity_amd import IVFPQIndex, MetadataFilter

    ix, q = built
    moved = [30_001, 30_005, 30_123]
    for doc in moved:
        ix.add_metadata(doc, {"group": 9})  # a category no list held at build time
    try:
        before = [ix.search_with_filter(q[0], 10, MetadataFilter.equals("group", g)) for g in (9, 1)]
        assert before[0][0].size == 0
        ix.save(tmp_path)
        loaded = IVFPQIndex.load(tmp_path)
        after = [loaded.search_with_filter(q[0], 10, MetadataFilter.equals("group", g)) for g in (9, 1)]
        for (ia, da), (ib, db) in zip(before, after):
            assert np.array_equal(ia, ib) and da.tobytes() == db.tobytes()
    finally:
        for doc in moved:
            ix.add_metadata(doc, {"group": (doc - 30_000) % 4, "label": f"doc-{doc - 30_000}"})


def test_compacted_snapshot_keeps_approximate_search_only(tmp_path):
    # search.rs:3027-3072
    from vicinity_amd import IVFPQIndex

    rng = np.random.default_rng(12)
    ix = IVFPQIndex(16, num_clusters=4, num_codebooks=4, codebook_size=16, nprobe=4, seed=124)
    ix.add_items(rng.random((200, 16), dtype=np.float32))
    ix.build(kmeans_max_iter=10)
    ix.compact()
    q = rng.random((8, 16), dtype=np.float32)
    before = ix.batch_search(q, 10)
    ix.save(tmp_path)
    loaded = IVFPQIndex.load(tmp_path)
    after = loaded.batch_search(q, 10)
    assert np.array_equal(before[0], after[0]) and before[1].tobytes() == after[1].tobytes()
    with pytest.raises(ValueError):
        loaded.batch_search(q, 10, rerank_pool=80)
    with pytest.raises(ValueError, match="save before build"):
        IVFPQIndex(16, num_clusters=4, num_codebooks=4, codebook_size=16).save(tmp_path / "x")
