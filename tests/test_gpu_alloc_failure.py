"""Device-allocation failures through the C ABI (the injection hook
vgpu_test_fail_device_allocations): a failed allocation in a search, an
upload, a build or a flat-index add returns VGPU_ERR_OUT_OF_MEMORY, leaves
the handle usable, and the same call succeeds once the hook is disarmed,
with results equal to the oracle's."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture
def fail():
    from vicinity_amd import _lib

    def arm(after, count=1):
        _lib.check(_lib.load().vgpu_test_fail_device_allocations(after, count))

    yield arm
    arm(0, 0)


def _oom(excinfo):
    from vicinity_amd import _lib

    assert excinfo.value.code == _lib.ERR_OUT_OF_MEMORY
    assert "injected" in str(excinfo.value)


def _oracle_index(oracle, art):
    return oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                        art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"])


def test_search_upload_and_build_recover_from_allocation_failure(oracle, fail):
    import vicinity_amd as v
    from vicinity_amd import VicinityGpuError

    assert v.device_available(), "no gfx950 device visible"
    w = v.datagen.ivfpq_small(n=6000, nq=200)
    _print_case("alloc failure: build 6000 x 32, nlist 32 with the 4th allocation failing")
    ix = v.IVFPQIndex(32, num_clusters=32, num_codebooks=8, codebook_size=256, nprobe=4, seed=3)
    ix.add_items(w.base)
    fail(3)
    with pytest.raises(VicinityGpuError) as e:
        ix.build(kmeans_max_iter=5)
    _oom(e)
    fail(0, 0)
    assert not ix.is_built
    ix.build(kmeans_max_iter=5)
    art = ix.export()
    oix, _ = oracle.ivfpq_build(oracle.normalize_rows(w.base), 32, 8, 256, 3, 0, 5)
    assert art["codes"].tobytes() == oix.codes.tobytes()
    assert art["centroids"].tobytes() == oix.centroids.tobytes()

    _print_case("alloc failure: first search on the handle (workspace allocation)")
    fail(0)
    with pytest.raises(VicinityGpuError) as e:
        ix.batch_search(w.queries, 10)
    _oom(e)
    fail(0, 0)
    ids, dists = ix.batch_search(w.queries, 10)
    oids, odists = _oracle_index(oracle, art).search_batch(w.queries, 10, 4)
    assert np.array_equal(ids, oids) and dists.tobytes() == odists.tobytes()

    _print_case("alloc failure: load_artifacts with the 3rd upload failing")
    ix2 = v.IVFPQIndex(32, num_clusters=32, num_codebooks=8, codebook_size=256, nprobe=4)
    args = (art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"], art["codes"])
    fail(2)
    with pytest.raises(VicinityGpuError) as e:
        ix2.load_artifacts(*args, vectors=art["vectors"])
    _oom(e)
    fail(0, 0)
    ix2.load_artifacts(*args, vectors=art["vectors"])
    ids2, dists2 = ix2.batch_search(w.queries, 10, rerank_pool=30)
    oids2, odists2 = _oracle_index(oracle, art).search_batch(w.queries, 10, 4, 30)
    assert np.array_equal(ids2, oids2) and dists2.tobytes() == odists2.tobytes()


def test_flat_add_recovers_from_allocation_failure(oracle, fail):
    from vicinity_amd import FlatIndex, VicinityGpuError

    _print_case("alloc failure: flat add 3000 x 48")
    rng = np.random.default_rng(4)
    base = rng.standard_normal((3000, 48)).astype(np.float32)
    q = rng.standard_normal((40, 48)).astype(np.float32)
    fx = FlatIndex(48, "l2")
    fail(0)
    with pytest.raises(VicinityGpuError) as e:
        fx.add(base[:1000])
    _oom(e)
    fail(0, 0)
    fx.add(base[:1000])
    # the second add's norm buffer fails after its rows were uploaded: the
    # index goes back to its first 1000 rows
    fail(1)
    with pytest.raises(VicinityGpuError) as e:
        fx.add(base[1000:])
    _oom(e)
    fail(0, 0)
    ids, dists = fx.search(q, 10)
    oids, odists = oracle.flat_search(base[:1000], q, 10, metric=0)
    assert np.array_equal(ids, oids) and dists.tobytes() == odists.tobytes()
    fx.add(base[1000:])
    ids, dists = fx.search(q, 10)
    oids, odists = oracle.flat_search(base, q, 10, metric=0)
    assert np.array_equal(ids, oids) and dists.tobytes() == odists.tobytes()
