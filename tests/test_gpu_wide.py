"""Searches past the fast path's shapes: nprobe up to nlist (the reference
clamps nprobe to nlist, search.rs:1610, and its full-probe invariant is
search.rs:2589-2645) and k or rerank pools above 2048 (the reference accepts
any k, search.rs:64-75).  Such searches choose their probes from the exact
score of every list and scan in EXACT mode (FastScan for ksub 16) with the
probe slots read from global memory.  Ids equal the oracle's and float32
distances are bit-identical; probe lists equal the oracle's, in order."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


def _oracle_index(oracle, art):
    return oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                        art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"])


@pytest.fixture(scope="module")
def wide_ix(oracle):
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    _print_case("wide: GPU build 40000 x 32, nlist 4096, M 8, ksub 256")
    rng = np.random.default_rng(31)
    base = rng.standard_normal((40_000, 32)).astype(np.float32)
    ix = v.IVFPQIndex(32, num_clusters=4096, num_codebooks=8, codebook_size=256, nprobe=8, seed=9)
    ix.add_items(base)
    ix.build(kmeans_max_iter=4)
    return ix, _oracle_index(oracle, ix.export()), rng


@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_full_probe_nprobe_equals_nlist(wide_ix, mode):
    ix, oix, rng = wide_ix
    _print_case(f"wide: nprobe 4096 of 4096, k 10, mode {mode}")
    ix.set_mode(mode)
    q = rng.standard_normal((48, 32)).astype(np.float32)
    ids, dists = ix.batch_search(q, 10, nprobe=4096)
    oids, odists = oix.search_batch(q, 10, 4096)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()
    # nprobe above nlist clamps to nlist (search.rs:1610)
    ids2, dists2 = ix.batch_search(q, 10, nprobe=100_000)
    assert np.array_equal(ids2, ids) and dists2.tobytes() == dists.tobytes()
    ix.set_mode("fast")


def test_wide_probe_lists_in_order(wide_ix):
    ix, oix, rng = wide_ix
    _print_case("wide: probe lists for nprobe 1500 and 4096")
    q = rng.standard_normal((12, 32)).astype(np.float32)
    for P in (1500, 4096):
        got = ix.probe(q, P)
        for i in range(q.shape[0]):
            assert np.array_equal(got[i], oix.probe(q[i], P)[0]), (P, i)


@pytest.mark.parametrize("k,nprobe,pool", [(4096, 1024, 0), (2500, 300, 0), (10, 256, 5000),
                                           (3000, 2000, 0)])
def test_large_k_and_rerank_pool(wide_ix, k, nprobe, pool):
    ix, oix, rng = wide_ix
    _print_case(f"wide: k {k}, nprobe {nprobe}, rerank pool {pool}")
    q = rng.standard_normal((24, 32)).astype(np.float32)
    ids, dists = ix.batch_search(q, k, nprobe=nprobe, rerank_pool=pool or None)
    oids, odists = oix.search_batch(q, k, nprobe, pool)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()


def test_fastscan_full_probe(oracle):
    import vicinity_amd as v

    _print_case("wide: FastScan 20000 x 32, nlist 1100 (lists below and above 16 entries), nprobe 1100")
    rng = np.random.default_rng(41)
    base = rng.standard_normal((20_000, 32)).astype(np.float32)
    ix = v.IVFPQIndex(32, num_clusters=1100, num_codebooks=8, codebook_size=16, nprobe=8, seed=4)
    ix.add_items(base)
    ix.build(kmeans_max_iter=4)
    oix = _oracle_index(oracle, ix.export())
    q = rng.standard_normal((32, 32)).astype(np.float32)
    for k, P in ((10, 1100), (20, 1050)):
        ids, dists = ix.batch_search(q, k, nprobe=P)
        oids, odists = oix.search_batch(q, k, P)
        assert np.array_equal(ids, oids), (k, P)
        assert dists.tobytes() == odists.tobytes(), (k, P)
