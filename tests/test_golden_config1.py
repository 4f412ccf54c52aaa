"""Config-1 regression goldens (20,000 x 32, nlist 64, M 8 x 4, ksub 256,
nprobe 8, k 10), written by tests/golden/make_config1.py from the oracle.

CPU: the oracle rebuilds the index and reproduces the stored digests, probe
lists, per-entry ADC distances and top-10 bit for bit, and the stored
goldens agree among themselves (each top-10 is the ten smallest stored ADC
distances under total order with ties to the lower vector index,
search.rs:1378-1391).  GPU: the engine's build, probe lists and top-10 equal
the goldens."""

import hashlib
import os

import numpy as np
import pytest

from tests.golden import make_config1 as gen

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config1.npz")


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(GOLDEN, allow_pickle=False))


@pytest.fixture(scope="module")
def rebuilt(oracle):
    return gen.build_config1()


def _digests(centroids, codebooks, offsets, list_ids, codes):
    return [hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
            for a in (centroids, codebooks, offsets, list_ids, codes)]


def test_stored_goldens_are_self_consistent(golden):
    g = golden
    k = g["top_ids"].shape[1]
    for i in range(int(g["adc_query"].max()) + 1):
        sel = g["adc_query"] == i
        d = g["adc_dist"][sel]
        assert np.isfinite(d).all() and (d >= 0).all()
        assert sel.sum() >= k
        # the ten smallest ADC distances are the stored top-10 distances
        assert np.array_equal(np.sort(d)[:k], g["top_dists"][i])
    assert (np.diff(g["top_dists"], axis=1) >= 0).all()
    assert g["probes"].shape == (g["queries"].shape[0], 8)
    assert all(len(set(row)) == len(row) for row in g["probes"].tolist())


def test_oracle_reproduces_config1_goldens(golden, rebuilt):
    w, ix = rebuilt
    g = golden
    assert np.array_equal(w.queries[:g["queries"].shape[0]], g["queries"])
    assert _digests(ix.centroids, ix.codebooks, ix.list_offsets, ix.list_ids,
                    ix.codes) == g["digests"].tolist()
    for i in range(g["queries"].shape[0]):
        assert np.array_equal(ix.probe(g["queries"][i], 8)[0], g["probes"][i])
    ids, dists = ix.search_batch(g["queries"], 10, 8)
    assert np.array_equal(ids, g["top_ids"])
    assert dists.tobytes() == g["top_dists"].tobytes()
    got_pos, got_dist = [], []
    for i in range(int(g["adc_query"].max()) + 1):
        _, rows = gen.adc_rows(ix, g["queries"][i], 8)
        got_pos += [r[1] for r in rows]
        got_dist += [r[3] for r in rows]
    assert np.array_equal(np.asarray(got_pos, np.uint32), g["adc_pos"])
    assert np.asarray(got_dist, np.float32).tobytes() == g["adc_dist"].tobytes()


def test_top10_ids_are_the_stored_adc_minimisers(golden, rebuilt):
    _, ix = rebuilt
    g = golden
    for i in range(int(g["adc_query"].max()) + 1):
        sel = g["adc_query"] == i
        vidx = ix.list_ids[g["adc_pos"][sel]].astype(np.int64)
        d = g["adc_dist"][sel]
        order = np.lexsort((vidx, d))[:10]
        assert np.array_equal(vidx[order], g["top_ids"][i])


@pytest.mark.gpu
def test_gpu_matches_config1_goldens(golden):
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    print("[case] config-1 goldens: GPU build 20000 x 32, nlist 64, M 8, ksub 256", flush=True)
    g = golden
    w = v.datagen.ivfpq_small()
    ix = v.IVFPQIndex(32, num_clusters=64, num_codebooks=8, codebook_size=256, nprobe=8, seed=42)
    ix.add_items(w.base)
    ix.build(kmeans_max_iter=10)
    art = ix.export()
    assert _digests(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                    art["codes"]) == g["digests"].tolist()
    assert np.array_equal(ix.probe(g["queries"], 8), g["probes"])
    for mode in ("fast", "exact"):
        ix.set_mode(mode)
        ids, dists = ix.batch_search(g["queries"], 10, nprobe=8)
        assert np.array_equal(ids, g["top_ids"]), mode
        assert dists.tobytes() == g["top_dists"].tobytes(), mode
