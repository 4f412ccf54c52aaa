"""GPU build side (search.rs:546-787 with this project's k-means): the coarse
centroids, lists, codebooks and codes built on the GPU (assignment and
centroid updates in kernels) equal the oracle's build bit for bit across
shapes: the row width above the update kernel's 256 (host update), ds = 1,
ksub 16, a training sample, crowded k-means where clusters empty out, and a
sample of many row blocks for the update's member-list sort."""

import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vg():
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    return v


CASES = {
    "d300_host_coarse_update": dict(n=1500, d=300, L=24, M=3, K=64, sample=None, iters=12),
    "ds1": dict(n=1200, d=16, L=16, M=16, K=32, sample=None, iters=15),
    "ksub16_d128": dict(n=3000, d=128, L=32, M=16, K=16, sample=None, iters=10),
    "sampled": dict(n=5000, d=64, L=40, M=8, K=128, sample=1500, iters=10),
    "crowded": dict(n=600, d=24, L=300, M=4, K=128, sample=None, iters=30),
    # about 20 row blocks of the k-means update's member-list sort per pass
    "many_blocks": dict(n=20000, d=32, L=64, M=8, K=256, sample=None, iters=6),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_gpu_build_equals_oracle_build(vg, oracle, name):
    c = CASES[name]
    print(f"[case] build {name} {c}", flush=True)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    base = rng.standard_normal((c["n"], c["d"])).astype(np.float32)
    if name == "crowded":  # tight groups: many centroids lose every member
        base = base[rng.integers(0, 40, c["n"])] + rng.standard_normal(base.shape).astype(np.float32) * 1e-3
    ix = vg.IVFPQIndex(c["d"], num_clusters=c["L"], num_codebooks=c["M"], codebook_size=c["K"],
                       nprobe=4, seed=77)
    ix.add_items(base)
    ix.build(training_sample_size=c["sample"], kmeans_max_iter=c["iters"])
    art = ix.export()
    vecs = oracle.normalize_rows(base)
    oix, _ = oracle.ivfpq_build(vecs, c["L"], c["M"], c["K"], 77, c["sample"] or 0, c["iters"])
    assert art["centroids"].tobytes() == oix.centroids.tobytes()
    assert art["codebooks"].tobytes() == oix.codebooks.tobytes()
    assert np.array_equal(art["list_offsets"], oix.list_offsets)
    assert np.array_equal(art["list_ids"], oix.list_ids)
    assert np.array_equal(art["codes"], oix.codes)
    q = rng.standard_normal((64, c["d"])).astype(np.float32)
    ids, dists = ix.batch_search(q, 10, nprobe=4)
    oids, odists = oix.search_batch(q, 10, 4)
    assert np.array_equal(ids, oids) and dists.tobytes() == odists.tobytes()
