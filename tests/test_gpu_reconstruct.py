"""IVFPQIndex::reconstruct, memory_usage and generation snapshots on the GPU
index, against the oracle and the reference's own tests restated:

- reconstruct (search.rs:857-884) is the decoded residual plus the list's
  centroid, bit for bit with the oracle (pq.rs:284-290; OPQ: R^T of the
  decoded vector, opq.rs:134-139, 194-204), also after compact();
- full_probe_equals_an_exhaustive_adc_scan (search.rs:2589-2645): with
  nprobe = num_clusters the top-k equals a brute-force scan over the
  reconstructed vectors;
- adc_distance_matches_exact_l2_to_reconstructed_vector (search.rs:3295-3331):
  the search's distances equal the L2 distance to the reconstruction within
  1e-3 relative;
- memory_usage (search.rs:1552-1577) reports the raw vectors until compact();
- save_generation / load_generation (search.rs:918-943) round-trip the index."""

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


def _index(oracle, n=3000, d=32, L=24, M=8, K=64, seed=3, opq=False):
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    rng = np.random.default_rng(seed)
    vecs = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    oix, _ = oracle.ivfpq_build(vecs, L, M, K, seed, 0, 8, use_opq=opq)
    ix = v.IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=L, use_opq=opq)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                      vectors=vecs, rotation=oix.rotation)
    return ix, oix, vecs, rng


def _oracle_reconstruct(oracle, oix, i, d, M, K):
    pos = int(np.nonzero(oix.list_ids == i)[0][0])
    lst = int(np.searchsorted(oix.list_offsets.astype(np.int64), pos, side="right") - 1)
    dec = oracle.pq_reconstruct(oix.codebooks, M, K, d // M, oix.codes[i:i + 1].reshape(-1)).reshape(-1)
    if oix.rotation is not None:
        dec = oracle.matvec_t(oix.rotation, dec)
    return (dec + oix.centroids[lst]).astype(np.float32)


@pytest.mark.parametrize("opq", [False, True])
def test_reconstruct_is_centroid_plus_decoded_residual(oracle, opq):
    _print_case(f"reconstruct opq={opq}")
    d, M, K = 32, 8, 64
    ix, oix, vecs, _ = _index(oracle, opq=opq, seed=5 + opq)
    for i in (0, 1, 17, 999, 2999):
        got = ix.reconstruct(i)
        assert got.tobytes() == _oracle_reconstruct(oracle, oix, i, d, M, K).tobytes(), i
    # search.rs:3262-3288: the decode error stays within PQ quantization error
    errs = []
    for i in range(0, 3000, 7):
        pos = int(np.nonzero(oix.list_ids == i)[0][0])
        lst = int(np.searchsorted(oix.list_offsets.astype(np.int64), pos, side="right") - 1)
        res = np.linalg.norm(vecs[i] - oix.centroids[lst])
        errs.append(np.linalg.norm(vecs[i] - ix.reconstruct(i)) / max(res, 1e-9))
    assert np.mean(errs) <= 0.55 and max(errs) <= 0.85
    ix.compact()
    assert ix.reconstruct(17).tobytes() == _oracle_reconstruct(oracle, oix, 17, d, M, K).tobytes()
    with pytest.raises(ValueError, match="out of range"):
        ix.reconstruct(3000)


def test_reconstruct_before_build_is_an_error():
    import vicinity_amd as v

    ix = v.IVFPQIndex(16, num_clusters=4, num_codebooks=4, codebook_size=16)
    with pytest.raises(ValueError, match="built before reconstruct"):
        ix.reconstruct(0)


def test_full_probe_equals_exhaustive_scan_over_reconstructions(oracle):
    """search.rs:2589-2645: 256 vectors of dimension 16, 32 lists, M 4, ksub
    16, nprobe 32, k 10; lists under 16 entries take the exact float path."""
    import vicinity_amd as v

    _print_case("full probe vs exhaustive scan over reconstruct()")
    rng = np.random.default_rng(4242)
    x = oracle.normalize_rows(rng.random((256, 16), dtype=np.float32))
    ix = v.IVFPQIndex(16, num_clusters=32, num_codebooks=4, codebook_size=16, nprobe=32, seed=7)
    ix.add_items(x, ids=np.arange(256) + 60_000)
    ix.build()
    q = oracle.normalize_rows(rng.random((8, 16), dtype=np.float32))
    art = ix.export()
    recon = np.stack([ix.reconstruct(i) for i in range(256)])
    for qi in range(8):
        ids, _ = ix.search(q[qi], 10)
        d = ((q[qi][None, :] - recon) ** 2).sum(axis=1, dtype=np.float32)
        order = sorted(range(256), key=lambda i: (float(d[i]), int(art["doc_ids"][i])))
        assert ids.tolist() == [int(art["doc_ids"][i]) for i in order[:10]], qi


def test_search_distance_is_l2_to_reconstruction(oracle):
    """search.rs:3295-3331 on the GPU search's own distances."""
    _print_case("ADC distance vs L2 to reconstruct()")
    ix, oix, vecs, _ = _index(oracle, seed=9)
    worst = 0.0
    for qi in (0, 5, 42, 777):
        ids, dists = ix.batch_search(vecs[qi:qi + 1], 200, nprobe=3)
        for doc, dist in zip(ids[0], dists[0]):
            if doc < 0:
                continue
            r = ix.reconstruct(int(doc))
            exact = float(((vecs[qi] - r) ** 2).sum(dtype=np.float32))
            worst = max(worst, abs(float(dist) - exact) / max(exact, 1e-6))
    assert worst <= 1e-3, worst


def test_memory_usage_and_generation_round_trip(oracle, tmp_path):
    import vicinity_amd as v

    _print_case("memory_usage and save/load_generation")
    ix, oix, vecs, rng = _index(oracle, seed=11)
    mu = ix.memory_usage()
    n, d, M = 3000, 32, 8
    assert mu["vectors_bytes"] == n * d * 4 and mu["graph_bytes"] == 0
    assert mu["quantized_bytes"] >= n * M and mu["metadata_bytes"] >= n * 4 + 24 * d * 4
    assert mu["device_bytes"] > n * M and mu["total"] == (
        mu["vectors_bytes"] + mu["quantized_bytes"] + mu["metadata_bytes"])
    q = rng.standard_normal((40, d)).astype(np.float32)
    want = ix.batch_search(q, 10, nprobe=6, rerank_pool=30)
    root = tmp_path / "gens"
    ix.save_generation(root)
    first = (root / "CURRENT").read_text().strip()
    ix.save_generation(root)
    second = (root / "CURRENT").read_text().strip()
    assert first != second and os.path.isdir(root / "generations" / first)
    back = v.IVFPQIndex.load_generation(root)
    got = back.batch_search(q, 10, nprobe=6, rerank_pool=30)
    assert np.array_equal(got[0], want[0]) and got[1].tobytes() == want[1].tobytes()
    fs = v.IVFPQFileSearcher.load_generation(root)
    got = fs.batch_search(q, 10, nprobe=6, rerank_pool=30)
    assert np.array_equal(got[0], want[0]) and got[1].tobytes() == want[1].tobytes()
    with pytest.raises(FileNotFoundError):
        v.IVFPQIndex.load_generation(tmp_path / "none")
    ix.compact()
    assert ix.memory_usage()["vectors_bytes"] == 0
