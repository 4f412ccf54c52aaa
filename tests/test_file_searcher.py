"""IVFPQFileSearcher (src/ivf_pq/search.rs:247-282, 1620-2041; python.rs:857-1060):
a snapshot directory searched with its PQ codes and raw vectors left on disk.

CPU: the metadata-only snapshot read, the CURRENT-generation resolution, and
the format errors the library reports before any device work (missing
directory, half a list-code sidecar, truncated files).  GPU: results equal the
oracle's in-memory search on the snapshot's arrays (ids equal, float32
distances bit-identical) and the in-memory GPU index's, with and without the
list-code sidecar, for ksub 256 and 16 (FastScan), OPQ, reranked searches;
the per-query diagnostics equal the counts the reference computes
(search.rs:1904-1980) from the oracle's probe lists."""

import os
import shutil

import numpy as np
import pytest

from vicinity_amd.snapshot import SnapshotFormatError, read_snapshot, write_snapshot


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


def _oracle_snapshot(oracle, tmp_path, n=3000, d=32, L=24, M=8, K=64, seed=5, opq=False, name="snap",
                     raw=True):
    rng = np.random.default_rng(seed)
    base = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    oix, _ = oracle.ivfpq_build(base, L, M, K, seed, 0, 8, use_opq=opq)
    path = tmp_path / name
    doc_ids = (1000 + 3 * np.arange(n)).astype(np.uint32)
    write_snapshot(path, dimension=d,
                   params=dict(num_clusters=L, nprobe=4, num_codebooks=M, codebook_size=K,
                               use_opq=opq, seed=seed),
                   centroids=oix.centroids, codebooks=oix.codebooks, codebook_size=K,
                   num_codebooks=M, list_offsets=oix.list_offsets, list_ids=oix.list_ids,
                   codes=oix.codes, doc_ids=doc_ids, vectors=oix.vectors if raw else None,
                   rotation=oix.rotation)
    oix = oracle.Index(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                       doc_ids, oix.vectors, M, K, oix.rotation)
    return path, oix, rng


# ---- CPU ------------------------------------------------------------------------

def test_metadata_only_read_skips_codes_and_vectors(oracle, tmp_path):
    path, oix, _ = _oracle_snapshot(oracle, tmp_path)
    full = read_snapshot(path)
    meta = read_snapshot(path, arrays=False)
    assert meta["codes"] is None and meta["vectors"] is None
    assert meta["raw_vectors_present"] is True
    for key in ("centroids", "codebooks", "list_offsets", "list_ids", "doc_ids"):
        assert np.array_equal(meta[key], full[key]), key
    # a truncated codes file is a format error even when the codes are not read
    with open(os.path.join(path, "codes.bin"), "r+b") as f:
        f.truncate(10)
    with pytest.raises(SnapshotFormatError, match="codes.bin size mismatch"):
        read_snapshot(path, arrays=False)


def test_missing_directory_and_generation_pointer(tmp_path):
    from vicinity_amd import IVFPQFileSearcher
    from vicinity_amd.file_searcher import _current_generation

    with pytest.raises(FileNotFoundError):
        IVFPQFileSearcher.load(tmp_path / "missing")
    root = tmp_path / "root"
    (root / "generations" / "g-000001").mkdir(parents=True)
    (root / "CURRENT").write_text("g-000001\n")
    assert _current_generation(root) == os.path.join(root, "generations", "g-000001")
    (root / "CURRENT").write_text("../escape")
    with pytest.raises(SnapshotFormatError):
        _current_generation(root)


def test_half_a_list_code_sidecar_is_rejected_before_device_work(oracle, tmp_path):
    from vicinity_amd import IVFPQFileSearcher, _lib

    path, _, _ = _oracle_snapshot(oracle, tmp_path)
    os.remove(os.path.join(path, "list_codes.bin"))
    with pytest.raises(ValueError, match="partial IVF-PQ list-code sidecar") as e:
        IVFPQFileSearcher.load(path)
    assert e.value.code == _lib.ERR_INVALID_PARAMETER


def test_repeated_list_member_is_rejected_at_open(oracle, tmp_path):
    """A snapshot whose lists hold one vector twice (and another not at all)
    is reported when the searcher opens it, before any device work."""
    from vicinity_amd import IVFPQFileSearcher, _lib

    rng = np.random.default_rng(3)
    base = oracle.normalize_rows(rng.standard_normal((400, 16)).astype(np.float32))
    oix, _ = oracle.ivfpq_build(base, 8, 4, 16, 3, 0, 5)
    list_ids = oix.list_ids.copy()
    list_ids[1] = list_ids[0]
    path = tmp_path / "dup"
    write_snapshot(path, dimension=16,
                   params=dict(num_clusters=8, nprobe=2, num_codebooks=4, codebook_size=16,
                               use_opq=False, seed=3),
                   centroids=oix.centroids, codebooks=oix.codebooks, codebook_size=16,
                   num_codebooks=4, list_offsets=oix.list_offsets, list_ids=list_ids, codes=oix.codes,
                   doc_ids=np.arange(400, dtype=np.uint32), vectors=None, rotation=None)
    with pytest.raises(ValueError, match="permutation") as e:
        IVFPQFileSearcher.load(path)
    assert e.value.code == _lib.ERR_INVALID_PARAMETER


# ---- GPU ------------------------------------------------------------------------

@pytest.fixture
def vg_device():
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    return v


def _diag_expect(oix, q, P, kk, M, sidecar, pool):
    """search.rs:1904-1980 for one query, from the oracle's probe lists."""
    lists = oix.probe(q, P)[0]
    lens = [int(oix.list_offsets[l + 1] - oix.list_offsets[l]) for l in lists]
    scanned = sum(lens)
    retained = min(kk, scanned)
    return {"probed_lists": len(lists), "scanned_vectors": scanned,
            "code_reads": sum(1 if (ln >= 16 and sidecar) else ln for ln in lens),
            "code_bytes": scanned * M, "retained_candidates": retained,
            "raw_vector_reads": retained if pool else 0,
            "raw_vector_bytes": retained * q.shape[0] * 4 if pool else 0,
            "reranked_candidates": retained if pool else 0}


@pytest.mark.gpu
@pytest.mark.parametrize("sidecar", [True, False])
@pytest.mark.parametrize("K,opq", [(64, False), (256, False), (16, False), (64, True)])
def test_file_searcher_matches_oracle_and_memory_index(vg_device, oracle, tmp_path, K, opq, sidecar):
    from vicinity_amd import IVFPQFileSearcher, IVFPQIndex

    _print_case(f"file searcher K={K} opq={opq} sidecar={sidecar}")
    path, oix, rng = _oracle_snapshot(oracle, tmp_path, K=K, opq=opq, seed=K + opq)
    if not sidecar:  # codes.bin read row by row (search.rs:1963-1971)
        os.remove(os.path.join(path, "list_codes.bin"))
        os.remove(os.path.join(path, "list_offsets.bin"))
    fs = IVFPQFileSearcher.load(path)
    mem = IVFPQIndex.load(path)
    assert len(fs) == 3000 and fs.dimension == 32 and fs.num_clusters == 24
    assert fs.num_codebooks == 8 and fs.codebook_size == K and fs.nprobe == 4
    assert "IVFPQFileSearcher(" in repr(fs)
    q = rng.standard_normal((150, 32)).astype(np.float32)
    for k, nprobe, pool in ((10, 4, None), (1, 1, None), (40, 24, None), (7, 6, 30), (20, 3, 20)):
        ids, dists, diag = fs.batch_search_with_diagnostics(q, k, nprobe=nprobe, rerank_pool=pool)
        oids, odists = oix.search_batch(q, k, nprobe, pool or 0)
        assert np.array_equal(ids, oids), (k, nprobe, pool)
        assert dists.tobytes() == odists.tobytes(), (k, nprobe, pool)
        mids, mdists = mem.batch_search(q, k, nprobe=nprobe, rerank_pool=pool)
        assert np.array_equal(ids, mids) and dists.tobytes() == mdists.tobytes()
        kk = max(pool, k) if pool else k
        for i in (0, 17, 149):
            assert diag[i] == _diag_expect(oix, q[i], nprobe, kk, 8, sidecar, pool), (i, k, nprobe, pool)
        io = fs.last_io()
        assert io["reads"] > 0 and io["bytes"] > 0
    # the single-query surface and the default nprobe after set_nprobe
    fs.set_nprobe(6)
    assert fs.nprobe == 6
    ids, dists = fs.search(q[3], 5)
    oids, odists = oix.search(q[3], 5, 6)
    assert ids.tolist() == [int(x) for x in oids] and dists.tobytes() == odists.tobytes()


@pytest.mark.gpu
def test_file_searcher_generation_compacted_and_mmap_warning(vg_device, oracle, tmp_path):
    import warnings

    from vicinity_amd import IVFPQFileSearcher

    _print_case("file searcher: generation root, raw vectors absent, mmap warning")
    path, oix, rng = _oracle_snapshot(oracle, tmp_path, name="g-000007")
    root = tmp_path / "root"
    (root / "generations").mkdir(parents=True)
    shutil.move(str(path), str(root / "generations" / "g-000007"))
    (root / "CURRENT").write_text("g-000007\n")
    fs = IVFPQFileSearcher.load_generation(root)
    q = rng.standard_normal((20, 32)).astype(np.float32)
    ids, dists = fs.batch_search(q, 10)
    oids, odists = oix.search_batch(q, 10, 4)
    assert np.array_equal(ids, oids) and dists.tobytes() == odists.tobytes()
    with pytest.warns(DeprecationWarning, match="mmap"):
        IVFPQFileSearcher.load(root / "generations" / "g-000007", mmap=True)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        IVFPQFileSearcher.load(root / "generations" / "g-000007")
    # a snapshot without raw vectors: approximate search only (search.rs:1841-1847)
    path2, oix2, _ = _oracle_snapshot(oracle, tmp_path, name="noraw", raw=False)
    fs2 = IVFPQFileSearcher.load(path2)
    ids, dists = fs2.batch_search(q, 10)
    oids, odists = oix2.search_batch(q, 10, 4)
    assert np.array_equal(ids, oids)
    with pytest.raises(ValueError, match="without raw vectors"):
        fs2.batch_search(q, 10, rerank_pool=20)


@pytest.mark.gpu
def test_explicit_nprobe_zero_probes_nothing(vg_device, oracle, tmp_path):
    """python.rs:1085-1096 / 1127-1139: an explicit nprobe replaces the index
    default for the call, 0 included (no list is probed, every row is padding);
    None keeps the default, which is unchanged afterwards."""
    from vicinity_amd import MISSING_DISTANCE, MISSING_LABEL, IVFPQFileSearcher, IVFPQIndex

    _print_case("explicit nprobe 0: file searcher and in-memory index")
    path, oix, rng = _oracle_snapshot(oracle, tmp_path, seed=9)
    q = rng.standard_normal((20, 32)).astype(np.float32)
    fs = IVFPQFileSearcher.load(path)
    mem = IVFPQIndex.load(path)
    for ix in (fs, mem):
        for pool in (None, 30):
            ids, dists = ix.batch_search(q, 10, nprobe=0, rerank_pool=pool)
            assert (ids == MISSING_LABEL).all() and (dists == MISSING_DISTANCE).all()
            ids, dists = ix.search(q[0], 10, nprobe=0, rerank_pool=pool)
            assert ids.size == 0 and dists.size == 0
        assert ix.nprobe == 4
        ids, dists = ix.batch_search(q, 10)
        oids, odists = oix.search_batch(q, 10, 4)
        assert np.array_equal(ids, oids) and dists.tobytes() == odists.tobytes()
    _, _, diag = fs.batch_search_with_diagnostics(q, 10, nprobe=0)
    assert all(g["probed_lists"] == 0 and g["scanned_vectors"] == 0 for g in diag)
    # the reference's checks still apply: a non-finite query, and a rerank
    # after the raw vectors are dropped
    bad = q.copy()
    bad[3, 5] = np.nan
    with pytest.raises(ValueError, match="non-finite"):
        mem.batch_search(bad, 10, nprobe=0)
    mem.compact()
    with pytest.raises(ValueError, match="compact"):
        mem.batch_search(q, 10, nprobe=0, rerank_pool=30)
