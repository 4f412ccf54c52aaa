"""GPU parity at dimensions above the scan workgroup's 512 threads, where the
query, the residuals and the list ranges are staged in more than one pass per
thread: d 640 with 8 codebooks of width 80 and d 544 with 16 of width 34
(codewords read from memory per table, not held in registers), in FAST and
EXACT mode, and an OPQ index at d 576 (rotated residual tables,
search.rs:1242-1255, opq.rs:120-123).  The reference accepts any dimension
its codebooks divide (src/ivf_pq/pq.rs:44-55).  Indexes are built by the
oracle and uploaded, so the comparison covers the search alone; distances are
compared bit for bit."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


def _data(oracle, rng, n, d, nc=30):
    centres = rng.standard_normal((nc, d)).astype(np.float32)
    x = centres[rng.integers(0, nc, n)] + 0.4 * rng.standard_normal((n, d)).astype(np.float32)
    q = centres[rng.integers(0, nc, 48)] + 0.4 * rng.standard_normal((48, d)).astype(np.float32)
    return oracle.normalize_rows(x.astype(np.float32)), oracle.normalize_rows(q.astype(np.float32))


@pytest.mark.parametrize("d,M", [(640, 8), (544, 16)])
def test_large_dimension_against_oracle(oracle, d, M):
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    L, n, K = 16, 3000, 256
    _print_case(f"large d={d} M={M} ds={d // M} L={L} n={n}")
    rng = np.random.default_rng(2000 + d + M)
    vecs, q = _data(oracle, rng, n, d)
    oix, _ = oracle.ivfpq_build(vecs, L, M, K, 9, 0, 6)
    ix = v.IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=L // 2)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                      vectors=vecs)
    for k, nprobe in [(10, L // 2), (100, L)]:
        oids, odists = oix.search_batch(q, k, nprobe)
        for mode in ["fast", "exact"]:
            ix.set_mode(mode)
            ids, dists = ix.batch_search(q, k, nprobe=nprobe)
            assert np.array_equal(ids, oids), (mode, k, nprobe)
            assert dists.tobytes() == odists.tobytes(), (mode, k, nprobe)


def test_large_dimension_rotated_residuals_against_oracle(oracle):
    """An orthogonal rotation attached to a plain index: every table is built
    from R (q - c), whatever the codes were trained on, so the search's
    arithmetic is compared on its own."""
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    d, M, K, L, n = 576, 8, 64, 16, 2500
    _print_case(f"rotated residuals d={d} M={M} ksub={K} L={L} n={n}")
    rng = np.random.default_rng(577)
    vecs, q = _data(oracle, rng, n, d)
    oix, _ = oracle.ivfpq_build(vecs, L, M, K, 4, 0, 6)
    rot, _ = np.linalg.qr(rng.standard_normal((d, d)))
    rot = np.ascontiguousarray(rot.astype(np.float32))
    ix = v.IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=6, use_opq=True)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                      vectors=vecs, rotation=rot)
    art = ix.export()
    rix = oracle.Index(art["centroids"], art["codebooks"], art["list_offsets"], art["list_ids"],
                       art["codes"], art["doc_ids"], art["vectors"], art["M"], art["K"], rot)
    for k, nprobe in [(10, 6), (50, L)]:
        oids, odists = rix.search_batch(q, k, nprobe)
        ids, dists = ix.batch_search(q, k, nprobe=nprobe)
        assert np.array_equal(ids, oids), (k, nprobe)
        assert dists.tobytes() == odists.tobytes(), (k, nprobe)
