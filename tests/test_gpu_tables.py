"""The scan kernels' own residual tables, pinned through the scan: with one
probed list and k at least its length, a search returns every entry of the
list with its distance, the m-ordered sum of the table entries its codes
select (compute_adc_table_into src/ivf_pq/pq.rs:196-266, distance_with_table
:272-279; for ksub 16 the quantised table of quantize_lut_flat
src/pq_simd.rs:576-611 and acc * scale + offset * M, :721-769).  Every table
entry that some entry's code selects is therefore compared bit for bit with
the oracle: the EXACT kernel's per-(query, list) tables in LDS (ksub 256 and
64) and FastScan's per-list quantised tables (ksub 16)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("K,ds", [(256, 2), (64, 3), (16, 4)])
def test_scan_tables_through_whole_lists(oracle, K, ds):
    import vicinity_amd as v
    from vicinity_amd import IVFPQIndex

    assert v.device_available(), "no gfx950 device visible"
    M, L, n = 8, 3, 3000
    d = M * ds
    _print_case(f"tables through whole lists: M {M}, ksub {K}, ds {ds}, {L} lists of {n} vectors")
    rng = np.random.default_rng(K + ds)
    vecs = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    oix, _ = oracle.ivfpq_build(vecs, L, M, K, 3, 0, 8)
    ix = IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=1)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes, vectors=vecs)
    ix.set_mode("exact")
    lens = np.diff(oix.list_offsets.astype(np.int64))
    k = int(lens.max())
    q = rng.standard_normal((12, d)).astype(np.float32)
    ids, dists = ix.batch_search(q, k, nprobe=1)
    oids, odists = oix.search_batch(q, k, 1)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()
    # every entry of the probed list came back (the rest is -1 padding)
    probed = ix.probe(q, 1)[:, 0]
    assert np.array_equal((ids >= 0).sum(axis=1), lens[probed])
    # the lists' codes select most table entries of every subspace
    codes = oix.codes.reshape(-1, M)
    for m in range(M):
        assert len(np.unique(codes[:, m])) >= 0.9 * K, m
