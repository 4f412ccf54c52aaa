"""GPU parity of the FAST scan's other specialisations with ksub 256, against
the oracle in FAST and EXACT mode: 32 codebooks (transposed blocks at
subvector widths 4 and 2), 64 codebooks (row layout, width 2), 16 codebooks
of width 3 (row layout, subvector width read at run time) and 48 codebooks
of width 4 at d 192 (transposed blocks; the coarse step takes the path for
d > 128), d 64 with 16 or 8 codebooks, d 32 with 16 or 4 and d 96 with 16 or
32 (widths 4, 8, 2, 8, 6 and 3: in EXACT mode the kernels whose codeword
registers are a half, a quarter or three quarters of the widest width), and
the FAST row layout at compile-time widths 3, 6, 12 and 16 (d 96 with 8, 16 or
32 codebooks, d 48 with 16, 8 or 4, d 24 with 8 or 4, d 12 with 4, d 192 with
32, d 128 with 8, d 64 with 4).  The reference accepts any number of codebooks
(src/pq_simd.rs:314-327).  Indexes are built by the oracle and uploaded, so
the comparison covers the scan alone; distances are compared bit for bit."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("d,M", [(128, 32), (64, 32), (128, 64), (48, 16), (192, 48), (64, 16), (64, 8), (32, 16), (32, 4), (96, 16), (96, 32),
                                 (96, 8), (48, 8), (48, 4), (24, 8), (24, 4), (12, 4), (192, 32),
                                 (128, 8), (64, 4)])
def test_fast_scan_shapes_against_oracle(oracle, d, M):
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    L, n, K = 24, 6000, 256
    _print_case(f"FAST shape d={d} M={M} ds={d // M} L={L} n={n}")
    rng = np.random.default_rng(1000 + d + M)
    centres = rng.standard_normal((40, d)).astype(np.float32)
    x = centres[rng.integers(0, 40, n)] + 0.3 * rng.standard_normal((n, d)).astype(np.float32)
    vecs = oracle.normalize_rows(x.astype(np.float32))
    oix, _ = oracle.ivfpq_build(vecs, L, M, K, 5, 0, 8)
    ix = v.IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=L // 2)
    ix.load_artifacts(oix.centroids, oix.codebooks, oix.list_offsets, oix.list_ids, oix.codes,
                      vectors=vecs)
    q = oracle.normalize_rows(
        (centres[rng.integers(0, 40, 64)] + 0.3 * rng.standard_normal((64, d))).astype(np.float32))
    for k, nprobe in [(10, L // 2), (100, L // 2), (10, L)]:
        oids, odists = oix.search_batch(q, k, nprobe)
        for mode in ["fast", "exact"]:
            ix.set_mode(mode)
            ids, dists = ix.batch_search(q, k, nprobe=nprobe)
            assert np.array_equal(ids, oids), (mode, k, nprobe)
            assert dists.tobytes() == odists.tobytes(), (mode, k, nprobe)
