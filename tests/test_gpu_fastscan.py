"""FastScan (ksub 16) over lists of chosen lengths: empty lists, lists under
16 entries (the exact float path, search.rs:1261 and :1355-1375), exactly 16
and 17 entries, block boundaries (31, 32, 33) and long lists, probed in an
order whose lists a wave scans as one stream of 32-entry blocks.  The probe
count is not a multiple of the four waves.  Ids equal the oracle's and
float32 distances are bit-identical (fastscan_block_portable
src/pq_simd.rs:629-654, fastscan_batch_quantized :721-769)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SIZES = [0, 1, 15, 16, 17, 31, 32, 33, 48, 500, 513, 2, 16, 64, 65, 200, 0, 300, 17, 40, 1000, 96, 7]


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def chosen_lists(oracle):
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    rng = np.random.default_rng(77)
    d, M, K = 32, 8, 16
    L, n = len(SIZES), sum(SIZES)
    vecs = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    cent = oracle.normalize_rows(rng.standard_normal((L, d)).astype(np.float32))
    cb = (rng.standard_normal((M, K, d // M)) * 0.3).astype(np.float32)
    offsets = np.concatenate([[0], np.cumsum(SIZES)]).astype(np.uint64)
    list_ids = rng.permutation(n).astype(np.uint32)
    codes = rng.integers(0, K, (n, M)).astype(np.uint8)
    doc_ids = (np.arange(n, dtype=np.uint32) * 5 + 3).astype(np.uint32)
    ix = v.IVFPQIndex(d, num_clusters=L, num_codebooks=M, codebook_size=K, nprobe=L)
    ix.load_artifacts(cent, cb, offsets, list_ids, codes, doc_ids=doc_ids, vectors=vecs)
    oix = oracle.Index(cent, cb, offsets, list_ids, codes, doc_ids, vecs, M, K)
    return ix, oix, rng, d


@pytest.mark.parametrize("nprobe,k", [(23, 10), (23, 300), (7, 10), (10, 1), (5, 50)])
def test_fastscan_stream_list_sizes(chosen_lists, nprobe, k):
    ix, oix, rng, d = chosen_lists
    _print_case(f"fastscan chosen list sizes: nprobe {nprobe}, k {k}")
    q = rng.standard_normal((40, d)).astype(np.float32)
    ids, dists = ix.batch_search(q, k, nprobe=nprobe)
    oids, odists = oix.search_batch(q, k, nprobe)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()


def test_fastscan_stream_reranked(chosen_lists):
    ix, oix, rng, d = chosen_lists
    _print_case("fastscan chosen list sizes: nprobe 23, k 10, rerank pool 100")
    q = rng.standard_normal((40, d)).astype(np.float32)
    ids, dists = ix.batch_search(q, 10, nprobe=23, rerank_pool=100)
    oids, odists = oix.search_batch(q, 10, 23, 100)
    assert np.array_equal(ids, oids)
    assert dists.tobytes() == odists.tobytes()
