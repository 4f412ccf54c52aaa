"""The allocation-free batch search (vgpu_ivfpq_search_batch_device_noalloc)
against vgpu_ivfpq_search_batch_device on the same index and queries: ids
equal and float32 distances bit-identical, over two calls in a row (the
second with a smaller batch, so stale scratch contents from the first must
not leak), and a batch large enough to go through the static scratch in
several query chunks."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


def _noalloc(ix, q, k, nprobe=0, pool=0):
    import torch

    from vicinity_amd import _lib

    nq = q.shape[0]
    ids = torch.full((nq, k), -7, dtype=torch.int64, device="cuda:0")
    dists = torch.full((nq, k), -7.0, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    _lib.check(_lib.load().vgpu_ivfpq_search_batch_device_noalloc(
        ix._h, q.data_ptr(), nq, q.shape[1], k, nprobe, pool, ids.data_ptr(), dists.data_ptr(),
        None))
    return ids.cpu().numpy(), dists.cpu().numpy()


def _alloc(ix, q, k, nprobe=0, pool=None):
    ids, dists = ix.search_batch_device(q, k, nprobe or None, rerank_pool=pool)
    return ids.cpu().numpy(), dists.cpu().numpy()


@pytest.fixture(scope="module")
def small():
    import torch

    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    _print_case("no-alloc: build 20000 x 32, nlist 64, M 8, ksub 256")
    w = v.datagen.ivfpq_small()
    ix = v.IVFPQIndex(32, num_clusters=64, num_codebooks=8, codebook_size=256, nprobe=8, seed=11)
    ix.add_items(w.base)
    ix.build(kmeans_max_iter=10)
    return ix, torch.from_numpy(w.queries).to("cuda:0")


def test_two_calls_in_a_row_equal_the_allocating_entry_point(small):
    ix, q = small
    for nq, k, nprobe, pool in [(1000, 10, 8, 0), (37, 5, 3, 0), (600, 10, 8, 40), (3, 100, 64, 0)]:
        _print_case(f"no-alloc: nq {nq} k {k} nprobe {nprobe} pool {pool}")
        qq = q[:nq].contiguous()
        a_ids, a_d = _alloc(ix, qq, k, nprobe, pool or None)
        b_ids, b_d = _noalloc(ix, qq, k, nprobe, pool)
        assert np.array_equal(a_ids, b_ids)
        assert a_d.tobytes() == b_d.tobytes()


def test_exact_mode_and_fastscan(small):
    import torch

    import vicinity_amd as v

    ix, q = small
    ix.set_mode("exact")
    try:
        _print_case("no-alloc: EXACT mode, nq 500 then 20")
        for nq in (500, 20):
            qq = q[:nq].contiguous()
            a = _alloc(ix, qq, 16, 8)
            b = _noalloc(ix, qq, 16, 8)
            assert np.array_equal(a[0], b[0]) and a[1].tobytes() == b[1].tobytes()
    finally:
        ix.set_mode("fast")
    _print_case("no-alloc: ksub 16 FastScan, nq 400 then 9")
    w = v.datagen.ivfpq_small(n=6000, nq=400)
    f = v.IVFPQIndex(32, num_clusters=16, num_codebooks=16, codebook_size=16, nprobe=4, seed=2)
    f.add_items(w.base)
    f.build(kmeans_max_iter=5)
    fq = torch.from_numpy(w.queries).to("cuda:0")
    for nq in (400, 9):
        qq = fq[:nq].contiguous()
        a = _alloc(f, qq, 10, 4)
        b = _noalloc(f, qq, 10, 4)
        assert np.array_equal(a[0], b[0]) and a[1].tobytes() == b[1].tobytes()


def test_a_batch_that_takes_several_scratch_chunks(small):
    """About 2 KB of workspace per query at d 32, nprobe 8, k 100, so 70,000
    queries need more than the 64 MiB scratch and go in three chunks."""
    import torch

    ix, q = small
    _print_case("no-alloc: 70000 queries x k 100 (several scratch chunks), then 5000")
    g = torch.Generator(device="cuda:0").manual_seed(5)
    big = torch.rand((70_000, 32), generator=g, device="cuda:0", dtype=torch.float32)
    for nq in (70_000, 5000):
        qq = big[:nq].contiguous()
        a = _alloc(ix, qq, 100, 8)
        b = _noalloc(ix, qq, 100, 8)
        assert np.array_equal(a[0], b[0]) and a[1].tobytes() == b[1].tobytes()
