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


def test_two_threads_on_two_handles(small):
    """Every call on a GPU shares its one scratch array: the library's per-GPU
    lock makes concurrent synchronous calls (here on two handles from two
    threads) take turns, so both results equal the allocating entry point."""
    import threading

    import vicinity_amd as v

    ix, q = small
    _print_case("no-alloc: two threads, two handles, 40 calls each")
    w = v.datagen.ivfpq_small(n=8000, nq=300)
    other = v.IVFPQIndex(32, num_clusters=32, num_codebooks=8, codebook_size=256, nprobe=6, seed=9)
    other.add_items(w.base)
    other.build(kmeans_max_iter=5)
    cases = [(ix, q[:900].contiguous(), 10, 8), (other, q[:700].contiguous(), 20, 6)]
    want = [_alloc(h, qq, k, p) for h, qq, k, p in cases]
    errors = []

    def run(i):
        import torch

        torch.cuda.set_device(0)
        h, qq, k, p = cases[i]
        try:
            for _ in range(40):
                got = _noalloc(h, qq, k, p)
                if not (np.array_equal(got[0], want[i][0]) and got[1].tobytes() == want[i][1].tobytes()):
                    errors.append(f"thread {i}: result differs")
                    return
        except Exception as e:  # reported below
            errors.append(f"thread {i}: {e!r}")

    ts = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors


def test_graph_capture_and_replay(small):
    """The call under stream capture records its kernels without waiting;
    each replay of the graph (with eager work and synchronisations between
    replays) equals the allocating entry point on the replay's queries."""
    import torch

    from vicinity_amd import _lib

    ix, q = small
    nq, k, nprobe = 800, 10, 8
    _print_case(f"no-alloc: capture nq {nq} k {k} nprobe {nprobe}, four replays")
    qbuf = q[:nq].clone()
    ids = torch.full((nq, k), -7, dtype=torch.int64, device="cuda:0")
    dists = torch.full((nq, k), -7.0, dtype=torch.float32, device="cuda:0")
    lib = _lib.load()
    # warm-up call outside capture: scratch address lookup, kernel attributes
    _noalloc(ix, qbuf, k, nprobe)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        rc = lib.vgpu_ivfpq_search_batch_device_noalloc(
            ix._h, qbuf.data_ptr(), nq, qbuf.shape[1], k, nprobe, 0, ids.data_ptr(),
            dists.data_ptr(), ctypes.c_void_p(side.cuda_stream))
    assert rc == 0, lib.vgpu_last_error()
    torch.cuda.synchronize()
    for rep in range(4):
        src = q[200:200 + nq] if rep % 2 else q[:nq]
        qbuf.copy_(src)
        ids.fill_(-7)
        dists.fill_(-7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = _alloc(ix, src.contiguous(), k, nprobe)
        assert np.array_equal(ids.cpu().numpy(), want[0]), f"replay {rep}"
        assert dists.cpu().numpy().tobytes() == want[1].tobytes(), f"replay {rep}"
    del g
