"""Concurrent searches on one handle (the reference's search takes &self,
src/ivf_pq/search.rs:1087): each call borrows its own device workspace and
stream, so threads searching one index at once get the results they would
get one at a time."""

import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _print_case(msg):
    print(f"[case] {msg}", flush=True)


def test_threads_searching_one_handle_get_sequential_results():
    import vicinity_amd as v

    assert v.device_available(), "no gfx950 device visible"
    _print_case("concurrent search: build 20000 x 32, nlist 64, M 8, ksub 256")
    w = v.datagen.ivfpq_small()
    ix = v.IVFPQIndex(32, num_clusters=64, num_codebooks=8, codebook_size=256, nprobe=8, seed=3)
    ix.add_items(w.base)
    ix.build(kmeans_max_iter=10)
    rng = np.random.default_rng(21)
    batches = [rng.random((int(rng.integers(1, 700)), 32), dtype=np.float32) for _ in range(12)]
    shapes = [(10, 8, None), (37, 3, None), (5, 16, 40)]  # (k, nprobe, rerank pool)
    want = [ix.batch_search(b, *shapes[i % 3]) for i, b in enumerate(batches)]
    got = [None] * len(batches)
    errors = []

    def worker(t):
        try:
            for rep in range(3):
                for i in range(t, len(batches), 4):
                    got[i] = ix.batch_search(batches[i], *shapes[i % 3])
                    if rep < 2:
                        assert np.array_equal(got[i][0], want[i][0])
        except Exception as e:  # surfaced in the main thread
            errors.append(e)

    _print_case("concurrent search: 4 threads x 3 passes")
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a search thread did not finish"
    assert not errors, errors
    for i in range(len(batches)):
        assert np.array_equal(got[i][0], want[i][0]), i
        assert got[i][1].tobytes() == want[i][1].tobytes(), i
    st = ix.last_stats()
    assert st["nq"] in {len(b) for b in batches}


def test_device_searches_on_separate_torch_streams():
    import torch

    import vicinity_amd as v

    _print_case("concurrent device search on two torch streams")
    w = v.datagen.ivfpq_small(n=8000, nq=2000)
    ix = v.IVFPQIndex(32, num_clusters=32, num_codebooks=8, codebook_size=256, nprobe=4, seed=5)
    ix.add_items(w.base)
    ix.build(kmeans_max_iter=5)
    q = torch.from_numpy(w.queries).to("cuda:0")
    ref_ids, ref_d = ix.batch_search(w.queries, 20)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()  # q is ready before the side streams read it
    outs = [None, None]

    def worker(j):
        with torch.cuda.stream(streams[j]):
            half = q[j * 1000:(j + 1) * 1000].contiguous()
            outs[j] = ix.search_batch_device(half, 20, stream=streams[j])

    threads = [threading.Thread(target=worker, args=(j,)) for j in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    torch.cuda.synchronize()
    ids = torch.cat([outs[0][0], outs[1][0]]).cpu().numpy()
    d = torch.cat([outs[0][1], outs[1][1]]).cpu().numpy()
    assert np.array_equal(ids, ref_ids) and d.tobytes() == ref_d.tobytes()
