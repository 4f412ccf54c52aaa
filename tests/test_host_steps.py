"""CPU tests of the library's host-side build steps through the C ABI (no
device needed): inverted lists from labels, the host k-means update, the OPQ
polar factor, and the errors raised when a label read back from the device
is out of range."""

import ctypes
import time

import numpy as np
import pytest


def _lib():
    from vicinity_amd import _lib

    return _lib, _lib.load()


def _host_lists(assign, L):
    lib, L_ = _lib()
    assign = np.ascontiguousarray(assign, np.uint32)
    off = np.empty(L + 1, np.uint64)
    ids = np.empty(max(len(assign), 1), np.uint32)
    st = L_.vgpu_test_host_lists(assign.ctypes.data, len(assign), L, off.ctypes.data, ids.ctypes.data)
    return st, off, ids[: len(assign)]


def test_host_lists_equal_the_oracle(oracle):
    rng = np.random.default_rng(3)
    for n, L in [(1, 1), (50, 7), (1000, 64)]:
        assign = rng.integers(0, L, n).astype(np.uint32)
        st, off, ids = _host_lists(assign, L)
        assert st == 0
        o_off, o_ids = oracle.build_lists(assign, L)
        assert np.array_equal(off, o_off.astype(np.uint64)) and np.array_equal(ids, o_ids)
        # search.rs:624-657: insertion order inside each list
        for l in range(L):
            seg = ids[off[l]:off[l + 1]]
            assert np.all(np.diff(seg.astype(np.int64)) > 0) and np.all(assign[seg] == l)


def test_host_lists_reject_a_label_outside_the_lists():
    from vicinity_amd._lib import ERR_DEVICE

    lib, L_ = _lib()
    assign = np.array([0, 3, 1, 4, 2], np.uint32)  # 4 is outside 0..3
    st, _, _ = _host_lists(assign, 4)
    assert st == ERR_DEVICE
    msg = L_.vgpu_last_error().decode()
    assert "row 3" in msg and "label 4" in msg
    st, _, _ = _host_lists(np.array([0xFFFFFFFF], np.uint32), 4)
    assert st == ERR_DEVICE


def _centroid_update(x, assign, cent):
    lib, L_ = _lib()
    x = np.ascontiguousarray(x, np.float32)
    assign = np.ascontiguousarray(assign, np.uint32)
    out = np.ascontiguousarray(cent, np.float32).copy()
    st = L_.vgpu_test_host_centroid_update(x.ctypes.data, x.shape[0], x.shape[1], assign.ctypes.data,
                                           out.shape[0], out.ctypes.data)
    return st, out


def test_host_centroid_update_is_the_float64_member_mean(oracle):
    rng = np.random.default_rng(4)
    n, d, k = 500, 300, 9  # d above the update kernel's 256-float rows
    x = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    assign = rng.integers(0, k - 1, n).astype(np.uint32)  # key k-1 stays empty
    cent = rng.standard_normal((k, d)).astype(np.float32)
    st, out = _centroid_update(x, assign, cent)
    assert st == 0
    for c in range(k - 1):
        mem = x[assign == c].astype(np.float64)
        s = np.zeros(d)
        for row in mem:  # member order
            s += row
        want = oracle.normalize_rows((s / len(mem)).astype(np.float32)[None, :])[0]
        assert out[c].tobytes() == want.tobytes()
    assert out[k - 1].tobytes() == cent[k - 1].tobytes()  # empty key keeps its row


def test_host_centroid_update_rejects_a_label_outside_the_keys():
    from vicinity_amd._lib import ERR_DEVICE

    x = np.ones((4, 3), np.float32)
    st, _ = _centroid_update(x, np.array([0, 1, 7, 0], np.uint32), np.zeros((2, 3), np.float32))
    assert st == ERR_DEVICE


def _polar(m):
    lib, L_ = _lib()
    m = np.ascontiguousarray(m, np.float32)
    r = np.empty_like(m)
    lib.check(L_.vgpu_test_polar_factor(m.ctypes.data, m.shape[0], r.ctypes.data))
    return r


@pytest.mark.parametrize("d", [3, 16, 64])
def test_polar_factor_equals_the_oracle_bit_for_bit(oracle, d):
    rng = np.random.default_rng(d)
    for kind in range(3):
        m = rng.standard_normal((d, d)).astype(np.float32)
        if kind == 1:
            m[:, 1] = 0.0  # rank deficient: the completion path
        if kind == 2:
            m[: d // 2] = 0.0
        assert _polar(m).tobytes() == oracle.polar(m).tobytes()


def test_polar_factor_build_cost_at_d512_and_d1024(oracle):
    """The OPQ build calls the polar factor ten times; column pairs are read
    as contiguous rows, which keeps d = 512 to about a second and d = 1024 to
    about a quarter minute on one host core."""
    rng = np.random.default_rng(9)
    m = rng.standard_normal((512, 512)).astype(np.float32)
    t = time.perf_counter()
    r = _polar(m)
    dt = time.perf_counter() - t
    assert r.tobytes() == oracle.polar(m).tobytes()
    assert dt < 10.0, dt
    m = rng.standard_normal((1024, 1024)).astype(np.float32)
    t = time.perf_counter()
    r = _polar(m).astype(np.float64)
    dt = time.perf_counter() - t
    assert np.abs(r @ r.T - np.eye(1024)).max() < 1e-5
    assert dt < 60.0, dt
