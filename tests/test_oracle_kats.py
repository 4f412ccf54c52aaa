"""Pins the oracle against the reference's own known-answer tests and
invariants (each test cites the reference test it restates), plus closed
forms and float64 brute force where the reference has no KAT."""

import numpy as np
import pytest

from tests.helpers import (f64_l2sq, pq_lcg_codes, pq_lcg_values, regression_lcg,
                           seq_normalize, total_cmp_key)


# ---- src/simd.rs:129-160 and src/distance.rs:148-165 ----------------------

def test_simd_closed_forms(oracle):
    assert oracle.dot([1, 2, 3], [4, 5, 6]) == np.float32(32.0)
    assert oracle.l2sq([0, 0], [3, 4]) == np.float32(25.0)
    n = oracle.normalize_rows(np.array([[3.0, 4.0]], np.float32))[0]
    assert n[0] == np.float32(3.0) / np.float32(5.0) and n[1] == np.float32(4.0) / np.float32(5.0)


def test_dot_is_sequential_float32(oracle):
    # A cancellation case where pairwise and sequential float32 sums differ.
    a = np.array([1e8, 1.0, -1e8, 1.0], np.float32)
    b = np.ones(4, np.float32)
    # sequential: ((1e8 + 1) - 1e8) + 1 = (1e8 - 1e8) + 1 = 1
    assert oracle.dot(a, b) == np.float32(1.0)
    rng = np.random.default_rng(0)
    for _ in range(20):
        x = rng.standard_normal(37).astype(np.float32)
        y = rng.standard_normal(37).astype(np.float32)
        s = np.float32(0)
        for u, v in zip(x, y):
            s = np.float32(s + np.float32(u * v))
        assert oracle.dot(x, y) == s


def test_normalize_rule(oracle):
    # search.rs:55-62: below 1e-10 the vector is returned unchanged.
    tiny = np.array([[1e-12, 0.0, 0.0]], np.float32)
    assert np.array_equal(oracle.normalize_rows(tiny), tiny)
    zero = np.zeros((1, 4), np.float32)
    assert np.array_equal(oracle.normalize_rows(zero), zero)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 33)).astype(np.float32)
    got = oracle.normalize_rows(x)
    for i in range(5):
        s = np.float32(0)
        for v in x[i]:
            s = np.float32(s + np.float32(v * v))
        want = (x[i] / np.float32(np.sqrt(s))).astype(np.float32)
        assert np.array_equal(got[i], want)


# ---- src/ivf_pq/pq.rs:335-372 ---------------------------------------------

def test_adc_table_one_dimensional_kat(oracle):
    t = oracle.adc_table(np.array([0.0, 1.0, 3.0, -1.0, 2.0, 4.0]), 2, 3, 1, [2.0, 1.0])
    assert t.tolist() == [4.0, 1.0, 1.0, 4.0, 1.0, 9.0]


def test_adc_table_small_multidimensional_kat(oracle):
    cb = np.array([0, 0, 0, 1, 1, 1, 2, 2, 2, 3, 3, 3], np.float32)
    t = oracle.adc_table(cb, 2, 2, 3, [1, 2, 3, 4, 5, 6])
    assert t.tolist() == [14.0, 5.0, 29.0, 14.0]


@pytest.mark.parametrize("ds", [1, 2, 8, 10, 16])
def test_adc_table_is_sequential_sub_mul_add(oracle, ds):
    # The three branches (pq.rs:211-263) all reduce to dist = 0; dist +=
    # (r - c)^2 in dimension order; restated here with numpy float32 scalars.
    rng = np.random.default_rng(ds)
    M, K = 3, 5
    cb = rng.standard_normal(M * K * ds).astype(np.float32)
    r = rng.standard_normal(M * ds).astype(np.float32)
    t = oracle.adc_table(cb, M, K, ds, r)
    for m in range(M):
        for k in range(K):
            acc = np.float32(0)
            for j in range(ds):
                diff = np.float32(r[m * ds + j] - cb[(m * K + k) * ds + j])
                acc = np.float32(acc + np.float32(diff * diff))
            assert t[m * K + k] == acc


def _fitted_pq(oracle, d, M, K, seed):
    """pq.rs:388-401 shape: 4*K (>=16) LCG vectors in [-1,1), PQ fit with the
    oracle's own k-means (the reference's clump fit is not reproducible)."""
    n = max(K * 4, 16)
    x, _ = pq_lcg_values(n * d, seed | 1)
    x = x.reshape(n, d)
    ds = d // M
    cbs = []
    for m in range(M):
        c, _ = oracle.kmeans(np.ascontiguousarray(x[:, m * ds:(m + 1) * ds]), K, 1, seed + m, 100)
        cbs.append(c.reshape(-1))
    return np.concatenate(cbs), min(K, n)


@pytest.mark.parametrize("M,ds,K,seed", [(1, 1, 4, 3), (2, 3, 7, 11), (3, 8, 16, 5),
                                         (4, 10, 9, 1234567), (2, 9, 16, 99)])
def test_adc_table_distance_equals_squared_l2_to_reconstruction(oracle, M, ds, K, seed):
    # pq.rs:435-478: sum of the table over random codes == ||q - decode||^2.
    d = M * ds
    cb, K = _fitted_pq(oracle, d, M, K, seed)
    q, _ = pq_lcg_values(d, (seed * 31 + 7) | 1)
    codes, _ = pq_lcg_codes(M, K, (seed * 17 + 3) | 1)
    table = oracle.adc_table(cb, M, K, ds, q)
    acc = oracle.distance_with_table(table, M, K, codes)
    rec = oracle.pq_reconstruct(cb, M, K, ds, codes)
    exact = f64_l2sq(q, rec)
    assert abs(float(acc) - exact) <= 1e-4 * max(abs(exact), 1.0)


@pytest.mark.parametrize("M,ds,K,seed", [(1, 2, 4, 1), (3, 4, 16, 2), (4, 10, 8, 3)])
def test_quantize_is_an_argmin(oracle, M, ds, K, seed):
    # pq.rs:485-524 and :529-551.
    d = M * ds
    cb, K = _fitted_pq(oracle, d, M, K, seed)
    x, _ = pq_lcg_values(d, (seed * 13) | 1)
    codes = oracle.pq_encode(cb, M, K, ds, x)[0]
    rec = oracle.pq_reconstruct(cb, M, K, ds, codes)
    cbm = cb.reshape(M, K, ds)
    for m in range(M):
        sub = x[m * ds:(m + 1) * ds]
        observed = f64_l2sq(sub, rec[m * ds:(m + 1) * ds])
        for k in range(K):
            assert observed <= f64_l2sq(sub, cbm[m, k]) * (1 + 1e-5) + 1e-6
        # strict `<`: the first minimum wins (pq.rs:145-155)
        dists = [oracle.l2sq(sub, cbm[m, k]) for k in range(K)]
        assert codes[m] == int(np.argmin(dists))
    again = oracle.pq_reconstruct(cb, M, K, ds, oracle.pq_encode(cb, M, K, ds, rec)[0])
    assert np.array_equal(again, rec)


def test_encode_tie_goes_to_lowest_code(oracle):
    cb = np.array([1.0, -1.0, 1.0], np.float32)  # M=1, K=3, ds=1
    assert oracle.pq_encode(cb, 1, 3, 1, np.array([0.0], np.float32))[0, 0] == 0
    assert oracle.pq_encode(cb, 1, 3, 1, np.array([0.9], np.float32))[0, 0] == 0


def test_finite_inputs_encode_to_finite_decodes(oracle):
    # pq.rs:556-591
    cb, K = _fitted_pq(oracle, 8, 2, 8, 42)
    x = np.array([1e30, -1e30, 3e29, 0, 5, -7e25, 1e-30, 2e30], np.float32)
    codes = oracle.pq_encode(cb, 2, K, 4, x)[0]
    assert (codes < K).all()
    assert np.isfinite(oracle.pq_reconstruct(cb, 2, K, 4, codes)).all()


# ---- src/pq_simd.rs tests -------------------------------------------------

def _test_lut(M, K):
    # pq_simd.rs:809-817: lut[m][c] = (m*K + c) as f32 * 0.1
    return (np.arange(M * K, dtype=np.float32) * np.float32(0.1)).astype(np.float32)


def test_adc_distance_basic(oracle):
    # pq_simd.rs:819-838
    d = oracle.distance_with_table(_test_lut(4, 256), 4, 256, [0, 1, 2, 3])
    assert abs(float(d) - (0.0 + 25.7 + 51.4 + 77.1)) < 0.01


def test_borrowed_lut_dispatch_matches_scalar(oracle):
    # pq_simd.rs:858-885
    M, n = 5, 257
    lut = _test_lut(M, 256)
    codes = (np.arange(n * M) * 37 % 256).astype(np.uint8)
    got = oracle.adc_scan(codes, M, 256, lut)
    for i in range(n):
        assert abs(got[i] - oracle.distance_with_table(lut, M, 256, codes[i * M:(i + 1) * M])) < 1e-4


@pytest.mark.parametrize("K", [256, 16])
@pytest.mark.parametrize("M", [1, 3, 5, 25])
def test_adc_batch_matches_naive_reference_at_odd_sizes(oracle, K, M):
    # pq_simd.rs:1108-1132: bitwise equality with the m-ordered float32 sum.
    i = np.arange(M * K)
    lut = (np.float32(0.25) + ((i * 7919) % 1009).astype(np.float32) * np.float32(0.003)).astype(np.float32)
    for n in [0, 1, 2, 3, 4, 5, 7, 8, 9, 15, 17, 33, 257]:
        codes = ((np.arange(n * M) * 131 + 17) % K).astype(np.uint8).reshape(n, M)
        want = np.zeros(n, np.float32)
        for m in range(M):
            want = (want + lut[m * K + codes[:, m].astype(np.int64)]).astype(np.float32)
        got = oracle.adc_scan(codes, M, K, lut)
        assert got.tobytes() == want.tobytes(), (K, M, n)


def test_fastscan_u16_accumulator_is_exact_at_the_codebook_limit(oracle):
    # pq_simd.rs:780-795
    M = 257
    packed = oracle.pack4(np.zeros(32 * M, np.uint8), 32, M)
    acc = oracle.fastscan_block(packed[:16 * M], np.full(M * 16, 255, np.uint8), M)
    assert (acc == 65535).all()


def test_fastscan_refuses_more_codebooks_than_the_u16_accumulator_holds(oracle):
    # pq_simd.rs:798-807
    M = 258
    packed = oracle.pack4(np.zeros(32 * M, np.uint8), 32, M)
    with pytest.raises(ValueError, match="overflow"):
        oracle.fastscan_batch(packed, 32, M, np.ones(M * 16, np.float32))


def test_packed_codes_4bit_roundtrip(oracle):
    # pq_simd.rs:1041-1077
    n, M = 5, 4
    idx = np.arange(n * M)
    codes = ((idx // M + idx % M) % 16).astype(np.uint8)
    packed = oracle.pack4(codes, n, M)
    assert packed.size == 16 * M
    for i in range(n):
        for m in range(M):
            byte = packed[m * 16 + (i % 16)]
            code = byte & 0x0F if i < 16 else byte >> 4
            assert code == codes[i * M + m]


def _np_pack4(codes, n, M):
    codes = codes.reshape(n, M)
    nb = (n + 31) // 32
    pad = np.zeros((nb * 32, M), np.uint8)
    pad[:n] = codes & 0x0F
    blocks = pad.reshape(nb, 2, 16, M)  # [block][half][lane][m]
    out = blocks[:, 0] | (blocks[:, 1] << 4)  # [block][lane][m]
    return np.ascontiguousarray(out.transpose(0, 2, 1)).reshape(-1)


@pytest.mark.parametrize("n,M", [(1, 1), (31, 3), (32, 5), (33, 2), (100, 8), (257, 50)])
def test_pack4_layout_matches_restatement(oracle, n, M):
    rng = np.random.default_rng(n * 100 + M)
    codes = rng.integers(0, 16, n * M, dtype=np.uint8)
    assert np.array_equal(oracle.pack4(codes, n, M), _np_pack4(codes, n, M))


def _create_4bit_lut(M):
    # pq_simd.rs:1024-1029: (m*16 + c) as f32 * 0.5
    return (np.arange(M * 16, dtype=np.float32) * np.float32(0.5)).astype(np.float32)


def test_quantize_lut_range(oracle):
    # pq_simd.rs:1160-1187
    lut = _create_4bit_lut(8)
    q, scale, offset = oracle.quantize_lut(lut, 8)
    assert q[0] == 0 and q[-1] == 255
    rec = q.astype(np.float32) * scale + offset
    assert (np.abs(rec - lut) <= scale / 2 + 1e-5).all()


def test_quantize_lut_rounds_half_away_and_degenerate_range(oracle):
    # Constant table: range < EPSILON -> scale 1, inv 0, all zeros.
    q, scale, offset = oracle.quantize_lut(np.full(32, 3.5, np.float32), 2)
    assert scale == 1.0 and offset == np.float32(3.5) and (q == 0).all()
    # (v - min) * inv == 0.5 exactly -> rounds to 1 (half away from zero).
    lut = np.zeros(16, np.float32)
    lut[1] = np.float32(0.5 / 255.0 * 255.0 / 255.0)
    lut[15] = np.float32(1.0)
    q, scale, offset = oracle.quantize_lut(lut, 1)
    inv = np.float32(255.0) / np.float32(1.0)
    assert q[1] == np.float32(np.floor(np.float32(lut[1] * inv) + np.float32(0.5)))


def _np_fastscan(codes, n, M, lut):
    # restates quantize_lut_flat + block accumulation + conversion in numpy
    lut = np.asarray(lut, np.float32)
    mn, mx = lut.min(), lut.max()
    rng_ = np.float32(mx - mn)
    if rng_ < np.float32(1.1920929e-07):
        scale, inv = np.float32(1.0), np.float32(0.0)
    else:
        scale, inv = np.float32(rng_ / np.float32(255.0)), np.float32(np.float32(255.0) / rng_)
    v = ((lut - mn) * inv).astype(np.float32)
    r = np.where(v >= 0, np.floor(v + np.float32(0.5)), np.ceil(v - np.float32(0.5)))  # half away
    q = np.clip(r, 0, 255).astype(np.uint16)
    c = codes.reshape(n, M).astype(np.int64)
    acc = np.zeros(n, np.uint16)
    for m in range(M):
        acc = (acc + q[m * 16 + c[:, m]]).astype(np.uint16)
    base = np.float32(mn * np.float32(M))
    return (acc.astype(np.float32) * scale + base).astype(np.float32)


@pytest.mark.parametrize("n,M", [(100, 8), (100, 4), (40, 5), (64, 50), (33, 1)])
def test_fastscan_matches_restatement_and_error_bound(oracle, n, M):
    # pq_simd.rs:1206-1318 (error <= M*scale/2 + 1e-3) and bitwise vs numpy.
    rng = np.random.default_rng(n + M)
    codes = rng.integers(0, 16, n * M, dtype=np.uint8)
    lut = rng.random(M * 16).astype(np.float32) * np.float32(3.0)
    got = oracle.fastscan_batch(oracle.pack4(codes, n, M), n, M, lut)
    assert got.tobytes() == _np_fastscan(codes, n, M, lut).tobytes()
    scalar = np.zeros(n, np.float32)
    for m in range(M):
        scalar = (scalar + lut[m * 16 + codes.reshape(n, M)[:, m].astype(np.int64)]).astype(np.float32)
    _, scale, _ = oracle.quantize_lut(lut, M)
    assert (np.abs(got - scalar) <= M * scale * 0.5 + 1e-3).all()


# ---- src/ivf_pq/search.rs:2047-2069 ----------------------------------------

def test_finish_top_k_keeps_sorted_prefix(oracle):
    ids = np.array([10, 11, 12, 13, 14, 15], np.uint32)
    d = np.array([5.0, 1.5, 3.0, 0.5, 2.0, 4.0], np.float32)
    oi, od = oracle.top_k(ids, d, 3)
    assert oi.tolist() == [13, 11, 14] and od.tolist() == [0.5, 1.5, 2.0]


def test_finish_top_k_handles_zero_and_short_inputs(oracle):
    assert oracle.top_k([1], [1.0], 0)[0].size == 0
    assert oracle.top_k([], [], 5)[0].size == 0
    oi, od = oracle.top_k([2, 1], [2.0, 1.0], 5)
    assert oi.tolist() == [1, 2] and od.tolist() == [1.0, 2.0]


def test_top_k_total_cmp_and_ties(oracle):
    rng = np.random.default_rng(5)
    for n, k in [(1000, 10), (5000, 100), (37, 36), (64, 64), (300, 1)]:
        d = rng.integers(0, 50, n).astype(np.float32)  # many exact ties
        d[::7] *= -1
        ids = rng.permutation(n).astype(np.uint32)
        oi, od = oracle.top_k(ids, d, k)
        order = np.lexsort((ids, total_cmp_key(d)))[:k]
        assert oi.tolist() == ids[order].tolist() and od.tolist() == d[order].tolist()
    d = np.array([np.nan, 1.0, -np.inf, np.inf, -0.0, 0.0], np.float32)
    oi, od = oracle.top_k(np.arange(6, dtype=np.uint32), d, 6)
    assert oi.tolist() == [2, 4, 5, 1, 3, 0]  # total_cmp: -0 < +0, NaN last


def test_nearest_centroids_brute_force(oracle):
    rng = np.random.default_rng(3)
    cent = np.ascontiguousarray(oracle.normalize_rows(rng.standard_normal((64, 16)).astype(np.float32)))
    for _ in range(10):
        q = oracle.normalize_rows(rng.standard_normal((1, 16)).astype(np.float32))[0]
        lists, scores = oracle.nearest_centroids(q, cent, 8)
        exact = np.array([np.float32(1.0) - oracle.dot(q, c) for c in cent], np.float32)
        order = np.lexsort((np.arange(64), exact))[:8]
        assert lists.tolist() == order.tolist()
        assert scores.tolist() == exact[order].tolist()
    lists, _ = oracle.nearest_centroids(q, cent, 100)  # nprobe clamped to L
    assert lists.size == 64


# ---- build side invariants -----------------------------------------------

def test_build_lists_keep_insertion_order(oracle):
    assign = np.array([2, 0, 2, 1, 0, 2], np.uint32)
    off, ids = oracle.build_lists(assign, 4)
    assert off.tolist() == [0, 2, 3, 6, 6]
    assert ids.tolist() == [1, 4, 3, 0, 2, 5]


def test_sample_indices(oracle):
    s = oracle.sample_indices(1000, 100, 42)
    assert s.size == 100 and np.all(np.diff(s.astype(np.int64)) > 0) and s.max() < 1000
    assert np.array_equal(s, oracle.sample_indices(1000, 100, 42))
    assert not np.array_equal(s, oracle.sample_indices(1000, 100, 43))
    assert np.array_equal(oracle.sample_indices(10, 0, 1), np.arange(10))


def _assign_f64_candidates(x, cent):
    """Rows of candidate sets for argmin_c (1 - x.c): every c whose float64
    score is within twice the float32 rounding bound of the float64 minimum.
    Bound per score: a sequential float32 dot of length d is within
    gamma_d * sum|x_j c_j| of the true dot (gamma_d = d u / (1 - d u),
    u = 2^-24), and 1 - dot adds one rounding of at most u * |1 - dot|."""
    d = x.shape[1]
    u = 2.0 ** -24
    gamma = d * u / (1 - d * u)
    x64, c64 = x.astype(np.float64), cent.astype(np.float64)
    s = 1.0 - x64 @ c64.T
    err = gamma * (np.abs(x64) @ np.abs(c64).T) + u * np.abs(s)
    out = []
    for i in range(x.shape[0]):
        lo = s[i].min()
        out.append(np.flatnonzero(s[i] - err[i] <= lo + err[i].max() * 1.0001))
    return out


@pytest.mark.parametrize("n,L,d", [(500, 37, 13), (300, 64, 32), (200, 9, 3), (150, 128, 97)])
def test_assign_cosine_is_the_argmin(oracle, n, L, d):
    """kmeans.rs:97-107 (called from search.rs:621, metric distance.rs:104-109):
    each vector goes to argmin over centroids of 1 - dot, first minimum wins.
    Checked against a float64 argmin wherever the float32 rounding bound
    separates the minimum, against the brute-force-pinned probe selection
    with nprobe 1, and on exact ties (duplicated centroids, a zero row)."""
    rng = np.random.default_rng(n + L + d)
    x = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    cent = oracle.normalize_rows(rng.standard_normal((L, d)).astype(np.float32))
    a = oracle.assign_cosine(x, cent)
    assert a.dtype == np.uint32 and a.shape == (n,)
    cands = _assign_f64_candidates(x, cent)
    unique = 0
    for i in range(n):
        assert a[i] in cands[i]
        if cands[i].size == 1:
            unique += 1
    assert unique >= n * 0.9  # the float64 check decides most rows
    for i in range(0, n, max(1, n // 40)):
        lists, _ = oracle.nearest_centroids(x[i], cent, 1)
        assert lists.tolist() == [a[i]]


def test_assign_cosine_ties_go_to_the_lowest_index(oracle):
    rng = np.random.default_rng(11)
    d = 21
    base = oracle.normalize_rows(rng.standard_normal((6, d)).astype(np.float32))
    # centroid rows 0..11: base rows, then the same rows again in reverse
    # order, so every score occurs twice at indices i and 11 - i.
    cent = np.ascontiguousarray(np.concatenate([base, base[::-1]]))
    x = oracle.normalize_rows(
        (base[rng.integers(0, 6, 200)] + 0.3 * rng.standard_normal((200, d))).astype(np.float32))
    a = oracle.assign_cosine(x, cent)
    assert a.max() < 6  # a `<=` rule would take the later copy
    for i in range(200):
        assert a[i] == np.argmin(1.0 - x[i].astype(np.float64) @ base.astype(np.float64).T) \
            or a[i] in _assign_f64_candidates(x[i:i + 1], base)[0]
    # A zero vector scores 1 against every centroid: index 0.
    z = np.zeros((1, d), np.float32)
    assert oracle.assign_cosine(z, cent).tolist() == [0]
    # All centroids equal: index 0 for every row.
    same = np.ascontiguousarray(np.repeat(base[:1], 9, axis=0))
    assert oracle.assign_cosine(x[:20], same).tolist() == [0] * 20
    # d = 1: rows are +-1, every score is exactly 0 or 2, and the answer is
    # the first centroid of the row's sign.
    c1 = np.array([[-1.0], [-1.0], [1.0], [-1.0], [1.0]], np.float32)
    x1 = np.array([[1.0], [-1.0], [1.0]], np.float32)
    assert oracle.assign_cosine(x1, c1).tolist() == [2, 0, 2]


@pytest.mark.parametrize("metric", [0, 1])
def test_kmeans_fixed_point(oracle, metric):
    rng = np.random.default_rng(metric)
    x = oracle.normalize_rows(rng.standard_normal((600, 8)).astype(np.float32))
    cent, it = oracle.kmeans(x, 12, metric, 7, 200)
    assert 0 < it < 200  # converged: assignments stopped changing
    if metric == 0:
        a = oracle.assign_cosine(x, cent)
    else:
        a = np.array([np.argmin([oracle.l2sq(v, c) for c in cent]) for v in x])
    for c in range(cent.shape[0]):
        mem = x[a == c].astype(np.float64)
        if mem.shape[0] == 0:
            continue
        mean = mem.sum(axis=0) / mem.shape[0]
        want = mean.astype(np.float32)
        if metric == 0:
            want = seq_normalize(want)
        np.testing.assert_array_equal(cent[c], want)


# ---- index-level invariants (search.rs tests, correctness_regression) ------

def _regression_index(oracle, n, dim, seed, L=None, M=8, K=64):
    vec, _ = regression_lcg(n * dim, seed)
    vecs = np.stack([seq_normalize(v) for v in vec.reshape(n, dim)])
    L = L if L is not None else min(16, n // 4)
    ix, _ = oracle.ivfpq_build(vecs, L, M, K, 42, 0, 100)
    return ix, vecs


def test_ivf_pq_self_retrieval(oracle):
    # correctness_regression/tests_feature_gated.rs:69-106
    ix, vecs = _regression_index(oracle, 400, 32, 1, L=16)
    found = sum(int(ix.search(v, 1, 16)[0][0] == i) for i, v in enumerate(vecs))
    assert found / 400 >= 0.8


def test_ivf_pq_query_scale_invariance_and_shape(oracle):
    # correctness_regression :109-163
    ix, _ = _regression_index(oracle, 200, 32, 2)
    vals, _ = regression_lcg(5 * 32, 888)
    for v in vals.reshape(5, 32):
        v = seq_normalize(v)
        a = ix.search(v, 5, 16)[0]
        b = ix.search((v * np.float32(5.3)).astype(np.float32), 5, 16)[0]
        assert a.tolist() == b.tolist()
    q = seq_normalize(regression_lcg(32, 42)[0])
    for k in [1, 3, 5, 10, 50]:
        ids, d = ix.search(q, k, 16)
        assert ids.size <= k
        assert (d >= -0.01).all() and (np.diff(d) >= 0).all()


def test_full_probe_equals_an_exhaustive_adc_scan(oracle):
    # search.rs:2589-2645: nprobe = num_clusters, lists below the batch
    # threshold, so results equal brute force over c + decode(codes).
    rng = np.random.default_rng(4242)
    n, d, L, M, K = 256, 16, 48, 4, 16
    x = oracle.normalize_rows(rng.random((n, d)).astype(np.float32))
    ix, assign = oracle.ivfpq_build(x, L, M, K, 7, 0, 100)
    # the reference keeps every list below the FastScan threshold (16)
    assert np.diff(ix.list_offsets.astype(np.int64)).max() < 16
    q = oracle.normalize_rows(rng.random((1, d)).astype(np.float32))[0]
    ids, dists = ix.search(q, 10, L)
    ds = d // M
    brute = []
    for i in range(n):
        rec = oracle.pq_reconstruct(ix.codebooks, M, K, ds, ix.codes[i]) + ix.centroids[assign[i]]
        brute.append(f64_l2sq(q, rec))
    brute = np.array(brute)
    order = np.argsort(brute, kind="stable")[:10]
    # equal except where float32 rounding reorders near-ties
    for j, i in enumerate(ids):
        assert abs(brute[i] - brute[order[j]]) <= 1e-5
    assert np.allclose(dists, brute[ids], rtol=1e-4, atol=1e-6)


def test_adc_distance_equals_distance_to_reconstruction(oracle):
    # search.rs:3294-3333 (faiss parity): ADC == ||q - (c + decode)||^2 within 1e-3
    rng = np.random.default_rng(9)
    n, d, L, M, K = 2000, 32, 16, 8, 256
    x = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    ix, assign = oracle.ivfpq_build(x, L, M, K, 3, 0, 20)
    for qi in range(5):
        q = x[qi * 37]
        ids, dists = ix.search(q, 10, 4)
        for i, dist in zip(ids, dists):
            rec = oracle.pq_reconstruct(ix.codebooks, M, K, d // M, ix.codes[i]) + ix.centroids[assign[i]]
            assert abs(float(dist) - f64_l2sq(q, rec)) <= 1e-3


def test_batch_search_padding(oracle):
    # python test_python.py:555-563 and python.rs:778-785
    rng = np.random.default_rng(0)
    x = oracle.normalize_rows(rng.standard_normal((16, 8)).astype(np.float32))
    ix, _ = oracle.ivfpq_build(x, 8, 4, 8, 0, 0, 5)
    ids, dists = ix.search_batch(x[:2], 20, 8, rerank_pool=16)
    assert ids.shape == (2, 20)
    assert (ids[:, 16:] == -1).all() and np.isinf(dists[:, 16:]).all()
    assert ids[0, 0] == 0 and abs(dists[0, 0]) < 1e-4


def test_reranked_distances_are_exact_cosine(oracle):
    rng = np.random.default_rng(2)
    x = oracle.normalize_rows(rng.standard_normal((500, 16)).astype(np.float32))
    ix, _ = oracle.ivfpq_build(x, 8, 4, 16, 1, 0, 10)
    q = x[3]
    ids, d = ix.search_reranked(q, 5, 50, 8)
    assert ids[0] == 3
    for i, dd in zip(ids, d):
        assert dd == np.float32(1.0) - oracle.dot(q, x[i])


# ---- flat exact search: src/distance.rs:78-83, 104-109; ground truth
# ---- search.rs:3376-3392 (brute force, ascending, ties by index) ---------

def test_flat_search_closed_forms(oracle):
    # l2_distance_squared: [1,2,3] to [4,5,6] is 27, to 0 is 14, to itself 0.
    base = np.array([[4, 5, 6], [1, 2, 3], [0, 0, 0]], np.float32)
    ids, d = oracle.flat_search(base, np.array([[1, 2, 3]], np.float32), 3, metric=0)
    assert ids.tolist() == [[1, 2, 0]] and d.tolist() == [[0.0, 14.0, 27.0]]
    # cosine_distance_normalized = 1 - dot on unit vectors.
    h = np.float32(np.sqrt(np.float32(0.5)))
    unit = np.array([[1, 0], [0, 1], [h, h]], np.float32)
    ids, d = oracle.flat_search(unit, np.array([[1, 0]], np.float32), 3, metric=1)
    assert ids.tolist() == [[0, 2, 1]]
    assert d.tolist() == [[0.0, float(np.float32(1) - h), 1.0]]


def test_flat_search_metric_branches_differ(oracle):
    # Unnormalised rows where squared L2 and 1 - dot rank in opposite orders:
    # a wrong metric branch fails one of the two assertions.
    base = np.array([[10, 0], [0.9, 0.1]], np.float32)
    q = np.array([[1, 0]], np.float32)
    assert oracle.flat_search(base, q, 2, metric=0)[0].tolist() == [[1, 0]]
    assert oracle.flat_search(base, q, 2, metric=1)[0].tolist() == [[0, 1]]


def test_flat_search_ties_padding_and_threads(oracle):
    rng = np.random.default_rng(5)
    base = rng.standard_normal((40, 6)).astype(np.float32)
    base[[3, 7, 11, 30]] = base[20]  # five equal rows: ties go to the lower index
    q = base[20:21].copy()
    for metric in (0, 1):
        ids, d = oracle.flat_search(base, q, 5, metric=metric)
        if metric == 0:
            assert ids.tolist() == [[3, 7, 11, 20, 30]]
            assert (d == 0).all()
        else:  # the equal rows keep index order wherever they fall in the row
            tied = [i for i in ids[0].tolist() if i in (3, 7, 11, 20, 30)]
            assert tied == sorted(tied)
    # k > n pads with (-1, +inf) (python.rs:778-785 convention)
    ids, d = oracle.flat_search(base[:4], q, 7, metric=0)
    assert ids[0, 4:].tolist() == [-1, -1, -1] and np.isinf(d[0, 4:]).all()
    assert sorted(ids[0, :4].tolist()) == [0, 1, 2, 3]
    # one thread and many give the same rows
    qs = rng.standard_normal((9, 6)).astype(np.float32)
    a = oracle.flat_search(base, qs, 6, metric=0, threads=1)
    b = oracle.flat_search(base, qs, 6, metric=0, threads=4)
    assert np.array_equal(a[0], b[0]) and a[1].tobytes() == b[1].tobytes()


@pytest.mark.parametrize("metric", [0, 1])
def test_flat_search_equals_float64_brute_force(oracle, metric):
    """Each returned distance is the sequential float32 primitive of its own
    (query, id) pair (a stride or pairing mistake fails), and the ranking
    equals float64 brute force wherever the float64 gap exceeds the float32
    rounding bound of the sums (d * 2^-23 * the sum of magnitudes)."""
    rng = np.random.default_rng(11 + metric)
    n, d, nq, k = 300, 19, 7, 12
    base = rng.standard_normal((n, d)).astype(np.float32)
    qs = rng.standard_normal((nq, d)).astype(np.float32)
    if metric == 1:
        base = oracle.normalize_rows(base)
        qs = oracle.normalize_rows(qs)
    ids, dist = oracle.flat_search(base, qs, k, metric=metric)
    for i in range(nq):
        for j in range(k):
            x = base[ids[i, j]]
            prim = oracle.l2sq(qs[i], x) if metric == 0 else np.float32(1) - oracle.dot(qs[i], x)
            assert dist[i, j] == np.float32(prim)
        q64, b64 = qs[i].astype(np.float64), base.astype(np.float64)
        if metric == 0:
            exact = ((b64 - q64) ** 2).sum(axis=1)
            mag = ((b64 - q64) ** 2).sum(axis=1)
        else:
            exact = 1.0 - b64 @ q64
            mag = np.abs(b64 * q64).sum(axis=1) + 1.0
        bound = d * 2.0 ** -23 * mag
        assert np.all(np.abs(dist[i].astype(np.float64) - exact[ids[i]]) <= bound[ids[i]])
        order = np.argsort(exact, kind="stable")
        # every id the float64 ranking puts clearly inside the top-k is returned
        kth = exact[order[k - 1]]
        clear = order[: k][exact[order[:k]] < kth - 2 * bound.max()]
        assert set(clear.tolist()) <= set(ids[i].tolist())
        # and nothing clearly outside it is
        outside = np.where(exact > kth + 2 * bound.max())[0]
        assert not set(outside.tolist()) & set(ids[i].tolist())
        assert np.all(np.diff(dist[i]) >= 0)
