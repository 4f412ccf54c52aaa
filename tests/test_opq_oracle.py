"""OPQ (src/ivf_pq/opq.rs, search.rs:732-749): the oracle's restatement,
pinned by the reference's own OPQ tests (opq.rs:309-453 and
tests/opq_vs_pq.rs), by an independent SVD (numpy's LAPACK) for the polar
factor, by closed forms (M = Q D gives R = Q), and for search by an exhaustive
float64 scan of ||R(q - c) - y||^2 at full probe.  The reference's rotation
comes from nalgebra 0.35's float32 SVD (absent): its bits are unpinned, the
polar factor it approximates is pinned."""

import math

import numpy as np
import pytest


def _orthogonal(rng, d):
    q, r = np.linalg.qr(rng.standard_normal((d, d)))
    return q * np.sign(np.diag(r))


# ---- matrix products (opq.rs:170-205, KATs :362-385) ----------------------

def test_matvec_kats(oracle):
    assert oracle.matvec(np.eye(2, dtype=np.float32), [3.0, 4.0]).tolist() == [3.0, 4.0]
    out = oracle.matvec(np.array([[0, -1], [1, 0]], np.float32), [1.0, 0.0])
    assert abs(out[0]) < 1e-6 and abs(out[1] - 1.0) < 1e-6
    v = np.arange(1, 9, dtype=np.float32)  # test_identity_rotation
    assert oracle.matvec(np.eye(8, dtype=np.float32), v).tolist() == v.tolist()
    # row-major R: out = R v, and matvec_t gives R^T v
    R = np.array([[1, 2], [3, 4]], np.float32)
    assert oracle.matvec(R, [1.0, 10.0]).tolist() == [21.0, 43.0]
    assert oracle.matvec_t(R, [1.0, 10.0]).tolist() == [31.0, 42.0]


def test_matvec_is_the_float64_product_to_rounding(oracle):
    rng = np.random.default_rng(3)
    for d in (4, 32, 128):
        R = _orthogonal(rng, d).astype(np.float32)
        v = rng.standard_normal(d).astype(np.float32)
        want = R.astype(np.float64) @ v.astype(np.float64)
        assert np.allclose(oracle.matvec(R, v), want, atol=1e-5 * math.sqrt(d))
        want_t = R.T.astype(np.float64) @ v.astype(np.float64)
        assert np.allclose(oracle.matvec_t(R, v), want_t, atol=1e-5 * math.sqrt(d))
    P = np.eye(16, dtype=np.float32)[np.random.default_rng(1).permutation(16)]
    v = rng.standard_normal(16).astype(np.float32)
    assert oracle.matvec(P, v).tobytes() == (P @ v).tobytes()  # a permutation is exact


# ---- the polar factor (opq.rs:232-295) ------------------------------------

def test_polar_matches_an_independent_svd(oracle):
    rng = np.random.default_rng(7)
    for d in (2, 5, 16, 64):
        M = rng.standard_normal((d, d)).astype(np.float32)
        U, _, Vt = np.linalg.svd(M.astype(np.float64))
        R = oracle.polar(M)
        assert np.allclose(R, U @ Vt, atol=2e-6), d
        assert np.allclose(R @ R.T, np.eye(d), atol=2e-6)
        S = R.T.astype(np.float64) @ M.astype(np.float64)  # = V S V^T: symmetric PSD
        assert np.allclose(S, S.T, atol=1e-4 * np.abs(S).max())
        assert np.linalg.eigvalsh((S + S.T) / 2).min() > -1e-4 * np.abs(S).max()


def test_polar_closed_form_and_rank_deficiency(oracle):
    rng = np.random.default_rng(11)
    Q = _orthogonal(rng, 12)
    D = np.diag(rng.uniform(0.5, 3.0, 12))
    R = oracle.polar((Q @ D).astype(np.float32))  # M = Q D: U = Q, V = I
    assert np.allclose(R, Q, atol=2e-6)
    # rank 3 in 8 dimensions: still orthogonal, still R^T M = V S V^T
    A = rng.standard_normal((8, 3)) @ rng.standard_normal((3, 8))
    M = A.astype(np.float32)
    R = oracle.polar(M)
    assert np.allclose(R @ R.T, np.eye(8), atol=2e-6)
    S = R.T.astype(np.float64) @ M.astype(np.float64)
    assert np.allclose(S, S.T, atol=1e-4 * np.abs(S).max())
    R0 = oracle.polar(np.zeros((4, 4), np.float32))
    assert np.allclose(R0 @ R0.T, np.eye(4), atol=1e-6)


# ---- training (opq.rs:65-109, tests :387-453) -------------------------------

def test_opq_training_rows_are_unit(oracle):
    n, d = 100, 16
    data = np.array([[((i * 7 + j * 3) % 100) / 100.0 for j in range(d)] for i in range(n)],
                    np.float32)
    R, cb, Ke = oracle.opq_fit(data, 4, 8, 2, 0)
    assert Ke == 8 and cb.size == 4 * 8 * 4
    assert np.allclose((R.astype(np.float64) ** 2).sum(axis=1), 1.0, atol=1e-5)
    assert np.allclose(R @ R.T, np.eye(d), atol=1e-5)


def test_opq_quantize_codes_are_in_range(oracle):
    n, d = 50, 8
    data = np.array([[((i + j) % 10) / 10.0 for j in range(d)] for i in range(n)], np.float32)
    R, cb, Ke = oracle.opq_fit(data, 2, 4, 2, 0)
    codes = oracle.pq_encode(cb, 2, Ke, 4, oracle.matvec(R, np.full(d, 0.5, np.float32)))
    assert codes.shape == (1, 2) and codes.max() < 4
    with pytest.raises(ValueError, match="at least 4 training vectors"):
        oracle.opq_fit(data[:3], 2, 4, 2, 0)


def test_decode_applies_the_transpose(oracle):
    # opq.rs:309-360 with a fixed 90-degree rotation of the first two axes
    rng = np.random.default_rng(11)
    data = rng.uniform(-1.0, 1.0, (64, 4)).astype(np.float32)
    _, cb, Ke = oracle.opq_fit(data, 2, 16, 1, 0)
    R = np.array([[0, -1, 0, 0], [1, 0, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1]], np.float32)
    x = rng.uniform(-1.0, 0.9, 4).astype(np.float32)
    codes = oracle.pq_encode(cb, 2, Ke, 2, oracle.matvec(R, x))[0]
    rotated_space = oracle.pq_reconstruct(cb, 2, Ke, 2, codes)
    decoded = oracle.matvec_t(R, rotated_space)
    assert np.allclose(decoded, R.T @ rotated_space, atol=1e-6)
    assert np.linalg.norm(x - decoded) < np.linalg.norm(x - rotated_space)


def test_the_last_rotation_follows_the_last_codebooks(oracle):
    # the rotation returned is the Procrustes step after the last PQ fit, so
    # it is polar(M) of that fit's reconstructions (opq.rs:94-106)
    rng = np.random.default_rng(5)
    data = rng.standard_normal((300, 8)).astype(np.float32)
    R1, cb1, K1 = oracle.opq_fit(data, 2, 8, 1, 9)
    M = np.zeros((8, 8), np.float32)
    for x in data:
        rec = oracle.pq_reconstruct(cb1, 2, K1, 4, oracle.pq_encode(cb1, 2, K1, 4, x)[0])
        M += np.outer(rec, x).astype(np.float32)
    assert np.allclose(R1, oracle.polar(M), atol=1e-5)
    R2, cb2, _ = oracle.opq_fit(data, 2, 8, 2, 9)
    # the second fit trains on the data rotated by R1
    rot = np.stack([oracle.matvec(R1, x) for x in data])
    cbm = [oracle.kmeans(np.ascontiguousarray(rot[:, 4 * m:4 * m + 4]), 8, 1, 9 + m, 100)[0]
           for m in range(2)]
    assert cb2.tobytes() == np.concatenate([c.ravel() for c in cbm]).tobytes()


# ---- tests/opq_vs_pq.rs: OPQ does not regress against PQ ------------------

class _Lcg:
    def __init__(self, seed):
        self.s = seed

    def next_f32(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        return np.float32(np.float32(self.s >> 33) / np.float32(np.float32(4294967295.0) / 2)) - np.float32(1)


def _normalize(v):
    n = np.float32(math.sqrt(float(np.dot(v.astype(np.float64), v.astype(np.float64)))))
    return v / n if n >= 1e-10 else np.zeros_like(v)


def _correlated(n, d, seed):
    rng = _Lcg(seed)
    mixing = np.array([rng.next_f32() for _ in range(d * 4)], np.float32)
    out = []
    for _ in range(n):
        f = [rng.next_f32() for _ in range(4)]
        v = np.zeros(d, np.float32)
        for j in range(d):
            for k in range(4):
                v[j] += mixing[j * 4 + k] * f[k]
            v[j] += rng.next_f32() * np.float32(0.1)
        out.append(_normalize(v))
    return np.array(out, np.float32)


def _uncorrelated(n, d, seed):
    rng = _Lcg(seed)
    return np.array([_normalize(np.array([rng.next_f32() for _ in range(d)], np.float32))
                     for _ in range(n)], np.float32)


def _mae(oracle, data, pairs, approx):
    rng = _Lcg(999)
    n = data.shape[0]
    tot, cnt = 0.0, 0
    for _ in range(pairs):
        i = int(np.float32(abs(rng.next_f32())) * np.float32(n)) % n
        j = int(np.float32(abs(rng.next_f32())) * np.float32(n)) % n
        if i == j:
            continue
        exact = 1.0 - float(np.dot(data[i].astype(np.float64), data[j].astype(np.float64)))
        tot += abs(exact - float(approx(data[i], data[j])))
        cnt += 1
    return tot / cnt


def _pq_codebooks(oracle, data, M, K, seed):
    ds = data.shape[1] // M
    return np.concatenate([oracle.kmeans(np.ascontiguousarray(data[:, m * ds:(m + 1) * ds]), K, 1,
                                         seed + m, 100)[0].ravel() for m in range(M)])


@pytest.mark.parametrize("kind", ["correlated", "uncorrelated"])
def test_opq_does_not_regress_against_pq(oracle, kind):
    if kind == "correlated":  # opq_vs_pq.rs:145-190
        d, M, K, n, iters, pairs, slack = 32, 4, 16, 500, 5, 2000, (1.2, 0.001)
        data = _correlated(n, d, 42)
    else:  # opq_vs_pq.rs:197-240
        d, M, K, n, iters, pairs, slack = 16, 4, 8, 200, 3, 1000, (1.5, 0.01)
        data = _uncorrelated(n, d, 123)
    ds = d // M
    cb = _pq_codebooks(oracle, data, M, K, 0)

    def pq_dist(q, x):
        return oracle.distance_with_table(oracle.adc_table(cb, M, K, ds, q), M, K,
                                          oracle.pq_encode(cb, M, K, ds, x)[0])

    R, ocb, Ke = oracle.opq_fit(data, M, K, iters, 0)

    def opq_dist(q, x):
        table = oracle.adc_table(ocb, M, Ke, ds, oracle.matvec(R, q))
        return oracle.distance_with_table(table, M, Ke, oracle.pq_encode(ocb, M, Ke, ds,
                                                                          oracle.matvec(R, x))[0])

    pq_mae = _mae(oracle, data, pairs, pq_dist)
    opq_mae = _mae(oracle, data, pairs, opq_dist)
    assert opq_mae <= pq_mae * slack[0] + slack[1], (opq_mae, pq_mae)


# ---- IVF-PQ with OPQ: build and search -----------------------------------

def _opq_index(oracle, n=600, d=16, L=8, M=4, K=16, seed=3):
    rng = np.random.default_rng(seed)
    vecs = oracle.normalize_rows(rng.standard_normal((n, d)).astype(np.float32))
    ix, assign = oracle.ivfpq_build(vecs, L, M, K, seed, 0, 20, use_opq=True)
    return ix, assign, rng


def test_build_encodes_the_rotated_residuals(oracle):
    ix, assign, _ = _opq_index(oracle)
    R = ix.rotation
    assert R is not None and np.allclose(R @ R.T, np.eye(ix.d), atol=1e-5)
    ds = ix.d // ix.M
    for v in range(0, ix.codes.shape[0], 7):
        res = ix.vectors[v] - ix.centroids[assign[v]]
        want = oracle.pq_encode(ix.codebooks, ix.M, ix.K, ds, oracle.matvec(R, res))[0]
        assert ix.codes[v].tolist() == want.tolist()


def test_identity_rotation_searches_like_pq(oracle):
    rng = np.random.default_rng(2)
    vecs = oracle.normalize_rows(rng.standard_normal((500, 16)).astype(np.float32))
    ix, _ = oracle.ivfpq_build(vecs, 8, 4, 256, 1, 0, 10)
    rot = oracle.Index(ix.centroids, ix.codebooks, ix.list_offsets, ix.list_ids, ix.codes,
                       ix.doc_ids, ix.vectors, ix.M, ix.K, np.eye(16, dtype=np.float32))
    q = rng.standard_normal((20, 16)).astype(np.float32)
    for pool in (0, 30):
        a, b = ix.search_batch(q, 10, 3, pool), rot.search_batch(q, 10, 3, pool)
        assert np.array_equal(a[0], b[0]) and a[1].tobytes() == b[1].tobytes()


@pytest.mark.parametrize("K", [16, 256])
def test_full_probe_equals_exhaustive_rotated_scan(oracle, K):
    ix, assign, rng = _opq_index(oracle, n=400, K=K, seed=4)
    R64 = ix.rotation.astype(np.float64)
    ds = ix.d // ix.M
    recon = np.stack([oracle.pq_reconstruct(ix.codebooks, ix.M, ix.K, ds, ix.codes[v])
                      for v in range(ix.codes.shape[0])]).astype(np.float64)
    for _ in range(6):
        q = oracle.normalize_rows(rng.standard_normal((1, ix.d)).astype(np.float32))[0]
        ids, dists = ix.search(q, 10, ix.centroids.shape[0])
        r = q.astype(np.float64)[None, :] - ix.centroids[assign].astype(np.float64)
        exact = (((r @ R64.T) - recon) ** 2).sum(axis=1)
        order = np.lexsort((np.arange(exact.size), exact))[:10]
        tol = 1e-4 if K == 256 else 2e-2  # K = 16 lists take FastScan's u8 table
        if K == 256:
            assert ids.tolist() == order.tolist()
        for i, dd in zip(ids.tolist(), dists):
            assert math.isclose(exact[i], float(dd), rel_tol=tol, abs_tol=tol)
