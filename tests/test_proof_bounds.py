"""The error bounds behind the exactness proofs, driven on the CPU with
adversarial float32 inputs: large centroid norms, tiny and cancelling
residuals, bfloat16 worst-case mantissas.  The bounds are the library's own
(vgpu_test_bound_*, the code the kernels run); the approximate scores are
numpy float32 emulations of the kernels' arithmetic in several summation
orders, the exact scores are the oracle's restatement of the reference
(pq.rs:232-276, simd.rs dot, distance.rs:78-109).

- FAST ranking value a = ||q - c||^2 + b(x) + sum_m T2[m][code_m] against the
  ADC distance e (k_scan8_fast.hip; bias_kernel in k_build.hip):
  |a - e| <= fast_tau.
- bf16x3 coarse score 1 - (qh.ch + qh.cl + ql.ch) against 1 - dot:
  |.| <= coarse_eps_bf16; the fp32 score within coarse_tau.
- flat ranking key ||x||^2 - 2 q.x (bf16x3, low mantissa bits replaced by a
  tile index) plus ||q||^2 against l2_distance_squared: <= flat_bf16_tau.

Each family also shows the inputs have teeth: the same case breaks a bound
with one term dropped, so a bound that lost that term would fail here."""

import ctypes

import numpy as np
import pytest

F32 = np.float32
U = 2.0 ** -24


def _lib():
    from vicinity_amd import _lib

    return _lib


def fast_tau(d, M, ds, qn, cmax, rmax, t0max):
    out = ctypes.c_float()
    _lib().check(_lib().load().vgpu_test_bound_fast_tau(d, M, ds, qn, cmax, rmax, t0max,
                                                        ctypes.byref(out)))
    return out.value


def coarse_bounds(d, qn, cmax):
    a, b = ctypes.c_float(), ctypes.c_float()
    _lib().check(_lib().load().vgpu_test_bound_coarse(d, qn, cmax, ctypes.byref(a), ctypes.byref(b)))
    return a.value, b.value


def flat_tau(d, metric, qn, xn, ib):
    out = ctypes.c_float()
    _lib().check(_lib().load().vgpu_test_bound_flat(d, metric, qn, xn, ib, ctypes.byref(out)))
    return out.value


# ---- float32 emulation helpers --------------------------------------------

def fma(a, b, c):
    """float32 fused multiply-add (exact product and sum, one rounding; the
    float64 sum of a float32 product and addend is exact here)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F32)


def seq_sum(terms, axis=-1):
    """Sequential float32 sum along axis."""
    terms = np.moveaxis(np.asarray(terms, F32), axis, 0)
    acc = np.zeros(terms.shape[1:], F32)
    for t in terms:
        acc = (acc + t).astype(F32)
    return acc


def tree_sum(terms, axis=-1):
    """Pairwise float32 sum along axis (the lane-exchange order)."""
    t = np.moveaxis(np.asarray(terms, F32), axis, 0)
    while t.shape[0] > 1:
        if t.shape[0] % 2:
            t = np.concatenate([t, np.zeros((1,) + t.shape[1:], F32)])
        t = (t[0::2] + t[1::2]).astype(F32)
    return t[0]


def bound_norm(x):
    """row_norm_bound (vgpu_index.cpp): float64 norm times 1.0001."""
    return F32(np.sqrt(np.sum(np.asarray(x, np.float64) ** 2)) * 1.0001 + 1e-30)


def bf16_split(x):
    """Round-to-nearest-even bfloat16 hi, then lo of the remainder."""
    x = np.asarray(x, F32)
    u = x.view(np.uint32)
    hb = ((u + np.uint32(0x7fff) + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    hi = (hb << 16).view(F32)
    rem = (x - hi).astype(F32)
    ru = rem.view(np.uint32)
    lb = ((ru + np.uint32(0x7fff) + ((ru >> 16) & 1)) >> 16).astype(np.uint32)
    lo = (lb << 16).view(F32)
    return hi, lo


def mfma_bf16x3(a, b, order):
    """sum_j a_j b_j as three bf16 MFMA passes (ah.bl, al.bh, ah.bh) over
    32-dimension steps.  Products of bf16 values are exact in float32; each
    step's 32 products are summed as `order` says: 'exact' (one rounding per
    step), 'seq' (float32 after every product), 'trunc' (sums rounded toward
    zero)."""
    ah, al = bf16_split(a)
    bh, bl = bf16_split(b)
    d = a.shape[-1]
    acc = np.zeros(np.broadcast_shapes(a.shape[:-1], b.shape[:-1]), F32)
    for t0 in range(0, d, 32):
        sl = slice(t0, min(d, t0 + 32))
        for x, y in ((ah, bl), (al, bh), (ah, bh)):
            prods = (x[..., sl].astype(np.float64) * y[..., sl].astype(np.float64))
            if order == "exact":
                acc = (acc.astype(np.float64) + prods.sum(-1)).astype(F32)
            elif order == "seq":
                for j in range(prods.shape[-1]):
                    acc = (acc + prods[..., j].astype(F32)).astype(F32)
            else:
                s = acc.astype(np.float64) + prods.sum(-1)
                r = s.astype(F32)
                too_big = np.abs(r.astype(np.float64)) > np.abs(s)
                acc = np.where(too_big, np.nextafter(r, F32(0)), r).astype(F32)
    return acc


# ---- FAST ranking value against the ADC distance ---------------------------

def _fast_case(rng, kind, d=32, M=8, K=32, n=400):
    ds = d // M
    if kind == "gaussian":
        q = rng.standard_normal(d)
        c = 0.3 * rng.standard_normal(d)
        cb = 0.5 * rng.standard_normal((M, K, ds))
    elif kind == "large_centroid":
        # loaded artifacts with centroid norm ~1e3 and residual codewords
        # that nearly cancel the residual: every term of a is ~1e6, e is small
        q = rng.standard_normal(d)
        c = 180.0 * rng.standard_normal(d)
        r = q - c
        cb = r.reshape(M, 1, ds) + 1e-2 * rng.standard_normal((M, K, ds))
    elif kind == "tiny_residual":
        q = rng.standard_normal(d)
        c = q + 1e-4 * rng.standard_normal(d)
        cb = 1e-4 * rng.standard_normal((M, K, ds))
    elif kind == "mantissa":
        # values one ulp around powers of two and halfway bf16 patterns
        base = rng.choice([1.0, -1.0, 0.5, 2.0], size=d) * (1 + rng.integers(0, 4, size=d) * 2.0 ** -23)
        q = base
        c = -base * (1 + 2.0 ** -9)
        cb = np.stack([np.stack([(q - c)[m * ds:(m + 1) * ds] * (1 + (k % 5) * 2.0 ** -8)
                                 for k in range(K)]) for m in range(M)])
    else:
        raise ValueError(kind)
    q = np.asarray(q, F32)
    q = (q / np.float32(np.sqrt(np.sum(q.astype(np.float64) ** 2)))).astype(F32)
    return (q, np.asarray(c, F32), np.asarray(cb, F32).reshape(M, K, ds),
            rng.integers(0, K, size=(n, M)).astype(np.uint8), d, M, K, ds)


def _round_toward_zero(s):
    """float64 sums rounded to float32 toward zero (a truncating adder)."""
    r = np.asarray(s).astype(F32)
    too_big = np.abs(r.astype(np.float64)) > np.abs(s)
    return np.where(too_big, np.nextafter(r, F32(0)), r).astype(F32)


def _t2_table(q, cb, M, ds, table):
    """T2[m][k] = -2 q_m . cw_mk as the kernels form it.  'fma': the scan's
    own build, -2 times an fma chain over the dimensions.  The pre-pass
    (t2_table_kernel): fp32 MFMA on (-2 q) and cw, exact products summed in
    float32 with sums that may truncate, either after every product
    ('mfma_seq') or once per step of four dimensions ('mfma_step')."""
    qm = q.reshape(M, ds)
    if table == "fma":
        t2 = np.zeros(cb.shape[:2], F32)
        for j in range(ds):
            t2 = fma(qm[:, None, j], cb[:, :, j], t2)
        return (F32(-2.0) * t2).astype(F32)
    prods = (F32(-2.0) * qm).astype(np.float64)[:, None, :] * cb.astype(np.float64)  # exact in float64
    acc = np.zeros(cb.shape[:2], F32)
    if table == "mfma_seq":
        for j in range(ds):
            acc = _round_toward_zero(acc.astype(np.float64) + prods[..., j])
    else:
        for j0 in range(0, ds, 4):
            acc = _round_toward_zero(acc.astype(np.float64) + prods[..., j0:j0 + 4].sum(-1))
    return acc


def _fast_a(q, c, cb, codes, d, M, ds, order, table="fma"):
    """The FAST kernel's ranking value for each entry (codes [n, M])."""
    diff = (q - c).astype(F32)
    acc = np.zeros(8, F32)  # term0: eight lanes, fma over j = lane mod 8, then a tree
    for j in range(d):
        acc[j % 8] = fma(diff[j], diff[j], acc[j % 8])
    term0 = tree_sum(acc, axis=0)
    t2 = _t2_table(q, cb, M, ds, table)
    # b(x) = sum_m (||cw||^2 + 2 c_m . cw), no FMA (bias_kernel)
    cw = cb[np.arange(M)[None, :], codes]  # [n, M, ds]
    e1 = np.zeros(codes.shape, F32)
    e2 = np.zeros(codes.shape, F32)
    cm = c.reshape(M, ds)
    for j in range(ds):
        e1 = (e1 + (cw[..., j] * cw[..., j]).astype(F32)).astype(F32)
        e2 = (e2 + (cm[None, :, j] * cw[..., j]).astype(F32)).astype(F32)
    b = seq_sum((e1 + (F32(2.0) * e2).astype(F32)).astype(F32), axis=1)
    terms = t2[np.arange(M)[None, :], codes]
    S = tree_sum(terms, axis=1) if order == "tree" else seq_sum(terms, axis=1)
    if order == "tree":
        return ((term0 + b).astype(F32) + S).astype(F32), term0
    return (term0 + (b + S).astype(F32)).astype(F32), term0


@pytest.mark.parametrize("table", ["fma", "mfma_seq", "mfma_step"])
@pytest.mark.parametrize("kind", ["gaussian", "large_centroid", "tiny_residual", "mantissa"])
def test_fast_ranking_value_within_fast_tau(oracle, kind, table):
    rng = np.random.default_rng({"gaussian": 1, "large_centroid": 2, "tiny_residual": 3,
                                 "mantissa": 4}[kind])
    worst = 0.0
    for ds_case in (4, 8):
        q, c, cb, codes, d, M, K, ds = _fast_case(rng, kind, M=32 // ds_case)
        r = (q - c).astype(F32)
        e = oracle.adc_scan(codes, M, K, oracle.adc_table(cb.reshape(-1), M, K, ds, r))
        rmax = F32(np.sqrt(np.sum(np.max(np.sum(cb.astype(np.float64) ** 2, -1), -1))) * 1.0001 + 1e-30)
        for order in ("tree", "seq"):
            a, term0 = _fast_a(q, c, cb, codes, d, M, ds, order, table)
            tau = fast_tau(d, M, ds, bound_norm(q), bound_norm(c), rmax, float(term0))
            err = np.abs(a.astype(np.float64) - e.astype(np.float64)).max()
            assert err <= tau, (kind, order, err, tau)
            worst = max(worst, err / tau)
    assert worst > 0.0 or kind == "tiny_residual"


# ---- bf16x3 and fp32 coarse scores ------------------------------------------

def _coarse_case(rng, kind, d, nq=64, L=48):
    if kind == "gaussian":
        Q = rng.standard_normal((nq, d))
        C = rng.standard_normal((L, d)) / np.sqrt(d)
    elif kind == "large_centroid":
        Q = rng.standard_normal((nq, d))
        C = 100.0 * rng.standard_normal((L, d))
    elif kind == "cancelling":
        # q.c ~ 0 with |q_j c_j| large: centroids orthogonal to a common
        # query direction, queries within 1e-3 of it
        q0 = np.abs(rng.standard_normal(d)) + 0.5
        q0 /= np.linalg.norm(q0)
        Q = q0 + 1e-3 * rng.standard_normal((nq, d))
        C = 30.0 * rng.standard_normal((L, d))
        C -= np.outer(C @ q0, q0)
    elif kind == "mantissa":
        # bf16 halfway patterns: low 16 bits 0x8000 (ties to even) and 0x7fff
        bits = rng.integers(0x3f000000, 0x40800000, size=(nq + L, d), dtype=np.int64)
        bits = (bits & ~0xffff) | rng.choice([0x8000, 0x7fff, 0xffff, 0x0001], size=(nq + L, d))
        X = bits.astype(np.uint32).view(F32) * rng.choice([1, -1], size=(nq + L, d)).astype(F32)
        Q, C = X[:nq], X[nq:]
    else:
        raise ValueError(kind)
    Q = np.asarray(Q, F32)
    Q = (Q / np.sqrt(np.sum(Q.astype(np.float64) ** 2, 1, keepdims=True))).astype(F32)
    return Q, np.asarray(C, F32)


@pytest.mark.parametrize("d", [2, 3, 7, 32, 96, 128])
@pytest.mark.parametrize("kind", ["gaussian", "large_centroid", "cancelling", "mantissa"])
def test_coarse_bf16x3_score_within_eps(oracle, kind, d):
    rng = np.random.default_rng(d * 7 + len(kind))
    Q, C = _coarse_case(rng, kind, d, nq=96 if d < 8 else 64, L=96 if d < 8 else 48)
    cmax = max(bound_norm(c) for c in C)
    qn = 1.0001  # normalised queries (the fused kernel's bound)
    eps, tau32 = coarse_bounds(d, qn, cmax)
    ref = np.array([[F32(1.0) - oracle.dot(q, c) for c in C] for q in Q], F32)
    for order in ("exact", "seq", "trunc"):
        approx = (F32(1.0) - mfma_bf16x3(Q[:, None, :], C[None, :, :], order)).astype(F32)
        err = np.abs(approx.astype(np.float64) - ref.astype(np.float64)).max()
        assert err <= eps, (kind, d, order, err, eps)
    # the fp32 GEMM path: products and sums in float32, any order
    for order in ("seq", "tree"):
        prods = (Q[:, None, :] * C[None, :, :]).astype(F32)
        dots = seq_sum(prods, axis=2) if order == "seq" else tree_sum(prods, axis=2)
        err = np.abs((F32(1.0) - dots).astype(np.float64) - ref.astype(np.float64)).max()
        assert err <= tau32, (kind, d, order, err, tau32)


def test_coarse_eps_split_term_needs_2_to_the_minus_16(oracle):
    """bfloat16 rounds within 2^-8 relative, so the split remainder is within
    2^-16 |x|, not 2^-18: a centroid component just above a power of two
    (256.94 -> hi 256, lo 0.9414, remainder 1.6e-3) with a query component
    near a bf16 midpoint makes the dropped terms exceed 3.01 * 2^-18
    sum|q_j c_j|.  The bound with 2^-18 fails here; the library's holds."""
    q = np.array([[0.9781833, 0.20774342]], F32)
    c = np.array([[256.94305, -10.729167]], F32)
    ref = F32(1.0) - oracle.dot(q[0], c[0])
    approx = (F32(1.0) - mfma_bf16x3(q[:, None, :], c[None, :, :], "exact"))[0, 0]
    err = abs(float(approx) - float(ref))
    qc = 1.0001 * float(bound_norm(c[0]))
    old_bound = (3.01 * 2.0 ** -18 + 7.0 * 2 * U) * qc + 2 * U * (1 + qc)
    eps, _ = coarse_bounds(2, 1.0001, float(bound_norm(c[0])))
    assert err > old_bound
    assert err <= eps


# ---- flat bf16x3 ranking key --------------------------------------------------

@pytest.mark.parametrize("kind", ["gaussian", "large_norm", "near_duplicate"])
@pytest.mark.parametrize("d", [33, 96, 128])
def test_flat_key_within_flat_tau(oracle, kind, d):
    rng = np.random.default_rng(d + len(kind))
    n, nq, ib = 96, 24, 8
    if kind == "gaussian":
        X = rng.standard_normal((n, d))
        Q = rng.standard_normal((nq, d))
    elif kind == "large_norm":
        X = 300.0 * rng.standard_normal((n, d))
        Q = 300.0 * rng.standard_normal((nq, d))
    else:
        X = rng.standard_normal((n, d))
        Q = X[rng.integers(0, n, nq)] + 1e-5 * rng.standard_normal((nq, d))
    X, Q = np.asarray(X, F32), np.asarray(Q, F32)
    xnorm = seq_sum((X * X).astype(F32), axis=1)  # flat_norms_kernel: no FMA
    qn = max(bound_norm(q) for q in Q)
    xn = max(bound_norm(x) for x in X)
    tau = flat_tau(d, 0, qn, xn, ib)
    ref = np.array([[oracle.l2sq(q, x) for x in X] for q in Q], F32)
    q2 = seq_sum((Q * Q).astype(F32), axis=1)
    for order in ("exact", "seq", "trunc"):
        acc = mfma_bf16x3((F32(-2.0) * Q)[:, None, :].astype(F32), X[None, :, :], order)
        v = (xnorm[None, :] + acc).astype(F32)
        # worst packing: the low ib bits replaced by all ones or all zeros
        for tile in (0, (1 << ib) - 1):
            key = ((v.view(np.uint32) & np.uint32(~((1 << ib) - 1) & 0xffffffff)) | np.uint32(tile)).view(F32)
            err = np.abs(key.astype(np.float64) + q2[:, None].astype(np.float64) - ref.astype(np.float64)).max()
            assert err <= tau, (kind, d, order, tile, err, tau)
