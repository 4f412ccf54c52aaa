"""Seeded synthetic workloads for the five benchmark shapes.

The reference publishes no data for these shapes (its own generators use
rand::StdRng, which cannot be reproduced here), so these generators define
the data: numpy PCG64 streams with fixed seeds, float32 throughout.  Every
mixture draws its centres from one stream and its base vectors and queries
from two more, so queries come from the same mixture as the base.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Workload:
    name: str
    base: np.ndarray
    queries: np.ndarray
    params: dict = field(default_factory=dict)


def _mixture(rng_c, rng_x, n, d, centres, std, chunk=1 << 20, clamp_min=None, normalise=False):
    out = np.empty((n, d), np.float32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        lab = rng_x.integers(0, centres.shape[0], e - s)
        x = rng_x.standard_normal((e - s, d), dtype=np.float32)
        x *= np.float32(std)
        x += centres[lab]
        if clamp_min is not None:
            np.maximum(x, np.float32(clamp_min), out=x)
        if normalise:
            x /= np.maximum(np.linalg.norm(x, axis=1, keepdims=True), np.float32(1e-30))
        out[s:e] = x
    return out


def _unit_rows(rng, n, d):
    c = rng.standard_normal((n, d), dtype=np.float32)
    c /= np.linalg.norm(c, axis=1, keepdims=True)
    return c


def ivfpq_small(n=20_000, nq=1_000) -> Workload:
    """n x 32 uniform [0,1) from seed 0, queries from seed 1; nlist 64
    (10 k-means iterations), M 8 x 4 dims, ksub 256, nprobe 8, k 10."""
    base = np.random.default_rng(0).random((n, 32), dtype=np.float32)
    queries = np.random.default_rng(1).random((nq, 32), dtype=np.float32)
    return Workload("ivfpq_small_20k_d32", base, queries,
                    dict(num_clusters=64, num_codebooks=8, codebook_size=256, nprobe=8, k=10,
                         kmeans_max_iter=10, training_sample_size=None))


def flat_gaussian(n=100_000, nq=10_000, d=96) -> Workload:
    """n x 96 mixture of 100 centres uniform in [0,1)^96, std 0.05; squared L2."""
    rc = np.random.default_rng(20)
    centres = rc.random((100, d), dtype=np.float32)
    base = _mixture(rc, np.random.default_rng(21), n, d, centres, 0.05)
    queries = _mixture(rc, np.random.default_rng(22), nq, d, centres, 0.05)
    return Workload("flat_100k_d96", base, queries, dict(k=10, metric="l2"))


def ivfpq_1m(n=1_000_000, nq=10_000, d=128) -> Workload:
    """n x 128 mixture of 1000 centres uniform in [0,128)^128, std 8, clamped
    at 0; nlist 4096, M 16 x 8 dims, ksub 256, nprobe 32, k 100."""
    rc = np.random.default_rng(30)
    centres = (rc.random((1000, d), dtype=np.float32) * np.float32(128.0)).astype(np.float32)
    base = _mixture(rc, np.random.default_rng(31), n, d, centres, 8.0, clamp_min=0.0)
    queries = _mixture(rc, np.random.default_rng(32), nq, d, centres, 8.0, clamp_min=0.0)
    return Workload("ivfpq_1m_d128", base, queries,
                    dict(num_clusters=4096, num_codebooks=16, codebook_size=256, nprobe=32, k=100))


def ivfpq_10m_angular(n=10_000_000, nq=10_000, d=96) -> Workload:
    """n x 96 mixture of 10,000 centres on the unit sphere, std 0.1, rows
    normalised; nlist 16384, M 48 x 2 dims, ksub 256, nprobe 64, k 10."""
    rc = np.random.default_rng(40)
    centres = _unit_rows(rc, 10_000, d)
    base = _mixture(rc, np.random.default_rng(41), n, d, centres, 0.1, normalise=True)
    queries = _mixture(rc, np.random.default_rng(42), nq, d, centres, 0.1, normalise=True)
    return Workload("ivfpq_10m_d96_angular", base, queries,
                    dict(num_clusters=16384, num_codebooks=48, codebook_size=256, nprobe=64, k=10))


def ivfpq_4bit_rerank(n=1_000_000, nq=10_000, d=100) -> Workload:
    """n x 100 mixture of 500 centres on the unit sphere, std 0.1, rows
    normalised; nlist 2048, M 50 x 2 dims, ksub 16 (FastScan), nprobe 64,
    rerank pool 100, k 10."""
    rc = np.random.default_rng(50)
    centres = _unit_rows(rc, 500, d)
    base = _mixture(rc, np.random.default_rng(51), n, d, centres, 0.1, normalise=True)
    queries = _mixture(rc, np.random.default_rng(52), nq, d, centres, 0.1, normalise=True)
    return Workload("ivfpq_4bit_1m_d100", base, queries,
                    dict(num_clusters=2048, num_codebooks=50, codebook_size=16, nprobe=64, k=10,
                         rerank_pool=100))


WORKLOADS = {
    "ivfpq_small": ivfpq_small,
    "flat": flat_gaussian,
    "ivfpq_1m": ivfpq_1m,
    "ivfpq_10m": ivfpq_10m_angular,
    "ivfpq_4bit": ivfpq_4bit_rerank,
}
