"""Deterministic generators restated from the reference's own tests."""

from __future__ import annotations

import numpy as np

MASK64 = (1 << 64) - 1


def pq_lcg_values(count: int, state: int):
    """pq.rs:377-382: s = s*6364136223846793005 + 1; ((s>>33) as f32 / 2^31) - 1.

    Returns (values f32[count], new_state)."""
    out = np.empty(count, np.float32)
    two31 = np.float32(2.0 ** 31)
    one = np.float32(1.0)
    for i in range(count):
        state = (state * 6364136223846793005 + 1) & MASK64
        out[i] = np.float32(np.float32(state >> 33) / two31) - one
    return out, state


def pq_lcg_codes(count: int, K: int, state: int):
    """pq.rs:403-412: codes = state % codebook_size after each LCG step."""
    out = np.empty(count, np.uint8)
    for i in range(count):
        state = (state * 6364136223846793005 + 1) & MASK64
        out[i] = state % K
    return out, state


def regression_lcg(count: int, state: int):
    """tests/correctness_regression/tests_feature_gated.rs:17-33."""
    out = np.empty(count, np.float32)
    half = np.float32(np.float32(4294967295.0) / np.float32(2.0))
    one = np.float32(1.0)
    for i in range(count):
        state = (state * 6364136223846793005 + 1442695040888963407) & MASK64
        out[i] = np.float32(np.float32(state >> 33) / half) - one
    return out, state


def seq_normalize(v: np.ndarray) -> np.ndarray:
    """distance.rs:135-141 with the scalar norm: sequential float32 sum."""
    v = np.asarray(v, np.float32)
    s = np.float32(0.0)
    for x in v:
        s = np.float32(s + np.float32(x * x))
    n = np.float32(np.sqrt(s))
    if n < np.float32(1e-10):
        return np.zeros_like(v)
    return (v / n).astype(np.float32)


def f64_l2sq(a, b) -> float:
    d = np.asarray(a, np.float64) - np.asarray(b, np.float64)
    return float(np.dot(d, d))


def total_cmp_key(d) -> np.ndarray:
    """f32::total_cmp as an unsigned key (u32 order == total_cmp order)."""
    b = np.asarray(d, np.float32).view(np.uint32)
    return np.where(b & 0x80000000, ~b, b | 0x80000000).astype(np.uint32)
