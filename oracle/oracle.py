"""ctypes wrapper around the C oracle (vicinity_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, to check results against.  The product
(vicinity_amd/) never imports this module.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libvicinity_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_sz = ctypes.c_size_t


def build() -> str:
    """Compile the oracle with its Makefile (idempotent)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def use_native() -> str:
    """Build the -march=native copy for this host (bit-identical results) and
    make it the library every later call loads; call before the first use."""
    global _LIB_PATH
    if _lib is not None:
        raise RuntimeError("the oracle library is already loaded")
    subprocess.run(["make", "-s", "-C", _HERE, "native"], check=True)
    _LIB_PATH = os.path.join(_HERE, "_build", "native", "libvicinity_oracle.so")
    return _LIB_PATH


class _Index(ctypes.Structure):
    _fields_ = [
        ("d", _sz), ("L", _sz), ("M", _sz), ("K", _sz), ("ds", _sz), ("n", _sz),
        ("centroids", ctypes.c_void_p), ("codebooks", ctypes.c_void_p),
        ("list_offsets", ctypes.c_void_p), ("list_ids", ctypes.c_void_p),
        ("codes", ctypes.c_void_p), ("doc_ids", ctypes.c_void_p),
        ("vectors", ctypes.c_void_p), ("rotation", ctypes.c_void_p),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_dot.restype = ctypes.c_float
        L.or_dot.argtypes = [_f32p, _f32p, _sz]
        L.or_l2sq.restype = ctypes.c_float
        L.or_l2sq.argtypes = [_f32p, _f32p, _sz]
        L.or_normalize_rows.argtypes = [_f32p, _sz, _sz, _f32p]
        L.or_adc_table.argtypes = [_f32p, _sz, _sz, _sz, _f32p, _f32p]
        L.or_distance_with_table.restype = ctypes.c_float
        L.or_distance_with_table.argtypes = [_f32p, _sz, _sz, _u8p]
        L.or_adc_scan.argtypes = [_u8p, _sz, _sz, _sz, _f32p, _f32p]
        L.or_pq_encode.argtypes = [_f32p, _sz, _sz, _sz, _f32p, _sz, _u8p]
        L.or_pq_reconstruct.argtypes = [_f32p, _sz, _sz, _sz, _u8p, _f32p]
        L.or_pack4_size.restype = _sz
        L.or_pack4_size.argtypes = [_sz, _sz]
        L.or_pack4.argtypes = [_u8p, _sz, _sz, _u8p]
        L.or_quantize_lut.argtypes = [_f32p, _sz, _u8p, ctypes.POINTER(ctypes.c_float),
                                      ctypes.POINTER(ctypes.c_float)]
        L.or_fastscan_block.argtypes = [_u8p, _u8p, _sz, _u16p]
        L.or_fastscan_batch.restype = ctypes.c_int
        L.or_fastscan_batch.argtypes = [_u8p, _sz, _sz, _f32p, _f32p]
        L.or_nearest_centroids.restype = _sz
        L.or_nearest_centroids.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _u32p, _f32p]
        L.or_top_k.restype = _sz
        L.or_top_k.argtypes = [_u32p, _f32p, _sz, _sz, _u32p, _f32p]
        L.or_ivfpq_search.restype = ctypes.c_long
        L.or_ivfpq_search.argtypes = [ctypes.POINTER(_Index), _f32p, _sz, _sz, _u32p, _f32p]
        L.or_ivfpq_search_reranked.restype = ctypes.c_long
        L.or_ivfpq_search_reranked.argtypes = [ctypes.POINTER(_Index), _f32p, _sz, _sz, _sz,
                                               _u32p, _f32p]
        L.or_ivfpq_search_batch.restype = ctypes.c_int
        L.or_ivfpq_search_batch.argtypes = [ctypes.POINTER(_Index), _f32p, _sz, _sz, _sz, _sz,
                                            ctypes.c_int, _i64p, _f32p]
        L.or_ivfpq_search_filtered.restype = ctypes.c_long
        L.or_ivfpq_search_filtered.argtypes = [ctypes.POINTER(_Index), _u64p, _i8p, _f32p, _sz,
                                               _sz, ctypes.c_int, _u32p, _f32p]
        L.or_list_masks.argtypes = [ctypes.POINTER(_Index), _i8p, _u64p]
        L.or_ivfpq_probe.restype = _sz
        L.or_ivfpq_probe.argtypes = [ctypes.POINTER(_Index), _f32p, _sz, _u32p, _f32p]
        L.or_assign_cosine.argtypes = [_f32p, _sz, _f32p, _sz, _sz, _u32p]
        L.or_build_lists.argtypes = [_u32p, _sz, _sz, _u64p, _u32p]
        L.or_sample_indices.argtypes = [_sz, _sz, ctypes.c_uint64, _u32p]
        L.or_kmeans.restype = ctypes.c_long
        L.or_kmeans.argtypes = [_f32p, _sz, _sz, _sz, ctypes.c_int, ctypes.c_uint64, _sz, _f32p]
        L.or_ivfpq_build.restype = ctypes.c_int
        L.or_ivfpq_build.argtypes = [_f32p, _sz, _sz, _sz, _sz, _sz, ctypes.c_uint64, _sz, _sz,
                                     ctypes.c_int, _f32p, _f32p, _u32p, _u8p, _f32p,
                                     ctypes.POINTER(_sz)]
        L.or_matvec.argtypes = [_f32p, _f32p, _sz, _f32p]
        L.or_matvec_t.argtypes = [_f32p, _f32p, _sz, _f32p]
        L.or_polar.argtypes = [_f32p, _sz, _f32p]
        L.or_opq_fit.restype = ctypes.c_int
        L.or_opq_fit.argtypes = [_f32p, _sz, _sz, _sz, _sz, _sz, ctypes.c_uint64, _sz, _f32p,
                                 _f32p, ctypes.POINTER(_sz)]
        L.or_flat_search.restype = ctypes.c_int
        L.or_flat_search.argtypes = [_f32p, _sz, _sz, _f32p, _sz, _sz, ctypes.c_int, ctypes.c_int,
                                     _i64p, _f32p]
        _lib = L
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- scalar kernels ------------------------------------------------------

def dot(a, b) -> np.float32:
    a, b = _c(a, np.float32), _c(b, np.float32)
    return np.float32(lib().or_dot(a, b, a.size))


def l2sq(a, b) -> np.float32:
    a, b = _c(a, np.float32), _c(b, np.float32)
    return np.float32(lib().or_l2sq(a, b, a.size))


def normalize_rows(x) -> np.ndarray:
    x = _c(np.atleast_2d(x), np.float32)
    out = np.empty_like(x)
    lib().or_normalize_rows(x, x.shape[0], x.shape[1], out)
    return out


# ---- product quantiser ---------------------------------------------------

def adc_table(codebooks, M, K, ds, r) -> np.ndarray:
    out = np.empty(M * K, np.float32)
    lib().or_adc_table(_c(codebooks, np.float32), M, K, ds, _c(r, np.float32), out)
    return out


def distance_with_table(table, M, K, codes) -> np.float32:
    return np.float32(lib().or_distance_with_table(_c(table, np.float32), M, K, _c(codes, np.uint8)))


def adc_scan(codes, M, K, table) -> np.ndarray:
    codes = _c(codes, np.uint8).reshape(-1)
    n = codes.size // M
    out = np.empty(n, np.float32)
    lib().or_adc_scan(codes if codes.size else np.zeros(1, np.uint8), n, M, K,
                      _c(table, np.float32), out if n else np.zeros(1, np.float32))
    return out


def pq_encode(codebooks, M, K, ds, x) -> np.ndarray:
    x = _c(np.atleast_2d(x), np.float32)
    out = np.empty((x.shape[0], M), np.uint8)
    lib().or_pq_encode(_c(codebooks, np.float32), M, K, ds, x, x.shape[0], out)
    return out


def pq_reconstruct(codebooks, M, K, ds, codes) -> np.ndarray:
    out = np.empty(M * ds, np.float32)
    lib().or_pq_reconstruct(_c(codebooks, np.float32), M, K, ds, _c(codes, np.uint8), out)
    return out


# ---- FastScan ------------------------------------------------------------

def pack4(codes, n, M) -> np.ndarray:
    out = np.empty(lib().or_pack4_size(n, M), np.uint8)
    c = _c(codes, np.uint8).reshape(-1)
    lib().or_pack4(c if c.size else np.zeros(1, np.uint8), n, M, out)
    return out


def quantize_lut(lut, M):
    q = np.empty(M * 16, np.uint8)
    scale, offset = ctypes.c_float(), ctypes.c_float()
    lib().or_quantize_lut(_c(lut, np.float32), M, q, ctypes.byref(scale), ctypes.byref(offset))
    return q, np.float32(scale.value), np.float32(offset.value)


def fastscan_block(block, lutq, M) -> np.ndarray:
    acc = np.empty(32, np.uint16)
    lib().or_fastscan_block(_c(block, np.uint8), _c(lutq, np.uint8), M, acc)
    return acc


def fastscan_batch(packed, n, M, lut) -> np.ndarray:
    out = np.empty(max(n, 1), np.float32)
    rc = lib().or_fastscan_batch(_c(packed, np.uint8), n, M, _c(lut, np.float32), out)
    if rc != 0:
        raise ValueError(f"FastScan accumulates in u16: {M} codebooks would overflow")
    return out[:n]


# ---- selection -----------------------------------------------------------

def nearest_centroids(q, centroids, nprobe):
    centroids = _c(centroids, np.float32)
    L, d = centroids.shape
    lists = np.empty(max(min(nprobe, L), 1), np.uint32)
    scores = np.empty_like(lists, dtype=np.float32)
    m = lib().or_nearest_centroids(_c(q, np.float32), centroids, L, d, nprobe, lists, scores)
    return lists[:m], scores[:m]


def top_k(idx, dist, k):
    idx, dist = _c(idx, np.uint32), _c(dist, np.float32)
    n = idx.size
    oi = np.empty(max(k, 1), np.uint32)
    od = np.empty(max(k, 1), np.float32)
    m = lib().or_top_k(idx if n else np.zeros(1, np.uint32), dist if n else np.zeros(1, np.float32),
                       n, k, oi, od)
    return oi[:m], od[:m]


# ---- index ---------------------------------------------------------------

@dataclass
class Index:
    """The arrays of a built IVFPQIndex (search.rs:212-239)."""

    centroids: np.ndarray      # f32 [L, d]
    codebooks: np.ndarray      # f32 [M*K*ds]
    list_offsets: np.ndarray   # u64 [L+1]
    list_ids: np.ndarray       # u32 [n]
    codes: np.ndarray          # u8  [n, M] insertion order
    doc_ids: np.ndarray | None  # u32 [n]
    vectors: np.ndarray | None  # f32 [n, d] normalised
    M: int
    K: int
    rotation: np.ndarray | None = None  # f32 [d, d] OPQ rotation (opq.rs:37-38)

    def __post_init__(self):
        self.centroids = _c(self.centroids, np.float32)
        self.codebooks = _c(self.codebooks, np.float32).reshape(-1)
        self.list_offsets = _c(self.list_offsets, np.uint64)
        self.list_ids = _c(self.list_ids, np.uint32)
        self.codes = _c(self.codes, np.uint8).reshape(-1, self.M)
        if self.doc_ids is not None:
            self.doc_ids = _c(self.doc_ids, np.uint32)
        if self.vectors is not None:
            self.vectors = _c(self.vectors, np.float32)
        if self.rotation is not None:
            self.rotation = _c(self.rotation, np.float32)
        L, d = self.centroids.shape
        p = lambda a: a.ctypes.data if a is not None else None  # noqa: E731
        self._s = _Index(d, L, self.M, self.K, d // self.M, self.codes.shape[0],
                         p(self.centroids), p(self.codebooks), p(self.list_offsets),
                         p(self.list_ids), p(self.codes), p(self.doc_ids), p(self.vectors),
                         p(self.rotation))

    @property
    def d(self):
        return self.centroids.shape[1]

    def search(self, q, k, nprobe):
        ids = np.empty(max(k, 1), np.uint32)
        dists = np.empty(max(k, 1), np.float32)
        m = lib().or_ivfpq_search(ctypes.byref(self._s), _c(q, np.float32), k, nprobe, ids, dists)
        return ids[:m], dists[:m]

    def search_reranked(self, q, k, pool, nprobe):
        ids = np.empty(max(k, 1), np.uint32)
        dists = np.empty(max(k, 1), np.float32)
        m = lib().or_ivfpq_search_reranked(ctypes.byref(self._s), _c(q, np.float32), k, pool,
                                           nprobe, ids, dists)
        if m < 0:
            raise RuntimeError("rerank needs raw vectors")
        return ids[:m], dists[:m]

    def search_batch(self, queries, k, nprobe, rerank_pool=0, threads=0):
        queries = _c(queries, np.float32)
        nq = queries.shape[0]
        ids = np.empty((nq, k), np.int64)
        dists = np.empty((nq, k), np.float32)
        rc = lib().or_ivfpq_search_batch(ctypes.byref(self._s), queries, nq, k, nprobe,
                                         rerank_pool, threads, ids, dists)
        if rc != 0:
            raise RuntimeError("oracle batch search failed")
        return ids, dists

    def list_masks(self, cat):
        """search.rs:626-648: per-list category bitmask from per-vector categories."""
        masks = np.empty(max(self._s.L, 1), np.uint64)
        lib().or_list_masks(ctypes.byref(self._s), _c(cat, np.int8), masks)
        return masks[:self._s.L]

    def search_filtered(self, q, k, nprobe, category, cat, list_mask=None):
        """search.rs:1407-1549: cat = category per vector (-1 none); list_mask defaults
        to the masks of cat (lists built with the current metadata)."""
        cat = _c(cat, np.int8)
        if list_mask is None:
            list_mask = self.list_masks(cat)
        ids = np.empty(max(k, 1), np.uint32)
        dists = np.empty(max(k, 1), np.float32)
        m = lib().or_ivfpq_search_filtered(ctypes.byref(self._s), _c(list_mask, np.uint64), cat,
                                           _c(q, np.float32), k, nprobe, category, ids, dists)
        if m < 0:
            raise ValueError("category outside 0..63")
        return ids[:m], dists[:m]

    def probe(self, q, nprobe):
        lists = np.empty(max(nprobe, 1), np.uint32)
        scores = np.empty(max(nprobe, 1), np.float32)
        m = lib().or_ivfpq_probe(ctypes.byref(self._s), _c(q, np.float32), nprobe, lists, scores)
        return lists[:m], scores[:m]


# ---- build side ----------------------------------------------------------

def assign_cosine(x, centroids) -> np.ndarray:
    x, centroids = _c(x, np.float32), _c(centroids, np.float32)
    out = np.empty(x.shape[0], np.uint32)
    lib().or_assign_cosine(x, x.shape[0], centroids, centroids.shape[0], x.shape[1], out)
    return out


def build_lists(assign, L):
    assign = _c(assign, np.uint32)
    off = np.empty(L + 1, np.uint64)
    ids = np.empty(max(assign.size, 1), np.uint32)
    lib().or_build_lists(assign, assign.size, L, off, ids)
    return off, ids[:assign.size]


def sample_indices(n, sample, seed) -> np.ndarray:
    cnt = n if (sample == 0 or sample >= n) else sample
    out = np.empty(max(cnt, 1), np.uint32)
    lib().or_sample_indices(n, sample, seed, out)
    return out[:cnt]


def kmeans(x, k, metric, seed, max_iter):
    x = _c(x, np.float32)
    n, d = x.shape
    ke = min(k, n)
    out = np.empty((ke, d), np.float32)
    it = lib().or_kmeans(x, n, d, k, metric, seed, max_iter, out)
    return out, it


def ivfpq_build(vectors_normalised, L, M, K, seed, sample, max_iter, use_opq=False):
    """Train + assign + encode with this project's k-means; returns (Index, assign)."""
    v = _c(vectors_normalised, np.float32)
    n, d = v.shape
    nt = n if (sample == 0 or sample >= n) else sample
    Le = min(L, nt)
    cent = np.empty((Le, d), np.float32)
    cb = np.empty(M * K * (d // M), np.float32)
    assign = np.empty(n, np.uint32)
    codes = np.empty((n, M), np.uint8)
    rot = np.empty((d, d), np.float32)
    ka = _sz()
    rc = lib().or_ivfpq_build(v, n, d, L, M, K, seed, sample, max_iter, 1 if use_opq else 0, cent,
                              cb, assign, codes, rot, ctypes.byref(ka))
    if rc != 0:
        raise ValueError("invalid IVF-PQ build shape")
    K_actual = ka.value
    cb = cb[: M * K_actual * (d // M)]
    off, ids = build_lists(assign, Le)
    return Index(cent, cb, off, ids, codes, np.arange(n, dtype=np.uint32), v, M, K_actual,
                 rot if use_opq else None), assign


# ---- OPQ (opq.rs) --------------------------------------------------------

def matvec(R, v):
    R, v = _c(R, np.float32), _c(v, np.float32)
    out = np.empty(v.size, np.float32)
    lib().or_matvec(R, v, v.size, out)
    return out


def matvec_t(R, v):
    R, v = _c(R, np.float32), _c(v, np.float32)
    out = np.empty(v.size, np.float32)
    lib().or_matvec_t(R, v, v.size, out)
    return out


def polar(M):
    M = _c(M, np.float32)
    out = np.empty_like(M)
    lib().or_polar(M, M.shape[0], out)
    return out


def opq_fit(data, M, K, iterations, seed, max_iter=100):
    """(rotation [d, d], codebooks [M*Ke*ds], Ke) of OptimizedProductQuantizer::fit."""
    data = _c(data, np.float32)
    n, d = data.shape
    rot = np.empty((d, d), np.float32)
    cb = np.empty(M * K * (d // M), np.float32)
    ka = _sz()
    rc = lib().or_opq_fit(data, n, d, M, K, iterations, seed, max_iter, rot, cb, ctypes.byref(ka))
    if rc != 0:
        raise ValueError(f"need at least {K} training vectors, got {n}")
    return rot, cb[: M * ka.value * (d // M)], ka.value


def flat_search(base, queries, k, metric=0, threads=0):
    base, queries = _c(base, np.float32), _c(queries, np.float32)
    nq = queries.shape[0]
    ids = np.empty((nq, k), np.int64)
    dists = np.empty((nq, k), np.float32)
    lib().or_flat_search(base, base.shape[0], base.shape[1], queries, nq, k, metric, threads,
                         ids, dists)
    return ids, dists
