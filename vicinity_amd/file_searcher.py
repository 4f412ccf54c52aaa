"""IVFPQFileSearcher: read-only IVF-PQ search over a snapshot directory whose
PQ codes and raw vectors stay on disk and are read per search call.

Mirrors pyvicinity's ``IVFPQFileSearcher`` (src/python.rs:857-1060,
pyvicinity/_core.pyi): ``load(path, mmap=None)``, ``load_generation(root)``,
``set_nprobe``, ``search`` / ``batch_search`` with ``nprobe`` and
``rerank_pool``, the shape properties, ``len`` and ``repr``; plus the Rust
API's per-query diagnostics (``*_with_diagnostics``, search.rs:263-282,
1809-1891).  The routing metadata is read by the snapshot reader; the engine
(vgpu_ivfpq_file_*) reads the codes of each call's probed lists, and for
reranking the raw vectors of the candidates, from the directory.
"""

from __future__ import annotations

import ctypes
import os
import threading
import warnings

import numpy as np

from . import _lib
from .ivf_pq import MISSING_DISTANCE, MISSING_LABEL, _f32_2d
from .snapshot import open_current, read_snapshot


# open_current (generation.rs:191-205)
_current_generation = open_current


class IVFPQFileSearcher:
    """File-backed IVF-PQ searcher (search.rs:240-262)."""

    def __init__(self, path, _snap: dict):
        s = _snap
        p = s["params"]
        self._L = _lib.load()
        self._dim = int(s["dimension"])
        self._n = int(s["num_vectors"])
        self._num_clusters = int(p["num_clusters"])
        self._num_codebooks = int(p["num_codebooks"])
        self._codebook_size = int(p["codebook_size"])
        self._nprobe = int(p["nprobe"])
        self._search_lock = threading.Lock()  # python.rs:172, the per-call nprobe
        self._path = os.fspath(path)
        prm = _lib.Params(self._num_clusters, self._nprobe, self._num_codebooks,
                          self._codebook_size, int(p["seed"]),
                          int(bool(p["use_opq"]) or s["rotation"] is not None))
        centroids = np.ascontiguousarray(s["centroids"], np.float32)
        codebooks = np.ascontiguousarray(s["codebooks"], np.float32)
        offsets = np.ascontiguousarray(s["list_offsets"], np.uint64)
        list_ids = np.ascontiguousarray(s["list_ids"], np.uint32)
        doc_ids = np.ascontiguousarray(s["doc_ids"], np.uint32)
        rot = s["rotation"]
        if rot is not None:
            rot = np.ascontiguousarray(rot, np.float32).reshape(-1)
        h = ctypes.c_void_p()
        _lib.check(self._L.vgpu_ivfpq_file_open(
            self._dim, ctypes.byref(prm), _lib.ptr(centroids), centroids.shape[0], _lib.ptr(codebooks),
            self._codebook_size, _lib.ptr(offsets), _lib.ptr(list_ids), _lib.ptr(doc_ids), self._n,
            _lib.ptr(rot), self._path.encode(), int(s["raw_vectors_present"]), ctypes.byref(h)))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._L.vgpu_ivfpq_file_free(h)
            self._h = None

    # ---- loading (python.rs:865-900) ---------------------------------------
    @staticmethod
    def load(path, mmap: bool | None = None) -> "IVFPQFileSearcher":
        if mmap is not None:
            warnings.warn("IVFPQFileSearcher.load(mmap=...) is deprecated and ignored; "
                          "vicinity no longer memory-maps index files", DeprecationWarning,
                          stacklevel=2)
        return IVFPQFileSearcher(path, read_snapshot(path, arrays=False))

    @staticmethod
    def load_generation(root) -> "IVFPQFileSearcher":
        return IVFPQFileSearcher.load(_current_generation(root))

    def set_nprobe(self, nprobe: int) -> None:
        with self._search_lock:
            _lib.check(self._L.vgpu_ivfpq_file_set_nprobe(self._h, int(nprobe)))
            self._nprobe = int(nprobe)

    # ---- search (python.rs:921-1046) ---------------------------------------
    def _run(self, queries, k: int, nprobe, rerank_pool):
        q = np.asarray(queries)
        if q.ndim != 2:
            raise ValueError("queries must be a 2-D array")
        if q.shape[1] != self._dim:
            raise ValueError(f"queries dimension mismatch: index expects {self._dim}, "
                             f"got {q.shape[1]}")
        q = _f32_2d(q, "queries")
        nq = q.shape[0]
        ids = np.full((nq, k), MISSING_LABEL, np.int64)
        dists = np.full((nq, k), MISSING_DISTANCE, np.float32)
        diag = (_lib.FileDiagnostics * max(nq, 1))()
        pool = 0 if rerank_pool is None else max(int(rerank_pool), k, 1)
        # python.rs:1116-1142: under the search lock, an explicit nprobe (0
        # included: no list is probed) replaces the default for the call
        with self._search_lock:
            if nprobe is not None:
                _lib.check(self._L.vgpu_ivfpq_file_set_nprobe(self._h, int(nprobe)))
            try:
                _lib.check(self._L.vgpu_ivfpq_file_search_batch(
                    self._h, _lib.ptr(q) if nq else None, nq, self._dim, k, 0, pool,
                    _lib.ptr(ids) if ids.size else None, _lib.ptr(dists) if dists.size else None, diag))
            finally:
                if nprobe is not None:
                    _lib.check(self._L.vgpu_ivfpq_file_set_nprobe(self._h, self._nprobe))
        return ids, dists, [diag[i].as_dict() for i in range(nq)]

    def batch_search(self, queries, k: int, nprobe: int | None = None,
                     rerank_pool: int | None = None):
        """(ids int64[nq, k], dists float32[nq, k]) padded with
        (MISSING_LABEL, MISSING_DISTANCE)."""
        ids, dists, _ = self._run(queries, k, nprobe, rerank_pool)
        return ids, dists

    def batch_search_with_diagnostics(self, queries, k: int, nprobe: int | None = None,
                                      rerank_pool: int | None = None):
        return self._run(queries, k, nprobe, rerank_pool)

    def search(self, query, k: int, nprobe: int | None = None, rerank_pool: int | None = None):
        """(ids int64[m], dists float32[m]), m <= k."""
        ids, dists, _ = self.search_with_diagnostics(query, k, nprobe, rerank_pool)
        return ids, dists

    def search_with_diagnostics(self, query, k: int, nprobe: int | None = None,
                                rerank_pool: int | None = None):
        q = np.asarray(query)
        if q.ndim != 1 or q.dtype != np.float32:
            raise ValueError("query must be a 1-D float32 array")
        if q.shape[0] != self._dim:
            raise ValueError(f"query dimension mismatch: index expects {self._dim}, "
                             f"got {q.shape[0]}")
        ids, dists, diag = self._run(q.reshape(1, -1), k, nprobe, rerank_pool)
        m = int(np.sum(ids[0] != MISSING_LABEL))
        return ids[0, :m].copy(), dists[0, :m].copy(), diag[0]

    def last_io(self) -> dict:
        """File reads of the last search call: positional reads and bytes."""
        r, b = ctypes.c_uint64(), ctypes.c_uint64()
        _lib.check(self._L.vgpu_ivfpq_file_last_io(self._h, ctypes.byref(r), ctypes.byref(b)))
        return {"reads": int(r.value), "bytes": int(b.value)}

    # ---- properties (python.rs:1005-1060) ----------------------------------
    @property
    def num_vectors(self) -> int:
        return self._n

    @property
    def dimension(self) -> int:
        return self._dim

    @property
    def num_clusters(self) -> int:
        return self._num_clusters

    @property
    def num_codebooks(self) -> int:
        return self._num_codebooks

    @property
    def codebook_size(self) -> int:
        return self._codebook_size

    @property
    def nprobe(self) -> int:
        return self._nprobe

    def __len__(self) -> int:
        return self._n

    def __repr__(self) -> str:
        return (f"IVFPQFileSearcher(dim={self._dim}, n={self._n}, num_clusters={self._num_clusters}, "
                f"num_codebooks={self._num_codebooks}, codebook_size={self._codebook_size}, "
                f"nprobe={self._nprobe})")
