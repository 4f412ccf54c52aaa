"""FlatIndex: exact top-k over HBM-resident vectors (the ground-truth path,
src/distance.rs:78-109 brute force, src/ivf_pq/search.rs:3376-3392)."""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

METRICS = {"l2": 0, "cosine": 1}


class FlatIndex:
    """metric 'l2': squared L2 distance; 'cosine': 1 - dot (vectors and
    queries are used as given, as cosine_distance_normalized does)."""

    def __init__(self, dim: int, metric: str = "l2"):
        self._L = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(self._L.vgpu_flat_new(dim, METRICS[metric], ctypes.byref(h)))
        self._h = h
        self._dim = dim
        self._n = 0

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._L.vgpu_flat_free(h)
            self._h = None

    def add(self, vectors) -> None:
        x = np.ascontiguousarray(vectors, np.float32)
        if x.ndim != 2 or x.shape[1] != self._dim:
            raise ValueError(f"dimension mismatch: index expects {self._dim}")
        _lib.check(self._L.vgpu_flat_add(self._h, _lib.ptr(x), x.shape[0]))
        self._n += x.shape[0]

    def search(self, queries, k: int):
        q = np.ascontiguousarray(queries, np.float32)
        if q.ndim != 2 or q.shape[1] != self._dim:
            raise ValueError(f"queries dimension mismatch: index expects {self._dim}")
        nq = q.shape[0]
        ids = np.full((nq, k), -1, np.int64)
        dists = np.full((nq, k), np.inf, np.float32)
        _lib.check(self._L.vgpu_flat_search_batch(self._h, _lib.ptr(q) if nq else None, nq,
                                                  self._dim, k, _lib.ptr(ids) if ids.size else None,
                                                  _lib.ptr(dists) if dists.size else None))
        return ids, dists

    def search_device(self, queries, k: int, out_ids=None, out_dists=None, stream=None):
        import torch

        nq = queries.shape[0]
        if out_ids is None:
            out_ids = torch.empty((nq, k), dtype=torch.int64, device=queries.device)
        if out_dists is None:
            out_dists = torch.empty((nq, k), dtype=torch.float32, device=queries.device)
        s = stream.cuda_stream if stream is not None else None
        _lib.check(self._L.vgpu_flat_search_batch_device(
            self._h, queries.data_ptr(), nq, queries.shape[1], k, out_ids.data_ptr(),
            out_dists.data_ptr(), s))
        return out_ids, out_dists

    def last_fallbacks(self) -> int:
        """Queries of the last search answered by the exhaustive exact scan."""
        q = ctypes.c_uint32()
        _lib.check(self._L.vgpu_flat_last_fallbacks(self._h, ctypes.byref(q)))
        return q.value

    def last_ms(self):
        g, t = ctypes.c_float(), ctypes.c_float()
        _lib.check(self._L.vgpu_flat_last_ms(self._h, ctypes.byref(g), ctypes.byref(t)))
        return g.value, t.value

    def __len__(self) -> int:
        return self._n
