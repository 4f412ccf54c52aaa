"""IVFPQIndex: the Python surface of vicinity's IVF-PQ index, backed by the
MI355X engine through the C ABI.

Mirrors pyvicinity's ``IVFPQIndex`` (src/python.rs:523-793,
pyvicinity/_core.pyi:197-292): same constructor defaults, argument meaning,
padding sentinels and ValueError behaviour.  ``save`` / ``load`` read and
write the reference's directory snapshots (src/python.rs:655-681);
``load_artifacts`` takes the arrays of an index built elsewhere.  Filtered
search follows the Rust API (``with_filtering``, ``add_metadata``,
``search_with_filter``, src/ivf_pq/search.rs:413-475, 1407-1549).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import _lib
from .filtering import MetadataFilter, filter_category, metadata_category
from .snapshot import open_current, publish_generation, read_snapshot, write_snapshot

# python.rs:1303-1304 (faiss convention)
MISSING_LABEL = -1
MISSING_DISTANCE = float("inf")


def default_codebooks(dim: int) -> int:
    """python.rs:1145-1150: the largest divisor of dim that is <= 8."""
    for m in range(min(8, dim), 0, -1):
        if dim % m == 0:
            return m
    return 1


def _validate_shape(dim, num_clusters, num_codebooks, codebook_size, nprobe):
    """python.rs:1152-1179."""
    if dim == 0:
        raise ValueError("dim must be greater than 0")
    if num_clusters == 0:
        raise ValueError("num_clusters must be greater than 0")
    if num_codebooks == 0 or dim % num_codebooks != 0:
        raise ValueError("num_codebooks must be a non-zero divisor of dim "
                         f"(dim={dim}, num_codebooks={num_codebooks})")
    if codebook_size == 0 or codebook_size > 256:
        raise ValueError("codebook_size must be in the range 1..=256")
    if nprobe == 0:
        raise ValueError("nprobe must be greater than 0")


def _f32_2d(a, name: str) -> np.ndarray:
    a = np.asarray(a)
    if a.ndim != 2:
        raise ValueError(f"{name} must be a 2-D array")
    if a.dtype != np.float32:
        raise TypeError(f"{name} must be float32")
    if not a.flags.c_contiguous:
        raise ValueError(f"{name} must be contiguous (C-order)")
    return a


class IVFPQIndex:
    """IVF-PQ index for compressed approximate nearest-neighbor search."""

    def __init__(self, dim: int, num_clusters: int = 256, num_codebooks: int | None = None,
                 codebook_size: int = 256, nprobe: int = 1, use_opq: bool = False,
                 seed: int = 42, filter_field: str | None = None):
        if num_codebooks is None:
            num_codebooks = default_codebooks(dim)
        _validate_shape(dim, num_clusters, num_codebooks, codebook_size, nprobe)
        self._L = _lib.load()
        params = _lib.Params(num_clusters, nprobe, num_codebooks, codebook_size, seed,
                             1 if use_opq else 0)
        h = ctypes.c_void_p()
        _lib.check(self._L.vgpu_ivfpq_new(dim, ctypes.byref(params), ctypes.byref(h)))
        self._h = h
        self._dim = dim
        self._nprobe = nprobe
        self._num_clusters = num_clusters
        self._num_codebooks = num_codebooks
        self._codebook_size = codebook_size
        self._use_opq = use_opq
        self._used_ids: set[int] = set()
        # search.rs:236-238: the filter field and the documents' metadata
        self._seed = seed
        self._filter_field = filter_field
        self._metadata: dict[int, dict] = {}
        if filter_field is not None:
            _lib.check(self._L.vgpu_ivfpq_enable_filtering(self._h))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._L.vgpu_ivfpq_free(h)
            self._h = None

    # ---- mutation ---------------------------------------------------------
    def add_items(self, vectors, ids=None) -> None:
        """python.rs:582-620: rows are L2-normalised on insert; ids must be
        unique u32 values (checked before anything is added)."""
        arr = np.asarray(vectors)
        if arr.ndim != 2 or arr.shape[1] != self._dim:
            got = arr.shape[1] if arr.ndim == 2 else arr.shape
            raise ValueError(f"dimension mismatch: index expects {self._dim}, got {got}")
        arr = _f32_2d(arr, "vectors")
        n = arr.shape[0]
        if ids is not None:
            ids = np.asarray(ids)
            if ids.ndim != 1 or ids.shape[0] != n:
                raise ValueError(f"ids length {ids.shape[0] if ids.ndim == 1 else ids.shape} "
                                 f"!= vectors rows {n}")
            out = []
            batch: set[int] = set()
            for i, v in enumerate(ids.tolist()):
                if not (0 <= v <= 0xFFFFFFFF):
                    raise ValueError(f"ids[{i}] = {v} out of range [0, 2**32); "
                                     "IDs are stored as u32")
                if v in self._used_ids or v in batch:
                    raise ValueError(f"duplicate doc_id {v} (IDs must be unique within an index)")
                batch.add(v)
                out.append(v)
            id_u32 = np.asarray(out, dtype=np.uint32)
        else:
            out = []
            cand = len(self)
            while len(out) < n:
                if cand > 0xFFFFFFFF:
                    raise ValueError("implicit IDs exceed the u32 ID limit")
                if cand not in self._used_ids:
                    out.append(cand)
                cand += 1
            id_u32 = np.asarray(out, dtype=np.uint32)
        if n:
            _lib.check(self._L.vgpu_ivfpq_add(self._h, _lib.ptr(id_u32), _lib.ptr(arr), n))
        self._used_ids.update(id_u32.tolist())

    def build(self, training_sample_size: int | None = None, kmeans_max_iter: int = 100) -> None:
        """search.rs:534-544 (training_sample_size None = every vector)."""
        if training_sample_size == 0:
            raise ValueError("training_sample_size must be greater than 0")
        _lib.check(self._L.vgpu_ivfpq_build(self._h, training_sample_size or 0, kmeans_max_iter))

    def load_artifacts(self, centroids, codebooks, list_offsets, list_ids, codes,
                       doc_ids=None, vectors=None, rotation=None) -> None:
        """Upload an index built elsewhere (same arrays as IVFPQIndex holds
        after build(), search.rs:212-239); `rotation` (d x d) is the OPQ
        rotation of an index made with use_opq (opq.rs:37-38)."""
        centroids = np.ascontiguousarray(centroids, np.float32)
        codebooks = np.ascontiguousarray(codebooks, np.float32).reshape(-1)
        list_offsets = np.ascontiguousarray(list_offsets, np.uint64)
        list_ids = np.ascontiguousarray(list_ids, np.uint32)
        codes = np.ascontiguousarray(codes, np.uint8).reshape(-1)
        n = list_ids.shape[0]
        M = self._num_codebooks
        ds = self._dim // M
        K = codebooks.size // (M * ds)
        if doc_ids is not None:
            doc_ids = np.ascontiguousarray(doc_ids, np.uint32)
        if vectors is not None:
            vectors = np.ascontiguousarray(vectors, np.float32)
        if rotation is not None:
            rotation = np.ascontiguousarray(rotation, np.float32).reshape(-1)
            _lib.check(self._L.vgpu_ivfpq_set_rotation(self._h, _lib.ptr(rotation), rotation.size))
        _lib.check(self._L.vgpu_ivfpq_load(
            self._h, _lib.ptr(centroids), centroids.shape[0], _lib.ptr(codebooks), K,
            _lib.ptr(list_offsets), _lib.ptr(list_ids), _lib.ptr(codes), _lib.ptr(doc_ids),
            _lib.ptr(vectors), n))
        self._used_ids = set((doc_ids if doc_ids is not None else np.arange(n)).tolist())

    # ---- snapshots (src/python.rs:655-681, search.rs:906-1084) -------------
    def save(self, path) -> None:
        """Save the built index as a directory snapshot in the reference's
        format (IVFPQIndex::save_to_dir, search.rs:906-1002)."""
        self._save(path, False)

    def save_generation(self, path) -> None:
        """Publish the built index as an immutable generation below `path`
        (IVFPQIndex::save_to_generation, search.rs:918-936; python.rs:660-665)."""
        if not self._info().built:
            raise ValueError("IVF-PQ index: save before build")
        publish_generation(path, lambda staging: self._save(staging, True))

    @staticmethod
    def load_generation(path) -> "IVFPQIndex":
        """Load the generation named by ``path/CURRENT``
        (IVFPQIndex::load_from_generation, search.rs:938-943; python.rs:683-697)."""
        if not os.path.exists(os.path.join(path, "CURRENT")):
            raise FileNotFoundError(os.path.join(path, "CURRENT"))
        return IVFPQIndex.load(open_current(path))

    def _save(self, path, generation: bool) -> None:
        inf = self._info()
        if not inf.built:
            raise ValueError("IVF-PQ index: save before build")
        art = self.export()
        L = art["centroids"].shape[0]
        masks = np.zeros(L, np.uint64)
        if self._filter_field is not None and L:
            _lib.check(self._L.vgpu_ivfpq_get_list_masks(self._h, _lib.ptr(masks), L))
        write_snapshot(
            path, dimension=self._dim,
            params={"num_clusters": self._num_clusters, "nprobe": self._nprobe,
                    "num_codebooks": self._num_codebooks, "codebook_size": self._codebook_size,
                    "use_opq": self._use_opq, "seed": self._seed},
            centroids=art["centroids"], codebooks=art["codebooks"], codebook_size=art["K"],
            num_codebooks=art["M"], list_offsets=art["list_offsets"], list_ids=art["list_ids"],
            codes=art["codes"], doc_ids=art["doc_ids"], vectors=art["vectors"], list_masks=masks,
            filter_field=self._filter_field,
            filter_metadata=self._metadata if self._filter_field is not None else None,
            rotation=art["rotation"], generation_components=generation)

    @staticmethod
    def load(path) -> "IVFPQIndex":
        """Load a directory snapshot written by `save` or by the reference
        (IVFPQIndex::load_from_dir, search.rs:1034-1084): the lists, codes and
        codebooks as saved, the persisted list bitmasks and filter metadata."""
        snap = read_snapshot(path)
        p = snap["params"]
        ix = IVFPQIndex(snap["dimension"], num_clusters=int(p["num_clusters"]),
                        num_codebooks=int(p["num_codebooks"]),
                        codebook_size=int(p["codebook_size"]), nprobe=int(p["nprobe"]),
                        use_opq=bool(p["use_opq"]) or snap["rotation"] is not None,
                        seed=int(p["seed"]), filter_field=snap["filter_field"])
        for doc, md in snap["filter_metadata"].items():
            ix.add_metadata(doc, md)
        ix.load_artifacts(snap["centroids"], snap["codebooks"], snap["list_offsets"],
                          snap["list_ids"], snap["codes"], snap["doc_ids"], snap["vectors"],
                          snap["rotation"])
        if snap["filter_field"] is not None:
            masks = np.ascontiguousarray(snap["list_masks"], np.uint64)
            _lib.check(ix._L.vgpu_ivfpq_set_list_masks(ix._h, _lib.ptr(masks), masks.shape[0]))
        return ix

    def set_nprobe(self, nprobe: int) -> None:
        self._nprobe = nprobe
        _lib.check(self._L.vgpu_ivfpq_set_nprobe(self._h, nprobe))

    def set_mode(self, mode: str) -> None:
        """'fast' (decomposed ranking + exact rescoring) or 'exact'."""
        m = {"fast": _lib.MODE_FAST, "exact": _lib.MODE_EXACT}[mode]
        _lib.check(self._L.vgpu_ivfpq_set_mode(self._h, m))

    def set_profiling(self, enabled) -> None:
        """False/0 off, True/1 every phase, 2 the scan kernels only (two
        hipEvents per query chunk, the cheapest timing)."""
        level = int(enabled)
        if level not in (0, 1, 2):
            raise ValueError("profiling level must be 0, 1 or 2")
        _lib.check(self._L.vgpu_ivfpq_set_profiling(self._h, level))

    def compact(self) -> None:
        if not self.is_built:
            raise ValueError("index must be built before compact")
        _lib.check(self._L.vgpu_ivfpq_compact(self._h))

    # ---- filtered search (search.rs:413-475, 1407-1549) ---------------------
    @classmethod
    def with_filtering(cls, dim: int, filter_field: str, **params) -> "IVFPQIndex":
        """IVFPQIndex::with_filtering (search.rs:413-435)."""
        return cls(dim, filter_field=filter_field, **params)

    def add_metadata(self, doc_id: int, metadata: dict) -> None:
        """IVFPQIndex::add_metadata (search.rs:439-475): the filter field, if
        present, must hold an integer category 0..63.  Metadata replaces any
        earlier entry of the document.  Lists record their members'
        categories when they are built (search.rs:626-648)."""
        if self._filter_field is None:
            raise ValueError("Unsupported: filtered search "
                             "(rebuild the index with IVFPQIndex::with_filtering())")
        if not 0 <= int(doc_id) < (1 << 32):
            raise ValueError(f"doc_id {doc_id} out of range [0, 2**32)")
        cat = metadata_category(metadata, self._filter_field)
        _lib.check(self._L.vgpu_ivfpq_set_category(self._h, int(doc_id), cat))
        self._metadata[int(doc_id)] = dict(metadata)

    def search_with_filter(self, query, k: int, filter: MetadataFilter):
        """IVFPQIndex::search_with_filter (search.rs:1407-1549): (ids int64[m],
        dists float32[m]), m <= k, the documents whose filter field equals the
        filter's category.  The probe widens to every list when the probed
        ones hold fewer than k matches."""
        if not self.is_built:
            raise ValueError("IVF-PQ index: search before build")
        q = np.asarray(query)
        if q.ndim != 1 or q.dtype != np.float32:
            raise ValueError("query must be a 1-D float32 array")
        if q.shape[0] != self._dim:
            raise ValueError(f"query dimension mismatch: index expects {self._dim}, "
                             f"got {q.shape[0]}")
        cat = filter_category(filter, self._filter_field)
        q = np.ascontiguousarray(q)
        ids = np.empty(max(k, 1), np.uint32)
        dists = np.empty(max(k, 1), np.float32)
        m = ctypes.c_size_t(0)
        _lib.check(self._L.vgpu_ivfpq_search_filtered(self._h, _lib.ptr(q), self._dim, k, cat,
                                                      _lib.ptr(ids), _lib.ptr(dists),
                                                      ctypes.byref(m)))
        return ids[:m.value].astype(np.int64), dists[:m.value].copy()

    def batch_search_with_filter(self, queries, k: int, filters):
        """search_with_filter for a batch: ``filters`` is one MetadataFilter
        for every query or one per query.  Returns (ids int64[nq, k], dists
        float32[nq, k]) padded with (MISSING_LABEL, MISSING_DISTANCE); row i
        equals search_with_filter(queries[i], k, filter_i)."""
        if not self.is_built:
            raise ValueError("IVF-PQ index: search before build")
        q = np.asarray(queries)
        if q.ndim != 2:
            raise ValueError("queries must be a 2-D array")
        if q.shape[1] != self._dim:
            raise ValueError(f"queries dimension mismatch: index expects {self._dim}, "
                             f"got {q.shape[1]}")
        q = _f32_2d(q, "queries")
        nq = q.shape[0]
        if isinstance(filters, MetadataFilter):
            filters = [filters] * nq
        if len(filters) != nq:
            raise ValueError(f"{len(filters)} filters for {nq} queries")
        cats = np.array([filter_category(f, self._filter_field) for f in filters], np.int64)
        ids = np.full((nq, k), MISSING_LABEL, np.int64)
        dists = np.full((nq, k), MISSING_DISTANCE, np.float32)
        _lib.check(self._L.vgpu_ivfpq_search_filtered_batch(
            self._h, _lib.ptr(q) if nq else None, nq, self._dim, k,
            _lib.ptr(cats) if nq else None, _lib.ptr(ids) if ids.size else None,
            _lib.ptr(dists) if dists.size else None))
        return ids, dists

    # ---- search -----------------------------------------------------------
    def search(self, query, k: int, nprobe: int | None = None, rerank_pool: int | None = None):
        """python.rs:709-738: (ids int64[m], dists float32[m]), m <= k."""
        q = np.asarray(query)
        if q.ndim != 1 or q.dtype != np.float32:
            raise ValueError("query must be a 1-D float32 array")
        if q.shape[0] != self._dim:
            raise ValueError(f"query dimension mismatch: index expects {self._dim}, "
                             f"got {q.shape[0]}")
        ids, dists = self.batch_search(q.reshape(1, -1), k, nprobe, rerank_pool)
        m = int(np.sum(ids[0] != MISSING_LABEL))
        return ids[0, :m].copy(), dists[0, :m].copy()

    def batch_search(self, queries, k: int, nprobe: int | None = None,
                     rerank_pool: int | None = None):
        """python.rs:744-793: (ids int64[nq, k], dists float32[nq, k]) padded
        with (MISSING_LABEL, MISSING_DISTANCE)."""
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
        pool = 0 if rerank_pool is None else max(int(rerank_pool), k, 1)
        if nprobe is not None and int(nprobe) == 0:
            self._check_no_probe(q, rerank_pool)
            return ids, dists
        _lib.check(self._L.vgpu_ivfpq_search_batch(
            self._h, _lib.ptr(q) if nq else None, nq, self._dim, k, nprobe or 0, pool,
            _lib.ptr(ids) if ids.size else None, _lib.ptr(dists) if dists.size else None))
        return ids, dists

    def _check_no_probe(self, q, rerank_pool) -> None:
        """An explicit nprobe of 0 is the index's nprobe for the call
        (python.rs:1085-1096): find_nearest_centroids probes no list
        (search.rs:1610), so every row is padding once the reference's checks
        pass: built (search.rs:1181-1186), query values (checked by the engine,
        which searches nothing with k = 0), raw vectors for a rerank
        (search.rs:1137-1142)."""
        nq = q.shape[0]
        _lib.check(self._L.vgpu_ivfpq_search_batch(self._h, _lib.ptr(q) if nq else None, nq, self._dim,
                                                   0, 0, 0, None, None))
        if rerank_pool is not None and not self._info().has_vectors:
            err = ValueError("search_reranked after compact(): raw vectors were dropped")
            err.code = _lib.ERR_UNSUPPORTED  # type: ignore[attr-defined]
            raise err

    def search_batch_device(self, queries, k: int, nprobe: int | None = None,
                            rerank_pool: int | None = None, out_ids=None, out_dists=None,
                            stream=None):
        """Batch search on HBM-resident torch tensors (float32 [nq, d] on the
        GPU); returns (ids int64 [nq, k], dists float32 [nq, k]) on the GPU."""
        import torch

        if not (queries.is_cuda and queries.dtype == torch.float32 and queries.is_contiguous()):
            raise ValueError("queries must be a contiguous float32 GPU tensor")
        nq = queries.shape[0]
        if out_ids is None:
            out_ids = torch.empty((nq, k), dtype=torch.int64, device=queries.device)
        if out_dists is None:
            out_dists = torch.empty((nq, k), dtype=torch.float32, device=queries.device)
        pool = 0 if rerank_pool is None else max(int(rerank_pool), k, 1)
        s = stream.cuda_stream if stream is not None else None
        _lib.check(self._L.vgpu_ivfpq_search_batch_device(
            self._h, queries.data_ptr(), nq, queries.shape[1], k, nprobe or 0, pool,
            out_ids.data_ptr(), out_dists.data_ptr(), s))
        return out_ids, out_dists

    def probe(self, queries, nprobe: int | None = None) -> np.ndarray:
        """Probed lists per query in probe order (search.rs:1602-1617)."""
        q = _f32_2d(np.asarray(queries), "queries")
        P = nprobe or self._nprobe
        lists = np.zeros((q.shape[0], max(P, 1)), np.uint32)
        out_p = ctypes.c_size_t()
        _lib.check(self._L.vgpu_ivfpq_probe_batch(self._h, _lib.ptr(q), q.shape[0], q.shape[1], P,
                                                   _lib.ptr(lists), ctypes.byref(out_p)))
        return lists[:, :out_p.value]

    def reconstruct(self, idx: int) -> np.ndarray:
        """IVFPQIndex::reconstruct (search.rs:857-884): the vector the codes
        of insertion index `idx` approximate, the decoded residual plus its
        list's centroid (float32 [d]); works after compact()."""
        if idx < 0:
            raise ValueError(f"vector index {idx} out of range (num_vectors = {len(self)})")
        out = np.empty(self._dim, np.float32)
        _lib.check(self._L.vgpu_ivfpq_reconstruct(self._h, int(idx), _lib.ptr(out), out.size))
        return out

    def memory_usage(self) -> dict:
        """IVFPQIndex::memory_usage (search.rs:1552-1577): host bytes by the
        reference's MemoryReport categories and their total, plus
        device_bytes, the HBM the index and its search workspaces hold."""
        r = _lib.MemoryReport()
        _lib.check(self._L.vgpu_ivfpq_memory_usage(self._h, ctypes.byref(r)))
        return r.as_dict()

    def last_stats(self) -> dict:
        st = _lib.Stats()
        _lib.check(self._L.vgpu_ivfpq_last_stats(self._h, ctypes.byref(st)))
        return st.as_dict()

    def export(self) -> dict:
        """The built arrays (centroids, codebooks, list_offsets, list_ids,
        codes in insertion order, doc_ids, vectors or None, the OPQ rotation
        [d, d] or None)."""
        inf = self._info()
        if not inf.built:
            raise ValueError("index must be built before export")
        n, d, L = inf.num_vectors, inf.dimension, inf.num_clusters
        M, K, ds = inf.num_codebooks, inf.codebook_size, inf.subvector_dim
        out = {
            "centroids": np.empty((L, d), np.float32),
            "codebooks": np.empty(M * K * ds, np.float32),
            "list_offsets": np.empty(L + 1, np.uint64),
            "list_ids": np.empty(max(n, 1), np.uint32),
            "codes": np.empty((max(n, 1), M), np.uint8),
            "doc_ids": np.empty(max(n, 1), np.uint32),
            "vectors": np.empty((max(n, 1), d), np.float32) if inf.has_vectors else None,
        }
        _lib.check(self._L.vgpu_ivfpq_export(
            self._h, _lib.ptr(out["centroids"]), _lib.ptr(out["codebooks"]),
            _lib.ptr(out["list_offsets"]), _lib.ptr(out["list_ids"]), _lib.ptr(out["codes"]),
            _lib.ptr(out["doc_ids"]), _lib.ptr(out["vectors"])))
        for key in ("list_ids", "codes", "doc_ids", "vectors"):
            if out[key] is not None:
                out[key] = out[key][:n]
        out["M"], out["K"] = M, K
        rot = np.empty((d, d), np.float32)
        present = ctypes.c_int(0)
        _lib.check(self._L.vgpu_ivfpq_get_rotation(self._h, _lib.ptr(rot), rot.size,
                                                   ctypes.byref(present)))
        out["rotation"] = rot if present.value else None
        return out

    # ---- properties (pyvicinity/_core.pyi:262-292) -------------------------
    def _info(self) -> _lib.Info:
        inf = _lib.Info()
        _lib.check(self._L.vgpu_ivfpq_get_info(self._h, ctypes.byref(inf)))
        return inf

    @property
    def num_vectors(self) -> int:
        return self._info().num_vectors

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

    @property
    def use_opq(self) -> bool:
        return self._use_opq

    @property
    def is_built(self) -> bool:
        return bool(self._info().built)

    def __len__(self) -> int:
        return self.num_vectors

    def __repr__(self) -> str:
        return (f"IVFPQIndex(dim={self._dim}, num_clusters={self._num_clusters}, "
                f"num_codebooks={self._num_codebooks}, codebook_size={self._codebook_size}, "
                f"nprobe={self._nprobe}, num_vectors={len(self)})")
