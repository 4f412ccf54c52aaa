"""ctypes binding of libvicinity_gpu.so (the C ABI in include/vicinity_gpu.h).

The library is built in-tree by vicinity_amd/csrc/Makefile; importing this
module never builds it and never substitutes a CPU path: a missing library is
an ImportError-style failure at first use.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

# VGPU_LIB: another build of the library (for example an instrumented one) in
# place of the in-tree libvicinity_gpu.so.
LIB_PATH = os.environ.get("VGPU_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                      "libvicinity_gpu.so")

# status codes (src/error.rs:17-80)
OK = 0
ERR_EMPTY_INDEX = 1
ERR_INVALID_PARAMETER = 2
ERR_INVALID_CONFIG = 3
ERR_NOT_BUILT = 4
ERR_ALREADY_BUILT = 5
ERR_UNSUPPORTED = 6
ERR_DIMENSION_MISMATCH = 7
ERR_DEVICE = 8
ERR_OUT_OF_MEMORY = 9

MODE_FAST = 0
MODE_EXACT = 1


class VicinityGpuError(RuntimeError):
    """A failure reported by the C ABI (status code in .code)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class Params(ctypes.Structure):
    _fields_ = [("num_clusters", ctypes.c_size_t), ("nprobe", ctypes.c_size_t),
                ("num_codebooks", ctypes.c_size_t), ("codebook_size", ctypes.c_size_t),
                ("seed", ctypes.c_uint64), ("use_opq", ctypes.c_int)]


class Info(ctypes.Structure):
    _fields_ = [("dimension", ctypes.c_size_t), ("num_vectors", ctypes.c_size_t),
                ("num_clusters", ctypes.c_size_t), ("nprobe", ctypes.c_size_t),
                ("num_codebooks", ctypes.c_size_t), ("codebook_size", ctypes.c_size_t),
                ("subvector_dim", ctypes.c_size_t), ("built", ctypes.c_int),
                ("has_vectors", ctypes.c_int), ("mode", ctypes.c_int)]


class FileDiagnostics(ctypes.Structure):
    """IVFPQFileSearchDiagnostics (search.rs:263-282)."""
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "probed_lists", "scanned_vectors", "code_reads", "code_bytes", "retained_candidates",
        "raw_vector_reads", "raw_vector_bytes", "reranked_candidates")]

    def as_dict(self) -> dict:
        return {name: int(getattr(self, name)) for name, _ in self._fields_}


class MemoryReport(ctypes.Structure):
    """MemoryReport (src/memory.rs:4-14) plus the HBM the index holds."""
    _fields_ = [(name, ctypes.c_size_t) for name in (
        "vectors_bytes", "graph_bytes", "quantized_bytes", "metadata_bytes", "device_bytes")]

    def as_dict(self) -> dict:
        d = {name: int(getattr(self, name)) for name, _ in self._fields_}
        d["total"] = d["vectors_bytes"] + d["graph_bytes"] + d["quantized_bytes"] + d["metadata_bytes"]
        return d


class Stats(ctypes.Structure):
    _fields_ = [("ms_normalize", ctypes.c_float), ("ms_coarse", ctypes.c_float),
                ("ms_select", ctypes.c_float), ("ms_scan", ctypes.c_float),
                ("ms_fallback", ctypes.c_float), ("ms_rerank", ctypes.c_float),
                ("ms_total", ctypes.c_float), ("candidates", ctypes.c_uint64),
                ("scan_bytes", ctypes.c_uint64), ("fallback_queries", ctypes.c_uint32),
                ("coarse_overflow", ctypes.c_uint32), ("nq", ctypes.c_uint32),
                ("fast_flushes", ctypes.c_uint64), ("fast_appends", ctypes.c_uint64),
                ("fallback_ties", ctypes.c_uint32), ("fast_retries", ctypes.c_uint32),
                ("ms_table", ctypes.c_float)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
_H = ctypes.c_void_p
_i = ctypes.c_int
_ci = ctypes.c_int
_f = ctypes.c_float

# name -> (restype, argtypes); every symbol declared in include/vicinity_gpu.h.
SIGNATURES = {
    "vgpu_last_error": (ctypes.c_char_p, []),
    "vgpu_device_available": (_i, []),
    "vgpu_ivfpq_new": (_i, [_sz, ctypes.POINTER(Params), ctypes.POINTER(_H)]),
    "vgpu_ivfpq_free": (None, [_H]),
    "vgpu_ivfpq_add": (_i, [_H, _vp, _vp, _sz]),
    "vgpu_ivfpq_build": (_i, [_H, _sz, _sz]),
    "vgpu_ivfpq_load": (_i, [_H, _vp, _sz, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _sz]),
    "vgpu_ivfpq_set_nprobe": (_i, [_H, _sz]),
    "vgpu_ivfpq_set_mode": (_i, [_H, _i]),
    "vgpu_ivfpq_compact": (_i, [_H]),
    "vgpu_ivfpq_get_info": (_i, [_H, ctypes.POINTER(Info)]),
    "vgpu_ivfpq_search": (_i, [_H, _vp, _sz, _sz, _vp, _vp, ctypes.POINTER(_sz)]),
    "vgpu_ivfpq_search_reranked": (_i, [_H, _vp, _sz, _sz, _sz, _vp, _vp, ctypes.POINTER(_sz)]),
    "vgpu_ivfpq_search_batch": (_i, [_H, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp]),
    "vgpu_ivfpq_search_batch_device": (_i, [_H, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _vp]),
    "vgpu_ivfpq_search_batch_device_noalloc": (_i, [_H, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp,
                                                    _vp]),
    "vgpu_ivfpq_last_stats": (_i, [_H, ctypes.POINTER(Stats)]),
    "vgpu_ivfpq_set_profiling": (_i, [_H, _i]),
    "vgpu_ivfpq_enable_filtering": (_i, [_H]),
    "vgpu_ivfpq_set_category": (_i, [_H, ctypes.c_uint32, ctypes.c_int64]),
    "vgpu_ivfpq_search_filtered": (_i, [_H, _vp, _sz, _sz, ctypes.c_int64, _vp, _vp,
                                        ctypes.POINTER(_sz)]),
    "vgpu_ivfpq_search_filtered_batch": (_i, [_H, _vp, _sz, _sz, _sz, _vp, _vp, _vp]),
    "vgpu_ivfpq_get_list_masks": (_i, [_H, _vp, _sz]),
    "vgpu_ivfpq_set_list_masks": (_i, [_H, _vp, _sz]),
    "vgpu_ivfpq_get_rotation": (_i, [_H, _vp, _sz, _vp]),
    "vgpu_ivfpq_set_rotation": (_i, [_H, _vp, _sz]),
    "vgpu_ivfpq_probe_batch": (_i, [_H, _vp, _sz, _sz, _sz, _vp, ctypes.POINTER(_sz)]),
    "vgpu_ivfpq_export": (_i, [_H, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "vgpu_ivfpq_reconstruct": (_i, [_H, _sz, _vp, _sz]),
    "vgpu_ivfpq_memory_usage": (_i, [_H, ctypes.POINTER(MemoryReport)]),
    "vgpu_ivfpq_file_open": (_i, [_sz, ctypes.POINTER(Params), _vp, _sz, _vp, _sz, _vp, _vp, _vp, _sz, _vp,
                                  ctypes.c_char_p, _i, ctypes.POINTER(_H)]),
    "vgpu_ivfpq_file_free": (None, [_H]),
    "vgpu_ivfpq_file_set_nprobe": (_i, [_H, _sz]),
    "vgpu_ivfpq_file_search_batch": (_i, [_H, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _vp]),
    "vgpu_ivfpq_file_last_io": (_i, [_H, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "vgpu_flat_new": (_i, [_sz, _i, ctypes.POINTER(_H)]),
    "vgpu_flat_free": (None, [_H]),
    "vgpu_flat_add": (_i, [_H, _vp, _sz]),
    "vgpu_flat_search_batch": (_i, [_H, _vp, _sz, _sz, _sz, _vp, _vp]),
    "vgpu_flat_search_batch_device": (_i, [_H, _vp, _sz, _sz, _sz, _vp, _vp, _vp]),
    "vgpu_flat_last_ms": (_i, [_H, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]),
    "vgpu_flat_last_fallbacks": (_i, [_H, ctypes.POINTER(ctypes.c_uint32)]),
    "vgpu_test_host_lists": (_i, [_vp, _sz, _sz, _vp, _vp]),
    "vgpu_test_host_centroid_update": (_i, [_vp, _sz, _sz, _vp, _sz, _vp]),
    "vgpu_test_polar_factor": (_i, [_vp, _sz, _vp]),
    "vgpu_test_set_rres_limit": (_i, [_H, _sz]),
    "vgpu_test_fail_device_allocations": (_i, [_sz, _sz]),
    "vgpu_test_bound_fast_tau": (_i, [_sz, _sz, _sz, _f, _f, _f, _f, _vp]),
    "vgpu_test_bound_coarse": (_i, [_sz, _f, _f, _vp, _vp]),
    "vgpu_test_bound_flat": (_i, [_sz, _ci, _f, _f, _ci, _vp]),
    "vgpu_test_adc_tables": (_i, [_vp, _sz, _sz, _sz, _vp, _sz, _vp]),
    "vgpu_test_pq_encode": (_i, [_vp, _sz, _sz, _sz, _vp, _sz, _vp]),
    "vgpu_test_normalize": (_i, [_vp, _sz, _sz, _vp]),
    "vgpu_test_fastscan": (_i, [_vp, _sz, _sz, _vp, _vp]),
    "vgpu_test_coarse_dots": (_i, [_vp, _sz, _vp, _sz, _sz, _vp]),
    "vgpu_test_coarse_dots_bf16x3": (_i, [_vp, _sz, _vp, _sz, _sz, _vp]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libvicinity_gpu.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C vicinity_amd/csrc` "
                "(there is no CPU fallback)")
        # PyTorch's ROCm wheel carries its own HIP and HSA runtimes.  Loading
        # torch first makes this library bind to those same runtimes; loaded
        # the other way round, the process holds two HSA runtimes and the
        # second to initialise finds no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = load().vgpu_last_error().decode("utf-8", "replace")
        if status in (ERR_DEVICE, ERR_OUT_OF_MEMORY):
            raise VicinityGpuError(status, msg)
        err = ValueError(msg)
        err.code = status  # type: ignore[attr-defined]
        raise err


def ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def device_available() -> bool:
    return bool(load().vgpu_device_available())
