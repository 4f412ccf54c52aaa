"""vicinity_amd: batched IVF-PQ search for one AMD MI355X (gfx950).

The search path runs in hand-written HIP kernels behind the C ABI of
include/vicinity_gpu.h (libvicinity_gpu.so, built by vicinity_amd/csrc).
"""

from ._lib import LIB_PATH, VicinityGpuError, device_available
from .filtering import MetadataFilter
from .file_searcher import IVFPQFileSearcher
from .flat import FlatIndex
from . import datagen
from .ivf_pq import MISSING_DISTANCE, MISSING_LABEL, IVFPQIndex, default_codebooks

__all__ = [
    "IVFPQIndex",
    "IVFPQFileSearcher",
    "FlatIndex",
    "MetadataFilter",
    "MISSING_LABEL",
    "MISSING_DISTANCE",
    "VicinityGpuError",
    "default_codebooks",
    "device_available",
    "LIB_PATH",
    "build_library",
]


def build_library() -> str:
    """Compile libvicinity_gpu.so for gfx950 in-tree (make)."""
    import os
    import subprocess

    here = os.path.dirname(os.path.abspath(__file__))
    subprocess.run(["make", "-s", "-j8", "-C", os.path.join(here, "csrc")], check=True)
    return LIB_PATH
