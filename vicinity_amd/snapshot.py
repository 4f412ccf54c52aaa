"""Directory snapshots in the reference's IVF-PQ format, so an index saved by
vicinity (`IVFPQIndex::save_to_dir`, src/ivf_pq/search.rs:906-1002) loads
here and the other way round.

Files (src/ivf_pq/persistence.rs, manifest.rs, file_storage.rs):
- ``manifest.json``: version 1, shapes, the parameters, the quantizer
  (serde's externally tagged ``{"Product": {...}}``, codebooks flat and
  codebook-major, or ``{"Optimized": {..., "rotation": [d*d row-major],
  "pq": {...}}}`` for OPQ, src/ivf_pq/opq.rs:29-41), the filter field and the documents' filter metadata, sorted
  by doc id (search.rs:968-991);
- ``centroids.bin`` f32, ``doc_ids.bin`` u32, ``codes.bin`` u8 in insertion
  order, ``raw_vectors.bin`` f32 when the vectors are kept; all little-endian;
- ``clusters.bin``: magic ``VICIVF1\\0``, u64 list count, then per list its u64
  category bitmask, u64 length and u32 member indices (persistence.rs:51-68);
- ``list_offsets.bin`` (u64 byte offsets) and ``list_codes.bin`` (the codes
  list by list), the file searcher's sidecars (file_storage.rs:39-71); written
  for it, not read by load (search.rs:1034-1084 does not read them).

Generations (src/persistence/generation.rs): ``root/generations/<id>`` holds a
snapshot whose manifest lists its component files, plus ``GENERATION.json``
(each file's length and CRC-32); ``root/CURRENT`` names the published one.

Floats in the manifest are decimal strings; codebook values are read back to
the nearest float32 of the decimal (correctly rounded, no double rounding), so
a loaded index holds the saved codebooks bit for bit.
"""

from __future__ import annotations

import fcntl
import itertools
import json
import os
import re
import struct
import time
import zlib
from decimal import Decimal

import numpy as np

FORMAT_VERSION = 1          # persistence.rs:9
CLUSTER_MAGIC = b"VICIVF1\0"  # persistence.rs:10


class SnapshotFormatError(RuntimeError):
    """RetrieveError::FormatError: a snapshot that does not follow the format
    (pyvicinity raises RuntimeError for it, src/python.rs:67-70)."""


# ---- floats ---------------------------------------------------------------

def f32_from_decimal(tok: str) -> np.float32:
    """The float32 nearest to the decimal `tok` (ties to even).  The decimal is
    first rounded to float64; that can only mislead when the float64 lands
    exactly midway between two float32 neighbours, which is settled by
    comparing the decimal itself with the midpoint."""
    x = float(tok)
    f = np.float32(x)
    if not np.isfinite(f) or float(f) == x:
        return f
    if float(f) < x:
        lo, hi = f, np.nextafter(f, np.float32(np.inf))
    else:
        lo, hi = np.nextafter(f, np.float32(-np.inf)), f
    mid = (float(lo) + float(hi)) / 2.0  # exact: float32 neighbours
    if x != mid:
        return f
    d, m = Decimal(tok), Decimal(mid)
    if d > m:
        return hi
    if d < m:
        return lo
    return lo if (int(np.float32(lo).view(np.uint32)) & 1) == 0 else hi


def _f32_text(v: np.float32) -> str:
    """Shortest decimal that reads back as v (the form serde_json writes)."""
    return np.format_float_positional(np.float32(v), unique=True, trim="0")


# ---- metadata values (src/filtering/mod.rs:8-23, serde externally tagged) ---

def metadata_to_json(md: dict) -> dict:
    out = {}
    for k, v in md.items():
        if isinstance(v, bool):
            out[k] = {"Bool": v}
        elif isinstance(v, int):
            out[k] = {"Int": v}
        elif isinstance(v, float):
            out[k] = {"Float": v if np.isfinite(v) else None}
        elif isinstance(v, str):
            out[k] = {"Str": v}
        else:
            raise TypeError(f"unsupported metadata value type {type(v).__name__}")
    return out


def metadata_from_json(obj: dict) -> dict:
    out = {}
    for k, tagged in obj.items():
        if not isinstance(tagged, dict) or len(tagged) != 1:
            raise SnapshotFormatError(f"metadata value of {k!r} is not a tagged MetadataValue")
        (tag, v), = tagged.items()
        if tag == "Int" and isinstance(v, int) and not isinstance(v, bool):
            out[k] = v
        elif tag == "Float" and isinstance(v, (int, float, str)) and not isinstance(v, bool):
            out[k] = float(v)  # decimals arrive as text (the manifest is read with parse_float=str)
        elif tag == "Str" and isinstance(v, str):
            out[k] = v
        elif tag == "Bool" and isinstance(v, bool):
            out[k] = v
        else:
            raise SnapshotFormatError(f"metadata value of {k!r}: unknown variant {tag!r}")
    return out


# ---- writing (search.rs:944-1002) -------------------------------------------

def _write_atomic(path: str, data: bytes) -> None:
    """persistence.rs:70-93: write a temporary sibling, sync, rename."""
    tmp = f"{path}.tmp.{os.getpid()}"
    try:
        with open(tmp, "wb") as f:
            f.write(data)
            f.flush()
            os.fsync(f.fileno())
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise


def write_snapshot(path, *, dimension: int, params: dict, centroids, codebooks, codebook_size: int,
                   num_codebooks: int, list_offsets, list_ids, codes, doc_ids, vectors=None,
                   list_masks=None, filter_field=None, filter_metadata=None,
                   rotation=None, generation_components=False) -> None:
    """Write a built index's arrays as a snapshot directory.  `params` holds
    num_clusters, nprobe, num_codebooks, codebook_size, use_opq and seed as
    the index was configured; list_offsets / list_ids are the lists as entry
    offsets and member indices.  With use_opq the quantizer is written as
    Quantizer::Optimized holding `rotation` (d x d, or None).  A generation's
    manifest lists its component files (search.rs:991-995,
    manifest.rs:64-77)."""
    centroids = np.ascontiguousarray(centroids, np.float32).reshape(-1, dimension)
    codebooks = np.ascontiguousarray(codebooks, np.float32).reshape(-1)
    list_offsets = np.asarray(list_offsets, np.uint64)
    list_ids = np.ascontiguousarray(list_ids, np.uint32)
    codes = np.ascontiguousarray(codes, np.uint8).reshape(-1, num_codebooks)
    doc_ids = np.ascontiguousarray(doc_ids, np.uint32)
    n = doc_ids.shape[0]
    L = centroids.shape[0]
    nlists = max(int(params["num_clusters"]), L)  # search.rs:626: one list per configured cluster
    if list_masks is None:
        list_masks = np.zeros(L, np.uint64)
    if filter_metadata and filter_field is None:
        raise ValueError("InvalidConfig: filter_field must be set before enabling filter metadata")
    os.makedirs(path, exist_ok=True)
    ds = dimension // num_codebooks
    present = vectors is not None
    manifest = {
        "version": FORMAT_VERSION,
        "dimension": int(dimension),
        "num_vectors": int(n),
        "num_centroids": int(L),
        "raw_vectors_present": bool(present),
        "params": {
            "num_clusters": int(params["num_clusters"]),
            "nprobe": int(params["nprobe"]),
            "num_codebooks": int(params["num_codebooks"]),
            "codebook_size": int(params["codebook_size"]),
            "use_opq": bool(params.get("use_opq", False)),
            "seed": int(params["seed"]),
        },
        "quantizer": None,
        "filter_field": filter_field,
        "filter_metadata": [
            {"doc_id": int(doc), "metadata": metadata_to_json(md)}
            for doc, md in sorted((filter_metadata or {}).items())
        ],
    }
    product = {
        "dimension": int(dimension),
        "num_codebooks": int(num_codebooks),
        "codebook_size": int(codebook_size),
        "subvector_dim": int(ds),
        "codebooks": "@CODEBOOKS@",
    }
    if params.get("use_opq", False):
        # OptimizedProductQuantizer (opq.rs:31-41): its own codebook_size stays
        # the configured one; the inner pq's is the trained one.
        manifest["quantizer"] = {"Optimized": {
            "dimension": int(dimension),
            "num_codebooks": int(num_codebooks),
            "codebook_size": int(params["codebook_size"]),
            "rotation": None if rotation is None else "@ROTATION@",
            "pq": product,
        }}
    else:
        manifest["quantizer"] = {"Product": product}
    if generation_components:
        manifest["generation_components"] = _COMPONENTS + (["raw_vectors.bin"] if present else [])
    text = json.dumps(manifest, indent=2)
    text = text.replace('"@CODEBOOKS@"', "[" + ", ".join(_f32_text(v) for v in codebooks) + "]")
    if rotation is not None:
        rot = np.ascontiguousarray(rotation, np.float32).reshape(-1)
        if rot.size != dimension * dimension:
            raise ValueError("rotation must hold dimension * dimension floats")
        text = text.replace('"@ROTATION@"', "[" + ", ".join(_f32_text(v) for v in rot) + "]")
    _write_atomic(os.path.join(path, "manifest.json"), text.encode("utf-8"))
    _write_atomic(os.path.join(path, "centroids.bin"), centroids.astype("<f4").tobytes())
    _write_atomic(os.path.join(path, "doc_ids.bin"), doc_ids.astype("<u4").tobytes())
    _write_atomic(os.path.join(path, "codes.bin"), codes.tobytes())
    # lists: the index's lists, then empty ones up to the configured count
    parts, byte_offsets, body = [], [0], []
    for l in range(nlists):
        if l < L:
            ids = list_ids[int(list_offsets[l]):int(list_offsets[l + 1])]
            mask = int(list_masks[l])
        else:
            ids, mask = np.zeros(0, np.uint32), 0
        parts.append(struct.pack("<QQ", mask, ids.shape[0]) + ids.astype("<u4").tobytes())
        body.append(codes[ids].tobytes())  # file_storage.rs:39-71
        byte_offsets.append(byte_offsets[-1] + ids.shape[0] * num_codebooks)
    _write_atomic(os.path.join(path, "list_offsets.bin"),
                  np.asarray(byte_offsets, "<u8").tobytes())
    _write_atomic(os.path.join(path, "list_codes.bin"), b"".join(body))
    _write_atomic(os.path.join(path, "clusters.bin"),
                  CLUSTER_MAGIC + struct.pack("<Q", nlists) + b"".join(parts))
    if present:
        _write_atomic(os.path.join(path, "raw_vectors.bin"),
                      np.ascontiguousarray(vectors, np.float32).astype("<f4").tobytes())


# ---- reading (search.rs:1034-1084) ------------------------------------------

_COMPONENTS = ["centroids.bin", "clusters.bin", "codes.bin", "doc_ids.bin", "list_codes.bin",
               "list_offsets.bin"]  # manifest.rs:64-79


def _check_size(path: str, nbytes: int) -> None:
    size = os.path.getsize(path)
    if size != nbytes:
        raise SnapshotFormatError(f"{os.path.basename(path)} size mismatch: expected {nbytes} bytes, got {size}")


def _read_exact(path: str, dtype, count: int) -> np.ndarray:
    """persistence.rs:117-174: the file holds exactly `count` values."""
    with open(path, "rb") as f:
        data = f.read()
    want = count * np.dtype(dtype).itemsize
    if len(data) != want:
        raise SnapshotFormatError(f"{path} size mismatch: expected {want} bytes, got {len(data)}")
    return np.frombuffer(data, dtype=dtype).astype(np.dtype(dtype).newbyteorder("="), copy=True)


def read_snapshot(path, arrays: bool = True) -> dict:
    """Parse and check a snapshot directory; returns the manifest fields and
    the arrays (lists as entry offsets + member indices).  With arrays=False
    the codes and raw vectors are not read (their files' sizes are checked):
    what the file-backed searcher keeps in memory (search.rs:1679-1762)."""
    with open(os.path.join(path, "manifest.json"), "rb") as f:
        raw = f.read()
    try:
        man = json.loads(raw, parse_float=str, parse_int=int)
    except ValueError as e:
        raise SnapshotFormatError(str(e)) from None
    if not isinstance(man, dict):
        raise SnapshotFormatError("manifest is not a JSON object")
    try:
        version = int(man["version"])
        dim, n, L = int(man["dimension"]), int(man["num_vectors"]), int(man["num_centroids"])
        present = man["raw_vectors_present"]
        prm = man["params"]
        quant = man["quantizer"]
    except (KeyError, TypeError) as e:
        raise SnapshotFormatError(f"manifest field missing: {e}") from None
    # persistence.rs:176-199
    if version != FORMAT_VERSION:
        raise SnapshotFormatError(f"unsupported IVF-PQ format version {version}")
    if dim == 0:
        raise SnapshotFormatError("IVF-PQ manifest has zero dimension")
    if n == 0:
        raise SnapshotFormatError("IVF-PQ manifest has zero vectors")
    if L == 0:
        raise SnapshotFormatError("IVF-PQ manifest has zero centroids")
    comps = man.get("generation_components")
    if comps is not None:  # manifest.rs:81-98
        want = _COMPONENTS + (["raw_vectors.bin"] if present else [])
        if comps != want:
            raise SnapshotFormatError(
                f"IVF-PQ generation component inventory mismatch: expected {want}, got {comps}")
    rotation = None
    if isinstance(quant, dict) and list(quant) == ["Product"]:
        pq = quant["Product"]
    elif isinstance(quant, dict) and list(quant) == ["Optimized"]:
        try:
            pq = quant["Optimized"]["pq"]
            rot = quant["Optimized"]["rotation"]
        except (KeyError, TypeError) as e:
            raise SnapshotFormatError(f"manifest field missing: {e}") from None
        if rot is not None:
            if len(rot) != dim * dim:
                raise SnapshotFormatError("OPQ rotation is not dimension x dimension")
            rotation = np.array([f32_from_decimal(str(t)) for t in rot], np.float32).reshape(dim, dim)
    else:
        raise SnapshotFormatError("unknown quantizer (expected Product or Optimized)")
    M, K, ds = int(pq["num_codebooks"]), int(pq["codebook_size"]), int(pq["subvector_dim"])
    cb_tokens = pq["codebooks"]
    if len(cb_tokens) != M * K * ds or M * ds != dim:
        raise SnapshotFormatError("product quantizer shape does not match its codebooks")
    codebooks = np.array([f32_from_decimal(str(t)) for t in cb_tokens], np.float32)
    params = {key: prm[key] for key in ("num_clusters", "nprobe", "num_codebooks", "codebook_size",
                                        "use_opq", "seed")}
    filter_field = man.get("filter_field")
    filter_metadata = {}
    for entry in man.get("filter_metadata") or []:
        filter_metadata[int(entry["doc_id"])] = metadata_from_json(entry["metadata"])
    if filter_metadata and filter_field is None:
        raise SnapshotFormatError("IVF-PQ manifest has filter metadata without filter_field")

    doc_ids = _read_exact(os.path.join(path, "doc_ids.bin"), "<u4", n)
    centroids = _read_exact(os.path.join(path, "centroids.bin"), "<f4", L * dim).reshape(L, dim)
    codes = vectors = None
    if arrays:
        codes = _read_exact(os.path.join(path, "codes.bin"), np.uint8,
                            n * int(params["num_codebooks"])).reshape(n, -1)
        if present:
            vectors = _read_exact(os.path.join(path, "raw_vectors.bin"), "<f4", n * dim).reshape(n, dim)
    else:
        _check_size(os.path.join(path, "codes.bin"), n * int(params["num_codebooks"]))
        if present:
            _check_size(os.path.join(path, "raw_vectors.bin"), n * dim * 4)
    # clusters.bin (persistence.rs:201-248)
    with open(os.path.join(path, "clusters.bin"), "rb") as f:
        blob = f.read()
    if blob[:8] != CLUSTER_MAGIC:
        raise SnapshotFormatError("invalid IVF-PQ cluster file magic")
    pos = 8

    def take(nbytes):
        nonlocal pos
        if pos + nbytes > len(blob):
            raise SnapshotFormatError("unexpected end of IVF-PQ cluster file")
        out = blob[pos:pos + nbytes]
        pos += nbytes
        return out

    (count,) = struct.unpack("<Q", take(8))
    if count != int(params["num_clusters"]):
        raise SnapshotFormatError(
            f"cluster count mismatch: expected {params['num_clusters']}, got {count}")
    masks, offsets, ids = [], [0], []
    for _ in range(count):
        mask, length = struct.unpack("<QQ", take(16))
        if length > n:
            raise SnapshotFormatError(f"cluster length {length} exceeds vector count {n}")
        members = np.frombuffer(take(4 * length), "<u4").astype(np.uint32)
        if members.size and int(members.max()) >= n:
            raise SnapshotFormatError(f"cluster id {int(members.max())} exceeds vector count {n}")
        masks.append(mask)
        ids.append(members)
        offsets.append(offsets[-1] + length)
    if pos != len(blob):
        raise SnapshotFormatError("trailing bytes in IVF-PQ cluster file")
    # lists past the centroids can hold nothing (no centroid to assign to)
    if any(len(m) for m in ids[L:]):
        raise SnapshotFormatError("a list beyond the centroids holds members")
    list_ids = np.concatenate(ids[:L]) if L else np.zeros(0, np.uint32)
    return {
        "dimension": dim, "num_vectors": n, "params": params, "M": M, "K": K,
        "centroids": centroids, "codebooks": codebooks, "doc_ids": doc_ids, "codes": codes,
        "vectors": vectors, "list_offsets": np.asarray(offsets[:L + 1], np.uint64),
        "list_ids": list_ids.astype(np.uint32), "list_masks": np.asarray(masks[:L], np.uint64),
        "filter_field": filter_field, "filter_metadata": filter_metadata, "rotation": rotation,
        "raw_vectors_present": bool(present),
    }


# ---- generations (src/persistence/generation.rs) ----------------------------

_GEN_SEQUENCE = itertools.count()


def open_current(root) -> str:
    """open_current (generation.rs:191-205): root/CURRENT names a directory
    under root/generations."""
    with open(os.path.join(root, "CURRENT"), encoding="utf-8") as f:
        gen = f.read().strip()
    if not re.fullmatch(r"[A-Za-z0-9_.-]+", gen) or gen in (".", ".."):
        raise SnapshotFormatError(f"invalid generation id {gen!r}")
    path = os.path.join(root, "generations", gen)
    if os.path.islink(path) or not os.path.isdir(path):
        raise SnapshotFormatError(f"current generation {path} is not a directory")
    return path


def _fsync_dir(path) -> None:
    fd = os.open(path, os.O_RDONLY)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def generation_inventory(directory) -> dict:
    """write_inventory (generation.rs:389-449): every file below the
    generation but GENERATION.json, sorted by its '/'-separated path, with its
    length and CRC-32 (the reflected 0xEDB88320 polynomial, generation.rs:
    451-470, which zlib.crc32 computes).  Symlinks and other entries are
    format errors."""
    files = []
    for top, dirs, names in os.walk(directory, followlinks=False):
        for name in list(dirs) + names:
            full = os.path.join(top, name)
            if os.path.islink(full):
                raise SnapshotFormatError(f"generation contains symlink {full}")
        for name in names:
            full = os.path.join(top, name)
            rel = os.path.relpath(full, directory).replace(os.sep, "/")
            if rel == "GENERATION.json":
                continue
            if not os.path.isfile(full):
                raise SnapshotFormatError(f"generation contains unsupported entry {full}")
            crc, length = 0, 0
            with open(full, "rb") as f:
                for chunk in iter(lambda: f.read(1 << 20), b""):
                    crc = zlib.crc32(chunk, crc)
                    length += len(chunk)
            files.append({"path": rel, "length": length, "crc32": crc})
    files.sort(key=lambda e: e["path"].encode("utf-8"))
    return {"version": 1, "files": files}


def publish_generation(root, write) -> str:
    """GenerationWriter (generation.rs:36-140): write(staging) fills a hidden
    staging directory under root/generations, which is then checked by
    reading it back, inventoried (GENERATION.json), synced and renamed to
    generations/<id>; root/CURRENT is replaced last (temporary file, sync,
    rename), under the advisory lock root/.PUBLISH.lock, and only if CURRENT
    still names the generation it named when the writer started.  Returns the
    published directory."""
    root = os.fspath(root)
    gens = os.path.join(root, "generations")
    os.makedirs(gens, exist_ok=True)
    cur_path = os.path.join(root, "CURRENT")
    try:
        with open(cur_path, encoding="utf-8") as f:
            expected = f.read().strip()
    except FileNotFoundError:
        expected = None
    gen_id = f"{time.time_ns()}-{os.getpid()}-{next(_GEN_SEQUENCE)}"
    staging = os.path.join(gens, f".staging-{gen_id}")
    os.mkdir(staging)
    write(staging)
    read_snapshot(staging)  # validate_staged_generation (search.rs:1016-1031)
    with open(os.path.join(root, ".PUBLISH.lock"), "a") as lock:
        try:
            fcntl.flock(lock.fileno(), fcntl.LOCK_EX | fcntl.LOCK_NB)
        except BlockingIOError:
            raise SnapshotFormatError(
                f"{root}/.PUBLISH.lock: another generation publisher holds the advisory lock") from None
        try:
            try:
                with open(cur_path, encoding="utf-8") as f:
                    now = f.read().strip()
            except FileNotFoundError:
                now = None
            if now != expected:
                raise SnapshotFormatError(f"{cur_path}: CURRENT changed while this generation was being built")
            inv = os.path.join(staging, "GENERATION.json")
            if os.path.exists(inv):
                raise SnapshotFormatError("GENERATION.json is reserved for the generation inventory")
            _write_atomic(inv, json.dumps(generation_inventory(staging), indent=2).encode("utf-8"))
            for top, _, names in os.walk(staging):
                for name in names:
                    with open(os.path.join(top, name), "rb") as f:
                        os.fsync(f.fileno())
                _fsync_dir(top)
            published = os.path.join(gens, gen_id)
            os.rename(staging, published)
            _fsync_dir(gens)
            tmp = os.path.join(root, f".CURRENT.tmp.{os.getpid()}.{next(_GEN_SEQUENCE)}")
            try:
                with open(tmp, "w", encoding="utf-8") as f:
                    f.write(gen_id + "\n")
                    f.flush()
                    os.fsync(f.fileno())
                os.replace(tmp, cur_path)
            except BaseException:
                if os.path.exists(tmp):
                    os.remove(tmp)
                raise
            _fsync_dir(root)
        finally:
            fcntl.flock(lock.fileno(), fcntl.LOCK_UN)
    return published
