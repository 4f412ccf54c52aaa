"""Directory snapshots in the reference's format (src/ivf_pq/persistence.rs,
manifest.rs, file_storage.rs; search.rs:906-1084).  The writer's files are
checked against bytes packed by hand from the Rust writers, the reader against
a hand-written manifest in serde's shape, and the reference's own load tests
(search.rs:3076-3190) against the reader's errors."""

import json
import os
import struct

import numpy as np
import pytest

from vicinity_amd.snapshot import (CLUSTER_MAGIC, SnapshotFormatError, f32_from_decimal,
                                   read_snapshot, write_snapshot)


def _arrays(seed=0, n=50, d=8, L=4, M=2, K=16, with_vectors=True):
    rng = np.random.default_rng(seed)
    assign = rng.integers(0, L, n)
    order = np.argsort(assign, kind="stable")
    counts = np.bincount(assign, minlength=L)
    return {
        "centroids": rng.standard_normal((L, d)).astype(np.float32),
        "codebooks": (rng.standard_normal(M * K * (d // M)) * 10.0 ** rng.integers(-8, 8, M * K * (d // M))).astype(np.float32),
        "list_offsets": np.concatenate([[0], np.cumsum(counts)]).astype(np.uint64),
        "list_ids": order.astype(np.uint32),
        "codes": rng.integers(0, K, (n, M)).astype(np.uint8),
        "doc_ids": (1000 + rng.permutation(n)).astype(np.uint32),
        "vectors": rng.standard_normal((n, d)).astype(np.float32) if with_vectors else None,
        "M": M, "K": K, "d": d, "L": L, "n": n,
    }


def _write(path, a, params=None, **kw):
    params = params or {"num_clusters": a["L"], "nprobe": 3, "num_codebooks": a["M"],
                        "codebook_size": a["K"], "use_opq": False, "seed": 7}
    write_snapshot(path, dimension=a["d"], params=params, centroids=a["centroids"],
                   codebooks=a["codebooks"], codebook_size=a["K"], num_codebooks=a["M"],
                   list_offsets=a["list_offsets"], list_ids=a["list_ids"], codes=a["codes"],
                   doc_ids=a["doc_ids"], vectors=a["vectors"], **kw)


def test_decimal_to_float32_is_correctly_rounded():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 0x7f800000, 20000, dtype=np.uint32)  # positive finite, subnormals too
    vals = bits.view(np.float32)
    for v in vals[:20000:7]:
        for text in (np.format_float_positional(v, unique=True), repr(float(v)),
                     np.format_float_scientific(v, unique=True)):
            assert f32_from_decimal(text).view(np.uint32) == v.view(np.uint32)
    # a decimal just above the midpoint of two float32 neighbours that rounds to
    # the midpoint in float64: the float32 above it is the nearest
    a = np.float32(1.0)
    b = np.nextafter(a, np.float32(2.0))
    mid = (float(a) + float(b)) / 2.0
    from decimal import Decimal, localcontext
    with localcontext() as ctx:
        ctx.prec = 60
        just_above = str(Decimal(mid) + Decimal("1e-30"))
        just_below = str(Decimal(mid) - Decimal("1e-30"))
    assert float(just_above) == mid and np.float32(float(just_above)) == a  # the double-rounding trap
    assert f32_from_decimal(just_above) == b
    assert f32_from_decimal(just_below) == a
    assert f32_from_decimal(str(Decimal(mid))) == a  # the exact midpoint: ties to even
    assert f32_from_decimal(repr(mid)) == b  # float64's shortest text lies just above it


def test_cluster_and_list_files_are_the_rust_layout(tmp_path):
    a = _arrays()
    masks = np.array([0b101, 0, 1 << 63, 2], np.uint64)
    _write(tmp_path, a, params={"num_clusters": 6, "nprobe": 3, "num_codebooks": 2,
                                "codebook_size": 16, "use_opq": False, "seed": 7},
           list_masks=masks)
    # persistence.rs:51-68: magic, u64 count, per cluster u64 mask, u64 len, u32 ids
    want = CLUSTER_MAGIC + struct.pack("<Q", 6)
    codes_want, offs = b"", [0]
    for l in range(6):
        if l < 4:
            ids = a["list_ids"][a["list_offsets"][l]:a["list_offsets"][l + 1]]
            m = int(masks[l])
        else:
            ids, m = [], 0  # configured lists beyond the centroids are empty
        want += struct.pack("<QQ", m, len(ids)) + b"".join(struct.pack("<I", int(i)) for i in ids)
        for i in ids:  # file_storage.rs:39-71
            codes_want += bytes(a["codes"][int(i)])
        offs.append(len(codes_want))
    assert (tmp_path / "clusters.bin").read_bytes() == want
    assert (tmp_path / "list_codes.bin").read_bytes() == codes_want
    assert (tmp_path / "list_offsets.bin").read_bytes() == b"".join(struct.pack("<Q", o) for o in offs)
    assert (tmp_path / "codes.bin").read_bytes() == a["codes"].tobytes()
    assert (tmp_path / "doc_ids.bin").read_bytes() == b"".join(struct.pack("<I", int(x)) for x in a["doc_ids"])
    assert (tmp_path / "centroids.bin").read_bytes() == b"".join(struct.pack("<f", x) for x in a["centroids"].ravel())
    man = json.loads((tmp_path / "manifest.json").read_text())
    assert list(man) == ["version", "dimension", "num_vectors", "num_centroids",
                         "raw_vectors_present", "params", "quantizer", "filter_field",
                         "filter_metadata"]  # manifest.rs:44-61 field order
    assert man["quantizer"]["Product"]["subvector_dim"] == 4
    assert man["params"] == {"num_clusters": 6, "nprobe": 3, "num_codebooks": 2,
                             "codebook_size": 16, "use_opq": False, "seed": 7}


def test_round_trip_keeps_every_array_bit_for_bit(tmp_path):
    a = _arrays(seed=3)
    meta = {1001: {"group": 3, "w": 0.25, "name": "x", "ok": True}, 1000: {"label": "y"}}
    _write(tmp_path, a, list_masks=np.arange(4, dtype=np.uint64), filter_field="group",
           filter_metadata=meta)
    s = read_snapshot(tmp_path)
    for key in ("centroids", "codebooks", "list_offsets", "list_ids", "codes", "doc_ids", "vectors"):
        assert s[key].tobytes() == np.ascontiguousarray(a[key]).tobytes(), key
    assert s["list_masks"].tolist() == [0, 1, 2, 3]
    assert s["filter_field"] == "group" and s["filter_metadata"] == meta
    man = json.loads((tmp_path / "manifest.json").read_text())
    assert [e["doc_id"] for e in man["filter_metadata"]] == [1000, 1001]  # sorted, search.rs:980
    assert man["filter_metadata"][1]["metadata"]["group"] == {"Int": 3}   # serde tagging


def test_reads_a_hand_written_serde_manifest(tmp_path):
    # the manifest in the form serde_json writes (legacy: no filter fields,
    # manifest.rs:52-55 #[serde(default)]), plus binary files packed by hand
    cb = [0.5, -1.25, 3.0, 1e-5, 0.1, 2.0, -0.0, 7.5]  # M 2, K 2, ds 2
    (tmp_path / "manifest.json").write_text(json.dumps({
        "version": 1, "dimension": 4, "num_vectors": 3, "num_centroids": 2,
        "raw_vectors_present": False,
        "params": {"num_clusters": 2, "nprobe": 1, "num_codebooks": 2, "codebook_size": 2,
                   "use_opq": False, "seed": 42},
        "quantizer": {"Product": {"dimension": 4, "num_codebooks": 2, "codebook_size": 2,
                                  "subvector_dim": 2, "codebooks": cb}}}, indent=2))
    (tmp_path / "centroids.bin").write_bytes(struct.pack("<8f", *range(8)))
    (tmp_path / "doc_ids.bin").write_bytes(struct.pack("<3I", 7, 8, 9))
    (tmp_path / "codes.bin").write_bytes(bytes([0, 1, 1, 0, 1, 1]))
    (tmp_path / "clusters.bin").write_bytes(
        CLUSTER_MAGIC + struct.pack("<Q", 2) + struct.pack("<QQ2I", 0, 2, 2, 0) +
        struct.pack("<QQI", 0, 1, 1))
    s = read_snapshot(tmp_path)
    assert s["codebooks"].tolist() == [np.float32(x) for x in cb]
    assert s["list_offsets"].tolist() == [0, 2, 3] and s["list_ids"].tolist() == [2, 0, 1]
    assert s["vectors"] is None and s["filter_field"] is None and s["filter_metadata"] == {}
    assert s["codes"].tolist() == [[0, 1], [1, 0], [1, 1]]


def test_load_rejects_what_the_reference_rejects(tmp_path):
    a = _arrays(seed=5)

    def fresh(name):
        d = tmp_path / name
        _write(d, a)
        return d

    d = fresh("version")  # search.rs:3076-3114
    man = json.loads((d / "manifest.json").read_text())
    man["version"] = 2
    (d / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(SnapshotFormatError, match="unsupported IVF-PQ format version"):
        read_snapshot(d)
    d = fresh("magic")  # search.rs:3160-3190
    (d / "clusters.bin").write_bytes(b"not ivfpq")
    with pytest.raises(SnapshotFormatError, match="invalid IVF-PQ cluster file magic"):
        read_snapshot(d)
    d = fresh("trailing")  # persistence.rs:239-244
    with open(d / "clusters.bin", "ab") as f:
        f.write(b"\0")
    with pytest.raises(SnapshotFormatError, match="trailing bytes"):
        read_snapshot(d)
    d = fresh("size")  # persistence.rs:117-131
    (d / "doc_ids.bin").write_bytes(b"\0" * 12)
    with pytest.raises(SnapshotFormatError, match="size mismatch"):
        read_snapshot(d)
    d = fresh("count")  # persistence.rs:212-217
    blob = bytearray((d / "clusters.bin").read_bytes())
    blob[8:16] = struct.pack("<Q", 9)
    (d / "clusters.bin").write_bytes(bytes(blob))
    with pytest.raises(SnapshotFormatError, match="cluster count mismatch"):
        read_snapshot(d)
    d = fresh("inventory")  # manifest.rs:81-98
    man = json.loads((d / "manifest.json").read_text())
    man["generation_components"] = ["centroids.bin"]
    (d / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(SnapshotFormatError, match="inventory mismatch"):
        read_snapshot(d)
    d = fresh("filters")  # search.rs:1068-1073
    man = json.loads((d / "manifest.json").read_text())
    man["filter_metadata"] = [{"doc_id": 1, "metadata": {"g": {"Int": 1}}}]
    (d / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(SnapshotFormatError, match="without filter_field"):
        read_snapshot(d)
    with pytest.raises(FileNotFoundError):
        read_snapshot(tmp_path / "missing")
    assert not any(name.endswith(tuple(f".tmp.{os.getpid()}")) for name in os.listdir(tmp_path / "size"))


def test_opq_quantizer_is_serdes_optimized_variant(tmp_path):
    # opq.rs:29-41: Quantizer::Optimized { dimension, num_codebooks,
    # codebook_size (as configured), rotation (row-major or null), pq }
    a = _arrays(seed=8)
    rng = np.random.default_rng(2)
    q, r = np.linalg.qr(rng.standard_normal((a["d"], a["d"])))
    rot = (q * np.sign(np.diag(r))).astype(np.float32)
    params = {"num_clusters": a["L"], "nprobe": 2, "num_codebooks": a["M"], "codebook_size": 32,
              "use_opq": True, "seed": 1}
    _write(tmp_path, a, params=params, rotation=rot)
    man = json.loads((tmp_path / "manifest.json").read_text())
    opt = man["quantizer"]["Optimized"]
    assert list(opt) == ["dimension", "num_codebooks", "codebook_size", "rotation", "pq"]
    assert opt["codebook_size"] == 32 and opt["pq"]["codebook_size"] == a["K"]
    assert list(opt["pq"]) == ["dimension", "num_codebooks", "codebook_size", "subvector_dim",
                               "codebooks"]
    s = read_snapshot(tmp_path)
    assert s["rotation"].tobytes() == rot.tobytes()
    assert s["codebooks"].tobytes() == a["codebooks"].tobytes()
    assert s["params"]["use_opq"] is True
    # a Product snapshot has no rotation; an Optimized one may hold null
    opt["rotation"] = None
    (tmp_path / "manifest.json").write_text(json.dumps(man))
    assert read_snapshot(tmp_path)["rotation"] is None
    opt["rotation"] = [0.0] * 5
    (tmp_path / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(SnapshotFormatError, match="dimension x dimension"):
        read_snapshot(tmp_path)
    _write(tmp_path / "plain", a)
    assert read_snapshot(tmp_path / "plain")["rotation"] is None


def _crc32_bitwise(data: bytes) -> int:
    """checksum_file (src/persistence/generation.rs:451-470) restated bit by
    bit: reflected polynomial 0xEDB88320, initial and final inversion."""
    crc = 0xFFFFFFFF
    for byte in data:
        crc ^= byte
        for _ in range(8):
            crc = (crc >> 1) ^ (0xEDB88320 & (-(crc & 1) & 0xFFFFFFFF))
    return crc ^ 0xFFFFFFFF


def test_crc32_of_the_inventory_is_the_references():
    import zlib

    assert _crc32_bitwise(b"123456789") == 0xCBF43926  # the CRC-32 check value
    rng = np.random.default_rng(4)
    for n in (0, 1, 7, 300):
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert zlib.crc32(data) == _crc32_bitwise(data)


def test_generation_publication_layout(tmp_path):
    """GenerationWriter (generation.rs:36-140): CURRENT names the published
    generation, whose manifest lists its components (manifest.rs:64-77) and
    whose GENERATION.json holds each other file's length and CRC-32, sorted
    by path (serde's pretty JSON); a second publication replaces CURRENT and
    keeps the first generation."""
    from vicinity_amd.snapshot import open_current, publish_generation

    a = _arrays(seed=3)
    root = tmp_path / "root"
    g1 = publish_generation(root, lambda d: _write(d, a, generation_components=True))
    cur = (root / "CURRENT").read_text()
    assert cur.endswith("\n") and os.path.join(root, "generations", cur.strip()) == g1
    assert open_current(root) == g1
    man = json.loads(open(os.path.join(g1, "manifest.json")).read())
    assert man["generation_components"] == ["centroids.bin", "clusters.bin", "codes.bin", "doc_ids.bin",
                                             "list_codes.bin", "list_offsets.bin", "raw_vectors.bin"]
    inv_text = open(os.path.join(g1, "GENERATION.json")).read()
    inv = json.loads(inv_text)
    assert inv_text == json.dumps(inv, indent=2)
    assert inv["version"] == 1
    names = sorted(f for f in os.listdir(g1) if f != "GENERATION.json")
    assert [e["path"] for e in inv["files"]] == names
    for e in inv["files"]:
        data = open(os.path.join(g1, e["path"]), "rb").read()
        assert e["length"] == len(data) and e["crc32"] == _crc32_bitwise(data), e["path"]
    assert not [f for f in os.listdir(root / "generations") if f.startswith(".staging")]
    snap = read_snapshot(open_current(root))
    assert np.array_equal(snap["codes"], a["codes"])
    g2 = publish_generation(root, lambda d: _write(d, _arrays(seed=5), generation_components=True))
    assert open_current(root) == g2 != g1 and os.path.isdir(g1)


def test_generation_publication_refusals(tmp_path):
    """A contended publication lock and a CURRENT replaced while the
    generation was staged are errors that leave CURRENT as it was
    (generation.rs:142-188); a manifest whose component list disagrees with
    its files is refused on load (manifest.rs:79-98)."""
    import fcntl

    from vicinity_amd.snapshot import publish_generation

    a = _arrays(seed=6)
    root = tmp_path / "root"
    g1 = publish_generation(root, lambda d: _write(d, a, generation_components=True))
    cur = (root / "CURRENT").read_text()
    with open(root / ".PUBLISH.lock", "a") as held:
        fcntl.flock(held.fileno(), fcntl.LOCK_EX)
        with pytest.raises(SnapshotFormatError, match="advisory lock"):
            publish_generation(root, lambda d: _write(d, a, generation_components=True))
        fcntl.flock(held.fileno(), fcntl.LOCK_UN)
    assert (root / "CURRENT").read_text() == cur

    def racing_writer(d):
        _write(d, a, generation_components=True)
        (root / "CURRENT").write_text("someone-else\n")

    with pytest.raises(SnapshotFormatError, match="CURRENT changed"):
        publish_generation(root, racing_writer)
    man_path = os.path.join(g1, "manifest.json")
    man = json.loads(open(man_path).read())
    man["generation_components"] = man["generation_components"][:-1]
    open(man_path, "w").write(json.dumps(man, indent=2))
    with pytest.raises(SnapshotFormatError, match="component inventory mismatch"):
        read_snapshot(g1)
