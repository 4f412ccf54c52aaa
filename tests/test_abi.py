"""CPU-only checks of the C ABI library and the host-side Python mirror
(no compute calls: this container has no GPU)."""

import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vicinity_gpu.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vgpu_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from vicinity_amd import _lib

    lib = _lib.load()
    declared = _declared_symbols()
    assert len(declared) >= 25
    for name in declared:
        assert hasattr(lib, name), name
    # the Python binding types every declared symbol and nothing else
    assert sorted(_lib.SIGNATURES) == declared


def test_library_is_built_for_gfx950():
    from vicinity_amd import LIB_PATH

    blob = open(LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_last_error_is_empty_string_initially():
    from vicinity_amd import _lib

    assert isinstance(_lib.load().vgpu_last_error(), bytes)


def test_default_codebooks_matches_runner_default():
    # python.rs:1145-1150 and test_python.py:499-502
    from vicinity_amd import default_codebooks

    assert default_codebooks(25) == 5
    assert default_codebooks(32) == 8
    assert default_codebooks(7) == 7
    assert default_codebooks(11) == 1


def test_shape_validation_matches_python_binding():
    # python.rs:1152-1179
    from vicinity_amd.ivf_pq import _validate_shape

    _validate_shape(8, 8, 4, 8, 1)
    for args, msg in [((0, 8, 4, 8, 1), "dim"), ((8, 0, 4, 8, 1), "num_clusters"),
                      ((8, 8, 3, 8, 1), "num_codebooks"), ((8, 8, 4, 257, 1), "codebook_size"),
                      ((8, 8, 4, 0, 1), "codebook_size"), ((8, 8, 4, 8, 0), "nprobe")]:
        with pytest.raises(ValueError, match=msg):
            _validate_shape(*args)


def test_struct_layouts_match_header():
    from vicinity_amd import _lib

    assert ctypes.sizeof(_lib.Params) == 5 * 8 + 8
    assert ctypes.sizeof(_lib.Info) == 7 * 8 + 3 * 4 + 4
    # 7 floats, pad, 2 u64, 3 u32, pad, 2 u64 (flushes, appends), 2 u32,
    # ms_table, tail pad
    assert ctypes.sizeof(_lib.Stats) == 7 * 4 + 4 + 2 * 8 + 3 * 4 + 4 + 2 * 8 + 4 + 4 + 4 + 4
    assert _lib.Stats.ms_table.offset == 88


def test_datagen_shapes_and_determinism():
    from vicinity_amd import datagen

    w = datagen.ivfpq_small(n=500, nq=20)
    assert w.base.shape == (500, 32) and w.queries.shape == (20, 32)
    assert w.base.dtype == np.float32
    assert np.array_equal(w.base, datagen.ivfpq_small(n=500, nq=20).base)
    assert (w.base >= 0).all() and (w.base < 1).all()
    f = datagen.ivfpq_1m(n=300, nq=7)
    assert f.base.shape == (300, 128) and (f.base >= 0).all()
    a = datagen.ivfpq_10m_angular(n=200, nq=3)
    assert np.allclose(np.linalg.norm(a.base, axis=1), 1.0, atol=1e-5)
    b = datagen.ivfpq_4bit_rerank(n=100, nq=3)
    assert b.params["codebook_size"] == 16 and b.base.shape[1] == 100


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from vicinity_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(ImportError, match="no CPU fallback"):
        _lib.load()


def test_ctypes_structs_match_the_c_header_field_by_field(tmp_path):
    """Compile a probe against include/vicinity_gpu.h with gcc and compare every
    field offset and struct size with the ctypes mirror."""
    import shutil
    import subprocess

    from vicinity_amd import _lib

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    structs = {"vgpu_ivfpq_params": _lib.Params, "vgpu_ivfpq_info": _lib.Info,
               "vgpu_search_stats": _lib.Stats}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l}
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)


def test_static_archive_links_into_a_c_program(tmp_path):
    """libvicinity_gpu.a (what a Rust build.rs links statically) resolves
    every declared entry point and runs the host-side checks of a C program
    linked against it."""
    import shutil
    import subprocess

    archive = os.path.join(ROOT, "vicinity_amd", "libvicinity_gpu.a")
    assert os.path.exists(archive), "run make -C vicinity_amd/csrc"
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-g", "--defined-only", archive], capture_output=True,
                             text=True, check=True).stdout
        defined = set(re.findall(r" T (vgpu_[a-z0-9_]+)$", out, flags=re.M))
        assert set(_declared_symbols()) <= defined
    exe = str(tmp_path / "link_check")
    subprocess.run(["gcc", "-O1", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "static_link", "link_check.c"), archive,
                    "-L/opt/rocm/lib", "-lamdhip64", "-lstdc++", "-lm", "-lpthread",
                    "-Wl,-rpath,/opt/rocm/lib", "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "static link ok" in r.stdout
