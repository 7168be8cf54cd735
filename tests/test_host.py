"""CPU tests of the C++ host side (trellis.cpp_amd/host): its GGUF reader against files the test
writer produces, its host fp16 conversion against numpy, the symbols it exports, and -- where the
reference checkout is present -- that the reference's own callers of the sparse path compile
unchanged against its headers and link against its libraries."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from trellis_cpp_amd.gguf_writer import write as write_gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "trellis.cpp_amd", "host")
HOST_LIB = os.path.join(HOST, "libtrellis_host.so")
REF = "/root/reference"


def _need(path):
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (run __graft_entry__.build())")


def test_gguf_reader(tmp_path):
    _need(os.path.join(HOST, "bin", "gguf_dump"))
    rng = np.random.default_rng(0)
    tensors = {"blocks.0.0.conv.weight": rng.standard_normal((8, 27, 5)).astype(np.float32),
               "blocks.0.0.conv.bias": rng.standard_normal(8).astype(np.float32),
               "a.bf16": rng.standard_normal((3, 7)).astype(np.float32),
               "idx": np.arange(11, dtype=np.int32)}
    dtypes = {"a.bf16": "bf16", "idx": "i32"}
    path = str(tmp_path / "m.gguf")
    write_gguf(path, tensors, dtypes, arch="unit-arch", config_json='{"k": 1}')
    out = subprocess.run([os.path.join(HOST, "bin", "gguf_dump"), path], capture_output=True,
                         text=True, check=True, timeout=60).stdout.splitlines()
    assert out[0] == "arch unit-arch" and out[1] == 'config {"k": 1}'
    data_off = int(out[2].split()[1])
    assert data_off % 32 == 0
    blob = open(path, "rb").read()
    rows = [l.split() for l in out[3:]]
    assert [r[0] for r in rows] == list(tensors)
    types = {"f32": 0, "f16": 1, "bf16": 30, "i32": 26}
    for (name, t, ne, off, nbytes), (key, a) in zip(rows, tensors.items()):
        dt = dtypes.get(key, "f16" if a.ndim >= 2 else "f32")
        assert int(t) == types[dt]
        assert [int(v) for v in ne.split(",")] == list(reversed(a.shape)) + [1] * (4 - a.ndim)
        raw = blob[data_off + int(off): data_off + int(off) + int(nbytes)]
        if dt == "f16":
            assert np.array_equal(np.frombuffer(raw, np.float16), a.astype(np.float16).ravel())
        elif dt == "f32":
            assert np.array_equal(np.frombuffer(raw, np.float32), a.ravel())
        elif dt == "i32":
            assert np.array_equal(np.frombuffer(raw, np.int32), a.ravel())
        else:
            assert len(raw) == a.size * 2


def test_gguf_reader_rejects_bad_files(tmp_path):
    _need(os.path.join(HOST, "bin", "gguf_dump"))
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + b"\0" * 60)
    r = subprocess.run([os.path.join(HOST, "bin", "gguf_dump"), str(bad)], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode != 0 and "not a GGUF file" in r.stderr
    path = str(tmp_path / "trunc.gguf")
    write_gguf(path, {"w": np.ones((4, 4), np.float32)})
    data = open(path, "rb").read()
    (tmp_path / "trunc.gguf").write_bytes(data[:40])
    r = subprocess.run([os.path.join(HOST, "bin", "gguf_dump"), path], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode != 0


def test_host_fp16_conversion():
    """ggml_fp32_to_fp16 / ggml_fp16_to_fp32 (round to nearest even) against numpy on every
    half and on floats around the rounding boundaries, subnormals, overflow, inf and NaN."""
    _need(HOST_LIB)
    L = ctypes.CDLL(HOST_LIB)
    L.ggml_fp16_to_fp32_row.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    L.ggml_fp32_to_fp16_row.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = np.empty(65536, np.float32)
    L.ggml_fp16_to_fp32_row(h.ctypes.data, f.ctypes.data, h.size)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(f), nan)
    assert np.array_equal(f[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    rng = np.random.default_rng(1)
    mids = (ref[~nan][:-1].astype(np.float64) + ref[~nan][1:].astype(np.float64)) / 2
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 1000,
        (rng.standard_normal(100000) * 1e-6).astype(np.float32),
        mids[np.isfinite(mids)].astype(np.float32),
        np.array([65504, 65519.99, 65520, 70000, np.inf, -np.inf, 2 ** -25, 2 ** -24, 3e-8, 0.0,
                  -0.0], np.float32)])
    y = np.empty(x.size, np.uint16)
    L.ggml_fp32_to_fp16_row(x.ctypes.data, y.ctypes.data, x.size)
    with np.errstate(over="ignore"):
        assert np.array_equal(y, x.astype(np.float16).view(np.uint16))
    y1 = np.empty(1, np.uint16)
    L.ggml_fp32_to_fp16_row(np.array([np.nan], np.float32).ctypes.data, y1.ctypes.data, 1)
    assert np.isnan(y1.view(np.float16)[0])


def _header_decls():
    names = set()
    for h in ("ggml.h", "ggml-backend.h", "ggml-alloc.h", "gguf.h"):
        text = re.sub(r"/\*.*?\*/", "", open(os.path.join(HOST, "include", h)).read(), flags=re.S)
        names |= set(re.findall(r"\b((?:ggml|gguf)_[a-z0-9_]+)\s*\(", text))
    return names


def test_host_library_exports():
    _need(HOST_LIB)
    out = subprocess.run(["nm", "-D", "-C", "--defined-only", HOST_LIB], capture_output=True,
                         text=True, check=True).stdout
    for fn in _header_decls():
        assert re.search(rf"\b{fn}\b", out), fn
    for sym in ("trellis::build_neighbor_table(", "trellis::sparse_submconv(",
                "trellis::sparse_convnext(", "trellis::sparse_c2s(", "trellis::Model::load(",
                "trellis::Model::get(", "trellis::Model::try_get(", "trellis::Model::free()",
                "trellis::tensor_to_f32(", "trellis::g_sparse_cast_f32"):
        assert sym in out, sym


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")),
                    reason="the reference checkout is not present")
@pytest.mark.parametrize("src", ["shape_decoder.cpp", "test_sparse_conv.cpp", "test_c2s.cpp",
                                 "test_bigop.cpp"])
def test_reference_callers_compile_and_link_against_the_shim(src, tmp_path):
    """The reference's callers of the sparse path compile unchanged against this build's
    sparse.h, trellis_model.h and ggml-compatible headers and link against libtrellis_host.so
    (and through it libtrellis_sparse.so): the programs with a main() into executables, the
    decoder into a shared object with no undefined symbol left. Nothing is run."""
    lib_dir = os.path.join(ROOT, "trellis.cpp_amd", "host")
    if not os.path.exists(os.path.join(lib_dir, "libtrellis_host.so")):
        pytest.fail("libtrellis_host.so is not built")
    out = str(tmp_path / os.path.splitext(src)[0])
    shared = ["-shared", "-fPIC", "-Wl,--no-undefined"] if src == "shape_decoder.cpp" else []
    r = subprocess.run(["g++", "-std=c++17", *shared, "-I", os.path.join(HOST, "include"),
                        "-I", os.path.join(REF, "include"), os.path.join(REF, "src", src), "-o", out,
                        "-L", lib_dir, "-ltrellis_host",
                        "-Wl,-rpath-link," + os.path.join(ROOT, "trellis.cpp_amd") + ":/opt/rocm/lib"],
                       capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-3000:]
    assert os.path.getsize(out) > 0
