"""The CPU code that parses files or indexes buffers, under AddressSanitizer and
UndefinedBehaviorSanitizer (host-only builds; no GPU code is instrumented):

* the oracle (oracle/san_check.c drives every function on small sets, the empty set, a lone
  voxel at the end of the coordinate range and duplicates, and cross-checks the results);
* the GGUF and .npy readers of the host side (tests/host/san_parsers.cpp) over valid files and
  corrupted ones: every truncation point of a small file, a length or count field set to huge
  values, and random byte flips. A valid file must load, a truncated one must be rejected, and no
  file may make the sanitizers report anything (out-of-bounds access, leak, overflow)."""
from __future__ import annotations

import os
import struct
import subprocess

import numpy as np
import pytest

from trellis_cpp_amd.gguf_writer import write as write_gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "trellis.cpp_amd", "host")
SAN_ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=86",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=87")


def _make(d, target):
    r = subprocess.run(["make", "-s", "-C", d, target], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]


def _clean(r):
    text = r.stdout + r.stderr
    assert "AddressSanitizer" not in text and "runtime error" not in text and "LeakSanitizer" not in text, text[-4000:]
    assert r.returncode == 0, text[-4000:]


def test_oracle_under_sanitizers():
    _make(os.path.join(ROOT, "oracle"), "sanitize")
    r = subprocess.run([os.path.join(ROOT, "oracle", "_san", "san_check")], capture_output=True, text=True,
                       errors="replace", timeout=300, env=dict(SAN_ENV, OMP_NUM_THREADS="1"))
    _clean(r)
    assert "san_check: ok" in r.stdout


@pytest.fixture(scope="module")
def san_parsers():
    if not os.path.exists(os.path.join(HOST, "libtrellis_host.so")):
        pytest.fail("libtrellis_host.so is not built")
    _make(HOST, "sanitize")
    return os.path.join(HOST, "_san", "san_parsers")


def _run(tool, kind, paths):
    r = subprocess.run([tool, kind, *paths], capture_output=True, text=True, errors="replace", timeout=600,
                       env=SAN_ENV)
    _clean(r)
    res = {}
    for line in r.stdout.splitlines():        # "ok <path> (...)" or "reject <path>[: why]"
        status, path = line.split(" ", 2)[:2]
        res[path.rstrip(":")] = status
    return res


def _mutations(blob, rng, fields):
    """Corrupt copies of blob: each truncation, each u64 field at `fields` set to huge values,
    and random byte flips."""
    out = [blob[:k] for k in range(0, len(blob), max(1, len(blob) // 97))]
    for off in fields:
        for v in (2 ** 63 - 1, 2 ** 40, 2 ** 32 + 5, 2 ** 31 - 1):
            out.append(blob[:off] + struct.pack("<Q", v) + blob[off + 8:])
    for _ in range(60):
        b = bytearray(blob)
        for _ in range(rng.integers(1, 6)):
            b[rng.integers(0, len(b))] = rng.integers(0, 256)
        out.append(bytes(b))
    return out


def test_gguf_reader_under_sanitizers(san_parsers, tmp_path):
    rng = np.random.default_rng(3)
    good = str(tmp_path / "good.gguf")
    write_gguf(good, {"blocks.0.0.conv.weight": rng.standard_normal((4, 27, 3)).astype(np.float32),
                      "blocks.0.0.conv.bias": rng.standard_normal(4).astype(np.float32),
                      "x.bf16": rng.standard_normal((2, 5)).astype(np.float32)},
               {"x.bf16": "bf16"}, arch="trellis2-shape-dec", config_json='{"a": [1, 2]}')
    blob = open(good, "rb").read()
    # u64 fields: n_tensors (8), n_kv (16), the first key's length (24)
    paths, trunc = [good], []
    for i, m in enumerate(_mutations(blob, rng, (8, 16, 24))):
        p = str(tmp_path / f"m{i}.gguf")
        open(p, "wb").write(m)
        paths.append(p)
        if i < len(range(0, len(blob), max(1, len(blob) // 97))) and len(m) < 100:
            trunc.append(p)
    res = _run(san_parsers, "gguf", paths)
    assert res[good] == "ok"
    assert all(res[p] == "reject" for p in trunc)


def test_npy_reader_under_sanitizers(san_parsers, tmp_path):
    rng = np.random.default_rng(4)
    paths, good = [], []
    for name, a in (("f", rng.standard_normal((7, 5)).astype(np.float32)), ("i", np.arange(12, dtype=np.int32)),
                    ("u", (rng.random(40) < 0.5).astype(np.uint8)), ("e", np.zeros((0, 3), np.float32))):
        p = str(tmp_path / f"{name}.npy")
        np.save(p, a)
        good.append(p)
    blob = open(good[0], "rb").read()
    hdr = blob[:blob.index(b"\n") + 1]
    paths += good
    for i, m in enumerate(_mutations(blob, rng, ())):
        p = str(tmp_path / f"m{i}.npy")
        open(p, "wb").write(m)
        paths.append(p)
    # headers with bad shapes, descr and lengths
    for i, h in enumerate([b"{'descr': '<f4', 'fortran_order': False, 'shape': (-3, 5), }",
                           b"{'descr': '<f4', 'fortran_order': False, 'shape': (99999999999, 99999999999), }",
                           b"{'descr': '<f4', 'fortran_order': False, 'shape': (x), }",
                           b"{'descr': '<f8', 'fortran_order': False, 'shape': (2,), }",
                           b"{'descr: '<f4', 'fortran_order': False, 'shape': (2,), }",
                           b"{'descr': '<f4', 'fortran_order': True, 'shape': (2,), }",
                           b"{'descr'"]):
        p = str(tmp_path / f"h{i}.npy")
        open(p, "wb").write(b"\x93NUMPY\x01\x00" + struct.pack("<H", len(h)) + h + b"\0" * 16)
        paths.append(p)
    p = str(tmp_path / "hlen.npy")
    open(p, "wb").write(b"\x93NUMPY\x02\x00" + struct.pack("<I", 2 ** 31) + hdr[10:])
    paths.append(p)
    res = _run(san_parsers, "npy", paths)
    assert all(res[g] == "ok" for g in good)
    assert all(res[str(tmp_path / f"h{i}.npy")] == "reject" for i in range(7))
    assert res[p] == "reject"
