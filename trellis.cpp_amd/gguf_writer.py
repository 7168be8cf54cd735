"""Minimal GGUF v3 writer for synthetic models (the tests' fixtures and the decoder benchmark):
string metadata and F32 / F16 / BF16 / I32 tensors.

The layout is the published GGUF v3 one (magic "GGUF", u32 version, u64 tensor count, u64
key/value count, the key/value table, the tensor table, padding to general.alignment, data).
A numpy array of shape (d0, ..., dk) is stored with ggml dims ne = (dk, ..., d0), so row-major
numpy arrays keep their memory layout: a conv weight [Co, 27, Ci] becomes ggml [Ci, 27, Co]
(the layout tools/convert.py:143-146 writes), a linear weight [out, in] becomes ggml [in, out].
"""
from __future__ import annotations

import struct

import numpy as np

GGML_TYPE = {"f32": 0, "f16": 1, "i32": 26, "bf16": 30}
_VT_STRING, _VT_U32 = 8, 4
ALIGN = 32


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _bf16_bits(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def write(path: str, tensors: dict, dtypes: dict | None = None, arch: str = "trellis2-shape-dec",
          config_json: str = "{}") -> None:
    """tensors: name -> numpy array; dtypes: name -> "f32" | "f16" | "bf16" | "i32" (default: f16
    for arrays of 2 or more dims, f32 for 1-D, as the reference's converter stores them)."""
    dtypes = dtypes or {}
    kv = [("general.architecture", _VT_STRING, _str(arch)),
          ("trellis.config_json", _VT_STRING, _str(config_json)),
          ("general.alignment", _VT_U32, struct.pack("<I", ALIGN))]
    infos, blobs, off = [], [], 0
    for name, a in tensors.items():
        a = np.asarray(a)
        dt = dtypes.get(name, "f16" if a.ndim >= 2 else "f32")
        if dt == "f32":
            raw = np.ascontiguousarray(a, np.float32).tobytes()
        elif dt == "f16":
            raw = np.ascontiguousarray(a, np.float16).tobytes()
        elif dt == "bf16":
            raw = _bf16_bits(a).tobytes()
        elif dt == "i32":
            raw = np.ascontiguousarray(a, np.int32).tobytes()
        else:
            raise ValueError(dt)
        ne = list(reversed(a.shape)) or [1]
        infos.append(_str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
                     + struct.pack("<IQ", GGML_TYPE[dt], off))
        blobs.append(raw)
        off += len(raw)
        off = (off + ALIGN - 1) // ALIGN * ALIGN
    head = b"GGUF" + struct.pack("<IQQ", 3, len(infos), len(kv))
    head += b"".join(_str(k) + struct.pack("<I", t) + v for k, t, v in kv)
    head += b"".join(infos)
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * ((-len(head)) % ALIGN))
        for raw in blobs:
            f.write(raw)
            f.write(b"\0" * ((-len(raw)) % ALIGN))
