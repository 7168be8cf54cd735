"""CPU oracle for the sparse submanifold conv path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module. It is the checker the HIP library is compared against, never the thing that is
measured or shipped.

Integer / index work and the conv itself run in the C restatement (liboracle.so, built
from oracle.c by oracle/Makefile); the per-voxel block arithmetic (LayerNorm, SiLU,
linear layers) is restated here in numpy float64.

Layouts match the reference: coords int32 [N,3] (x,y,z); feats [N,C] row-major
(= ggml [C,N]); nbr int32 [27*N] tap-major with sentinel N (sparse.h:14-16);
conv weight [Co,27,Ci] (= ggml [Ci,27,Co], convert.py:143-146); bias [Co].
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


def build() -> str:
    """Compile liboracle.so with oracle/Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_neighbor_table_hash.argtypes = [_i32p, ctypes.c_int64, _i32p]
        L.orc_neighbor_table_hash.restype = ctypes.c_int
        L.orc_neighbor_table_grid.argtypes = [_i32p, ctypes.c_int64, _i32p, ctypes.c_int64]
        L.orc_neighbor_table_grid.restype = ctypes.c_int
        L.orc_count_pairs.argtypes = [_i32p, ctypes.c_int64]
        L.orc_count_pairs.restype = ctypes.c_int64
        L.orc_subm_conv_f32.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _i32p, _f32p, _f32p,
                                        ctypes.c_int, _f32p, ctypes.c_int]
        L.orc_subm_conv_f32.restype = None
        L.orc_subm_conv_f32_rows.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _i32p, _f32p,
                                             _f32p, ctypes.c_int, _f32p, ctypes.c_int64,
                                             ctypes.c_int64, ctypes.c_int]
        L.orc_subm_conv_f32_rows.restype = None
        L.orc_subm_conv_f64.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _i32p, _f32p, _f32p,
                                        ctypes.c_int, _f64p, ctypes.c_int, ctypes.c_int]
        L.orc_subm_conv_f64.restype = None
        L.orc_subm_conv_f64_rows.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _i32p, _f32p,
                                             _f32p, ctypes.c_int, _f64p,
                                             np.ctypeslib.ndpointer(dtype=np.int64,
                                                                    flags="C_CONTIGUOUS"),
                                             ctypes.c_int64, ctypes.c_int, ctypes.c_int]
        L.orc_subm_conv_f64_rows.restype = None
        L.orc_subdivide.argtypes = [_u8p, _i32p, ctypes.c_int64, _i32p, _i32p, _i32p]
        L.orc_subdivide.restype = ctypes.c_int64
        _lib = L
    return _lib


def _coords(coords) -> np.ndarray:
    c = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 3)
    return c


# ----------------------------------------------------------------------------------------
# Rulebook (sparse.cpp:21-39)
# ----------------------------------------------------------------------------------------
def neighbor_table(coords) -> np.ndarray:
    """Tap-major int32 [27*N] table via the hash-map restatement of build_neighbor_table."""
    c = _coords(coords)
    n = c.shape[0]
    out = np.empty(27 * n, np.int32)
    if lib().orc_neighbor_table_hash(c, n, out) != 0:
        raise ValueError("coordinates outside [-2^20, 2^20)")
    return out


def neighbor_table_grid(coords, max_cells: int = 1 << 31) -> np.ndarray:
    """The same table by brute force on a dense occupancy grid (independent check)."""
    c = _coords(coords)
    n = c.shape[0]
    out = np.empty(27 * n, np.int32)
    if lib().orc_neighbor_table_grid(c, n, out, max_cells) != 0:
        raise ValueError("bounding box too large for the dense-grid brute force")
    return out


def neighbor_table_sorted(coords) -> np.ndarray:
    """A third, vectorised statement: binary search of packed keys (max row wins on ties)."""
    c = _coords(coords).astype(np.int64)
    n = c.shape[0]
    out = np.full((27, n), n, np.int32)
    if n == 0:
        return out.reshape(-1)
    lo = c.min(0) - 1
    span = c.max(0) - lo + 2
    key = lambda p: ((p[:, 0] - lo[0]) * span[1] + (p[:, 1] - lo[1])) * span[2] + (p[:, 2] - lo[2])
    k = key(c)
    # stable sort by key; for duplicate keys the last occurrence (largest row) is the one kept
    order = np.lexsort((np.arange(n), k))
    ks = k[order]
    last = np.ones(n, bool)
    last[:-1] = ks[1:] != ks[:-1]
    ks, rows = ks[last], order[last]
    for t in range(27):
        off = np.array([t // 9 - 1, (t // 3) % 3 - 1, t % 3 - 1])
        q = key(c + off)
        pos = np.minimum(np.searchsorted(ks, q), len(ks) - 1)
        hit = ks[pos] == q
        out[t, hit] = rows[pos[hit]]
    return out.reshape(-1)


def count_pairs(nbr, n: int) -> int:
    nb = np.ascontiguousarray(nbr, dtype=np.int32)
    return int(lib().orc_count_pairs(nb, n))


# ----------------------------------------------------------------------------------------
# Submanifold conv (sparse.cpp:61-92)
# ----------------------------------------------------------------------------------------
def subm_conv_f32(feats, nbr, weight, bias, threads: int = 0) -> np.ndarray:
    """fp32, 27 taps in tap order against the zero sentinel row, bias last (sparse.cpp:64-79)."""
    f = np.ascontiguousarray(feats, dtype=np.float32)
    n, ci = f.shape
    w = np.ascontiguousarray(weight, dtype=np.float32)
    co = w.shape[0]
    assert w.shape == (co, 27, ci)
    b = np.ascontiguousarray(bias, dtype=np.float32).reshape(co)
    nb = np.ascontiguousarray(nbr, dtype=np.int32).reshape(27 * n)
    out = np.empty((n, co), np.float32)
    lib().orc_subm_conv_f32(f, n, ci, nb, w, b, co, out, threads)
    return out


def subm_conv_f32_rows(feats, nbr, weight, bias, r0: int, r1: int, threads: int = 0) -> np.ndarray:
    f = np.ascontiguousarray(feats, dtype=np.float32)
    n, ci = f.shape
    w = np.ascontiguousarray(weight, dtype=np.float32)
    co = w.shape[0]
    b = np.ascontiguousarray(bias, dtype=np.float32).reshape(co)
    nb = np.ascontiguousarray(nbr, dtype=np.int32).reshape(27 * n)
    out = np.zeros((n, co), np.float32)
    lib().orc_subm_conv_f32_rows(f, n, ci, nb, w, b, co, out, r0, r1, threads)
    return out


def _pad_mode(zero_pad: bool, row0) -> bool:
    """Whether the padding row is an exact zero row. row0: the float32 row 0 that 16-bit-rounded
    feats came from (the reference pads before ggml's mul_mat rounds, sparse.cpp:74, 81-85). A
    finite row0 gives a zero padding row even where its rounding overflows to Inf; a non-finite
    channel of row0 stays non-finite in the rounded row, and any NaN channel of the padding row
    makes every output channel of the rows that read it NaN, so the rounded row then stands for
    row0."""
    if zero_pad or row0 is None:
        return zero_pad
    return bool(np.isfinite(np.asarray(row0, np.float32)).all())


def subm_conv_f64(feats, nbr, weight, bias, threads: int = 0, zero_pad: bool = False,
                  row0=None) -> np.ndarray:
    """The same sum in fp64 over active taps only: the tolerance judge. Absent taps read the
    padding row 0 * feats[0] (NaN rows where feats[0] is not finite), or with zero_pad an exact
    zero row (the C2S conv2, sparse.cpp:289-306); row0 as in _pad_mode."""
    zero_pad = _pad_mode(zero_pad, row0)
    f = np.ascontiguousarray(feats, dtype=np.float32)
    n, ci = f.shape
    w = np.ascontiguousarray(weight, dtype=np.float32)
    co = w.shape[0]
    b = np.ascontiguousarray(bias, dtype=np.float32).reshape(co)
    nb = np.ascontiguousarray(nbr, dtype=np.int32).reshape(27 * n)
    out = np.empty((n, co), np.float64)
    lib().orc_subm_conv_f64(f, n, ci, nb, w, b, co, out, threads, 1 if zero_pad else 0)
    return out


def subm_conv_f64_rows(feats, nbr, weight, bias, rows, threads: int = 0,
                      zero_pad: bool = False, row0=None) -> np.ndarray:
    """fp64 conv for the listed output rows only -> [len(rows), Co]."""
    zero_pad = _pad_mode(zero_pad, row0)
    f = np.ascontiguousarray(feats, dtype=np.float32)
    n, ci = f.shape
    w = np.ascontiguousarray(weight, dtype=np.float32)
    co = w.shape[0]
    b = np.ascontiguousarray(bias, dtype=np.float32).reshape(co)
    nb = np.ascontiguousarray(nbr, dtype=np.int32).reshape(27 * n)
    r = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.empty((len(r), co), np.float64)
    lib().orc_subm_conv_f64_rows(f, n, ci, nb, w, b, co, out, r, len(r), threads, 1 if zero_pad else 0)
    return out


def rel_err(mine, ref) -> float:
    """max|d| / max|ref| -- the metric of test_sparse_conv.cpp:16-23."""
    mine = np.asarray(mine, np.float64)
    ref = np.asarray(ref, np.float64)
    g = np.abs(ref).max() if ref.size else 0.0
    d = np.abs(mine - ref).max() if ref.size else 0.0
    return float(d / g) if g > 0 else float(d)


# ----------------------------------------------------------------------------------------
# C2S subdivision index math (sparse.cpp:205-224)
# ----------------------------------------------------------------------------------------
def subdivide(mask, coords):
    """Returns (child_coords [M,3], gidx [M], mstart [N+1]) in parent-major, octant-ascending
    order (sparse.cpp:211-222)."""
    c = _coords(coords)
    n = c.shape[0]
    m8 = np.ascontiguousarray(mask, dtype=np.uint8).reshape(8 * n)
    cc = np.empty((8 * n, 3), np.int32)
    gi = np.empty(8 * n, np.int32)
    ms = np.empty(n + 1, np.int32)
    m = lib().orc_subdivide(m8, c, n, cc, gi, ms)
    return cc[:m].copy(), gi[:m].copy(), ms


def subdivide_vectorised(mask, coords):
    """Independent statement following the upstream SparseChannel2Spatial formulation
    (nonzero + repeat_interleave; docs/spec/22-sparse_conv.md section 5)."""
    c = _coords(coords).astype(np.int64)
    n = c.shape[0]
    sub = np.asarray(mask, np.uint8).reshape(n, 8) != 0
    n_leaf = sub.sum(1)
    parent, subidx = np.nonzero(sub)            # row-major: parent then octant ascending
    child = 2 * c[parent]
    for a in range(3):
        child[:, a] += (subidx >> a) & 1
    mstart = np.zeros(n + 1, np.int64)
    mstart[1:] = np.cumsum(n_leaf)
    return child.astype(np.int32), (parent * 8 + subidx).astype(np.int32), mstart.astype(np.int32)


# ----------------------------------------------------------------------------------------
# Block arithmetic (float64)
# ----------------------------------------------------------------------------------------
def round_f16(x):
    """x rounded to IEEE binary16 (nearest even) by way of float32, as a device rounds a float32
    value; returned as float64."""
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def round_bf16(x):
    """x rounded to bfloat16 (nearest even on the float32 bit pattern; NaN stays NaN); float64."""
    u = np.asarray(x, np.float64).astype(np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).astype(np.float64)
    nan = np.isnan(np.asarray(x, np.float64))
    return np.where(nan, np.nan, out)


def act_round(x, wtype, conv_weight: bool = False, cast_f32: bool = False):
    """The input of a matrix product with weights stored as `wtype` ("f16", "bf16", "f32" or None),
    rounded as ggml's mul_mat rounds it (sparse.cpp:74, 126, 128, 188; shape_decoder.cpp:71): to
    the weights' 16-bit type (the CPU backend's vec_dot type), unchanged for f32 weights. F16 conv
    weights under g_sparse_cast_f32 are cast to f32 first (w32, sparse.cpp:16-19) and leave the
    input unrounded; linear weights are never cast. Returns float64."""
    if wtype == "f16" and not (conv_weight and cast_f32):
        return round_f16(x)
    if wtype == "bf16":
        return round_bf16(x)
    return np.asarray(x, np.float64)


def layer_norm(x, weight=None, bias=None, eps: float = 1e-6):
    """Row LayerNorm over channels with biased variance (ggml_norm, sparse.cpp:124)."""
    x = np.asarray(x, np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if weight is not None:
        y = y * np.asarray(weight, np.float64)
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def silu(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def linear(x, w, b):
    """y = x @ w.T + b with w [out, in] (ggml mul_mat of ne [in, out], sparse.cpp:126)."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T + np.asarray(b, np.float64)


def _rounder(wt, cast_f32):
    """r(x, name, conv): act_round by the stored type of weight `name` (wt: name -> type; None
    rounds nothing)."""
    def r(x, name, conv=False):
        if wt is None:
            return np.asarray(x, np.float64)
        return act_round(x, wt.get(name), conv, cast_f32)
    return r


def convnext_block(feats, nbr, p: dict, prefix: str, wt=None, cast_f32: bool = False):
    """SparseConvNeXtBlock3d (sparse.cpp:102-137): conv -> LN(1e-6)+affine -> mlp.0 -> SiLU
    -> mlp.2 -> + block input. wt (weight name -> stored type) rounds each product's input as
    act_round says; p holds the weights' stored values. Returns float64 [N, C]."""
    r = _rounder(wt, cast_f32)
    x = np.asarray(feats, np.float32)
    xc = r(x, prefix + ".conv.weight", True).astype(np.float32)
    h = subm_conv_f64(xc, nbr, p[prefix + ".conv.weight"], p[prefix + ".conv.bias"], row0=x[0])
    h = layer_norm(h, p[prefix + ".norm.weight"], p[prefix + ".norm.bias"], 1e-6)
    h = linear(r(h, prefix + ".mlp.0.weight"), p[prefix + ".mlp.0.weight"], p[prefix + ".mlp.0.bias"])
    h = silu(h)
    h = linear(r(h, prefix + ".mlp.2.weight"), p[prefix + ".mlp.2.weight"], p[prefix + ".mlp.2.bias"])
    return h + x.astype(np.float64)


def convnext_block_rows(feats, nbr, p: dict, prefix: str, rows, wt=None, cast_f32: bool = False):
    """convnext_block for the listed output rows only -> float64 [len(rows), C]: the conv of those
    rows, then the row-local rest (sparse.cpp:121-135)."""
    r = _rounder(wt, cast_f32)
    x = np.asarray(feats, np.float32)
    rows = np.asarray(rows, np.int64)
    xc = r(x, prefix + ".conv.weight", True).astype(np.float32)
    h = subm_conv_f64_rows(xc, nbr, p[prefix + ".conv.weight"], p[prefix + ".conv.bias"], rows, row0=x[0])
    h = layer_norm(h, p[prefix + ".norm.weight"], p[prefix + ".norm.bias"], 1e-6)
    h = linear(r(h, prefix + ".mlp.0.weight"), p[prefix + ".mlp.0.weight"], p[prefix + ".mlp.0.bias"])
    h = silu(h)
    h = linear(r(h, prefix + ".mlp.2.weight"), p[prefix + ".mlp.2.weight"], p[prefix + ".mlp.2.bias"])
    return h + x[rows].astype(np.float64)


def c2s_block(feats, coords, p: dict, prefix: str, cout: int, ext_mask=None, wt=None,
              cast_f32: bool = False, logits_out=None):
    """SparseResBlockC2S3d (sparse.cpp:172-336). wt rounds each product's input as in
    convnext_block. Returns (out float64 [M,Cout], child_coords [M,3], mask_used uint8 [8N]).
    logits_out (a list), when given, receives the to_subdiv logits [N, 8] of this block's input,
    also where ext_mask decides the mask (for checking a predicted mask against them)."""
    rd = _rounder(wt, cast_f32)
    x = np.asarray(feats, np.float32)
    n, cin = x.shape
    c = _coords(coords)
    logits = None
    if ext_mask is None or logits_out is not None:
        logits = linear(rd(x, prefix + ".to_subdiv.weight"), p[prefix + ".to_subdiv.weight"],
                        p[prefix + ".to_subdiv.bias"])
        if logits_out is not None:
            logits_out.append(logits)
    if ext_mask is None:
        mask = (logits > 0).astype(np.uint8).reshape(-1)        # sparse.cpp:215
    else:
        mask = (np.asarray(ext_mask).reshape(-1) != 0).astype(np.uint8)
    child, gidx, _ = subdivide(mask, c)
    k = cin // 8
    r = cout // k
    nbr = neighbor_table(c)
    h = silu(layer_norm(x, p[prefix + ".norm1.weight"], p[prefix + ".norm1.bias"], 1e-6))
    h = subm_conv_f64(rd(h, prefix + ".conv1.weight", True).astype(np.float32), nbr, p[prefix + ".conv1.weight"],
                      p[prefix + ".conv1.bias"], row0=h[0].astype(np.float32))
    h = h.reshape(n * 8, cout)[gidx]                              # octant gather, :288
    h = silu(layer_norm(h, None, None, 1e-6))                     # norm2 without affine, :293
    nbr2 = neighbor_table(child)
    # conv2 reads hn padded with its zero column M (silu(norm(0)) = 0, :289-306), not 0 * hn[0]
    h = subm_conv_f64(rd(h, prefix + ".conv2.weight", True).astype(np.float32), nbr2, p[prefix + ".conv2.weight"],
                      p[prefix + ".conv2.bias"], zero_pad=True)
    xs = x.reshape(n * 8, k)[gidx].astype(np.float64)             # skip gather, :307
    skip = np.repeat(xs, r, axis=1)                               # repeat_interleave, :322
    return h + skip, child, mask


def decode_unet(latent, coords, p: dict, stages, out_ch: int, guide=None, wt=None,
                cast_f32: bool = False, logits_out=None):
    """SparseUnetVaeDecoder (shape_decoder.cpp:79-117): from_latent -> per stage, its ConvNeXt
    blocks on the stage's table then its C2S block (masks from `guide` when given, else
    predicted) -> LayerNorm(eps 1e-5, no affine, :116) -> output_layer. `stages` lists
    (block prefixes, (c2s prefix, cin, cout)); wt rounds each product's input as in
    convnext_block. The stream between blocks is float32 (ggml's F32 tensors). Returns (out
    float64 [M, out_ch], coords [M,3], masks used per stage). logits_out as in c2s_block, one
    entry per stage."""
    r = _rounder(wt, cast_f32)
    c = _coords(coords)
    h = linear(r(np.asarray(latent, np.float32), "from_latent.weight"), p["from_latent.weight"],
               p["from_latent.bias"])
    masks = []
    for si, (blocks, (c2s, _cin, cout)) in enumerate(stages):
        nbr = neighbor_table(c)
        for b in blocks:
            h = convnext_block(h.astype(np.float32), nbr, p, b, wt, cast_f32)
        h, c, m = c2s_block(h.astype(np.float32), c, p, c2s, cout,
                            None if guide is None else guide[si], wt, cast_f32, logits_out)
        masks.append(m)
    h = layer_norm(h.astype(np.float32), None, None, 1e-5)
    out = linear(r(h, "output_layer.weight"), p["output_layer.weight"], p["output_layer.bias"])
    return out, c, masks


def _lookup(coords):
    """A row lookup for the voxels of coords: returns find(q [K,3]) -> rows [K] (-1 where absent;
    the largest row for duplicated coordinates, as build_neighbor_table keeps the last insert)."""
    c = _coords(coords).astype(np.int64)
    n = c.shape[0]
    key = lambda p: ((p[:, 0] + 1) << 42) | ((p[:, 1] + 1) << 21) | (p[:, 2] + 1)
    k = key(c)
    order = np.lexsort((np.arange(n), k))
    ks = k[order]
    last = np.ones(n, bool)
    last[:-1] = ks[1:] != ks[:-1]
    ks, rows = ks[last], order[last]

    def find(q):
        q = np.asarray(q, np.int64).reshape(-1, 3)
        ok = (q >= 0).all(1)
        kq = key(np.where(ok[:, None], q, 0))
        pos = np.minimum(np.searchsorted(ks, kq), len(ks) - 1) if len(ks) else np.zeros(len(kq), np.int64)
        hit = ok & (len(ks) > 0) & (ks[pos] == kq if len(ks) else False)
        return np.where(hit, rows[pos] if len(ks) else -1, -1)
    return find


def _conv_rows(get, find, coords_rows, weight, bias, pad_row):
    """fp64 submanifold conv of the voxels at coords_rows over the set `find` looks up: bias +
    sum_t W_t . get(neighbour rows) (pad_row where a neighbour is absent) -> [K, Co]."""
    w = np.asarray(weight, np.float64)                      # [Co, 27, Ci]
    q = np.asarray(coords_rows, np.int64).reshape(-1, 3)
    out = np.tile(np.asarray(bias, np.float64), (len(q), 1))
    for t in range(27):
        off = np.array([t // 9 - 1, (t // 3) % 3 - 1, t % 3 - 1])
        r = find(q + off)
        src = np.tile(pad_row[None, :], (len(q), 1))
        if (r >= 0).any():
            src[r >= 0] = get(r[r >= 0])
        out += src @ w[:, t, :].T
    return out


def _compact(n, rows, values):
    """get(r) over a few rows of an n-row array: values[i] is row rows[i]."""
    pos = np.full(n, -1, np.int64)
    pos[rows] = np.arange(len(rows))

    def get(r):
        i = pos[r]
        assert (i >= 0).all(), "row outside the computed set"
        return values[i]
    return get


def c2s_block_rows(feats, coords, p: dict, prefix: str, cout: int, mask, rows, wt=None,
                   cast_f32: bool = False):
    """c2s_block's output for the child rows `rows` only (same arithmetic and rounding, with the
    mask given), for sets too large to run whole: conv2 of each child reads its neighbouring
    children's conv1 octant slices, each from its parent's conv1 row, which reads the parent's
    neighbours' normalised inputs. Returns (out float64 [len(rows), Cout], child_coords [M,3])."""
    rd = _rounder(wt, cast_f32)
    x = np.asarray(feats, np.float32)
    n, cin = x.shape
    c = _coords(coords)
    mask = (np.asarray(mask).reshape(-1) != 0).astype(np.uint8)
    child, gidx, _ = subdivide(mask, c)
    m = len(child)
    rows = np.asarray(rows, np.int64)
    k = cin // 8
    r = cout // k
    offs = [np.array([t // 9 - 1, (t // 3) % 3 - 1, t % 3 - 1]) for t in range(27)]
    find_p, find_c = _lookup(c), _lookup(child)
    # children whose norm2 outputs the sampled rows read, and their parents' conv1 rows
    need = np.stack([find_c(child[rows].astype(np.int64) + o) for o in offs], 1)
    kids = np.unique(need[need >= 0])
    parents = np.unique(gidx[kids] // 8)
    # the normalised inputs of those parents' neighbours (and row 0, the padding row's source)
    near = np.unique(np.concatenate([find_p(c[parents].astype(np.int64) + o) for o in offs] +
                                    [np.zeros(1, np.int64)]))
    near = near[near >= 0]
    hn = silu(layer_norm(x[near], p[prefix + ".norm1.weight"], p[prefix + ".norm1.bias"], 1e-6))
    xin = rd(hn.astype(np.float32), prefix + ".conv1.weight", True)
    pad1 = 0.0 * hn[0].astype(np.float32).astype(np.float64)       # 0 * row 0 (near[0] == 0)
    h1 = _conv_rows(_compact(n, near, xin), find_p, c[parents], p[prefix + ".conv1.weight"],
                    p[prefix + ".conv1.bias"], pad1)
    slot = _compact(n, parents, np.arange(len(parents)))
    g = gidx[kids]
    y = h1[slot(g // 8)[:, None], (g % 8)[:, None] * cout + np.arange(cout)[None, :]]
    y = silu(layer_norm(y, None, None, 1e-6))
    h2 = rd(y.astype(np.float32), prefix + ".conv2.weight", True)
    out = _conv_rows(_compact(m, kids, h2), find_c, child[rows], p[prefix + ".conv2.weight"],
                     p[prefix + ".conv2.bias"], np.zeros(cout))
    xs = x.reshape(n * 8, k)[gidx[rows]].astype(np.float64)
    return out + np.repeat(xs, r, axis=1), child


def decoder_head_rows(h, p: dict, wt=None, cast_f32: bool = False):
    """decode_unet's head on some rows: LayerNorm (eps 1e-5, no affine, shape_decoder.cpp:116),
    then output_layer, its input rounded as the stored weight type says."""
    r = _rounder(wt, cast_f32)
    hn = layer_norm(np.asarray(h, np.float32), None, None, 1e-5)
    return linear(r(hn, "output_layer.weight"), p["output_layer.weight"], p["output_layer.bias"])
