"""CPU tests of the C ABI boundary: the library loads, exports every symbol the header declares
(unmangled, extern "C"), and rejects bad arguments with a status code and a message before any
device work -- no GPU needed."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trellis_sparse.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tsp_[a-z0-9_]+)\s*\(", text)))


def test_header_lists_match(pkg):
    assert header_functions() == sorted(pkg.EXPORTS)


def test_library_exports_every_declared_symbol(pkg):
    L = pkg.lib()
    for name in header_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", pkg.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in header_functions() if n not in exported]
    assert not missing, missing


def test_version_and_error_string(pkg):
    L = pkg.lib()
    assert L.tsp_version() >= 100
    assert isinstance(L.tsp_last_error(), bytes)


FAKE = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails validation first
NULL = ctypes.c_void_p(0)


def _err(pkg):
    return pkg.lib().tsp_last_error().decode()


def test_rulebook_validation(pkg):
    L = pkg.lib()
    assert L.tsp_rulebook_build(FAKE, -1, FAKE, FAKE, 1 << 20, NULL, NULL) == 1
    assert "out of range" in _err(pkg)
    assert L.tsp_rulebook_build(NULL, 0, NULL, NULL, 0, NULL, NULL) == 0       # empty: no-op
    assert L.tsp_rulebook_build(NULL, 10, FAKE, FAKE, 1 << 20, NULL, NULL) == 1
    ws = L.tsp_rulebook_workspace_bytes(1000)
    assert L.tsp_rulebook_build(FAKE, 1000, FAKE, FAKE, ws - 1, NULL, NULL) == 5
    assert "workspace" in _err(pkg)
    assert L.tsp_rulebook_count_pairs(FAKE, -3, FAKE, NULL) == 1
    # the table and the ordered plan in one call: the plan buffer is checked first
    pb = L.tsp_conv_plan_bytes(1000)
    assert L.tsp_rulebook_build_planned(FAKE, -1, FAKE, FAKE, ws, NULL, FAKE, pb, NULL) == 1
    assert L.tsp_rulebook_build_planned(NULL, 0, NULL, NULL, 0, NULL, NULL, 0, NULL) == 0
    assert L.tsp_rulebook_build_planned(FAKE, 1000, FAKE, FAKE, ws, NULL, NULL, pb, NULL) == 1
    assert "null plan" in _err(pkg)
    assert L.tsp_rulebook_build_planned(FAKE, 1000, FAKE, FAKE, ws, NULL, FAKE, pb - 1, NULL) == 5
    assert "plan buffer" in _err(pkg)
    assert L.tsp_rulebook_build_planned(FAKE, 1000, FAKE, FAKE, ws - 1, NULL, FAKE, pb, NULL) == 5
    assert "workspace" in _err(pkg)


def test_workspace_sizes(pkg):
    L = pkg.lib()
    prev = 0
    for n in (0, 1, 1000, 10**5, 10**6, 4 * 10**6):
        b = L.tsp_rulebook_workspace_bytes(n)
        assert b >= 12 * 2 * n and b >= prev
        prev = b
    assert L.tsp_subdivide_workspace_bytes(10**6) >= 4 * (10**6 // 1024)


def test_conv_validation(pkg):
    L = pkg.lib()
    f = lambda **kw: L.tsp_subm_conv3x3(
        kw.get("feats", FAKE), kw.get("fdt", 2), kw.get("n", 100), kw.get("ci", 64),
        kw.get("nbr", FAKE), kw.get("w", FAKE), kw.get("wdt", 2), kw.get("bias", FAKE),
        kw.get("co", 64), kw.get("out", ctypes.c_void_p(0x2000)), kw.get("odt", 0),
        kw.get("algo", 0), NULL)
    assert f(n=-1) == 1
    assert f(ci=0) == 1 and f(co=-4) == 1
    assert f(fdt=7) == 1 and f(odt=9) == 1
    assert f(algo=7) == 1
    assert f(algo=5) == 4 and "thin matrix-core" in _err(pkg)     # THIN_MFMA: ci=64 is not its shape
    assert f(algo=6) == 4 and "fp32 matrix-core" in _err(pkg)     # F32_MFMA: bf16 feats
    assert f(algo=6, fdt=0, wdt=2) == 4                             # f32 feats, bf16 weights
    assert f(algo=6, fdt=0, wdt=0, ci=40) == 4                      # ci % 16 != 0
    assert f(algo=6, fdt=0, wdt=0, co=48) == 4                      # co % 32 != 0
    assert f(nbr=NULL) == 1
    assert f(out=FAKE) == 1 and "alias" in _err(pkg)
    assert f(n=0) == 0                                              # empty: no-op
    assert f(algo=1, ci=48) == 4 and "MFMA" in _err(pkg)            # ci % 32 != 0
    assert f(algo=1, fdt=0, wdt=0) == 4                             # fp32 has no MFMA path here
    assert f(algo=1, co=96) == 4                                    # co % 64 != 0


def test_plan_and_pack_validation(pkg):
    L = pkg.lib()
    assert L.tsp_conv_plan_build(FAKE, -1, FAKE, 1 << 30, NULL) == 1
    assert L.tsp_conv_plan_build(NULL, 0, NULL, 0, NULL) == 0
    pb = L.tsp_conv_plan_bytes(100000)
    assert pb > 27 * 2 * 100000
    assert L.tsp_conv_plan_build(FAKE, 100000, FAKE, pb - 1, NULL) == 5
    assert L.tsp_conv_weight_pack(FAKE, 0, 64, 64, ctypes.c_void_p(0x2000), NULL) == 4   # f32
    assert L.tsp_conv_weight_pack(FAKE, 2, 40, 64, ctypes.c_void_p(0x2000), NULL) == 4   # ci%16
    assert L.tsp_conv_weight_pack(FAKE, 2, 64, 48, ctypes.c_void_p(0x2000), NULL) == 4   # co%32
    assert L.tsp_conv_weight_pack(FAKE, 2, 64, 64, FAKE, NULL) == 1                      # aliased
    # the packed values, then the 256-byte trailer (the non-finite flag)
    assert L.tsp_conv_weight_packed_bytes(64, 128) == 27 * 64 * 128 * 2 + 256
    assert L.tsp_conv_weight_packed_bytes(0, 64) == 0 and L.tsp_conv_weight_packed_bytes(64, -1) == 0
    p = lambda **kw: L.tsp_subm_conv3x3_planned(
        kw.get("feats", FAKE), kw.get("dt", 2), kw.get("n", 100), kw.get("ci", 64), FAKE,
        FAKE, FAKE, FAKE, kw.get("co", 64), kw.get("out", ctypes.c_void_p(0x2000)),
        kw.get("odt", 0), NULL)
    assert p(dt=0) == 4 and p(odt=1) == 4 and p(ci=40) == 4 and p(co=96) == 4
    assert p(n=-5) == 1 and p(out=FAKE) == 1 and p(n=0) == 0


def test_subdivide_validation(pkg):
    L = pkg.lib()
    assert L.tsp_subdivide(FAKE, FAKE, -1, FAKE, FAKE, FAKE, FAKE, FAKE, 64, NULL) == 1
    assert L.tsp_subdivide(FAKE, FAKE, 1 << 29, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 30, NULL) == 1
    ws = L.tsp_subdivide_workspace_bytes(5000)
    assert L.tsp_subdivide(FAKE, FAKE, 5000, FAKE, FAKE, FAKE, FAKE, FAKE, ws - 1, NULL) == 5
    # the allocation-free variant: the same argument checks, no workspace
    assert L.tsp_subdivide_noalloc(FAKE, FAKE, -1, FAKE, FAKE, FAKE, FAKE, NULL) == 1
    assert L.tsp_subdivide_noalloc(FAKE, FAKE, 1 << 28, FAKE, FAKE, FAKE, FAKE, NULL) == 1
    assert "out of range" in _err(pkg)
    assert L.tsp_subdivide_noalloc(NULL, NULL, 10, FAKE, FAKE, FAKE, FAKE, NULL) == 1
    assert L.tsp_subdivide_noalloc(FAKE, FAKE, 10, FAKE, FAKE, FAKE, NULL, NULL) == 1


def test_python_binding_rejects_host_tensors(pkg):
    import torch
    with pytest.raises(ValueError):
        pkg.rulebook_build(torch.zeros((4, 3), dtype=torch.int32))


def test_linear_ex_validation(pkg):
    """tsp_linear_ex: argument checks, and TSP_ERR_UNSUPPORTED (4) -- the caller's cue to fall
    back to tsp_linear -- for f32 inputs, mixed dtypes, widths not a multiple of 8, misalignment
    and a residual with 16-bit output, all before any device work."""
    L = pkg.lib()
    X, W, O, R = (ctypes.c_void_p(a) for a in (0x1000, 0x2000, 0x3000, 0x4000))
    f = lambda **kw: L.tsp_linear_ex(
        kw.get("x", X), kw.get("xdt", 2), kw.get("n", 100), kw.get("ci", 64), kw.get("w", W),
        kw.get("wdt", 2), NULL, kw.get("co", 256), kw.get("act", 0), kw.get("res", NULL),
        kw.get("out", O), kw.get("odt", 2), NULL)
    assert f(n=-1) == 1 and f(act=7) == 1 and f(xdt=9) == 1
    assert f(n=0) == 0                                   # empty: no-op
    assert f(x=NULL) == 1 and f(out=X) == 1              # null / aliased
    assert f(xdt=0, wdt=0, odt=0) == 4                   # f32: not a library GEMM here
    assert f(wdt=1) == 4                                 # mixed 16-bit dtypes
    assert f(ci=36) == 4 and f(co=250) == 4              # widths not multiples of 8
    assert f(x=ctypes.c_void_p(0x1008)) == 4             # misaligned
    assert f(res=R) == 4                                 # residual needs f32 output
    assert f(res=ctypes.c_void_p(0x4004), odt=0) == 1    # misaligned residual
    assert "residual" in _err(pkg)


def test_linear_row_split(pkg):
    """tsp_linear_rows_per_call: the rows tsp_linear / tsp_linear_ex hand hipBLASLt per call. For
    every dtype pair, residual or not, and widths up to 4096 (plus 2^20 and 2^29 to reach the
    one-row and no-row ends), no operand of one call -- x [rows][ci], out [rows][co], the f32
    residual [rows][co] -- spans 2^31 bytes or more; the chunk is a multiple of 256 rows wherever
    256 rows fit, and as large as that allows (one more block of 256 rows would break the bound).
    The chunk walk over n = INT32_MAX - 1 rows covers every row exactly once."""
    L = pkg.lib()
    size = {0: 4, 1: 2, 2: 2}
    limit = 2 ** 31
    widths = [8, 16, 64, 128, 256, 512, 1000, 1024, 2048, 4096, 1 << 20, 1 << 29]
    for xdt in (0, 1, 2):
        for odt in (0, 1, 2):
            for res in (0, 1):
                for ci in widths:
                    for co in widths:
                        rows = L.tsp_linear_rows_per_call(ci, co, xdt, odt, res)
                        row_bytes = max(ci * size[xdt], co * size[odt], co * 4 if res else 0)
                        if row_bytes >= limit:
                            assert rows == 0
                            continue
                        assert rows >= 1
                        assert rows * row_bytes < limit, (ci, co, xdt, odt, res)
                        if rows >= 256:
                            assert rows % 256 == 0 and (rows + 256) * row_bytes >= limit
                        else:
                            assert (rows + 1) * row_bytes >= limit
    assert L.tsp_linear_rows_per_call(0, 64, 2, 2, 0) == 0 and L.tsp_linear_rows_per_call(64, 64, 9, 2, 0) == 0
    # the decoder's widest hidden layer: 2.45 M rows of 4 x 128 f32 channels (2.5 GB) take 3 calls
    rows = L.tsp_linear_rows_per_call(128, 512, 2, 0, 0)
    n = 2_445_586
    assert rows == 1_048_320 and -(-n // rows) == 3
    n = 2 ** 31 - 2
    rows = L.tsp_linear_rows_per_call(4096, 4096, 2, 0, 1)
    covered = sum(min(rows, n - r0) for r0 in range(0, n, rows))
    assert covered == n


def test_planned_octants_validation(pkg):
    """tsp_subm_conv3x3_planned_octants: argument checks before any device work -- range and dtype
    (1 / 4), cout not a multiple of 64 and ci not a multiple of 16 (4), the empty case (0), null,
    aliased and misaligned pointers (1)."""
    L = pkg.lib()
    F, NB, P, W, B, M, S, O = (ctypes.c_void_p(a) for a in
                               (0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 0x7000, 0x8000))
    f = lambda **kw: L.tsp_subm_conv3x3_planned_octants(
        kw.get("f", F), kw.get("dt", 2), kw.get("n", 100), kw.get("ci", 64), kw.get("nbr", NB),
        kw.get("plan", P), kw.get("w", W), kw.get("b", B), kw.get("cout", 64), kw.get("mask", M),
        kw.get("mstart", S), kw.get("out", O), NULL)
    assert f(n=-1) == 1 and f(ci=0) == 1 and f(cout=0) == 1
    assert f(dt=0) == 4                                    # f32 features: not the MFMA kernel
    assert f(cout=96) == 4 and f(ci=40) == 4               # cout % 64, ci % 16
    assert f(n=0) == 0                                     # empty: no-op
    assert f(mask=NULL) == 1 and f(mstart=NULL) == 1 and f(plan=NULL) == 1
    assert f(out=F) == 1                                   # out aliases feats
    assert f(mask=ctypes.c_void_p(0x6004)) == 1            # mask not 8-byte aligned
    assert "aligned" in _err(pkg)


def test_planned_skip_validation(pkg):
    """tsp_subm_conv3x3_planned_skip: argument checks before any device work -- range (1), dtype
    and shape limits (4: f32 features, co % 64, cin % 8, a repeat co / (cin / 8) not a multiple
    of 4), the empty case (0), null and aliased pointers (1)."""
    L = pkg.lib()
    F, NB, P, W, B, X, G, O = (ctypes.c_void_p(a) for a in
                               (0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 0x7000, 0x8000))
    f = lambda **kw: L.tsp_subm_conv3x3_planned_skip(
        kw.get("f", F), kw.get("dt", 2), kw.get("n", 100), kw.get("ci", 64), kw.get("nbr", NB),
        kw.get("plan", P), kw.get("w", W), kw.get("b", B), kw.get("co", 64), kw.get("x", X),
        kw.get("cin", 128), kw.get("gidx", G), kw.get("out", O), NULL)
    assert f(n=-1) == 1 and f(cin=0) == 1 and f(co=0) == 1
    assert f(dt=0) == 4 and f(co=96) == 4                  # f32 features; co % 64
    assert f(cin=12) == 4                                  # cin % 8
    assert f(cin=256) == 4                                 # R = 64 / 32 = 2: not a multiple of 4
    assert f(n=0) == 0                                     # empty: no-op
    assert f(x=NULL) == 1 and f(gidx=NULL) == 1
    assert f(out=X) == 1                                   # out aliases x
    assert "alias" in _err(pkg)


def test_conv_ex_flags_validation(pkg):
    """The *_ex convs: unknown flag bits are rejected (1) before any device work; flags 0 takes
    the same checks as the plain calls."""
    L = pkg.lib()
    O = ctypes.c_void_p(0x2000)
    f = lambda flags, **kw: L.tsp_subm_conv3x3_ex(
        FAKE, 2, kw.get("n", 100), 64, FAKE, FAKE, 2, FAKE, 64, kw.get("out", O), 0, 0, flags,
        kw.get("row0", NULL), NULL)
    assert f(2) == 1 and "flags" in _err(pkg)
    assert f(1, n=0) == 0 and f(0, n=0) == 0 and f(0, n=0, row0=FAKE) == 0
    assert f(1, out=FAKE) == 1 and "alias" in _err(pkg)
    p = lambda flags, **kw: L.tsp_subm_conv3x3_planned_ex(
        FAKE, kw.get("dt", 2), kw.get("n", 100), 64, FAKE, FAKE, FAKE, FAKE, 64, O, 0, flags,
        kw.get("row0", NULL), NULL)
    assert p(4) == 1 and "flags" in _err(pkg)
    assert p(1, dt=0) == 4
    assert p(1, n=0) == 0 and p(0, n=0, row0=FAKE) == 0


def test_python_conv_argument_checks(pkg):
    """The binding checks every buffer the kernels index before any launch: a caller's out (shape,
    dtype, contiguity), the table's size and dtype, the plan's size against tsp_conv_plan_bytes,
    the packed weight's dtype and size. Host tensors reach each check (they run before the device
    check), so the ValueError names the problem."""
    import torch
    n, ci, co = 100, 64, 64
    f = torch.zeros((n, ci), dtype=torch.bfloat16)
    nbr = torch.zeros(27 * n, dtype=torch.int32)
    w = torch.zeros((co, 27, ci), dtype=torch.bfloat16)
    b = torch.zeros(co, dtype=torch.float32)
    with pytest.raises(ValueError, match="shape"):
        pkg.subm_conv3x3(f, nbr, w, b, out=torch.zeros((n - 1, co)))
    with pytest.raises(ValueError, match="must be torch.float32"):
        pkg.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, out=torch.zeros((n, co), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="contiguous"):
        pkg.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, out=torch.zeros((co, n)).t())
    with pytest.raises(ValueError, match="27\\*N"):
        pkg.subm_conv3x3(f, nbr[:-1], w, b)
    with pytest.raises(ValueError, match="27\\*N"):
        pkg.subm_conv3x3(f, nbr.to(torch.int64), w, b)
    plan_ok = torch.zeros(pkg.lib().tsp_conv_plan_bytes(n), dtype=torch.uint8)
    packed = torch.zeros(pkg.lib().tsp_conv_weight_packed_bytes(ci, co) // 2, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="plan holds"):
        pkg.subm_conv3x3_planned(f, nbr, plan_ok[:-1], packed, b, co)
    with pytest.raises(ValueError, match="packed weight is"):
        pkg.subm_conv3x3_planned(f, nbr, plan_ok, packed.to(torch.float16), b, co)
    with pytest.raises(ValueError, match="packed weight size"):
        pkg.subm_conv3x3_planned(f, nbr, plan_ok, packed[:-8], b, co)
    with pytest.raises(ValueError, match="shape"):
        pkg.subm_conv3x3_planned(f, nbr, plan_ok, packed, b, co, out=torch.zeros((n, co + 1)))
    with pytest.raises(ValueError, match="row0"):
        pkg.subm_conv3x3_planned(f, nbr, plan_ok, packed, b, co, row0=torch.zeros(ci - 1))
    with pytest.raises(ValueError, match="GPU"):   # every check passed: only the device is wrong
        pkg.subm_conv3x3_planned(f, nbr, plan_ok, packed, b, co)


def test_composite_validation(pkg):
    """tsp_convnext / tsp_c2s reject bad arguments before any device work: no weights, unknown
    flags, a 16-bit x of another type than the conv input, a short workspace, mismatched plans."""
    L = pkg.lib()
    w = pkg.ConvNextWeights(FAKE, 2, FAKE, None, FAKE, FAKE, FAKE, 2, FAKE, FAKE, 2, FAKE)
    nb = L.tsp_convnext_workspace_bytes(1000, 64, 0, ctypes.byref(w), 1, 0)
    plain = L.tsp_convnext_workspace_bytes(1000, 64, 0, ctypes.byref(w), 0, 0)
    # without a plan: the rounded conv input, the f32 conv output and the norm's output (+ the MLP
    # chunk); with one, the conv and the norm are one kernel (no f32 conv output) and the weights
    # are packed into the workspace
    assert plain >= 1000 * 64 * (2 + 4 + 2) and nb % 256 == 0 and plain % 256 == 0
    a256 = lambda b: (b + 255) // 256 * 256
    assert nb == plain - a256(1000 * 64 * 4) + a256(L.tsp_conv_weight_packed_bytes(64, 64))
    cn = lambda **kw: L.tsp_convnext(FAKE, kw.get("xdt", 0), 1000, 64, FAKE, kw.get("plan", FAKE),
                                     kw.get("w", ctypes.byref(w)), ctypes.c_void_p(0x2000), FAKE,
                                     kw.get("ws", nb), kw.get("flags", 0), NULL)
    assert cn(w=None) == 1
    assert cn(flags=4) == 1 and "flags" in _err(pkg)
    assert cn(xdt=1) == 4                     # f16 x for bf16 conv weights
    assert cn(ws=nb - 1) == 5 and "workspace" in _err(pkg)
    c = pkg.C2SWeights(FAKE, FAKE, FAKE, 2, FAKE, None, FAKE, 2, FAKE, None)
    cb = L.tsp_c2s_workspace_bytes(500, 1200, 128, 64, ctypes.byref(c), 1, 1, 0)
    assert cb > 0
    cs = lambda **kw: L.tsp_c2s(FAKE, 500, kw.get("cin", 128), FAKE, kw.get("plan", FAKE), FAKE, FAKE, FAKE,
                                kw.get("m", 1200), 64, FAKE, kw.get("cplan", FAKE), ctypes.byref(c),
                                ctypes.c_void_p(0x2000), FAKE, kw.get("ws", cb), 0, NULL)
    assert cs(cin=60) == 1                    # Cin % 8
    assert cs(m=4001) == 1                    # M > 8 N
    assert L.tsp_c2s_workspace_bytes(500, 1200, 128, 64, ctypes.byref(c), 1, 0, 0) != cb
    assert cs(ws=cb - 1) == 5
    assert cs(m=0) == 0
    # the rounded copies of the _ex forms: x16 only with f32 x, out16 bf16 or f16, 16-byte aligned,
    # not aliasing the block's other buffers
    cx = lambda **kw: L.tsp_convnext_ex(FAKE, kw.get("xdt", 0), kw.get("x16", None), 1000, 64, FAKE, FAKE,
                                        ctypes.byref(w), ctypes.c_void_p(0x2000), kw.get("o16", None),
                                        kw.get("o16dt", 2), FAKE, nb, 0, NULL)
    assert cx(xdt=2, x16=FAKE) == 1 and "rounded copy of x" in _err(pkg)
    assert cx(o16=ctypes.c_void_p(0x3000), o16dt=0) == 1
    assert cx(x16=ctypes.c_void_p(0x3008)) == 1 and "aligned" in _err(pkg)
    assert cx(o16=ctypes.c_void_p(0x2000)) == 1 and "alias" in _err(pkg)
    cx2 = lambda **kw: L.tsp_c2s_ex(FAKE, 500, 128, FAKE, FAKE, FAKE, FAKE, FAKE, 1200, 64, FAKE, FAKE,
                                    ctypes.byref(c), ctypes.c_void_p(0x2000), kw.get("o16", None),
                                    kw.get("o16dt", 2), FAKE, cb, 0, NULL)
    assert cx2(o16=ctypes.c_void_p(0x3000), o16dt=3) == 1
    assert cx2(o16=ctypes.c_void_p(0x2000)) == 1 and "alias" in _err(pkg)
    # tsp_c2s_part: the part, and a tile range only for the conv2 part
    cp = lambda **kw: L.tsp_c2s_part(FAKE, 500, 128, FAKE, FAKE, FAKE, FAKE, FAKE, 1200, 64, FAKE, FAKE,
                                     ctypes.byref(c), ctypes.c_void_p(0x2000), None, 2, FAKE, kw.get("ws", cb), 0,
                                     kw.get("part", 3), kw.get("t0", 0), kw.get("nt", -1), NULL)
    assert cp(part=0) == 1 and "part" in _err(pkg)
    assert cp(part=4) == 1
    assert cp(part=2, t0=-1) == 1 and cp(part=2, nt=-2) == 1
    assert cp(part=1, t0=3) == 1 and "conv2 part" in _err(pkg)
    assert cp(part=2, t0=1, nt=2, ws=cb - 1) == 5


def test_convnext_mlp_validation(pkg):
    """tsp_convnext_mlp / _pack: C = 128 only (wider blocks keep the library GEMMs), 16-bit dtypes,
    null and misaligned pointers, an output aliasing xn -- all refused before any launch; n = 0
    is a no-op."""
    L = pkg.lib()
    assert L.tsp_convnext_mlp_packed_bytes(128) == 2 * 4 * 128 * 128 * 2
    assert L.tsp_convnext_mlp_pack(FAKE, FAKE, 2, 256, FAKE, NULL) == 4 and "C=256" in _err(pkg)
    assert L.tsp_convnext_mlp_pack(FAKE, FAKE, 0, 128, FAKE, NULL) == 4      # f32 weights
    assert L.tsp_convnext_mlp_pack(FAKE, ctypes.c_void_p(0x1008), 2, 128, FAKE, NULL) == 1
    mlp = lambda **kw: L.tsp_convnext_mlp(kw.get("xn", FAKE), kw.get("dt", 2), kw.get("n", 1000), kw.get("c", 128),
                                          kw.get("packed", FAKE), NULL, NULL, FAKE, kw.get("out", ctypes.c_void_p(0x2000)),
                                          NULL)
    assert mlp(c=256) == 4 and mlp(c=64) == 4
    assert mlp(dt=0) == 4
    assert mlp(n=-1) == 1
    assert mlp(packed=NULL) == 1
    assert mlp(xn=ctypes.c_void_p(0x1008)) == 1 and "aligned" in _err(pkg)
    assert mlp(out=FAKE) == 1 and "alias" in _err(pkg)
    assert mlp(n=0, packed=NULL) == 0
