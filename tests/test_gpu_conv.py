"""GPU parity of the submanifold conv against the oracle.

Tolerance: max|gpu - ref| / max|ref| (the metric of test_sparse_conv.cpp:16-23) <= 1e-3 for
16-bit features with fp32 accumulation, against the fp64 oracle on identical (already
rounded) inputs; fp32 runs are held to 1e-5. bf16/f16 outputs are additionally rounded once,
so they are held to 4e-3 (2^-8 = one bf16 ulp at the largest element)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_16 = 1e-3
TOL_32 = 1e-5
TOL_16_OUT = 4e-3


def _case(name):
    print(f"[conv] {name}", flush=True)


def _dev(a, dtype):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(dtype).cuda()


def _run(pkg, coords, feats, weight, bias, dtype, wdtype=None, out_dtype=None, algo="auto"):
    import torch
    c = torch.from_numpy(np.ascontiguousarray(coords, np.int32)).cuda()
    nbr = pkg.rulebook_build(c)
    f = _dev(feats, dtype)
    w = _dev(weight, wdtype or dtype)
    b = _dev(bias, torch.float32)
    out = pkg.subm_conv3x3(f, nbr, w, b, out_dtype=out_dtype or torch.float32, algo=algo)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), nbr


def test_golden_fp32(gpu_lib, golden):
    _case("conv_rand800_c32 f32")
    import torch
    g = golden("conv_rand800_c32.npz")
    out, _ = _run(gpu_lib, g["coords"], g["feats"], g["weight"], g["bias"], torch.float32)
    assert out.shape == g["out"].shape
    err = float(np.abs(out - g["out"]).max() / np.abs(g["out"]).max())
    assert err < TOL_32, err


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_golden_16bit(gpu_lib, golden, orc, shells, dtype_name):
    _case(f"conv_rand800_c32 {dtype_name}")
    import torch
    dt = getattr(torch, dtype_name)
    g = golden("conv_rand800_c32.npz")
    key = "bf16" if dt == torch.bfloat16 else "f16"
    f, w = shells.round_to(g["feats"], key), shells.round_to(g["weight"], key)
    ref = orc.subm_conv_f64(f, orc.neighbor_table(g["coords"]), w, g["bias"])
    out, _ = _run(gpu_lib, g["coords"], f, w, g["bias"], dt)
    assert orc.rel_err(out, ref) < TOL_16


def _rand_case(shells, rng, n_hint, ci, co, dtype):
    coords = shells.sphere_shell(48, 24.0, 14.0, 16.0)
    coords = coords[:n_hint] if n_hint else coords
    feats = shells.round_to(rng.standard_normal((len(coords), ci)).astype(np.float32), dtype)
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / np.sqrt(27 * ci)).astype(np.float32), dtype)
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    return coords, feats, weight, bias


@pytest.mark.parametrize("ci,co,n", [(64, 64, 0), (128, 128, 0), (256, 256, 3000), (32, 64, 257),
                                     (96, 192, 1000), (128, 320, 511), (64, 128, 1),
                                     (512, 64, 700)])
@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_mfma_vs_oracle(gpu_lib, orc, shells, ci, co, n, dtype_name):
    _case(f"mfma ci={ci} co={co} n={n} {dtype_name}")
    import torch
    dt = getattr(torch, dtype_name)
    key = "bf16" if dt == torch.bfloat16 else "f16"
    rng = np.random.default_rng(ci * 1000 + co + n)
    coords, feats, weight, bias = _rand_case(shells, rng, n, ci, co, key)
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    for algo in ("mfma", "mfma_gather", "narrow"):
        out, _ = _run(gpu_lib, coords, feats, weight, bias, dt, algo=algo)
        assert orc.rel_err(out, ref) < TOL_16, algo


def _run_planned(pkg, coords, feats, weight, bias, dtype, out_dtype=None):
    import torch
    c = torch.from_numpy(np.ascontiguousarray(coords, np.int32)).cuda()
    nbr = pkg.rulebook_build(c)
    plan = pkg.conv_plan_build(nbr, len(coords))
    pw = pkg.conv_weight_pack(_dev(weight, dtype))
    out = pkg.subm_conv3x3_planned(_dev(feats, dtype), nbr, plan, pw, _dev(bias, torch.float32),
                                   weight.shape[0], out_dtype=out_dtype or torch.float32)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("ci,co,n", [(64, 64, 0), (128, 128, 0), (48, 64, 900), (256, 256, 2100),
                                     (32, 192, 513), (16, 128, 1)])
@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_planned_vs_oracle(gpu_lib, orc, shells, ci, co, n, dtype_name):
    _case(f"planned ci={ci} co={co} n={n} {dtype_name}")
    import torch
    dt = getattr(torch, dtype_name)
    key = "bf16" if dt == torch.bfloat16 else "f16"
    rng = np.random.default_rng(ci * 7 + co + n)
    coords, feats, weight, bias = _rand_case(shells, rng, n, ci, co, key)
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    assert orc.rel_err(_run_planned(gpu_lib, coords, feats, weight, bias, dt), ref) < TOL_16
    out16 = _run_planned(gpu_lib, coords, feats, weight, bias, dt, out_dtype=dt)
    assert orc.rel_err(out16, ref) < TOL_16_OUT



@pytest.mark.parametrize("ci,cout,n,keep", [(32, 64, 0, 0.5), (64, 128, 1500, 0.3), (16, 64, 513, 1.0),
                                           (48, 64, 700, 0.0)])
@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_planned_octants(gpu_lib, orc, shells, ci, cout, n, keep, dtype_name):
    """The C2S conv1 with the octant gather in its stores (sparse.cpp:263-291) against the planned
    conv to 8*cout channels followed by the gather: bit for bit. And against the oracle's conv
    plus the reference's gather (out[m] = h[gidx/8][(gidx%8)*cout, +cout)) within TOL_16. Masks
    keep a random fraction of octants, with some parents dropped whole and some kept whole, and
    mark kept octants with bytes other than 1; keep 0 drops every child."""
    _case(f"planned octants ci={ci} cout={cout} n={n} keep={keep} {dtype_name}")
    import torch
    dt = getattr(torch, dtype_name)
    key = "bf16" if dt == torch.bfloat16 else "f16"
    rng = np.random.default_rng(ci * 31 + cout + n)
    coords, feats, weight, bias = _rand_case(shells, rng, n, ci, 8 * cout, key)
    nv = len(coords)
    mask = np.where(rng.random((nv, 8)) < keep, rng.integers(1, 256, (nv, 8)), 0).astype(np.uint8)
    if 0 < keep < 1:
        mask[::7] = 0
        mask[3::11] = 0x80
    c = torch.from_numpy(np.ascontiguousarray(coords, np.int32)).cuda()
    nbr = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr, nv)
    pw = gpu_lib.conv_weight_pack(_dev(weight, dt))
    f, b = _dev(feats, dt), _dev(bias, torch.float32)
    mask_t = torch.from_numpy(mask.reshape(-1)).cuda()
    _, gidx, mstart = gpu_lib.subdivide(mask_t, c)
    m = len(gidx)
    assert m == int(np.count_nonzero(mask))
    if m == 0:
        return
    fused = gpu_lib.subm_conv3x3_planned_octants(f, nbr, plan, pw, b, cout, mask_t, mstart, m)
    full = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, 8 * cout, out_dtype=torch.float32)
    assert torch.equal(fused, gpu_lib.c2s_gather(full, gidx, cout))
    h = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    ref = h.reshape(nv * 8, cout)[gidx.cpu().numpy()]
    assert orc.rel_err(fused.cpu().numpy(), ref) < TOL_16



@pytest.mark.parametrize("cin,ci,co,n", [(128, 64, 64, 0), (256, 128, 128, 1500), (64, 32, 64, 513)])
@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_planned_skip(gpu_lib, orc, shells, cin, ci, co, n, dtype_name):
    """The C2S conv2 with the skip added by its stores (sparse.cpp:302-323) against the planned
    conv followed by the skip pass: bit for bit. And against the oracle's conv plus the
    reference's repeat-interleaved octant block of x within TOL_16. The children come from a
    random subdivision of random parents, so gidx reaches every octant."""
    _case(f"planned skip cin={cin} ci={ci} co={co} n={n} {dtype_name}")
    import torch
    dt = getattr(torch, dtype_name)
    key = "bf16" if dt == torch.bfloat16 else "f16"
    rng = np.random.default_rng(cin + ci * 3 + co + n)
    pcoords = shells.sphere_shell(24, 12.0, 7.0, 9.0)
    pcoords = pcoords[:max(1, (n or 4000) // 4)]
    npar = len(pcoords)
    mask = (rng.random(npar * 8) < 0.5).astype(np.uint8)
    _, gidx, _ = gpu_lib.subdivide(torch.from_numpy(mask).cuda(),
                                   torch.from_numpy(np.ascontiguousarray(pcoords, np.int32)).cuda())
    child = np.ascontiguousarray(orc.subdivide(mask, pcoords)[0], np.int32)
    m = len(child)
    feats = shells.round_to(rng.standard_normal((m, ci)).astype(np.float32), key)
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / np.sqrt(27 * ci)).astype(np.float32), key)
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    x = rng.standard_normal((npar, cin)).astype(np.float32)
    c = torch.from_numpy(child).cuda()
    nbr = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr, m)
    pw = gpu_lib.conv_weight_pack(_dev(weight, dt))
    f, b, xt = _dev(feats, dt), _dev(bias, torch.float32), _dev(x, torch.float32)
    fused = gpu_lib.subm_conv3x3_planned_skip(f, nbr, plan, pw, b, co, xt, gidx)
    two_pass = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, co, out_dtype=torch.float32)
    gpu_lib.c2s_skip_add(xt, gidx, two_pass)
    assert torch.equal(fused, two_pass)
    k = cin // 8
    g = gidx.cpu().numpy()
    skip = np.repeat(x.reshape(npar * 8, k)[g], co // k, axis=1)
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(child), weight, bias) + skip
    assert orc.rel_err(fused.cpu().numpy(), ref) < TOL_16



def _column_split_tiles(n_tiles, nct, cus):
    """The tile where the planned conv at co = 128 nct hands the rest of its tiles to 64-channel
    units (0: one launch): the whole rounds of its persistent grid (cus / 8 workgroups per XCD,
    rounded down to a multiple of nct), when the tiles left fill at most one round of the
    64-channel grid."""
    g = 8 * max(1, cus // 8 // nct) * nct
    rounds = n_tiles * nct // g
    if rounds < 1:
        return 0
    t = rounds * (g // nct)
    left = n_tiles - t
    fit64 = max(1, cus // 8 // (2 * nct)) * (2 * nct)
    return t if 0 < left and -(-left * 2 * nct // 8) <= fit64 else 0


@pytest.mark.parametrize("kind,ci,co,shell,dtype_name,out16", [
    ("plain", 64, 1024, (64, 32.0, 28.5, 31.5), "bfloat16", False),
    ("plain", 64, 512, (64, 32.0, 28.5, 31.5), "float16", True),
    ("plain", 128, 128, (112, 56.0, 49.0, 53.5), "bfloat16", True),
    ("plain", 64, 256, (112, 56.0, 49.0, 53.5), "float16", False),
    ("octants", 64, 1024, (64, 32.0, 28.5, 31.5), "bfloat16", False),
    ("octants", 32, 512, (64, 32.0, 28.5, 31.5), "float16", False),
    ("skip", 64, 256, (64, 32.0, 28.5, 31.5), "float16", False),
    ("skip", 128, 128, (64, 32.0, 28.5, 31.5), "bfloat16", False)])
def test_planned_column_split(gpu_lib, shells, kind, ci, co, shell, dtype_name, out16):
    """Planned convs whose 128-channel units leave a thin last round of the persistent grid run
    that round's tiles as 64-channel units in a second launch: bit for bit the unplanned conv
    (plain), the unplanned conv then the gather (C2S conv1's octant stores), the unplanned conv
    then the skip pass (C2S conv2's skip stores), on Morton plans of shells sized so that the
    split happens on this device."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    dt = getattr(torch, dtype_name)
    key = "bf16" if dt == torch.bfloat16 else "f16"
    rng = np.random.default_rng(ci + co + len(kind))
    pcoords = np.ascontiguousarray(shells.sphere_shell(*shell), np.int32)
    if kind == "skip":
        mask = (rng.random(len(pcoords) * 8) < 0.5).astype(np.uint8)
        _, gidx, _ = gpu_lib.subdivide(torch.from_numpy(mask).cuda(), torch.from_numpy(pcoords).cuda())
        coords = np.ascontiguousarray(shells.children(mask, pcoords), np.int32)
    else:
        coords = pcoords
    n = len(coords)
    t_split = _column_split_tiles(-(-n // 512), co // 128, cus)
    _case(f"column split {kind} ci={ci} co={co} n={n} {dtype_name} out16={out16}: tiles [0, {t_split}) "
          f"at 128 channels, the rest at 64 ({cus} CUs)")
    if cus == 256:
        assert t_split > 0, "the shell was sized to split on 256 compute units"
    feats = shells.round_to(rng.standard_normal((n, ci)).astype(np.float32), key)
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / np.sqrt(27 * ci)).astype(np.float32), key)
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr, n, coords=c)
    f, w, b = _dev(feats, dt), _dev(weight, dt), _dev(bias, torch.float32)
    pw = gpu_lib.conv_weight_pack(w)
    if kind == "plain":
        odt = dt if out16 else torch.float32
        out = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, co, out_dtype=odt)
        ref = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=odt, algo="mfma")
    elif kind == "octants":
        cout = co // 8
        mask = np.where(rng.random((n, 8)) < 0.4, rng.integers(1, 256, (n, 8)), 0).astype(np.uint8)
        mask_t = torch.from_numpy(mask.reshape(-1)).cuda()
        _, g8, mstart = gpu_lib.subdivide(mask_t, c)
        out = gpu_lib.subm_conv3x3_planned_octants(f, nbr, plan, pw, b, cout, mask_t, mstart, len(g8))
        full = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma")
        ref = gpu_lib.c2s_gather(full, g8, cout)
    else:
        cin = 128
        x = _dev(rng.standard_normal((len(pcoords), cin)).astype(np.float32), torch.float32)
        out = gpu_lib.subm_conv3x3_planned_skip(f, nbr, plan, pw, b, co, x, gidx)
        ref = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma")
        gpu_lib.c2s_skip_add(x, gidx, ref)
    torch.cuda.synchronize()
    assert out.shape == ref.shape and bool(torch.isfinite(out.float()).all())
    assert torch.equal(out, ref)


@pytest.mark.parametrize("bad", ["inf", "nan"])
@pytest.mark.parametrize("path", ["planned", "auto", "mfma_gather", "narrow", "f32", "f32_narrow", "unsorted"])
def test_nonfinite_row0(gpu_lib, orc, shells, path, bad):
    """Absent taps read the padding row 0 * feats[0] (sparse.cpp:81-85). With an Inf or a NaN in
    row 0 every output row that has an absent tap is NaN in every channel, on every kernel path
    (the LDS-staged kernel with and without a stored plan, its direct path on unsorted rows, the
    gather kernel, the VALU kernel in 16 and 32 bits, the fp32 matrix-core kernel that AUTO takes
    for f32); rows whose 27 taps are all present keep their finite values (checked against the
    oracle away from row 0's own neighbours)."""
    _case(f"non-finite row 0 {path} {bad}")
    import torch
    rng = np.random.default_rng(23)
    coords = np.concatenate([shells.sphere_shell(24, 12.0, 7.0, 9.0),
                             np.stack(np.meshgrid(*[np.arange(40, 45)] * 3, indexing="ij"), -1).reshape(-1, 3)])
    if path == "unsorted":
        coords = np.concatenate([coords[:1], rng.permutation(coords[1:])])
    coords = np.ascontiguousarray(coords, np.int32)
    n, ci, co = len(coords), 32, 64
    key = "f32" if path.startswith("f32") else "bf16"
    feats = rng.standard_normal((n, ci)).astype(np.float32)
    feats[0, 7] = np.inf if bad == "inf" else np.nan
    weight = (rng.standard_normal((co, 27, ci)) / 30).astype(np.float32)
    if key == "bf16":
        feats, weight = shells.round_to(feats, "bf16"), shells.round_to(weight, "bf16")
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    ref = orc.subm_conv_f64(feats, nbr, weight, bias)
    dt = torch.float32 if key == "f32" else torch.bfloat16
    if path == "planned":
        out = _run_planned(gpu_lib, coords, feats, weight, bias, dt)
    else:
        algo = {"auto": "auto", "unsorted": "mfma", "mfma_gather": "mfma_gather", "narrow": "narrow",
                "f32": "auto", "f32_narrow": "narrow"}[path]
        out, _ = _run(gpu_lib, coords, feats, weight, bias, dt, algo=algo)
    t = nbr.reshape(27, n)
    absent = (t == n).any(axis=0)
    near0 = (t == 0).any(axis=0)
    assert absent.any() and (~absent & ~near0).any()
    assert np.isnan(out[absent]).all()
    keep = ~absent & ~near0
    assert np.isfinite(out[keep]).all()
    assert orc.rel_err(out[keep], ref[keep]) < (TOL_32 if key == "f32" else TOL_16)


def test_weight_pack_layout(gpu_lib):
    """packed[((c32*nkc + kc)*27 + t)*64 + lane][e] = W[32*c32 + lane%32][t][16*kc + 8*(lane//32) + e]"""
    _case("weight pack layout")
    import torch
    ci, co = 48, 96
    w = torch.arange(co * 27 * ci, dtype=torch.float32).reshape(co, 27, ci)
    w16 = (w % 2048).to(torch.float16)        # exactly representable, all distinct per 2048
    flat = gpu_lib.conv_weight_pack(w16.cuda()).cpu()
    assert flat.numel() == co * 27 * ci + 128                 # + the 256-byte trailer
    packed = flat[:co * 27 * ci].reshape(co // 32, ci // 16, 27, 2, 32, 8)
    ref = w16.reshape(co // 32, 32, 27, ci // 16, 2, 8).permute(0, 3, 2, 4, 1, 5)
    assert torch.equal(packed, ref)
    trailer = flat[co * 27 * ci:].view(torch.int32)
    assert int(trailer[0]) == 0 and not trailer.any()         # finite weights


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("bad", ["none", "inf", "-inf", "nan", "max"])
def test_weight_pack_nonfinite_flag(gpu_lib, dt, bad):
    """The trailer's first word is nonzero exactly when some weight is an Inf or a NaN (the
    largest finite value does not count), wherever it sits."""
    _case(f"weight pack trailer {dt} {bad}")
    import torch
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    ci, co = 32, 64
    w = torch.randn(co, 27, ci).to(tdt)
    if bad != "none":
        val = {"inf": float("inf"), "-inf": float("-inf"), "nan": float("nan"),
               "max": torch.finfo(tdt).max}[bad]
        w[co - 1, 26, ci - 1] = val            # the last element of the last pack block
        w[3, 13, 17] = val
    flat = gpu_lib.conv_weight_pack(w.cuda()).cpu()
    flag = int(flat[co * 27 * ci:].view(torch.int32)[0])
    assert (flag != 0) == (bad in ("inf", "-inf", "nan"))



@pytest.mark.parametrize("n_shell", ["r14", "r22"])
def test_mfma_unsorted_inputs(gpu_lib, orc, shells, n_shell):
    """Row order scattered at random: a 512-voxel tile then references far more distinct rows
    than LDS holds (r14: ~23K voxels, span fits but the set does not) or a row range wider
    than the bitmap (r22: ~92K voxels), so the MFMA kernel's direct path runs."""
    _case(f"unsorted {n_shell}")
    import torch
    rng = np.random.default_rng(61)
    r = 14.0 if n_shell == "r14" else 22.0
    coords = rng.permutation(shells.sphere_shell(64, 32.0, r, r + 2.0))
    n = len(coords)
    feats = shells.round_to(rng.standard_normal((n, 64)).astype(np.float32), "bf16")
    weight = shells.round_to((rng.standard_normal((128, 27, 64)) / 40).astype(np.float32), "bf16")
    bias = (rng.standard_normal(128) * 0.1).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    rows = np.unique(np.concatenate([np.arange(600), rng.integers(0, n, 2000)]))
    ref = orc.subm_conv_f64_rows(feats, nbr, weight, bias, rows)
    for algo in ("mfma", "mfma_gather"):
        out, _ = _run(gpu_lib, coords, feats, weight, bias, torch.bfloat16, algo=algo)
        assert orc.rel_err(out[rows], ref) < TOL_16, algo
    out = _run_planned(gpu_lib, coords, feats, weight, bias, torch.bfloat16)
    assert orc.rel_err(out[rows], ref) < TOL_16


@pytest.mark.parametrize("ci,co", [(3, 5), (16, 8), (64, 64), (33, 70)])
def test_narrow_fp32_ragged(gpu_lib, orc, shells, ci, co):
    _case(f"narrow f32 ci={ci} co={co}")
    import torch
    rng = np.random.default_rng(ci + 100 * co)
    coords, feats, weight, bias = _rand_case(shells, rng, 1500, ci, co, "f32")
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    out, _ = _run(gpu_lib, coords, feats, weight, bias, torch.float32, algo="narrow")
    assert orc.rel_err(out, ref) < TOL_32


def test_f32_feats_with_16bit_weights(gpu_lib, orc, shells):
    """The reference's default: f32 activations with f16 weights (sparse.cpp:17-19)."""
    _case("f32 feats x f16/bf16 weights")
    import torch
    rng = np.random.default_rng(31)
    for wdt, key in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        coords, feats, weight, bias = _rand_case(shells, rng, 2000, 64, 64, "f32")
        weight = shells.round_to(weight, key)
        ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
        out, _ = _run(gpu_lib, coords, feats, weight, bias, torch.float32, wdtype=wdt)
        assert orc.rel_err(out, ref) < TOL_32


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_16bit_output(gpu_lib, orc, shells, dtype_name):
    _case(f"16-bit output {dtype_name}")
    import torch
    dt = getattr(torch, dtype_name)
    key = "bf16" if dt == torch.bfloat16 else "f16"
    rng = np.random.default_rng(41)
    coords, feats, weight, bias = _rand_case(shells, rng, 4000, 128, 128, key)
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    for algo in ("mfma", "narrow"):
        out, _ = _run(gpu_lib, coords, feats, weight, bias, dt, out_dtype=dt, algo=algo)
        assert orc.rel_err(out, ref) < TOL_16_OUT


def test_isolated_voxels_and_empty(gpu_lib, orc):
    _case("isolated + empty")
    import torch
    rng = np.random.default_rng(51)
    coords = (np.arange(300, dtype=np.int32)[:, None] * 3).repeat(3, 1)   # no two adjacent
    feats = rng.standard_normal((300, 64)).astype(np.float32)
    weight = rng.standard_normal((64, 27, 64)).astype(np.float32)
    bias = rng.standard_normal(64).astype(np.float32)
    out, _ = _run(gpu_lib, coords, feats, weight, bias, torch.float32)
    ref = feats.astype(np.float64) @ weight[:, 13, :].T.astype(np.float64) + bias   # W_13 f + b
    assert orc.rel_err(out, ref) < TOL_32
    empty = gpu_lib.subm_conv3x3(
        torch.zeros((0, 64), dtype=torch.bfloat16, device="cuda"),
        torch.zeros(0, dtype=torch.int32, device="cuda"),
        torch.zeros((64, 27, 64), dtype=torch.bfloat16, device="cuda"),
        torch.zeros(64, dtype=torch.float32, device="cuda"))
    assert empty.shape == (0, 64)


def test_shell64_fp32_workload(gpu_lib, orc, shells):
    """The fp32 64^3 shell on AUTO's kernel (the fp32 matrix-core one) and on the VALU kernel."""
    _case("shell64-c64-f32")
    import torch
    w = shells.workload("shell64-c64-f32")
    ref = orc.subm_conv_f64(w.feats, orc.neighbor_table(w.coords), w.weight, w.bias)
    for algo in ("auto", "f32_mfma", "narrow"):
        out, _ = _run(gpu_lib, w.coords, w.feats, w.weight, w.bias, torch.float32, algo=algo)
        assert orc.rel_err(out, ref) < TOL_32, algo


@pytest.mark.parametrize("ci,co,n", [(16, 32, 1500), (64, 64, 0), (48, 96, 3000), (32, 128, 40000),
                                     (64, 64, 380934), (128, 96, 200000)])
def test_f32_mfma_vs_oracle(gpu_lib, orc, shells, ci, co, n):
    """The fp32 matrix-core kernel (algo="f32_mfma", AUTO's choice for f32 layers with Ci % 16 == 0
    and Co % 32 == 0, after the thin kernels' shapes) in both launch shapes it picks by size -- the
    taps of 32-row tiles split over 4 waves (up to 40 K voxels here), one wave per 64-row tile
    (200 K and 381 K voxels) -- with 32- and 64-channel column tiles, against the fp64 oracle
    (every row, or 4000 sampled rows plus the first and last tiles at the larger sizes), against
    the VALU kernel on every row, bitwise repeatable and equal to AUTO, and with bf16 and f16
    outputs."""
    _case(f"f32 mfma ci={ci} co={co} n={n}")
    import torch
    rng = np.random.default_rng(7 * ci + co)
    if n > 6000:
        coords = shells.sphere_shell(160, 70.0, 50.0, 60.0)[:n]
    else:
        coords = shells.sphere_shell(48, 24.0, 14.0, 16.0)[:n or None]
    coords = np.ascontiguousarray(coords, np.int32)
    n = len(coords)
    feats = rng.standard_normal((n, ci)).astype(np.float32)
    weight = (rng.standard_normal((co, 27, ci)) / np.sqrt(27 * ci)).astype(np.float32)
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    f, w, b = _dev(feats, torch.float32), _dev(weight, torch.float32), _dev(bias, torch.float32)
    out = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="f32_mfma")
    out2 = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="f32_mfma")
    auto = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="auto")
    outn = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="narrow")
    o16 = {dt: gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=dt, algo="f32_mfma")
           for dt in (torch.bfloat16, torch.float16)}
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    if not (co <= 32 and ci * co <= 512):    # AUTO's choice unless the thin VALU kernel takes the shape
        assert torch.equal(out, auto)
    got = out.cpu().numpy()
    nbr_h = nbr.cpu().numpy()
    if n > 6000:
        rows = np.unique(np.concatenate([np.arange(64), np.arange(n - 64, n), rng.integers(0, n, 4000)]))
        ref = orc.subm_conv_f64_rows(feats, nbr_h, weight, bias, rows)
    else:
        rows = np.arange(n)
        ref = orc.subm_conv_f64(feats, nbr_h, weight, bias)
    assert orc.rel_err(got[rows], ref) < TOL_32
    assert orc.rel_err(got, outn.cpu().numpy()) < TOL_32
    for dt, o in o16.items():
        assert orc.rel_err(o.float().cpu().numpy()[rows], ref) < TOL_16_OUT, dt


def test_f32_mfma_rejects(gpu_lib, shells):
    """algo="f32_mfma" outside its shapes: 16-bit features, mixed dtypes, Ci % 16 != 0, Co % 32 != 0."""
    _case("f32 mfma rejects")
    import torch
    coords = np.ascontiguousarray(shells.sphere_shell(24, 12.0, 7.0, 9.0), np.int32)
    n = len(coords)
    nbr = gpu_lib.rulebook_build(torch.from_numpy(coords).cuda())
    b = torch.zeros(64, dtype=torch.float32, device="cuda")
    for fdt, wdt, ci, co in ((torch.bfloat16, torch.bfloat16, 64, 64), (torch.float32, torch.float16, 64, 64),
                             (torch.float32, torch.float32, 40, 64), (torch.float32, torch.float32, 64, 48)):
        f = torch.zeros((n, ci), dtype=fdt, device="cuda")
        w = torch.zeros((co, 27, ci), dtype=wdt, device="cuda")
        with pytest.raises(gpu_lib.TspError, match="fp32 matrix-core"):
            gpu_lib.subm_conv3x3(f, nbr, w, b[:co], out_dtype=torch.float32, algo="f32_mfma")


@pytest.mark.parametrize("name", ["ellipsoids128-c256-bf16", "shells256-c128-bf16"])
def test_full_size_sampled_rows(gpu_lib, orc, shells, name):
    """Full-size workloads: every output row of a deterministic sample (the first and last
    tiles plus 3000 random rows) against the fp64 oracle, MFMA and VALU kernels against each
    other on all rows, and bitwise reproducibility."""
    _case(name)
    import torch
    w = shells.workload(name)
    c = torch.from_numpy(w.coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    f = _dev(w.feats, torch.bfloat16)
    wt = _dev(w.weight, torch.bfloat16)
    b = _dev(w.bias, torch.float32)
    out = gpu_lib.subm_conv3x3(f, nbr, wt, b, out_dtype=torch.float32, algo="mfma")
    out2 = gpu_lib.subm_conv3x3(f, nbr, wt, b, out_dtype=torch.float32, algo="mfma")
    outg = gpu_lib.subm_conv3x3(f, nbr, wt, b, out_dtype=torch.float32, algo="mfma_gather")
    outn = gpu_lib.subm_conv3x3(f, nbr, wt, b, out_dtype=torch.float32, algo="narrow")
    plan = gpu_lib.conv_plan_build(nbr, w.n, coords=c)
    outp = gpu_lib.subm_conv3x3_planned(f, nbr, plan, gpu_lib.conv_weight_pack(wt), b, w.co,
                                        out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    assert torch.equal(outp, out)        # same MFMA order: the stored plan changes nothing
    assert orc.rel_err(outg.cpu().numpy(), out.cpu().numpy()) < TOL_16
    rng = np.random.default_rng(0)
    rows = np.unique(np.concatenate([np.arange(512), np.arange(w.n - 512, w.n),
                                     rng.integers(0, w.n, 3000)]))
    nbr_h = nbr.cpu().numpy()
    ref = orc.subm_conv_f64_rows(w.feats, nbr_h, w.weight, w.bias, rows)
    got = out.cpu().numpy()
    assert orc.rel_err(got[rows], ref) < TOL_16
    assert orc.rel_err(got, outn.cpu().numpy()) < TOL_16


def _nan_aware(out, ref, tol):
    """Non-finite entries at the same places (NaN vs Inf not distinguished); the finite rest
    within tol of max|ref| over the finite reference entries."""
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(out), fin)
    err = np.abs(out[fin] - ref[fin]).max() / max(np.abs(ref[fin]).max(), 1e-30)
    assert err < tol, err


@pytest.mark.parametrize("bad", ["inf", "nan"])
@pytest.mark.parametrize("path", ["planned", "auto", "mfma_gather", "narrow", "f32", "f32_narrow", "unsorted",
                                  "skip"])
def test_zero_padding_row(gpu_lib, orc, shells, path, bad):
    """TSP_CONV_ZERO_PAD: absent taps read an exact zero row, as the C2S conv2 reads hn's zero
    padding column (sparse.cpp:289-306). With an Inf or a NaN in feature row 0, only the rows
    that reference row 0 become non-finite; every other row keeps its finite value, against the
    oracle's zero-padded conv. "skip" is the fused C2S conv2 (always zero padded)."""
    _case(f"zero padding row {path} {bad}")
    import torch
    rng = np.random.default_rng(29)
    coords = np.concatenate([shells.sphere_shell(24, 12.0, 7.0, 9.0),
                             np.stack(np.meshgrid(*[np.arange(40, 45)] * 3, indexing="ij"), -1).reshape(-1, 3)])
    if path == "unsorted":
        coords = np.concatenate([coords[:1], rng.permutation(coords[1:])])
    coords = np.ascontiguousarray(coords, np.int32)
    n, ci, co = len(coords), 32, 64
    key = "f32" if path.startswith("f32") else "bf16"
    feats = rng.standard_normal((n, ci)).astype(np.float32)
    feats[0, 5] = np.inf if bad == "inf" else np.nan
    weight = (rng.standard_normal((co, 27, ci)) / 30).astype(np.float32)
    if key == "bf16":
        feats, weight = shells.round_to(feats, "bf16"), shells.round_to(weight, "bf16")
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    ref = orc.subm_conv_f64(feats, nbr, weight, bias, zero_pad=True)
    dt = torch.float32 if key == "f32" else torch.bfloat16
    c = torch.from_numpy(coords).cuda()
    nbr_d = gpu_lib.rulebook_build(c)
    f, w, b = _dev(feats, dt), _dev(weight, dt), _dev(bias, torch.float32)
    if path in ("planned", "skip"):
        plan = gpu_lib.conv_plan_build(nbr_d, n)
        pw = gpu_lib.conv_weight_pack(w)
        if path == "planned":
            out = gpu_lib.subm_conv3x3_planned(f, nbr_d, plan, pw, b, co, out_dtype=torch.float32,
                                               zero_pad=True)
        else:
            # children of n // 8 parents: every child m has gidx = m, so x row m // 8 feeds it
            cin = 128
            x = rng.standard_normal((n // 8 + 1, cin)).astype(np.float32)
            gidx = torch.arange(n, dtype=torch.int32, device="cuda")
            out = gpu_lib.subm_conv3x3_planned_skip(f, nbr_d, plan, pw, b, co, _dev(x, torch.float32), gidx)
            k = cin // 8
            ref = ref + np.repeat(x.reshape(-1, k)[np.arange(n)], co // k, axis=1)
    else:
        algo = {"auto": "auto", "unsorted": "mfma", "mfma_gather": "mfma_gather", "narrow": "narrow",
                "f32": "auto", "f32_narrow": "narrow"}[path]
        out = gpu_lib.subm_conv3x3(f, nbr_d, w, b, out_dtype=torch.float32, algo=algo, zero_pad=True)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    t = nbr.reshape(27, n)
    refs0 = (t == 0).any(axis=0)
    absent = (t == n).any(axis=0)
    assert (absent & ~refs0).any()
    assert np.isfinite(out[~refs0]).all()
    _nan_aware(out, ref, TOL_32 if key == "f32" else TOL_16)


@pytest.mark.parametrize("path", ["planned", "mfma", "mfma_gather", "narrow"])
def test_padding_row_from_f32_source(gpu_lib, orc, shells, path):
    """A finite f32 row 0 beyond the f16 range rounds to Inf. The reference forms its padding row
    0 * feats[0] in F32 before ggml's F16 mul_mat rounds the activations (sparse.cpp:74, 81-85), so
    the padding row is zero: given the f32 row 0 (row0=), only rows that reference row 0 turn
    non-finite. Without it the rounded Inf row makes every row with an absent tap NaN. On every
    kernel path."""
    _case(f"padding row from the f32 source row: {path}")
    import torch
    rng = np.random.default_rng(37)
    coords = np.ascontiguousarray(shells.sphere_shell(24, 12.0, 7.0, 9.0), np.int32)
    n, ci, co = len(coords), 32, 64
    feats32 = rng.standard_normal((n, ci)).astype(np.float32)
    feats32[0, 3] = 1.0e5                                   # finite, > 65504
    feats16 = shells.round_to(feats32, "f16")
    assert np.isinf(feats16[0, 3])
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / 30).astype(np.float32), "f16")
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    c = torch.from_numpy(coords).cuda()
    nbr_d = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr_d, n)
    pw = gpu_lib.conv_weight_pack(_dev(weight, torch.float16))
    f, b = _dev(feats16, torch.float16), _dev(bias, torch.float32)
    r0 = _dev(feats32[0], torch.float32)
    if path == "planned":
        with_src = gpu_lib.subm_conv3x3_planned(f, nbr_d, plan, pw, b, co, out_dtype=torch.float32, row0=r0)
        without = gpu_lib.subm_conv3x3_planned(f, nbr_d, plan, pw, b, co, out_dtype=torch.float32)
    else:
        w = _dev(weight, torch.float16)
        with_src = gpu_lib.subm_conv3x3(f, nbr_d, w, b, out_dtype=torch.float32, algo=path, row0=r0)
        without = gpu_lib.subm_conv3x3(f, nbr_d, w, b, out_dtype=torch.float32, algo=path)
    torch.cuda.synchronize()
    _nan_aware(with_src.cpu().numpy(), orc.subm_conv_f64(feats16, nbr, weight, bias, zero_pad=True), TOL_16)
    absent = (nbr.reshape(27, n) == n).any(axis=0)
    assert np.isnan(without.cpu().numpy()[absent]).all()


def _plan_parts(plan, n):
    """Views of a plan buffer's tile records (layout of tile_plan.hpp's carve_plan)."""
    al = lambda b: (b + 255) // 256 * 256
    t = (n + 511) // 512
    raw = plan.cpu().numpy()
    off, parts = 0, {}
    for name, nbytes, dt, shape in (("hdr", t * 16, np.int32, (t, 4)), ("rowof", t * 2048 * 4, np.int32, (t, 2048)),
                                    ("slots", t * 27 * 512 * 2, np.uint16, (t, 27, 4, 32, 4)),
                                    ("vox", t * 512 * 4, np.int32, (t, 512)),
                                    ("act", t * 64, np.uint32, (t, 4, 4))):
        parts[name] = raw[off:off + nbytes].view(dt).reshape(shape)
        off += al(nbytes)
    return parts


def _check_plan(p, table, n, order):
    """What a plan promises the conv: the tiles' positions hold every voxel once (a tile of a
    plan without coordinates holds consecutive rows); inside each 32-row block the voxels come
    first, ordered by their set of present corner taps (then by row, for a plan without
    coordinates), then the empty positions; the act bits of each
    (row group, block, tap) say exactly whether a voxel of the block has the tap; each (tap,
    position) slot names the row the table gives, through the tile's list of distinct rows (sorted
    for row tiles; in cell-grid position order for Morton tiles), or the zero slot. Returns the
    tiles' distinct-row counts and the number of clear act bits."""
    vox = p["vox"].reshape(-1)
    assert np.array_equal(np.sort(vox[vox >= 0]), np.arange(n))
    assert (vox < 0).sum() == p["vox"].size - n
    H = p["hdr"][:, 0]
    present = table != n                                   # [27, n]
    corners = [0, 2, 6, 8, 18, 20, 24, 26]                 # taps (+-1, +-1, +-1)
    cset = (present[corners].astype(np.int64) << np.arange(8)[:, None]).sum(0)
    clear = 0
    for t in range(p["vox"].shape[0]):
        v = p["vox"][t]
        k = int((v >= 0).sum())
        if order == "rows":
            assert np.array_equal(np.sort(v[v >= 0]), np.arange(512 * t, 512 * t + k))
        for g in range(4):
            bits = sum(int(p["act"][t, g, w]) << (32 * w) for w in range(4))
            for b in range(4):
                blk = v[g * 128 + b * 32: g * 128 + b * 32 + 32]
                m = int((blk >= 0).sum())
                assert (blk[:m] >= 0).all() and (blk[m:] < 0).all()
                assert np.all(np.diff(cset[blk[:m]]) >= 0)
                if order == "rows":
                    assert np.all(np.diff((cset[blk[:m]] << 32) | blk[:m]) > 0)
                for tap in range(27):
                    want = bool(m) and bool(present[tap, blk[:m]].any())
                    assert ((bits >> (4 * tap + b)) & 1) == want, (t, g, b, tap)
                    clear += not want
        if p["hdr"][t, 1]:
            continue
        rows = p["rowof"][t, :H[t]]
        if order == "rows":
            assert np.all(np.diff(rows) > 0)
        else:
            assert len(np.unique(rows)) == H[t] and rows.min() >= 0 and rows.max() < n
        for tap in (0, 4, 13, 22, 26):
            sl = p["slots"][t, tap].transpose(0, 2, 1).reshape(512)   # [group][block][row] = position order
            got = np.where(sl == 2048, n, rows[np.minimum(sl, max(H[t] - 1, 0))])
            want = np.where(v >= 0, table[tap][np.maximum(v, 0)], n)
            assert np.array_equal(got, want), (t, tap)
    return H, clear


@pytest.mark.parametrize("order", ["rows", "morton"])
def test_plan_records(gpu_lib, orc, shells, order):
    """The plan's records checked on the host (see _check_plan); Morton tiles reference fewer
    distinct rows than row tiles on a thin shell, every tile fits the LDS stage, and grouping
    voxels by tap set clears act bits (absent taps skipped by whole blocks)."""
    _case(f"plan records {order}")
    import torch
    coords = np.ascontiguousarray(shells.sphere_shell(64, 32.0, 20.0, 22.0), np.int32)
    n = len(coords)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr, n, coords=c if order == "morton" else None)
    torch.cuda.synchronize()
    p = _plan_parts(plan, n)
    H, clear = _check_plan(p, nbr.cpu().numpy().reshape(27, n), n, order)
    assert (p["hdr"][:, 1] == 0).all()
    print(f"{order}: distinct rows per voxel {H.sum() / n:.2f}, (block, tap) pairs skipped "
          f"{clear / (len(H) * 16 * 27):.3f}", flush=True)
    assert clear > 0.05 * len(H) * 16 * 27
    if order == "morton":
        rplan = gpu_lib.conv_plan_build(nbr, n)
        assert H.sum() < 0.8 * _plan_parts(rplan, n)["hdr"][:, 0].sum()


@pytest.mark.parametrize("order", ["rows", "morton"])
def test_plan_wide_row_span(gpu_lib, orc, shells, order):
    """Half a compact cube in the first rows, the other half in the last, a dense box of 2.2M
    voxels in between. Row tiles: the first tile (the cube's first half and the box's first rows)
    references rows at both ends of the range, more than the two-level bitmap's 2^21, so the
    planner cuts the empty stretch out and the tile still stages its rows in LDS. Morton tiles: the
    cube is one 8^3 cell and one tile of its own, with the first and the last rows. Records of that
    tile checked as in test_plan_records; the conv equals the unplanned one bit for bit and the
    oracle on the cube's rows."""
    _case(f"plan: wide row span, {order}")
    import torch
    cube = np.stack(np.meshgrid(*[np.arange(8)] * 3, indexing="ij"), -1).reshape(-1, 3).astype(np.int32)
    box = (np.stack(np.meshgrid(*[np.arange(131)] * 3, indexing="ij"), -1).reshape(-1, 3) + 100).astype(np.int32)
    coords = np.ascontiguousarray(np.concatenate([cube[:256], box, cube[256:]]))
    n = len(coords)
    assert n - 256 > (1 << 21)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr, n, coords=c if order == "morton" else None)
    torch.cuda.synchronize()
    p = _plan_parts(plan, n)
    table = nbr.cpu().numpy().reshape(27, n)
    first = np.nonzero((p["vox"] == 0).any(axis=1))[0][0]          # the tile holding row 0
    assert p["hdr"][first, 1] == 0
    if order == "morton":
        assert (p["vox"][first] == n - 1).any()                     # ... and the last row
        assert (p["hdr"][:, 1] == 0).all()
    H = p["hdr"][first, 0]
    rows = p["rowof"][first, :H]
    assert rows[0] == 0 and rows[-1] >= n - 256 and np.all(np.diff(rows) > 0)
    v = p["vox"][first]
    for tap in range(27):
        sl = p["slots"][first, tap].transpose(0, 2, 1).reshape(512)
        got = np.where(sl == 2048, n, rows[np.minimum(sl, H - 1)])
        assert np.array_equal(got, np.where(v >= 0, table[tap][np.maximum(v, 0)], n)), tap
    rng = np.random.default_rng(9)
    feats = shells.round_to(rng.standard_normal((n, 32)).astype(np.float32), "bf16")
    weight = shells.round_to((rng.standard_normal((64, 27, 32)) / 30).astype(np.float32), "bf16")
    bias = (rng.standard_normal(64) * 0.1).astype(np.float32)
    f, w, b = _dev(feats, torch.bfloat16), _dev(weight, torch.bfloat16), _dev(bias, torch.float32)
    out = gpu_lib.subm_conv3x3_planned(f, nbr, plan, gpu_lib.conv_weight_pack(w), b, 64, out_dtype=torch.float32)
    ref_d = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma")
    torch.cuda.synchronize()
    assert torch.equal(out, ref_d)
    rows_chk = np.concatenate([np.arange(256), np.arange(n - 256, n)])
    ref = orc.subm_conv_f64_rows(feats, nbr.cpu().numpy(), weight, bias, rows_chk)
    assert orc.rel_err(out.cpu().numpy()[rows_chk], ref) < TOL_16


def test_ordered_plan_duplicates_unsorted(gpu_lib, orc, shells):
    """Morton tiles of an unsorted shell with duplicated coordinates: the cell walk places each
    coordinate's largest row in its cell and the other duplicates after all cells; every voxel
    sits in the plan once, each slot names the table's row, and the planned conv equals the
    unplanned one bit for bit."""
    _case("ordered plan: duplicates, unsorted")
    import torch
    rng = np.random.default_rng(31)
    shell = shells.sphere_shell(48, 24.0, 14.0, 16.0)
    dup = shell[rng.choice(len(shell), size=700, replace=False)]
    coords = np.ascontiguousarray(rng.permutation(np.concatenate([shell, dup])), np.int32)
    n = len(coords)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr, n, coords=c)
    torch.cuda.synchronize()
    table = nbr.cpu().numpy().reshape(27, n)
    assert np.array_equal(table, orc.neighbor_table(coords).reshape(27, n))
    p = _plan_parts(plan, n)
    H, _ = _check_plan(p, table, n, "morton")
    # the largest row of each coordinate is placed by its cell; the duplicates' other rows fill the
    # last walk positions [n - 700, n), so tiles past the one holding position n - 700 hold only them
    _, last = np.unique(coords[::-1], axis=0, return_index=True)
    losers = np.setdiff1d(np.arange(n), n - 1 - last)
    assert len(losers) == 700
    t0 = (n - 700) // 512
    tail = p["vox"][t0 + 1:].reshape(-1)
    assert np.isin(tail[tail >= 0], losers).all()
    head = p["vox"][:t0].reshape(-1)
    assert not np.isin(head[head >= 0], losers).any()
    assert (p["hdr"][:t0, 1] == 0).all()       # the cells' tiles stage their rows in LDS
    feats = shells.round_to(rng.standard_normal((n, 64)).astype(np.float32), "bf16")
    weight = shells.round_to((rng.standard_normal((64, 27, 64)) / 40).astype(np.float32), "bf16")
    bias = (rng.standard_normal(64) * 0.1).astype(np.float32)
    f, w, b = _dev(feats, torch.bfloat16), _dev(weight, torch.bfloat16), _dev(bias, torch.float32)
    out = gpu_lib.subm_conv3x3_planned(f, nbr, plan, gpu_lib.conv_weight_pack(w), b, 64, out_dtype=torch.float32)
    ref_d = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma")
    torch.cuda.synchronize()
    assert torch.equal(out, ref_d)


@pytest.mark.parametrize("kind", ["shell", "duplicates", "scattered-box"])
def test_table_and_plan_in_one_call(gpu_lib, shells, kind):
    """tsp_rulebook_build_planned: the table of tsp_rulebook_build and the records of
    tsp_conv_plan_build_ordered, from one cell grid (a brick hash and row tiles for the scattered
    set), also when the buffers are reused."""
    _case(f"table + plan in one call: {kind}")
    import torch
    rng = np.random.default_rng(43)
    if kind == "shell":
        coords = shells.sphere_shell(80, 40.0, 30.0, 32.0)
    elif kind == "duplicates":
        sh = shells.sphere_shell(48, 24.0, 14.0, 16.0)
        coords = rng.permutation(np.concatenate([sh, sh[rng.choice(len(sh), 500, replace=False)]]))
    else:
        coords = rng.integers(0, 400, size=(20000, 3))
    coords = np.ascontiguousarray(coords, np.int32)
    n = len(coords)
    c = torch.from_numpy(coords).cuda()
    nbr, plan = gpu_lib.rulebook_build_planned(c)
    ref_nbr = gpu_lib.rulebook_build(c)
    ref_plan = gpu_lib.conv_plan_build(ref_nbr, n, coords=c)
    nbr2, plan2 = gpu_lib.rulebook_build_planned(c, nbr=torch.full_like(nbr, -7),
                                                 plan=torch.full_like(plan, 255))
    torch.cuda.synchronize()
    assert torch.equal(nbr, ref_nbr) and torch.equal(nbr2, ref_nbr)
    b = _plan_parts(ref_plan, n)
    for got in (_plan_parts(plan, n), _plan_parts(plan2, n)):
        for k in ("hdr", "vox", "act"):
            assert np.array_equal(got[k], b[k]), k
        for t in range(b["hdr"].shape[0]):
            if b["hdr"][t, 1] == 0:
                H = b["hdr"][t, 0]
                assert np.array_equal(got["rowof"][t, :H], b["rowof"][t, :H])
                assert np.array_equal(got["slots"][t], b["slots"][t])


@pytest.mark.parametrize("kind", ["far-flung", "scattered-box"])
def test_ordered_plan_fallback(gpu_lib, shells, kind):
    """Coordinates whose cell grid does not fit the plan's space -- a bounding box wider than the
    directory allows (far-flung), or more occupied cells than the blocks' space (scattered-box):
    the ordered build falls back to row tiles on the device, and its records equal the plan
    without coordinates."""
    _case(f"ordered plan fallback: {kind}")
    import torch
    rng = np.random.default_rng(41)
    if kind == "far-flung":
        coords = rng.integers(0, (1 << 21) - 3, size=(3000, 3)).astype(np.int32)
    else:
        coords = rng.integers(0, 400, size=(20000, 3)).astype(np.int32)
    n = len(coords)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    a = _plan_parts(gpu_lib.conv_plan_build(nbr, n, coords=c), n)
    b = _plan_parts(gpu_lib.conv_plan_build(nbr, n), n)
    for k in ("hdr", "vox", "act"):
        assert np.array_equal(a[k], b[k]), k
    for t in range(a["hdr"].shape[0]):
        if a["hdr"][t, 1] == 0:
            H = a["hdr"][t, 0]
            assert np.array_equal(a["rowof"][t, :H], b["rowof"][t, :H])
            assert np.array_equal(a["slots"][t], b["slots"][t])


def _grid_blocks(coords):
    """Blocks of the plan's cell grid for coords (8^3 cells; a cell above or below a voxel at the
    top or bottom of its cell also gets one, inside the directory's power-of-two box)."""
    c = np.asarray(coords, np.int64)
    cell = c >> 3
    lo = cell.min(0)
    side = 1 << int(np.ceil(np.log2(max(int((cell.max(0) - lo).max()) + 1, 1))))
    keys = {tuple(v) for v in cell.tolist()}
    for v, z in zip(cell.tolist(), c[:, 2].tolist()):
        for dz, hit in ((-1, z & 7 == 0), (1, z & 7 == 7)):
            if hit and 0 <= v[2] + dz - lo[2] < side:
                keys.add((v[0], v[1], v[2] + dz))
    return len(keys)


@pytest.mark.parametrize("n,box", [(2000, 256), (5000, 400)])
def test_ordered_plan_scattered_more_blocks_than_voxels(gpu_lib, orc, shells, n, box):
    """Scattered voxels whose cell grid has more blocks than voxels (a voxel can add a halo-only
    block), which the plan's per-block scratch must hold: the conv on the Morton plan equals the
    conv on the row plan and without a plan bit for bit, and the oracle within TOL_16; the table
    and plan built in one call give the same conv."""
    import torch
    rng = np.random.default_rng(n)
    coords = np.ascontiguousarray(rng.integers(0, box, size=(n, 3)), np.int32)
    nb = _grid_blocks(coords)
    assert nb > n, (nb, n)   # the case the scratch was once too small for
    _case(f"ordered plan, scattered n={n} in [0,{box})^3: {nb} grid blocks")
    ci = co = 64
    feats = shells.round_to(rng.standard_normal((n, ci)).astype(np.float32), "bf16")
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / np.sqrt(27 * ci)).astype(np.float32), "bf16")
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    f, w, b = _dev(feats, torch.bfloat16), _dev(weight, torch.bfloat16), _dev(bias, torch.float32)
    pw = gpu_lib.conv_weight_pack(w)
    outs = {}
    for name, pc in (("morton", c), ("rows", None)):
        plan = gpu_lib.conv_plan_build(nbr, n, coords=pc)
        outs[name] = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, co, out_dtype=torch.float32)
    nbr1, plan1 = gpu_lib.rulebook_build_planned(c)
    outs["one-call"] = gpu_lib.subm_conv3x3_planned(f, nbr1, plan1, pw, b, co, out_dtype=torch.float32)
    outs["none"] = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma")
    torch.cuda.synchronize()
    assert torch.equal(nbr1, nbr)
    for k in ("morton", "rows", "one-call"):
        assert torch.equal(outs[k], outs["none"]), k
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    assert orc.rel_err(outs["morton"].cpu().numpy(), ref) < TOL_16


def test_table_and_plan_dense_random_blocks(gpu_lib, shells):
    """2,000,000 random voxels in [0,295)^3 (~40 per occupied 8^3 cell): the neighbour table's
    workspace holds their cell grid, whose presence bitmaps (64 bytes a block) the plan built in
    the same call must hold too. The one-call table equals tsp_rulebook_build's, and the conv on its
    plan equals the conv without a plan bit for bit."""
    import torch
    rng = np.random.default_rng(295)
    n = 2_000_000
    coords = np.ascontiguousarray(rng.integers(0, 295, size=(n, 3)), np.int32)
    _case(f"table + plan in one call: {n} random voxels in [0,295)^3")
    c = torch.from_numpy(coords).cuda()
    nbr1, plan1 = gpu_lib.rulebook_build_planned(c)
    nbr = gpu_lib.rulebook_build(c)
    assert torch.equal(nbr1, nbr)
    ci = co = 64
    f = (torch.randn((n, ci), device="cuda")).to(torch.bfloat16)
    w = (torch.randn((co, 27, ci), device="cuda") / 40).to(torch.bfloat16)
    b = torch.zeros(co, device="cuda")
    out = gpu_lib.subm_conv3x3_planned(f, nbr1, plan1, gpu_lib.conv_weight_pack(w), b, co, out_dtype=torch.float32)
    ref = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma")
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("ci,co", [(128, 128), (64, 64), (256, 64)])
def test_ordered_plan_results(gpu_lib, orc, shells, ci, co):
    """The planned conv on Morton tiles, on row tiles and without a plan: the same bits, and the
    fp64 oracle within TOL_16. Ordering and skipping dead taps change nothing in any row's sum."""
    _case(f"ordered plan ci={ci} co={co}")
    import torch
    rng = np.random.default_rng(ci + 3 * co)
    coords = np.ascontiguousarray(rng.permutation(shells.sphere_shell(64, 32.0, 18.0, 20.5)), np.int32)
    n = len(coords)
    feats = shells.round_to(rng.standard_normal((n, ci)).astype(np.float32), "bf16")
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / np.sqrt(27 * ci)).astype(np.float32), "bf16")
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    f, w, b = _dev(feats, torch.bfloat16), _dev(weight, torch.bfloat16), _dev(bias, torch.float32)
    pw = gpu_lib.conv_weight_pack(w)
    outs = {}
    for name, pc in (("morton", c), ("rows", None)):
        plan = gpu_lib.conv_plan_build(nbr, n, coords=pc)
        outs[name] = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, co, out_dtype=torch.float32)
    outs["none"] = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma")
    torch.cuda.synchronize()
    assert torch.equal(outs["morton"], outs["none"]) and torch.equal(outs["rows"], outs["none"])
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    assert orc.rel_err(outs["morton"].cpu().numpy(), ref) < TOL_16


@pytest.mark.parametrize("bad", ["inf", "nan"])
def test_nonfinite_weight_runs_every_tap(gpu_lib, shells, bad):
    """Absent taps multiply the zero slot by W: zero for finite weights, NaN where W holds an Inf
    or a NaN (as the reference's padding row times W gives). The planned conv on Morton tiles
    matches the unplanned kernel NaN for NaN and value for value."""
    _case(f"non-finite weight {bad}")
    import torch
    rng = np.random.default_rng(71)
    coords = np.ascontiguousarray(shells.sphere_shell(40, 20.0, 12.0, 14.0), np.int32)
    n, ci, co = len(coords), 64, 128
    feats = shells.round_to(rng.standard_normal((n, ci)).astype(np.float32), "bf16")
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / 30).astype(np.float32), "bf16")
    weight[5, 0, 3] = np.inf if bad == "inf" else np.nan      # tap 0: absent for most voxels
    bias = np.zeros(co, np.float32)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    f, w, b = _dev(feats, torch.bfloat16), _dev(weight, torch.bfloat16), _dev(bias, torch.float32)
    plan = gpu_lib.conv_plan_build(nbr, n, coords=c)
    got = gpu_lib.subm_conv3x3_planned(f, nbr, plan, gpu_lib.conv_weight_pack(w), b, co,
                                       out_dtype=torch.float32).cpu().numpy()
    want = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma").cpu().numpy()
    assert np.isnan(want[:, 5]).any()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(want)], want[~np.isnan(want)])


@pytest.mark.parametrize("ci,co", [(4, 4), (8, 8), (16, 16), (32, 16), (16, 32), (64, 8), (128, 4)])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16", "f32xf16"])
def test_thin_vs_oracle(gpu_lib, orc, shells, ci, co, dt):
    """The thin-channel VALU kernel (one voxel's output row per thread) at every width it takes,
    for f32, bf16, f16 and f32 features with f16 weights, by algo="thin"; AUTO's choice for the
    same shapes (the thin matrix-core kernel for 16-bit Ci in {8, 16, 32}, else this one) within
    the same bar."""
    _case(f"thin ci={ci} co={co} {dt}")
    import torch
    rng = np.random.default_rng(ci * 7 + co)
    fkey, wkey = {"f32": ("f32", "f32"), "bf16": ("bf16", "bf16"), "f16": ("f16", "f16"),
                  "f32xf16": ("f32", "f16")}[dt]
    coords, feats, weight, bias = _rand_case(shells, rng, 3000, ci, co, "f32")
    feats, weight = shells.round_to(feats, fkey), shells.round_to(weight, wkey)
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    out, nbr = _run(gpu_lib, coords, feats, weight, bias, tdt[fkey], wdtype=tdt[wkey])
    tol = TOL_32 if fkey == "f32" and wkey == "f32" else (TOL_32 if fkey == "f32" else TOL_16)
    assert orc.rel_err(out, ref) < tol
    out2, _ = _run(gpu_lib, coords, feats, weight, bias, tdt[fkey], wdtype=tdt[wkey], algo="thin")
    assert orc.rel_err(out2, ref) < tol
    if not (fkey == wkey and fkey != "f32" and ci in (8, 16, 32)):
        assert np.array_equal(out, out2)   # AUTO took the VALU kernel
    if fkey != "f32":   # 16-bit output: one rounding more
        o16, _ = _run(gpu_lib, coords, feats, weight, bias, tdt[fkey], out_dtype=tdt[fkey], algo="thin")
        assert orc.rel_err(o16, ref) < TOL_16_OUT


THIN_MFMA_SHAPES = [(8, 4), (8, 8), (8, 16), (8, 32), (16, 8), (16, 16), (16, 32), (32, 4), (32, 8), (32, 16)]


@pytest.mark.parametrize("ci,co", THIN_MFMA_SHAPES)
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_thin_mfma_vs_oracle(gpu_lib, orc, shells, ci, co, dt):
    """The thin matrix-core kernel (the 27 taps folded into K = 27 Ci of 16 x 16 x 32 steps, each
    lane gathering its neighbour row piece straight into the operand) at every shape it takes, on
    a ragged voxel count (not a multiple of its 16- or 32-voxel chunks), f32 and 16-bit output,
    against the fp64 oracle; AUTO picks it for these shapes (the same bits)."""
    _case(f"thin mfma ci={ci} co={co} {dt}")
    import torch
    rng = np.random.default_rng(ci * 11 + co)
    coords, feats, weight, bias = _rand_case(shells, rng, 2999, ci, co, dt)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    out, _ = _run(gpu_lib, coords, feats, weight, bias, tdt, algo="thin_mfma")
    assert orc.rel_err(out, ref) < TOL_16
    auto, _ = _run(gpu_lib, coords, feats, weight, bias, tdt)
    assert np.array_equal(out, auto)
    o16, _ = _run(gpu_lib, coords, feats, weight, bias, tdt, out_dtype=tdt, algo="thin_mfma")
    assert orc.rel_err(o16, ref) < TOL_16_OUT
    # the 16-bit output is the f32 output rounded once
    assert np.array_equal(o16, torch.from_numpy(out).to(tdt).float().numpy())


def test_thin_mfma_full_size_shells256_c8(gpu_lib, orc, shells):
    """The thin workload at full size (1,694,162 voxels, Ci = Co = 8, bf16): the thin matrix-core
    kernel on every row against the thin VALU kernel, a deterministic row sample against the fp64
    oracle, bitwise reproducibility, and the bf16 output equal to the f32 output rounded once."""
    _case("thin mfma full size shells256-c8-bf16")
    import torch
    w = shells.workload("shells256-c8-bf16")
    nbr = gpu_lib.rulebook_build(torch.from_numpy(w.coords).cuda())
    f, wt, b = _dev(w.feats, torch.bfloat16), _dev(w.weight, torch.bfloat16), _dev(w.bias, torch.float32)
    out = gpu_lib.subm_conv3x3(f, nbr, wt, b, out_dtype=torch.float32, algo="thin_mfma")
    out2 = gpu_lib.subm_conv3x3(f, nbr, wt, b, out_dtype=torch.float32, algo="thin_mfma")
    o16 = gpu_lib.subm_conv3x3(f, nbr, wt, b, out_dtype=torch.bfloat16, algo="thin_mfma")
    outv = gpu_lib.subm_conv3x3(f, nbr, wt, b, out_dtype=torch.float32, algo="thin")
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    assert torch.equal(o16, out.to(torch.bfloat16))
    got = out.cpu().numpy()
    assert orc.rel_err(got, outv.cpu().numpy()) < TOL_16
    rng = np.random.default_rng(8)
    rows = np.unique(np.concatenate([np.arange(64), np.arange(w.n - 64, w.n), rng.integers(0, w.n, 4000)]))
    ref = orc.subm_conv_f64_rows(w.feats, nbr.cpu().numpy(), w.weight, w.bias, rows)
    assert orc.rel_err(got[rows], ref) < TOL_16


def test_thin_mfma_rejects(gpu_lib, shells):
    """algo="thin_mfma" outside its shapes: f32 features, Ci = 4 or 64, Co = 64, mixed dtypes."""
    import torch
    rng = np.random.default_rng(3)
    for ci, co, fdt, wdt in ((8, 8, torch.float32, torch.float32), (4, 8, torch.bfloat16, torch.bfloat16),
                             (64, 8, torch.bfloat16, torch.bfloat16), (8, 64, torch.bfloat16, torch.bfloat16),
                             (8, 8, torch.float16, torch.bfloat16)):
        coords, feats, weight, bias = _rand_case(shells, rng, 100, ci, co, "f32")
        with pytest.raises(gpu_lib.TspError, match="UNSUPPORTED"):
            _run(gpu_lib, coords, feats, weight, bias, fdt, wdtype=wdt, algo="thin_mfma")


@pytest.mark.parametrize("algo", ["thin", "thin_mfma"])
@pytest.mark.parametrize("mode", ["nan_row0", "zero_pad", "row0_source"])
def test_thin_padding_row(gpu_lib, orc, shells, mode, algo):
    """The thin kernel's padding row: a NaN in row 0 makes every row with an absent tap NaN;
    TSP_CONV_ZERO_PAD reads an exact zero row (only row 0's neighbours turn non-finite); an f32
    source row that is finite gives a zero padding row although its f16 rounding overflows."""
    _case(f"thin padding {mode} {algo}")
    import torch
    rng = np.random.default_rng(41)
    coords = np.ascontiguousarray(np.concatenate([shells.sphere_shell(24, 12.0, 7.0, 9.0),
                                                  np.stack(np.meshgrid(*[np.arange(40, 45)] * 3, indexing="ij"),
                                                           -1).reshape(-1, 3)]), np.int32)
    n, ci, co = len(coords), 16, 16
    feats = rng.standard_normal((n, ci)).astype(np.float32)
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / 20).astype(np.float32), "f16")
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    t = nbr.reshape(27, n)
    absent, refs0 = (t == n).any(axis=0), (t == 0).any(axis=0)
    c = torch.from_numpy(coords).cuda()
    nbr_d = gpu_lib.rulebook_build(c)
    w, b = _dev(weight, torch.float16), _dev(bias, torch.float32)
    if mode == "nan_row0":
        feats[0, 3] = np.nan
        f16 = shells.round_to(feats, "f16")
        out = gpu_lib.subm_conv3x3(_dev(f16, torch.float16), nbr_d, w, b, out_dtype=torch.float32, algo=algo)
        out = out.cpu().numpy()
        assert np.isnan(out[absent]).all()
        keep = ~absent & ~refs0
        assert orc.rel_err(out[keep], orc.subm_conv_f64(f16, nbr, weight, bias)[keep]) < TOL_16
    elif mode == "zero_pad":
        feats[0, 3] = np.inf
        f16 = shells.round_to(feats, "f16")
        out = gpu_lib.subm_conv3x3(_dev(f16, torch.float16), nbr_d, w, b, out_dtype=torch.float32, algo=algo,
                                   zero_pad=True).cpu().numpy()
        assert np.isfinite(out[~refs0]).all()
        _nan_aware(out, orc.subm_conv_f64(f16, nbr, weight, bias, zero_pad=True), TOL_16)
    else:
        feats[0, 3] = 1.0e5                         # finite, > 65504: rounds to Inf
        f16 = shells.round_to(feats, "f16")
        out = gpu_lib.subm_conv3x3(_dev(f16, torch.float16), nbr_d, w, b, out_dtype=torch.float32, algo=algo,
                                   row0=_dev(feats[0], torch.float32)).cpu().numpy()
        assert np.isfinite(out[~refs0]).all()
        _nan_aware(out, orc.subm_conv_f64(f16, nbr, weight, bias, row0=feats[0]), TOL_16)


@pytest.mark.parametrize("ci,co", [(64, 64), (32, 128), (128, 128)])
@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_planned_ln_vs_oracle(gpu_lib, orc, shells, ci, co, dtype_name):
    """The conv with its LayerNorm done by the stores (the ConvNeXt block's conv + norm,
    sparse.cpp:121-128) against the fp64 oracle's conv followed by its norm (eps 1e-6, affine),
    both through a plan; one 16-bit rounding of the output."""
    _case(f"planned conv+norm ci={ci} co={co} {dtype_name}")
    import torch
    dt = getattr(torch, dtype_name)
    key = "bf16" if dt == torch.bfloat16 else "f16"
    rng = np.random.default_rng(ci + 3 * co)
    coords, feats, weight, bias = _rand_case(shells, rng, 0, ci, co, key)
    nw = (1 + 0.1 * rng.standard_normal(co)).astype(np.float32)
    nb = (0.1 * rng.standard_normal(co)).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    ref = orc.layer_norm(orc.subm_conv_f64(feats, nbr, weight, bias), nw, nb, 1e-6)
    c = torch.from_numpy(coords).cuda()
    nbr_d = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr_d, len(coords), coords=c)
    pw = gpu_lib.conv_weight_pack(_dev(weight, dt))
    out = gpu_lib.subm_conv3x3_planned_ln(_dev(feats, dt), nbr_d, plan, pw, _dev(bias, torch.float32), co,
                                          _dev(nw, torch.float32), _dev(nb, torch.float32))
    assert out.dtype == dt
    assert orc.rel_err(out.float().cpu().numpy(), ref) < TOL_16_OUT


@pytest.mark.parametrize("co", [64, 128])
def test_planned_ln_vs_separate_full_size(gpu_lib, shells, co):
    """On the ~640K-voxel shell set (1,257 tiles: several per workgroup of the persistent grid, so
    the row-norm stores also run after the cross-tile prefetch): the fused conv + norm against the
    planned conv's f32 rows normalised by the LayerNorm kernel, within one 16-bit rounding."""
    _case(f"planned conv+norm full size co={co}")
    import torch
    w = shells.workload("shells600k-c128-bf16")
    rng = np.random.default_rng(co)
    n, ci = w.n, 128
    c = torch.from_numpy(w.coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr, n, coords=c)
    f = torch.from_numpy(w.feats).to(torch.bfloat16).cuda()
    wt = torch.from_numpy(w.weight[:co]).to(torch.bfloat16).cuda()
    pw = gpu_lib.conv_weight_pack(wt)
    b = torch.from_numpy(w.bias[:co]).cuda()
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(co)).astype(np.float32)).cuda()
    nb = torch.from_numpy((0.1 * rng.standard_normal(co)).astype(np.float32)).cuda()
    fused = gpu_lib.subm_conv3x3_planned_ln(f, nbr, plan, pw, b, co, nw, nb).float()
    h = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, co, out_dtype=torch.float32)
    ref = gpu_lib.layer_norm(h, nw, nb, eps=1e-6, out_dtype=torch.float32)
    torch.cuda.synchronize()
    d = (fused - ref).abs()
    # a bf16 rounding moves a value by at most 2^-9 of it; the two f32 norms differ by far less
    assert bool((d <= ref.abs() * 2.0 ** -8 + 1e-6).all()), float((d / (ref.abs() + 1e-6)).max())


def test_planned_ln_nonfinite_row0(gpu_lib, orc, shells):
    """A NaN in feature row 0 makes every row with an absent tap NaN before the norm (the
    reference's padding row 0 * feats[0]), so those rows are NaN after it; the rest match the
    oracle."""
    _case("planned conv+norm non-finite row 0")
    import torch
    rng = np.random.default_rng(77)
    coords, feats, weight, bias = _rand_case(shells, rng, 0, 64, 64, "bf16")
    feats[0, 3] = np.nan
    n = len(coords)
    nbr = orc.neighbor_table(coords)
    t = nbr.reshape(27, n)
    absent, refs0 = (t == n).any(axis=0), (t == 0).any(axis=0)
    c = torch.from_numpy(coords).cuda()
    nbr_d = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr_d, n, coords=c)
    pw = gpu_lib.conv_weight_pack(_dev(weight, torch.bfloat16))
    nw, nb = np.ones(64, np.float32), np.zeros(64, np.float32)
    out = gpu_lib.subm_conv3x3_planned_ln(_dev(feats, torch.bfloat16), nbr_d, plan, pw, _dev(bias, torch.float32),
                                          64, _dev(nw, torch.float32), _dev(nb, torch.float32)).float().cpu().numpy()
    assert np.isnan(out[absent]).all()
    keep = ~absent & ~refs0
    ref = orc.layer_norm(orc.subm_conv_f64(feats, nbr, weight, bias), nw, nb, 1e-6)
    assert orc.rel_err(out[keep], ref[keep]) < TOL_16_OUT


@pytest.mark.parametrize("seed", list(range(12)))
def test_planned_random_shapes(gpu_lib, orc, shells, seed):
    """Seeded random shapes through the planned conv with a Morton plan: channel counts whose
    slice count is odd (the tile loop without cross-tile pipelining) or even (with it), output
    widths of one to five column tiles, band or scattered voxel sets of 1 to ~12 K voxels, bf16
    and f16, f32 and 16-bit output. Against the fp64 oracle, and bit for bit against the
    unplanned matrix-core conv (the same accumulation order per output, tiles of consecutive
    rows built inside the kernel, which takes Ci % 32 == 0)."""
    import torch
    rng = np.random.default_rng(1000 + seed)
    ci = int(rng.choice([16, 32, 48, 64, 80, 96, 112, 128, 144, 192, 256]))
    co = int(rng.choice([64, 128, 192, 256, 320]))
    key = "bf16" if seed % 2 == 0 else "f16"
    dt = torch.bfloat16 if key == "bf16" else torch.float16
    if seed % 3 == 2:
        coords = shells.random_distinct_voxels(int(rng.integers(1, 6000)), 96, seed)
    else:
        shapes = shells.random_shapes(rng, 48, 2, 6.0, 16.0, boxes=seed % 3 == 1)
        coords = shells.band_voxels(shapes, 48, 2.0)
        coords = coords[: int(rng.integers(1, len(coords) + 1))]
    coords = np.ascontiguousarray(coords, np.int32)
    n = len(coords)
    _case(f"planned random seed={seed} n={n} ci={ci} co={co} {key}")
    feats = shells.round_to(rng.standard_normal((n, ci)).astype(np.float32), key)
    weight = shells.round_to((rng.standard_normal((co, 27, ci)) / np.sqrt(27 * ci)).astype(np.float32), key)
    bias = (rng.standard_normal(co) * 0.1).astype(np.float32)
    c = torch.from_numpy(coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    plan = gpu_lib.conv_plan_build(nbr, n, coords=c)
    f, b = _dev(feats, dt), _dev(bias, torch.float32)
    pw = gpu_lib.conv_weight_pack(_dev(weight, dt))
    odt = torch.float32 if seed % 4 < 2 else dt
    out = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, co, out_dtype=odt)
    unplanned = gpu_lib.subm_conv3x3(f, nbr, _dev(weight, dt), b, out_dtype=odt, algo="mfma") if ci % 32 == 0 \
        else None
    torch.cuda.synchronize()
    ref = orc.subm_conv_f64(feats, orc.neighbor_table(coords), weight, bias)
    assert orc.rel_err(out.float().cpu().numpy(), ref) < (TOL_16 if odt == torch.float32 else TOL_16_OUT)
    assert unplanned is None or torch.equal(out, unplanned)
