"""GPU parity of the composite C-ABI blocks, tsp_convnext and tsp_c2s (the ConvNeXt block and the
C2S block's features in one call each), against the oracle's blocks with the same rounding of
each product's input (oracle.act_round). Bar max|d|/max|ref| <= max(2e-4, 1.5 x the case's
rounding noise floor): the later products' inputs are rounded on both sides from float32 values
computed in different orders, so where one lands within that difference of a rounding boundary it
rounds the other way on one side (one ulp of the 16-bit type: 2^-11 for f16, 2^-8 for bf16). The
floor is measured per case on the oracle itself (host_cases.rounding_noise_floor: the oracle
against itself with every product input perturbed by a relative 1e-7 before its rounding), so it
is what two correct evaluation orders differ by; f16 floors sit at ~1e-4, bf16 floors at
~7e-4. The plan-less calls run the unplanned kernels, and must agree with the planned ones to the
same bar."""
from __future__ import annotations

import numpy as np
import pytest

from host_cases import rounding_noise_floor

pytestmark = pytest.mark.gpu

TOL_BLOCK = 2e-4
DT = {"f16": "float16", "bf16": "bfloat16", "f32": "float32"}


def _bar(floor):
    return max(TOL_BLOCK, 1.5 * floor)


def _case(name):
    print(f"[composite] {name}", flush=True)


def _dev(a, dt=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(getattr(torch, DT[dt])) if dt else t


def _params(rng, shapes, wtype):
    """name -> (stored values, device tensor): matrices in wtype, vectors f32."""
    from trellis_cpp_amd.shells import round_to
    out = {}
    for k, (shape, scale, off) in shapes.items():
        v = (rng.standard_normal(shape) * scale + off).astype(np.float32)
        if len(shape) >= 2 and wtype != "f32":
            v = round_to(v, wtype)
        out[k] = (v, _dev(v, wtype if len(shape) >= 2 else None))
    return out


@pytest.mark.parametrize("c,wtype,cast,planned", [(64, "bf16", False, True), (64, "bf16", False, False),
                                                  (128, "f16", False, True), (48, "f16", False, False),
                                                  (64, "f16", True, True), (32, "f32", False, False),
                                                  (128, "bf16", False, True), (256, "bf16", False, False),
                                                  (256, "f16", False, True)])
def test_convnext(gpu_lib, orc, shells, c, wtype, cast, planned):
    _case(f"convnext c={c} {wtype} cast={cast} planned={planned}")
    rng = np.random.default_rng(c + len(wtype))
    coords = np.ascontiguousarray(shells.sphere_shell(20, 10.0, 6.0, 7.5), np.int32)
    n = len(coords)
    x = rng.standard_normal((n, c)).astype(np.float32)
    P = _params(rng, {"conv.weight": ((c, 27, c), 1 / np.sqrt(27 * c), 0), "conv.bias": ((c,), 0.1, 0),
                      "norm.weight": ((c,), 0.1, 1), "norm.bias": ((c,), 0.1, 0),
                      "mlp.0.weight": ((4 * c, c), 1 / np.sqrt(c), 0), "mlp.0.bias": ((4 * c,), 0.1, 0),
                      "mlp.2.weight": ((c, 4 * c), 1 / np.sqrt(4 * c), 0), "mlp.2.bias": ((c,), 0.1, 0)}, wtype)
    nbr = gpu_lib.rulebook_build(_dev(coords))
    plan = gpu_lib.conv_plan_build(nbr, n) if planned else None
    out = gpu_lib.convnext(_dev(x), nbr, {k: v[1] for k, v in P.items()}, plan=plan, cast_f32=cast)
    q = {"blk." + k: v[0] for k, v in P.items()}
    wt = {"blk." + k: (wtype if v[0].ndim >= 2 else "f32") for k, v in P.items()}
    tab = orc.neighbor_table(coords)
    ref, floor = rounding_noise_floor(orc, lambda: orc.convnext_block(x, tab, q, "blk", wt, cast), runs=3)
    err = orc.rel_err(out.cpu().numpy(), ref)
    print(f"convnext rel={err:.3e} floor={floor:.3e}", flush=True)
    assert err < _bar(floor)


def _tail_split_units(n, c, cus):
    """The (tile, column tile) units the planned conv's tail split cuts into parts, for n voxels,
    C = c and `cus` compute units (the library's arithmetic: 8 XCDs, each walking its share of the
    units with cus / 8 workgroups rounded down to a multiple of the column tiles)."""
    nct = c // 128 if c % 128 == 0 else c // 64
    total = -(-n // 512) * nct
    per_xcd = -(-total // 8)
    g = min(per_xcd, max(1, cus // 8 // nct) * nct)
    units = []
    for x in range(8):
        lo = x * per_xcd
        p = min(per_xcd, total - lo)
        if p <= 0:
            continue
        r, t = divmod(p, g)
        if 0 < t and 2 * t <= g:
            units += [lo + r * g + i for i in range(t)]
    return units, nct


@pytest.mark.skip(reason="the planned conv's tail split (the last, thin round of units cut by input-channel "
                         "ranges over the idle CUs) made an illegal memory access on the GPU at C = 256, "
                         "N = 70000 and its cause was not found; the split is not in the library")
@pytest.mark.parametrize("c,n", [(1024, 16600), (256, 70000)])
def test_convnext_tail_split(gpu_lib, orc, shells, c, n):
    """The ConvNeXt conv on a stored plan at sizes whose last round of (tile, column tile) units is
    thin, so that its units are cut by input-channel ranges over the idle CUs and their parts added
    by a second pass (the decoder's 33.5 K-voxel level at C = 1024 is such a size): rows of every
    split unit's tile and random rows against the oracle's block, at the block bar, and two runs
    bit-identical."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    units, nct = _tail_split_units(n, c, cus)
    _case(f"convnext tail split c={c} n={n}: {len(units)} split units on {cus} CUs")
    assert units, "the size was chosen to split"
    rng = np.random.default_rng(c + n)
    coords = np.ascontiguousarray(shells.sphere_shell(140, 70.0, 40.0, 52.0)[:n], np.int32)
    assert len(coords) == n
    x = rng.standard_normal((n, c)).astype(np.float32)
    P = _params(rng, {"conv.weight": ((c, 27, c), 1 / np.sqrt(27 * c), 0), "conv.bias": ((c,), 0.1, 0),
                      "norm.weight": ((c,), 0.1, 1), "norm.bias": ((c,), 0.1, 0),
                      "mlp.0.weight": ((4 * c, c), 1 / np.sqrt(c), 0), "mlp.0.bias": ((4 * c,), 0.1, 0),
                      "mlp.2.weight": ((c, 4 * c), 1 / np.sqrt(4 * c), 0), "mlp.2.bias": ((c,), 0.1, 0)}, "bf16")
    nbr = gpu_lib.rulebook_build(_dev(coords))
    plan = gpu_lib.conv_plan_build(nbr, n)          # row tiles: tile t holds rows [512 t, 512 t + 512)
    wd = {k: v[1] for k, v in P.items()}
    out = gpu_lib.convnext(_dev(x), nbr, wd, plan=plan)
    out2 = gpu_lib.convnext(_dev(x), nbr, wd, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    tiles = sorted({u // nct for u in units})
    rows = np.unique(np.concatenate([np.concatenate([rng.choice(np.arange(512 * t, min(n, 512 * t + 512)), 24,
                                                                replace=False) for t in tiles]),
                                     rng.integers(0, n, 200)]))
    q = {"blk." + k: v[0] for k, v in P.items()}
    wt = {"blk." + k: ("bf16" if v[0].ndim >= 2 else "f32") for k, v in P.items()}
    tab = orc.neighbor_table(coords)
    ref, floor = rounding_noise_floor(orc, lambda: orc.convnext_block_rows(x, tab, q, "blk", rows, wt), runs=2)
    err = orc.rel_err(out.cpu().numpy()[rows], ref)
    print(f"tail split rel={err:.3e} floor={floor:.3e} rows={len(rows)}", flush=True)
    assert err < _bar(floor)


@pytest.mark.parametrize("c,dt,n", [(128, "bf16", 1), (128, "bf16", 5001), (128, "f16", 300),
                                    (128, "bf16", 40001), (128, "f16", 8192 + 33)])
def test_convnext_mlp(gpu_lib, orc, c, dt, n):
    """tsp_convnext_mlp (mlp.0, SiLU, mlp.2 and the block input in one kernel; a workgroup per CU
    walks 32-row blocks, so n > 32 x CUs takes several blocks a workgroup) against a float64
    statement of the same products with the hidden layer rounded to the input's type, as the
    stored hidden layer of the two-GEMM path is; also in place (out = x), and against that path
    (tsp_linear_ex twice) on the same inputs. Bar: max|d|/max|ref| <= max(TOL_BLOCK, 1.5 x the
    statement's rounding noise floor) (a hidden value may round the other way where the SiLU
    lands within the two computations' difference of a rounding boundary)."""
    import torch
    from trellis_cpp_amd.shells import round_to
    _case(f"convnext mlp c={c} {dt} n={n}")
    rng = np.random.default_rng(c + n)
    xn = round_to(rng.standard_normal((n, c)).astype(np.float32), dt)
    w0 = round_to((rng.standard_normal((4 * c, c)) / np.sqrt(c)).astype(np.float32), dt)
    w2 = round_to((rng.standard_normal((c, 4 * c)) / np.sqrt(4 * c)).astype(np.float32), dt)
    b0 = (rng.standard_normal(4 * c) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal(c) * 0.1).astype(np.float32)
    x = rng.standard_normal((n, c)).astype(np.float32)
    def statement():
        hpre = xn.astype(np.float64) @ w0.astype(np.float64).T + b0
        hid = orc.act_round(hpre / (1.0 + np.exp(-hpre)), dt)   # the hidden layer, rounded as stored
        return x + b2 + hid @ w2.astype(np.float64).T
    ref, floor = rounding_noise_floor(orc, statement, runs=3)
    packed = gpu_lib.convnext_mlp_pack(_dev(w0, dt), _dev(w2, dt))
    out = gpu_lib.convnext_mlp(_dev(xn, dt), packed, _dev(b0), _dev(b2), _dev(x))
    xd = _dev(x)
    inplace = gpu_lib.convnext_mlp(_dev(xn, dt), packed, _dev(b0), _dev(b2), xd, out=xd)
    torch.cuda.synchronize()
    scale = np.abs(ref).max()
    err = np.abs(out.cpu().numpy() - ref).max() / scale
    two = gpu_lib.linear_ex(gpu_lib.linear_ex(_dev(xn, dt), _dev(w0, dt), _dev(b0), act="silu"), _dev(w2, dt),
                            _dev(b2), residual=_dev(x), out_dtype=torch.float32)
    err2 = np.abs(out.cpu().numpy() - two.cpu().numpy()).max() / scale
    print(f"mlp rel={err:.3e} vs two GEMMs {err2:.3e}", flush=True)
    print(f"mlp floor={floor:.3e}", flush=True)
    assert err < _bar(floor) and err2 < _bar(floor)
    assert torch.equal(inplace, out)


@pytest.mark.parametrize("cin,cout,wtype,planned", [(128, 64, "bf16", True), (128, 64, "bf16", False),
                                                    (64, 32, "f16", True), (32, 16, "f32", False),
                                                    (64, 64, "f16", True), (256, 128, "bf16", True),
                                                    (128, 128, "f16", True)])
def test_c2s(gpu_lib, orc, shells, cin, cout, wtype, planned):
    """After the caller's subdivision (mask, subdivide, the children's table): octant stores and
    skip stores on the planned path at Cout = 64 and 128, where conv1's stores also normalise the
    children and apply SiLU (one wave, or both column waves of a workgroup, holding whole child
    rows); gather and skip passes elsewhere."""
    import torch
    _case(f"c2s {cin}->{cout} {wtype} planned={planned}")
    rng = np.random.default_rng(cin + cout)
    coords = np.ascontiguousarray(shells.sphere_shell(16, 8.0, 5.0, 6.5), np.int32)
    n = len(coords)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    mask = (rng.random(8 * n) < 0.4).astype(np.uint8)
    P = _params(rng, {"norm1.weight": ((cin,), 0.1, 1), "norm1.bias": ((cin,), 0.1, 0),
                      "conv1.weight": ((8 * cout, 27, cin), 1 / np.sqrt(27 * cin), 0),
                      "conv1.bias": ((8 * cout,), 0.1, 0),
                      "conv2.weight": ((cout, 27, cout), 1 / np.sqrt(27 * cout), 0),
                      "conv2.bias": ((cout,), 0.1, 0)}, wtype)
    cc, mt = _dev(coords), _dev(mask)
    nbr = gpu_lib.rulebook_build(cc)
    child, gidx, mstart = gpu_lib.subdivide(mt, cc)
    m = len(gidx)
    cnbr = gpu_lib.rulebook_build(child)
    plans = (gpu_lib.conv_plan_build(nbr, n), gpu_lib.conv_plan_build(cnbr, m)) if planned else (None, None)
    out = gpu_lib.c2s(_dev(x), nbr, mt, mstart, gidx, m, cout, cnbr, {k: v[1] for k, v in P.items()},
                      plan=plans[0], child_plan=plans[1])
    torch.cuda.synchronize()
    q = {"c2s." + k: v[0] for k, v in P.items()}
    wt = {"c2s." + k: (wtype if v[0].ndim >= 2 else "f32") for k, v in P.items()}
    (ref, rchild, _), floor = rounding_noise_floor(orc, lambda: orc.c2s_block(x, coords, q, "c2s", cout, mask, wt),
                                                   runs=3)
    assert np.array_equal(child.cpu().numpy(), rchild)
    err = orc.rel_err(out.cpu().numpy(), ref)
    print(f"c2s rel={err:.3e} floor={floor:.3e}", flush=True)
    assert err < _bar(floor)


@pytest.mark.parametrize("cin,cout,wtype,o16", [(128, 64, "bf16", None), (256, 128, "f16", "f16"),
                                               (128, 64, "f16", "bf16")])
def test_c2s_in_parts(gpu_lib, shells, cin, cout, wtype, o16):
    """tsp_c2s_part: the front part once, then conv2 over ranges of the child plan's tiles (a plan
    without coordinates: tile t holds children [512 t, 512 t + 512)), in an order other than
    ascending and with an empty range, equals tsp_c2s_ex bit for bit (out and its rounded copy);
    a range past the last tile is refused, and so is a conv2 range where conv2 does not store the
    skip itself (Cout = 32: no matrix-core conv2)."""
    import torch
    _case(f"c2s in parts {cin}->{cout} {wtype} out16={o16}")
    rng = np.random.default_rng(cin + 3 * cout)
    coords = np.ascontiguousarray(shells.sphere_shell(40, 20.0, 15.0, 17.5), np.int32)
    n = len(coords)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    mask = (rng.random(8 * n) < 0.45).astype(np.uint8)
    P = _params(rng, {"norm1.weight": ((cin,), 0.1, 1), "norm1.bias": ((cin,), 0.1, 0),
                      "conv1.weight": ((8 * cout, 27, cin), 1 / np.sqrt(27 * cin), 0),
                      "conv1.bias": ((8 * cout,), 0.1, 0),
                      "conv2.weight": ((cout, 27, cout), 1 / np.sqrt(27 * cout), 0),
                      "conv2.bias": ((cout,), 0.1, 0)}, wtype)
    p = {k: v[1] for k, v in P.items()}
    cc, mt = _dev(coords), _dev(mask)
    nbr = gpu_lib.rulebook_build(cc)
    child, gidx, mstart = gpu_lib.subdivide(mt, cc)
    m = len(gidx)
    cnbr = gpu_lib.rulebook_build(child)
    plan, cplan = gpu_lib.conv_plan_build(nbr, n, coords=cc), gpu_lib.conv_plan_build(cnbr, m)
    t16 = None if o16 is None else getattr(torch, DT[o16])
    xd = _dev(x)
    args = (xd, nbr, mt, mstart, gidx, m, cout, cnbr, p)
    whole = gpu_lib.c2s(*args, plan=plan, child_plan=cplan, out16_dtype=t16)
    nt = -(-m // 512)
    assert nt >= 6, "enough child tiles for several ranges"
    ranges = [(nt // 2, nt - nt // 2), (0, 0), (3, nt // 2 - 3), (0, 3)]
    parts = gpu_lib.c2s(*args, plan=plan, child_plan=cplan, out16_dtype=t16, conv2_tiles=ranges)
    torch.cuda.synchronize()
    if t16 is None:
        assert torch.equal(parts, whole)
    else:
        assert torch.equal(parts[0], whole[0]) and torch.equal(parts[1].view(torch.int16), whole[1].view(torch.int16))
    with pytest.raises(gpu_lib.TspError, match="tiles"):
        gpu_lib.c2s(*args, plan=plan, child_plan=cplan, conv2_tiles=[(nt - 1, 2)])
    P32 = _params(rng, {"norm1.weight": ((cin,), 0.1, 1), "norm1.bias": ((cin,), 0.1, 0),
                        "conv1.weight": ((8 * 32, 27, cin), 1 / np.sqrt(27 * cin), 0),
                        "conv1.bias": ((8 * 32,), 0.1, 0),
                        "conv2.weight": ((32, 27, 32), 1 / np.sqrt(27 * 32), 0),
                        "conv2.bias": ((32,), 0.1, 0)}, wtype)
    with pytest.raises(gpu_lib.TspError, match="range of tiles"):
        gpu_lib.c2s(xd, nbr, mt, mstart, gidx, m, 32, cnbr, {k: v[1] for k, v in P32.items()}, plan=plan,
                    child_plan=cplan, conv2_tiles=[(0, 1)])
    torch.cuda.synchronize()


@pytest.mark.parametrize("c,wtype,planned,o16", [(128, "bf16", True, "bf16"), (128, "f16", True, "f16"),
                                                 (128, "bf16", True, "f16"), (256, "bf16", True, "bf16"),
                                                 (64, "bf16", False, "bf16")])
def test_convnext_rounded_copies(gpu_lib, shells, c, wtype, planned, o16):
    """tsp_convnext_ex: the rounded copy of out equals out rounded to nearest even, bit for bit (the
    fused MLP's stores at C = 128, a rounding pass elsewhere); out itself is the same as without
    the copy; and giving x's rounded copy (x16) leaves out unchanged, bit for bit."""
    import torch
    _case(f"convnext copies c={c} {wtype} planned={planned} out16={o16}")
    rng = np.random.default_rng(7 * c + len(wtype))
    coords = np.ascontiguousarray(shells.sphere_shell(20, 10.0, 6.0, 7.5), np.int32)
    n = len(coords)
    x = rng.standard_normal((n, c)).astype(np.float32)
    P = _params(rng, {"conv.weight": ((c, 27, c), 1 / np.sqrt(27 * c), 0), "conv.bias": ((c,), 0.1, 0),
                      "norm.weight": ((c,), 0.1, 1), "norm.bias": ((c,), 0.1, 0),
                      "mlp.0.weight": ((4 * c, c), 1 / np.sqrt(c), 0), "mlp.0.bias": ((4 * c,), 0.1, 0),
                      "mlp.2.weight": ((c, 4 * c), 1 / np.sqrt(4 * c), 0), "mlp.2.bias": ((c,), 0.1, 0)}, wtype)
    p = {k: v[1] for k, v in P.items()}
    nbr = gpu_lib.rulebook_build(_dev(coords))
    plan = gpu_lib.conv_plan_build(nbr, n) if planned else None
    xd = _dev(x)
    t16 = getattr(torch, DT[o16])
    base = gpu_lib.convnext(xd, nbr, p, plan=plan)
    out, out16 = gpu_lib.convnext(xd, nbr, p, plan=plan, out16_dtype=t16)
    with_x16 = gpu_lib.convnext(xd, nbr, p, plan=plan, x16=xd.to(getattr(torch, DT[wtype])))
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    assert torch.equal(out16.view(torch.int16), out.cpu().to(t16).cuda().view(torch.int16))
    assert torch.equal(with_x16, base)


@pytest.mark.parametrize("cin,cout,wtype,o16", [(256, 128, "bf16", "bf16"), (128, 64, "f16", "f16"),
                                                (64, 32, "bf16", "bf16")])
def test_c2s_rounded_copy(gpu_lib, shells, cin, cout, wtype, o16):
    """tsp_c2s_ex: the rounded copy of out equals out rounded to nearest even, bit for bit -- from
    conv2's skip stores (Cout / (Cin / 8) a multiple of 4) or from a rounding pass (64 -> 32) --
    and out is the same as without the copy."""
    import torch
    _case(f"c2s copy {cin}->{cout} {wtype} out16={o16}")
    rng = np.random.default_rng(cin + 3 * cout)
    coords = np.ascontiguousarray(shells.sphere_shell(16, 8.0, 5.0, 6.5), np.int32)
    n = len(coords)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    mask = (rng.random(8 * n) < 0.4).astype(np.uint8)
    P = _params(rng, {"norm1.weight": ((cin,), 0.1, 1), "norm1.bias": ((cin,), 0.1, 0),
                      "conv1.weight": ((8 * cout, 27, cin), 1 / np.sqrt(27 * cin), 0),
                      "conv1.bias": ((8 * cout,), 0.1, 0),
                      "conv2.weight": ((cout, 27, cout), 1 / np.sqrt(27 * cout), 0),
                      "conv2.bias": ((cout,), 0.1, 0)}, wtype)
    p = {k: v[1] for k, v in P.items()}
    cc, mt = _dev(coords), _dev(mask)
    nbr = gpu_lib.rulebook_build(cc)
    child, gidx, mstart = gpu_lib.subdivide(mt, cc)
    m = len(gidx)
    cnbr = gpu_lib.rulebook_build(child)
    plans = (gpu_lib.conv_plan_build(nbr, n), gpu_lib.conv_plan_build(cnbr, m))
    t16 = getattr(torch, DT[o16])
    base = gpu_lib.c2s(_dev(x), nbr, mt, mstart, gidx, m, cout, cnbr, p, plan=plans[0], child_plan=plans[1])
    out, out16 = gpu_lib.c2s(_dev(x), nbr, mt, mstart, gidx, m, cout, cnbr, p, plan=plans[0], child_plan=plans[1],
                             out16_dtype=t16)
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    assert torch.equal(out16.view(torch.int16), out.cpu().to(t16).cuda().view(torch.int16))


def _region_mask(coords, rng, p_keep=0.5):
    """A subdivision mask whose kept octants depend on the parent's 8^3 region, so that whole
    32-parent blocks of a tile keep none of some octants (those blocks' conv1 MFMAs for that
    octant are skipped)."""
    reg = (coords[:, 0] >> 3) * 73 + (coords[:, 1] >> 3) * 31 + (coords[:, 2] >> 3) * 7
    keep_reg = np.stack([(np.random.default_rng(o).random(reg.max() + 1) < p_keep)[reg] for o in range(8)], 1)
    return (keep_reg & (rng.random((len(coords), 8)) < 0.8)).astype(np.uint8).reshape(-1)


@pytest.mark.parametrize("cin,cout,wtype", [(256, 256, "bf16"), (512, 256, "f16")])
def test_c2s_octant_skip_bitexact(gpu_lib, shells, cin, cout, wtype):
    """tsp_c2s at Cout >= 256 (conv1 with octant stores, no child norm) skips conv1's MFMAs for
    row blocks whose parents keep none of a wave's octant; its output equals, bit for bit, the
    same block composed from the single entry points (norm1 + SiLU, the octant conv without the
    skip, norm2 + SiLU, the skip conv), on a mask that empties whole blocks' octants."""
    import torch
    _case(f"c2s octant skip {cin}->{cout} {wtype}")
    rng = np.random.default_rng(cin + cout + 1)
    coords = np.ascontiguousarray(shells.sphere_shell(40, 20.0, 12.0, 15.0), np.int32)
    n = len(coords)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    mask = _region_mask(coords, rng)
    P = _params(rng, {"norm1.weight": ((cin,), 0.1, 1), "norm1.bias": ((cin,), 0.1, 0),
                      "conv1.weight": ((8 * cout, 27, cin), 1 / np.sqrt(27 * cin), 0),
                      "conv1.bias": ((8 * cout,), 0.1, 0),
                      "conv2.weight": ((cout, 27, cout), 1 / np.sqrt(27 * cout), 0),
                      "conv2.bias": ((cout,), 0.1, 0)}, wtype)
    p = {k: v[1] for k, v in P.items()}
    cc, mt = _dev(coords), _dev(mask)
    nbr = gpu_lib.rulebook_build(cc)
    child, gidx, mstart = gpu_lib.subdivide(mt, cc)
    m = len(gidx)
    cnbr = gpu_lib.rulebook_build(child)
    plan, cplan = gpu_lib.conv_plan_build(nbr, n, coords=cc), gpu_lib.conv_plan_build(cnbr, m, coords=child)
    xd = _dev(x)
    out = gpu_lib.c2s(xd, nbr, mt, mstart, gidx, m, cout, cnbr, p, plan=plan, child_plan=cplan)
    t16 = getattr(torch, DT[wtype])
    h0 = gpu_lib.layer_norm(xd, p["norm1.weight"], p["norm1.bias"], 1e-6, silu=True, out_dtype=t16)
    g = gpu_lib.subm_conv3x3_planned_octants(h0, nbr, plan, gpu_lib.conv_weight_pack(p["conv1.weight"]),
                                             p["conv1.bias"], cout, mt, mstart, m)
    h2 = gpu_lib.layer_norm(g, None, None, 1e-6, silu=True, out_dtype=t16)
    ref = gpu_lib.subm_conv3x3_planned_skip(h2, cnbr, cplan, gpu_lib.conv_weight_pack(p["conv2.weight"]),
                                            p["conv2.bias"], cout, xd, gidx)
    torch.cuda.synchronize()
    assert m > 0 and torch.equal(out, ref)


@pytest.mark.parametrize("cin,cout,wtype", [(128, 64, "bf16"), (256, 128, "f16"), (512, 256, "bf16")])
def test_c2s_octant_skip_vs_oracle(gpu_lib, orc, shells, cin, cout, wtype):
    """The same skip in the norm-in-stores kernels (Cout = 64, 128) and the plain octant stores,
    against the oracle's block, on masks that empty whole blocks' octants."""
    import torch
    _case(f"c2s octant skip oracle {cin}->{cout} {wtype}")
    rng = np.random.default_rng(cin + 5 * cout)
    coords = np.ascontiguousarray(shells.sphere_shell(24, 12.0, 7.0, 9.0), np.int32)
    n = len(coords)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    mask = _region_mask(coords, rng)
    P = _params(rng, {"norm1.weight": ((cin,), 0.1, 1), "norm1.bias": ((cin,), 0.1, 0),
                      "conv1.weight": ((8 * cout, 27, cin), 1 / np.sqrt(27 * cin), 0),
                      "conv1.bias": ((8 * cout,), 0.1, 0),
                      "conv2.weight": ((cout, 27, cout), 1 / np.sqrt(27 * cout), 0),
                      "conv2.bias": ((cout,), 0.1, 0)}, wtype)
    cc, mt = _dev(coords), _dev(mask)
    nbr = gpu_lib.rulebook_build(cc)
    child, gidx, mstart = gpu_lib.subdivide(mt, cc)
    m = len(gidx)
    cnbr = gpu_lib.rulebook_build(child)
    plans = (gpu_lib.conv_plan_build(nbr, n, coords=cc), gpu_lib.conv_plan_build(cnbr, m, coords=child))
    out = gpu_lib.c2s(_dev(x), nbr, mt, mstart, gidx, m, cout, cnbr, {k: v[1] for k, v in P.items()},
                      plan=plans[0], child_plan=plans[1])
    torch.cuda.synchronize()
    q = {"c2s." + k: v[0] for k, v in P.items()}
    wt = {"c2s." + k: (wtype if v[0].ndim >= 2 else "f32") for k, v in P.items()}
    (ref, rchild, _), floor = rounding_noise_floor(orc, lambda: orc.c2s_block(x, coords, q, "c2s", cout, mask, wt),
                                                   runs=3)
    assert np.array_equal(child.cpu().numpy(), rchild)
    err = orc.rel_err(out.cpu().numpy(), ref)
    print(f"c2s skip rel={err:.3e} floor={floor:.3e}", flush=True)
    assert err < _bar(floor)
