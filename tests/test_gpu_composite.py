"""GPU parity of the composite C-ABI blocks, tsp_convnext and tsp_c2s (the ConvNeXt block and the
C2S block's features in one call each), against the oracle's blocks with the same rounding of
each product's input (oracle.act_round). Bar max|d|/max|ref| <= 2e-4, the block bar: the later
products' inputs are rounded on both sides from float32 values computed in different orders.
The plan-less calls run the unplanned kernels, and must agree with the planned ones to the same
bar."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_BLOCK = 2e-4
DT = {"f16": "float16", "bf16": "bfloat16", "f32": "float32"}


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
                                                  (64, "f16", True, True), (32, "f32", False, False)])
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
    ref = orc.convnext_block(x, orc.neighbor_table(coords), q, "blk", wt, cast)
    err = orc.rel_err(out.cpu().numpy(), ref)
    print(f"convnext rel={err:.3e}", flush=True)
    assert err < TOL_BLOCK


@pytest.mark.parametrize("cin,cout,wtype,planned", [(128, 64, "bf16", True), (128, 64, "bf16", False),
                                                    (64, 32, "f16", True), (32, 16, "f32", False)])
def test_c2s(gpu_lib, orc, shells, cin, cout, wtype, planned):
    """After the caller's subdivision (mask, subdivide, the children's table): octant stores and
    skip stores on the planned path at (128, 64); gather and skip passes elsewhere."""
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
    ref, rchild, _ = orc.c2s_block(x, coords, q, "c2s", cout, mask, wt)
    assert np.array_equal(child.cpu().numpy(), rchild)
    err = orc.rel_err(out.cpu().numpy(), ref)
    print(f"c2s rel={err:.3e}", flush=True)
    assert err < TOL_BLOCK
