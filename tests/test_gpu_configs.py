"""GPU parity at the shapes of the two benchmark configurations the other conv tests do not reach:

* band512-c64-bf16 at its full size: the seed-3 256^3 shell set subdivided 2x and pruned to the
  thickness-2 band at 512^3 (5.87 M voxels, the ext-mask route of sparse.cpp:215), then a C = 64
  submanifold conv. Subdivision and neighbour table bit-exact; the planned MFMA conv on sampled
  rows against the fp64 oracle.
* the decoder stack's first widths (shape_decoder.cpp:88-90: 1024 -> 512): a ConvNeXt block at
  C = 1024 (conv, mlp.0 1024 -> 4096 with SiLU, mlp.2 4096 -> 1024 with the residual) and the C2S
  convs (conv1 1024 -> 8 x 512 with octant stores, conv2 512 -> 512 with the skip), on a small
  shell so the fp64 oracle stays fast.

Bars as elsewhere: exact for integer work; max|d|/max|ref| <= 1e-3 for 16-bit inputs with fp32
accumulation against the fp64 oracle on the same rounded inputs (a 16-bit output one rounding
more: 4e-3)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_16 = 1e-3
TOL_16_OUT = 4e-3


def _case(name):
    print(f"[configs] {name}", flush=True)


def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def test_band512_full_size(gpu_lib, orc, shells):
    import torch
    _case("band512: parents and mask")
    rng, parents, mask = shells.band512_parents()
    pc, mt = _t(parents), _t(mask)
    child, gidx, mstart = gpu_lib.subdivide(mt, pc)
    rchild, rgidx, rmstart = orc.subdivide(mask, parents)
    _case(f"band512: {len(parents)} parents -> {len(rchild)} children")
    assert np.array_equal(child.cpu().numpy(), rchild)
    assert np.array_equal(gidx.cpu().numpy(), rgidx)
    assert np.array_equal(mstart.cpu().numpy(), rmstart)
    n = len(rchild)
    assert n > 5_000_000

    _case("band512: neighbour table")
    nbr = gpu_lib.rulebook_build(child)
    ref_nbr = orc.neighbor_table(rchild)
    assert np.array_equal(nbr.cpu().numpy(), ref_nbr)

    _case("band512: planned C=64 conv")
    feats, weight, bias = shells.conv_inputs(rng, n, 64, 64, 1 / np.sqrt(27 * 64), "bf16", 0.1)
    f, w, b = _t(feats, torch.bfloat16), _t(weight, torch.bfloat16), _t(bias)
    plan = gpu_lib.conv_plan_build(nbr, n)
    pw = gpu_lib.conv_weight_pack(w)
    out = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, 64, out_dtype=torch.float32)
    out16 = gpu_lib.subm_conv3x3_planned(f, nbr, plan, pw, b, 64, out_dtype=torch.bfloat16)
    direct = gpu_lib.subm_conv3x3(f, nbr, w, b, out_dtype=torch.float32, algo="mfma")
    torch.cuda.synchronize()
    assert torch.equal(out, direct)      # the stored plan only reorders the same sums
    sample = np.random.default_rng(3)
    rows = np.unique(np.concatenate([np.arange(512), np.arange(n - 512, n), sample.integers(0, n, 4000)]))
    ref = orc.subm_conv_f64_rows(feats, ref_nbr, weight, bias, rows)
    assert orc.rel_err(out.cpu().numpy()[rows], ref) < TOL_16
    assert orc.rel_err(out16.float().cpu().numpy()[rows], ref) < TOL_16_OUT


def _round(shells, a, key="bf16"):
    return shells.round_to(np.asarray(a, np.float32), key)


def test_decoder_widths_convnext_1024(gpu_lib, orc, shells):
    """ConvNeXt block at C = 1024 as the decoder runs it (sparse.cpp:102-137): the planned conv on
    bf16 features, LayerNorm + affine rounded to bf16, mlp.0 (1024 -> 4096) with its bias and SiLU
    in one GEMM rounded to bf16, mlp.2 (4096 -> 1024) with its bias and the f32 block input. Each
    piece against the oracle on the same rounded inputs, then the block against the oracle that
    rounds at the same three points."""
    import torch
    _case("ConvNeXt C=1024")
    rng = np.random.default_rng(4)
    coords = np.ascontiguousarray(shells.sphere_shell(16, 8.0, 5.0, 6.5), np.int32)
    n, c = len(coords), 1024
    x = rng.standard_normal((n, c)).astype(np.float32)
    std = 0.02
    p = {"conv.weight": _round(shells, rng.standard_normal((c, 27, c)) * std),
         "conv.bias": (rng.standard_normal(c) * std).astype(np.float32),
         "norm.weight": (1 + rng.standard_normal(c) * 0.1).astype(np.float32),
         "norm.bias": (rng.standard_normal(c) * 0.1).astype(np.float32),
         "mlp.0.weight": _round(shells, rng.standard_normal((4 * c, c)) * std),
         "mlp.0.bias": (rng.standard_normal(4 * c) * std).astype(np.float32),
         "mlp.2.weight": _round(shells, rng.standard_normal((c, 4 * c)) * std),
         "mlp.2.bias": (rng.standard_normal(c) * std).astype(np.float32)}
    P = {k: _t(v, torch.bfloat16 if v.ndim >= 2 else torch.float32) for k, v in p.items()}
    nbr_h = orc.neighbor_table(coords)
    nbr = gpu_lib.rulebook_build(_t(coords))
    x16 = _round(shells, x)

    # conv 1024 -> 1024
    plan = gpu_lib.conv_plan_build(nbr, n)
    pw = gpu_lib.conv_weight_pack(P["conv.weight"])
    h = gpu_lib.subm_conv3x3_planned(_t(x16, torch.bfloat16), nbr, plan, pw, P["conv.bias"], c,
                                     out_dtype=torch.float32)
    h_ref = orc.subm_conv_f64(x16, nbr_h, p["conv.weight"], p["conv.bias"])
    assert orc.rel_err(h.cpu().numpy(), h_ref) < TOL_16

    # LayerNorm + affine, rounded to bf16 (mlp.0's input)
    hn = gpu_lib.layer_norm(h, P["norm.weight"], P["norm.bias"], 1e-6, out_dtype=torch.bfloat16)
    # mlp.0: 1024 -> 4096, bias and SiLU in the GEMM, bf16 out
    hid = gpu_lib.linear_ex(hn, P["mlp.0.weight"], P["mlp.0.bias"], act="silu")
    hid_ref = orc.silu(orc.linear(hn.float().cpu().numpy(), p["mlp.0.weight"], p["mlp.0.bias"]))
    assert orc.rel_err(hid.float().cpu().numpy(), hid_ref) < 8e-3       # one bf16 rounding of the output
    # mlp.2: 4096 -> 1024, bias and the f32 block input in the GEMM
    y = gpu_lib.linear_ex(hid, P["mlp.2.weight"], P["mlp.2.bias"], residual=_t(x), out_dtype=torch.float32)
    y_ref = orc.linear(hid.float().cpu().numpy(), p["mlp.2.weight"], p["mlp.2.bias"]) + x
    assert orc.rel_err(y.cpu().numpy(), y_ref) < 1e-5
    torch.cuda.synchronize()

    # the block against the oracle rounding at the same points
    r = orc.layer_norm(h_ref, p["norm.weight"], p["norm.bias"], 1e-6)
    r = orc.silu(orc.linear(_round(shells, r), p["mlp.0.weight"], p["mlp.0.bias"]))
    r = orc.linear(_round(shells, r), p["mlp.2.weight"], p["mlp.2.bias"]) + x
    err = orc.rel_err(y.cpu().numpy(), r)
    print(f"ConvNeXt C=1024 block rel={err:.3e}", flush=True)
    assert err < TOL_16


def test_decoder_widths_c2s_1024_to_512(gpu_lib, orc, shells):
    """The first C2S block's convs at the decoder's widths (sparse.cpp:172-336; 1024 -> 512):
    conv1 1024 -> 8 x 512 with its octant gather in the stores, and conv2 512 -> 512 on the
    children (exact zero padding row) with the repeat-interleaved skip (K = 128, R = 4) added by
    its stores, against the oracle's conv, gather and skip on the same bf16 inputs."""
    import torch
    _case("C2S 1024 -> 512")
    rng = np.random.default_rng(5)
    coords = np.ascontiguousarray(shells.sphere_shell(16, 8.0, 5.0, 6.5), np.int32)
    n, cin, cout = len(coords), 1024, 512
    std = 0.02
    h0 = _round(shells, rng.standard_normal((n, cin)))                     # LN1 + SiLU output, bf16
    w1 = _round(shells, rng.standard_normal((8 * cout, 27, cin)) * std)
    b1 = (rng.standard_normal(8 * cout) * std).astype(np.float32)
    w2 = _round(shells, rng.standard_normal((cout, 27, cout)) * std)
    b2 = (rng.standard_normal(cout) * std).astype(np.float32)
    x = rng.standard_normal((n, cin)).astype(np.float32)                   # the block input
    mask = (rng.random(8 * n) < 0.45).astype(np.uint8)
    cc = _t(coords)
    nbr = gpu_lib.rulebook_build(cc)
    plan = gpu_lib.conv_plan_build(nbr, n)
    mt = _t(mask)
    child, gidx, mstart = gpu_lib.subdivide(mt, cc)
    m = len(gidx)
    g = gpu_lib.subm_conv3x3_planned_octants(_t(h0, torch.bfloat16), nbr, plan,
                                             gpu_lib.conv_weight_pack(_t(w1, torch.bfloat16)), _t(b1), cout,
                                             mt, mstart, m)
    # conv1 rows of the first 160 parents, gathered to their children
    nbr_h = orc.neighbor_table(coords)
    parents = np.arange(160)
    h1 = orc.subm_conv_f64_rows(h0, nbr_h, w1, b1, parents)
    gi = gidx.cpu().numpy()
    mine = gi // 8 < 160
    ref1 = h1.reshape(160 * 8, cout)[gi[mine]]
    assert orc.rel_err(g.cpu().numpy()[mine], ref1) < TOL_16

    # conv2 on the children with the skip
    h2 = _round(shells, rng.standard_normal((m, cout)))                    # norm2 + SiLU output, bf16
    cnbr = gpu_lib.rulebook_build(child)
    cplan = gpu_lib.conv_plan_build(cnbr, m)
    out = gpu_lib.subm_conv3x3_planned_skip(_t(h2, torch.bfloat16), cnbr, cplan,
                                            gpu_lib.conv_weight_pack(_t(w2, torch.bfloat16)), _t(b2), cout,
                                            _t(x), gidx)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(min(m, 400)), np.random.default_rng(1).integers(0, m, 400)]))
    k = cin // 8
    skip = np.repeat(x.reshape(n * 8, k)[gi[rows]], cout // k, axis=1)
    ref2 = orc.subm_conv_f64_rows(h2, orc.neighbor_table(child.cpu().numpy()), w2, b2, rows,
                                  zero_pad=True) + skip
    assert orc.rel_err(out.cpu().numpy()[rows], ref2) < TOL_16
