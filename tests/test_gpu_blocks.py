"""GPU parity of the per-voxel block pieces (linear, LayerNorm, C2S gather / skip, mask) and of
whole ConvNeXt / C2S blocks composed from the C ABI, against the oracle (fp64).

Tolerance: max|d| / max|ref| <= 1e-5 for fp32 paths; gather, skip and mask are copies, sums
and comparisons and must be exact."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_32 = 1e-5


def _case(name):
    print(f"[blocks] {name}", flush=True)


def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


@pytest.mark.parametrize("n,ci,co", [(1, 8, 3), (300, 64, 256), (1000, 256, 64), (777, 33, 17)])
def test_linear(gpu_lib, orc, n, ci, co):
    _case(f"linear n={n} ci={ci} co={co}")
    import torch
    rng = np.random.default_rng(n + ci + co)
    x = rng.standard_normal((n, ci)).astype(np.float32)
    w = rng.standard_normal((co, ci)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32)
    ref = orc.linear(x, w, b)
    out = gpu_lib.linear(_t(x), _t(w), _t(b)).cpu().numpy()
    assert orc.rel_err(out, ref) < TOL_32
    out_nb = gpu_lib.linear(_t(x), _t(w)).cpu().numpy()      # no bias
    assert orc.rel_err(out_nb, x.astype(np.float64) @ w.T.astype(np.float64)) < TOL_32
    # f32 activations x f16 weights (the reference's default weight dtype)
    w16 = w.astype(np.float16)
    out16 = gpu_lib.linear(_t(x), _t(w16), _t(b)).cpu().numpy()
    assert orc.rel_err(out16, orc.linear(x, w16.astype(np.float32), b)) < TOL_32
    # 16-bit x and weights of one dtype: the matrix-core path when ci % 32 == 0 and co % 64 == 0
    for tdt in (torch.float16, torch.bfloat16):
        xr, wr = _t(x).to(tdt), _t(w).to(tdt)
        ref = orc.linear(xr.float().cpu().numpy(), wr.float().cpu().numpy(), b)
        out = gpu_lib.linear(xr, wr, _t(b), out_dtype=torch.float32).cpu().numpy()
        assert orc.rel_err(out, ref) < TOL_32, tdt
        out_nb = gpu_lib.linear(xr, wr, out_dtype=torch.float32).cpu().numpy()
        assert orc.rel_err(out_nb, ref - b.astype(np.float64)) < TOL_32, tdt



@pytest.mark.parametrize("n,ci,co", [(1000, 64, 256), (777, 128, 512), (3, 32, 64), (4096, 256, 64)])
def test_linear_ex(gpu_lib, orc, n, ci, co):
    """The fused MLP pieces: silu(x W^T + b) rounded to x's dtype (mlp.0 -> SiLU, rounded as
    mlp.2's input) and x W^T + b + residual in f32 (mlp.2 -> + block input), against the oracle
    on the same 16-bit inputs."""
    _case(f"linear_ex n={n} ci={ci} co={co}")
    import torch
    rng = np.random.default_rng(n * 3 + ci + co)
    for tdt in (torch.bfloat16, torch.float16):
        xr = _t(rng.standard_normal((n, ci)).astype(np.float32)).to(tdt)
        wr = _t((rng.standard_normal((co, ci)) / np.sqrt(ci)).astype(np.float32)).to(tdt)
        b = rng.standard_normal(co).astype(np.float32)
        res = rng.standard_normal((n, co)).astype(np.float32)
        pre = orc.linear(xr.float().cpu().numpy(), wr.float().cpu().numpy(), b)
        h = gpu_lib.linear_ex(xr, wr, _t(b), act="silu").float().cpu().numpy()
        ref = orc.silu(pre)
        # one 16-bit rounding of the output on top of fp32 accumulation
        assert orc.rel_err(h, ref) < (8e-3 if tdt == torch.bfloat16 else 1e-3), tdt
        y = gpu_lib.linear_ex(xr, wr, _t(b), residual=_t(res), out_dtype=torch.float32).cpu().numpy()
        assert orc.rel_err(y, pre + res) < TOL_32, tdt
        y0 = gpu_lib.linear_ex(xr, wr, out_dtype=torch.float32).cpu().numpy()   # no bias
        assert orc.rel_err(y0, pre - b.astype(np.float64)) < TOL_32, tdt
    # f32 inputs are not a library GEMM here: the caller falls back to tsp_linear
    with pytest.raises(gpu_lib.TspError, match="UNSUPPORTED"):
        gpu_lib.linear_ex(_t(np.ones((4, 32), np.float32)), _t(np.ones((64, 32), np.float32)))


def test_linear_ex_chunked_over_2gib(gpu_lib, orc):
    """tsp_linear_ex where one operand spans more than 2 GiB: the decoder's last-stage ConvNeXt
    hidden layer, 2,445,586 rows x (128 -> 512) bf16 with f32 output (5.0 GB), which the library
    cuts into calls of tsp_linear_rows_per_call rows (3 here) so that no operand of one hipBLASLt
    call reaches 2^31 bytes. Sampled rows -- both chunk boundaries, the first and last rows and a
    random sample -- against the fp64 oracle: the SiLU output and the residual output."""
    import torch
    n, ci, co = 2_445_586, 128, 512
    L = gpu_lib.lib()
    rows = L.tsp_linear_rows_per_call(ci, co, 2, 0, 0)
    assert rows * co * 4 < 2 ** 31 and n * co * 4 > 2 ** 31 and -(-n // rows) == 3
    _case(f"linear_ex chunked n={n} ci={ci} co={co} rows/call={rows}")
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((n, ci), generator=g, device="cuda").to(torch.bfloat16)
    rng = np.random.default_rng(7)
    w = _t((rng.standard_normal((co, ci)) / np.sqrt(ci)).astype(np.float32)).to(torch.bfloat16)
    b = rng.standard_normal(co).astype(np.float32)
    edges = [0, 1, rows - 1, rows, rows + 1, 2 * rows - 1, 2 * rows, n - 2, n - 1]
    sample = np.unique(np.concatenate([edges, rng.integers(0, n, 3000)]))
    xs = x[torch.from_numpy(sample).cuda()].float().cpu().numpy()
    pre = orc.linear(xs, w.float().cpu().numpy(), b)
    h = gpu_lib.linear_ex(x, w, _t(b), act="silu", out_dtype=torch.float32)
    hs = h[torch.from_numpy(sample).cuda()].cpu().numpy()
    del h
    assert orc.rel_err(hs, orc.silu(pre)) < 1e-4
    res = torch.randn((n, co), generator=g, device="cuda")
    y = gpu_lib.linear_ex(x, w, _t(b), residual=res, out_dtype=torch.float32)
    idx = torch.from_numpy(sample).cuda()
    ys, rs = y[idx].cpu().numpy(), res[idx].cpu().numpy()
    assert orc.rel_err(ys, pre + rs) < TOL_32

@pytest.mark.parametrize("c", [7, 64, 128, 256, 512, 1024, 2048, 4096])
def test_layer_norm(gpu_lib, orc, c):
    _case(f"layer_norm c={c}")
    rng = np.random.default_rng(c)
    x = (rng.standard_normal((333, c)) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(c).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    for affine in (False, True):
        for silu in (False, True):
            ref = orc.layer_norm(x, g if affine else None, b if affine else None, 1e-6)
            if silu:
                ref = orc.silu(ref)
            out = gpu_lib.layer_norm(_t(x), _t(g) if affine else None, _t(b) if affine else None,
                                     1e-6, silu).cpu().numpy()
            assert orc.rel_err(out, ref) < TOL_32, (affine, silu)


def test_c2s_gather_and_skip(gpu_lib, golden):
    _case("c2s gather / skip")
    import torch
    g = golden("subdivide_rand600.npz")
    n = len(g["coords"])
    gidx = g["gidx"]
    m = len(gidx)
    rng = np.random.default_rng(2)
    cout, cin = 24, 32
    h = rng.standard_normal((n, 8 * cout)).astype(np.float32)
    out = gpu_lib.c2s_gather(_t(h), _t(gidx), cout).cpu().numpy()
    assert np.array_equal(out, h.reshape(n * 8, cout)[gidx])
    x = rng.standard_normal((n, cin)).astype(np.float32)
    acc0 = rng.standard_normal((m, cout)).astype(np.float32)
    acc = _t(acc0.copy())
    gpu_lib.c2s_skip_add(_t(x), _t(gidx), acc)
    k = cin // 8
    skip = np.repeat(x.reshape(n * 8, k)[gidx], cout // k, axis=1)
    assert np.array_equal(acc.cpu().numpy(), acc0 + skip)


@pytest.mark.parametrize("rep", [1, 4])
def test_bf16_store_rounding(gpu_lib, rep):
    """fp32 -> bf16 stores round to nearest even, bit for bit: the C2S skip into a zeroed bf16
    accumulator stores bf16(x + 0) for every element of x (rep 4 takes the vectorized kernel,
    rep 1 the scalar one). The expected bits come from torch's CPU conversion. Inputs: random
    finite bit patterns, exact ties (low half 0x8000) on even and odd bf16 values, the patterns
    next to them, subnormals, values that round up to the next binade or to infinity, and
    +-infinity."""
    _case(f"bf16 rounding rep={rep}")
    import torch
    rng = np.random.default_rng(11 + rep)
    hi = rng.integers(0, 1 << 16, 1 << 16, dtype=np.uint32)
    parts = [rng.integers(0, 1 << 32, 1 << 18, dtype=np.uint64).astype(np.uint32)]
    parts += [(hi << 16) | low for low in (0x8000, 0x7FFF, 0x8001, 0xFFFF, 0x0000)]
    parts.append(rng.integers(1, 1 << 23, 1 << 14, dtype=np.uint32) | (rng.integers(0, 2, 1 << 14, dtype=np.uint32) << 31))
    parts.append(np.arange(0x7F7F7F00, 0x7F800000, dtype=np.uint32))
    parts.append(np.array([0x7F800000, 0xFF800000, 0x3F7FFFFF, 0x3F7F8000, 0x00008000], np.uint32))
    bits = np.concatenate(parts)
    bits = bits[(bits & 0x7FFFFFFF) <= 0x7F800000]      # NaN excluded: x + 0 may requiet it
    k = 16
    bits = np.concatenate([bits, np.zeros((-len(bits)) % (8 * k), np.uint32)])
    x = bits.view(np.float32).reshape(-1, 8 * k)
    m = x.shape[0] * 8
    gidx = np.arange(m, dtype=np.int32)
    acc = torch.zeros((m, k * rep), dtype=torch.bfloat16, device="cuda")
    gpu_lib.c2s_skip_add(_t(x), _t(gidx), acc)
    want = torch.from_numpy(np.repeat(x.reshape(m, k) + np.float32(0), rep, axis=1)).to(torch.bfloat16)
    got = acc.cpu()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_mask_positive(gpu_lib):
    _case("mask")
    x = np.array([[-1.0, 0.0, 2.0, -0.0, 1e-30, -1e-30, np.inf, -np.inf]], np.float32)
    assert gpu_lib.mask_positive(_t(x)).cpu().numpy().tolist() == [[0, 0, 1, 0, 1, 0, 1, 0]]


def _params(rng, c, cout=None, scale=0.05):
    s = lambda *shape: (rng.standard_normal(shape) * scale).astype(np.float32)
    p = {"blk.conv.weight": s(c, 27, c), "blk.conv.bias": s(c),
         "blk.norm.weight": 1 + s(c), "blk.norm.bias": s(c),
         "blk.mlp.0.weight": s(4 * c, c), "blk.mlp.0.bias": s(4 * c),
         "blk.mlp.2.weight": s(c, 4 * c), "blk.mlp.2.bias": s(c)}
    if cout:
        p.update({"c2s.to_subdiv.weight": s(8, c) * 20, "c2s.to_subdiv.bias": s(8),
                  "c2s.norm1.weight": 1 + s(c), "c2s.norm1.bias": s(c),
                  "c2s.conv1.weight": s(8 * cout, 27, c), "c2s.conv1.bias": s(8 * cout),
                  "c2s.conv2.weight": s(cout, 27, cout), "c2s.conv2.bias": s(cout)})
    return p


def test_convnext_block_composed(gpu_lib, orc, shells):
    """conv -> LN(1e-6)+affine -> mlp.0 -> SiLU -> mlp.2 -> + x (sparse.cpp:102-137), fp32."""
    _case("convnext block")
    import torch
    rng = np.random.default_rng(4)
    coords = shells.sphere_shell(40, 20.0, 12.0, 14.0)
    c = 32
    x = rng.standard_normal((len(coords), c)).astype(np.float32)
    p = _params(rng, c)
    nbr = gpu_lib.rulebook_build(_t(coords))
    P = {k: _t(v) for k, v in p.items()}
    h = gpu_lib.subm_conv3x3(_t(x), nbr, P["blk.conv.weight"], P["blk.conv.bias"])
    h = gpu_lib.layer_norm(h, P["blk.norm.weight"], P["blk.norm.bias"], 1e-6)
    h = gpu_lib.linear(h, P["blk.mlp.0.weight"], P["blk.mlp.0.bias"])
    h = h * torch.sigmoid(h)           # SiLU in torch (test composition only)
    h = gpu_lib.linear(h, P["blk.mlp.2.weight"], P["blk.mlp.2.bias"]) + _t(x)
    ref = orc.convnext_block(x, orc.neighbor_table(coords), p, "blk")
    assert orc.rel_err(h.cpu().numpy(), ref) < 1e-4


@pytest.mark.parametrize("ext", [False, True])
def test_c2s_block_composed(gpu_lib, orc, shells, ext):
    """to_subdiv -> mask -> subdivide; LN+SiLU -> conv1 -> octant gather -> LN+SiLU -> conv2 on
    the children -> + repeat_interleave skip (sparse.cpp:172-336), fp32."""
    _case(f"c2s block ext={ext}")
    import torch
    rng = np.random.default_rng(5)
    coords = shells.random_distinct_voxels(500, 12, 5)
    n, cin, cout = len(coords), 32, 16
    x = rng.standard_normal((n, cin)).astype(np.float32)
    p = _params(rng, cin, cout)
    P = {k: _t(v) for k, v in p.items()}
    ext_mask = (rng.random(8 * n) < 0.3).astype(np.uint8) if ext else None
    xc, cc = _t(x), _t(coords)
    if ext:
        mask = _t(ext_mask)
    else:
        mask = gpu_lib.mask_positive(gpu_lib.linear(xc, P["c2s.to_subdiv.weight"],
                                                    P["c2s.to_subdiv.bias"])).reshape(-1)
    child, gidx, _ = gpu_lib.subdivide(mask, cc)
    h = gpu_lib.layer_norm(xc, P["c2s.norm1.weight"], P["c2s.norm1.bias"], 1e-6, silu=True)
    h = gpu_lib.subm_conv3x3(h, gpu_lib.rulebook_build(cc), P["c2s.conv1.weight"],
                             P["c2s.conv1.bias"])
    h = gpu_lib.layer_norm(gpu_lib.c2s_gather(h, gidx, cout), None, None, 1e-6, silu=True)
    out = gpu_lib.subm_conv3x3(h, gpu_lib.rulebook_build(child), P["c2s.conv2.weight"],
                               P["c2s.conv2.bias"], zero_pad=True)
    gpu_lib.c2s_skip_add(xc, gidx, out)
    ref, rchild, rmask = orc.c2s_block(x, coords, p, "c2s", cout, ext_mask)
    assert np.array_equal(mask.cpu().numpy().reshape(-1), rmask)
    assert np.array_equal(child.cpu().numpy(), rchild)
    assert orc.rel_err(out.cpu().numpy(), ref) < 1e-4
