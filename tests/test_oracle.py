"""CPU tests that pin the oracle: golden fixtures, independent statements of each result,
closed forms, library routines and invariants. Each check is chosen so that a plausible
mistake (wrong tap order, transposed weight, dropped term, off-by-one octant) fails it; the
`*_planted` tests plant such mistakes in the oracle's inputs and assert the checks notice."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from host_cases import decode_closed_form, zero_weight_decoder


# ------------------------------------------------------------------------------------------
# Rulebook
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("fixture", ["rulebook_rand800.npz", "rulebook_edges.npz"])
def test_rulebook_golden(orc, golden, fixture):
    g = golden(fixture)
    for fn in (orc.neighbor_table, orc.neighbor_table_grid, orc.neighbor_table_sorted):
        assert np.array_equal(fn(g["coords"]), g["nbr"])


def test_rulebook_three_way_random(orc, shells):
    rng = np.random.default_rng(11)
    sets = [
        shells.sphere_shell(24, 12.0, 7.0, 9.0),
        rng.integers(0, 12, size=(3000, 3)).astype(np.int32),        # many duplicates
        rng.integers(0, 1 << 20, size=(2000, 3)).astype(np.int32),   # sparse, huge coords
        np.zeros((0, 3), np.int32),
        np.array([[3, 4, 5]], np.int32),
    ]
    for c in sets:
        a = orc.neighbor_table(c)
        c_small = c if (len(c) == 0 or c.max() < 4096) else None
        if c_small is not None:
            assert np.array_equal(a, orc.neighbor_table_grid(c))
        assert np.array_equal(a, orc.neighbor_table_sorted(c))


def test_rulebook_tap_convention(orc):
    # tap t = kd*9 + kh*3 + kw reads the voxel at (x+kd-1, y+kh-1, z+kw-1) (sparse.h:14-16)
    c = np.array([[5, 5, 5], [6, 5, 4], [4, 6, 5]], np.int32)
    nbr = orc.neighbor_table(c).reshape(27, 3)
    t_b = 2 * 9 + 1 * 3 + 0          # offset (+1, 0, -1) from voxel 0
    t_c = 0 * 9 + 2 * 3 + 1          # offset (-1, +1, 0) from voxel 0
    assert nbr[t_b, 0] == 1 and nbr[t_c, 0] == 2
    assert nbr[26 - t_b, 1] == 0     # the mirror tap sees voxel 0 from voxel 1
    assert all(nbr[t, 0] == 3 for t in range(27) if t not in (t_b, t_c, 13))
    assert nbr[13].tolist() == [0, 1, 2]


def test_rulebook_special_cases(orc):
    iso = np.array([[10, 10, 10], [20, 20, 20]], np.int32)
    nbr = orc.neighbor_table(iso).reshape(27, 2)
    assert nbr[13].tolist() == [0, 1] and (np.delete(nbr, 13, 0) == 2).all()
    cube = np.array([(x, y, z) for x in range(3) for y in range(3) for z in range(3)], np.int32)
    nbr = orc.neighbor_table(cube).reshape(27, 27)
    centre = 13                     # voxel (1,1,1) is row 13 in x-major order
    assert nbr[:, centre].tolist() == list(range(27))
    dup = np.array([[1, 1, 1], [2, 1, 1], [1, 1, 1], [1, 1, 1]], np.int32)
    nbr = orc.neighbor_table(dup).reshape(27, 4)
    assert nbr[13].tolist() == [3, 1, 3, 3]          # last insert wins (sparse.cpp:26)
    assert nbr[9 * 2 + 3 + 1, 0] == 1                 # (+1,0,0) neighbour
    assert nbr[0 * 9 + 3 + 1, 1] == 3                 # (-1,0,0) from (2,1,1) -> last dup
    assert orc.neighbor_table(np.zeros((0, 3), np.int32)).size == 0


def test_rulebook_planted(orc):
    """A table built with the z and x offsets swapped must fail the fixture check."""
    c = np.array([[5, 5, 5], [6, 5, 5], [5, 5, 6]], np.int32)
    good = orc.neighbor_table(c)
    swapped = orc.neighbor_table(c[:, ::-1].copy())   # planted: axes reversed
    assert not np.array_equal(good, swapped)


def test_count_pairs(orc, golden):
    g = golden("rulebook_rand800.npz")
    n = len(g["coords"])
    assert orc.count_pairs(g["nbr"], n) == int((g["nbr"] != n).sum())


# ------------------------------------------------------------------------------------------
# Conv
# ------------------------------------------------------------------------------------------
def _dense_box(rng, dims, ci):
    X, Y, Z = dims
    coords = np.array([(x, y, z) for x in range(X) for y in range(Y) for z in range(Z)],
                      np.int32)
    feats = rng.standard_normal((len(coords), ci)).astype(np.float32)
    return coords, feats


def _conv3d_reference(coords, feats, weight, bias, dims):
    """torch.nn.functional.conv3d with zero padding 1 on the dense box (a textbook routine):
    on a fully occupied box the submanifold conv is exactly this cross-correlation."""
    X, Y, Z = dims
    ci = feats.shape[1]
    co = weight.shape[0]
    dense = torch.zeros(1, ci, X, Y, Z, dtype=torch.float64)
    cc = torch.from_numpy(coords.astype(np.int64))
    dense[0, :, cc[:, 0], cc[:, 1], cc[:, 2]] = torch.from_numpy(feats).double().T
    w = torch.from_numpy(weight).double().reshape(co, 3, 3, 3, ci).permute(0, 4, 1, 2, 3)
    out = F.conv3d(dense, w.contiguous(), torch.from_numpy(bias).double(), padding=1)
    return out[0, :, cc[:, 0], cc[:, 1], cc[:, 2]].T.numpy()


def test_conv_dense_box_equals_conv3d(orc):
    rng = np.random.default_rng(5)
    dims = (5, 4, 6)
    coords, feats = _dense_box(rng, dims, 8)
    weight = rng.standard_normal((7, 27, 8)).astype(np.float32)
    bias = rng.standard_normal(7).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    ref = _conv3d_reference(coords, feats, weight, bias, dims)
    assert np.allclose(orc.subm_conv_f64(feats, nbr, weight, bias), ref, rtol=1e-12, atol=1e-10)
    assert orc.rel_err(orc.subm_conv_f32(feats, nbr, weight, bias), ref) < 1e-6


def test_conv_zero_pad_dense_box(orc):
    """zero_pad: absent taps read an exact zero row. On a dense box the only absent taps point
    out of the box, where conv3d's zero padding reads zeros too, so with an Inf at one voxel the
    zero-padded sparse conv equals conv3d, NaN and Inf positions included: only that voxel's
    neighbours are non-finite. The reference padding 0 * feats[0] instead makes every boundary
    voxel NaN when the Inf sits in row 0, so it must differ from conv3d there."""
    rng = np.random.default_rng(8)
    dims = (4, 5, 4)
    coords, feats = _dense_box(rng, dims, 6)
    weight = rng.standard_normal((5, 27, 6)).astype(np.float32)
    bias = rng.standard_normal(5).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    for row in (0, 37):
        f = feats.copy()
        f[row, 2] = np.inf
        with np.errstate(invalid="ignore"):
            ref = _conv3d_reference(coords, f, weight, bias, dims)
        got = orc.subm_conv_f64(f, nbr, weight, bias, zero_pad=True)
        assert np.array_equal(np.isfinite(got), np.isfinite(ref))
        fin = np.isfinite(ref)
        assert np.allclose(got[fin], ref[fin], rtol=1e-12, atol=1e-10)
        assert (~np.isfinite(got)).any(axis=1).sum() == (nbr.reshape(27, -1) == row).any(axis=0).sum()
        rows = np.arange(0, len(coords), 3)
        assert np.array_equal(np.isfinite(orc.subm_conv_f64_rows(f, nbr, weight, bias, rows, zero_pad=True)),
                              np.isfinite(got[rows]))
    f0 = feats.copy()
    f0[0, 2] = np.inf
    default = orc.subm_conv_f64(f0, nbr, weight, bias)
    boundary = (nbr.reshape(27, -1) == len(coords)).any(axis=0)
    assert np.isnan(default[boundary]).all()


def test_conv_dense_box_planted(orc):
    """Weights with the tap axis mirrored (a transposed kernel) must fail the conv3d check."""
    rng = np.random.default_rng(6)
    dims = (4, 4, 4)
    coords, feats = _dense_box(rng, dims, 4)
    weight = rng.standard_normal((3, 27, 4)).astype(np.float32)
    bias = np.zeros(3, np.float32)
    nbr = orc.neighbor_table(coords)
    ref = _conv3d_reference(coords, feats, weight, bias, dims)
    planted = weight[:, ::-1, :].copy()
    assert orc.rel_err(orc.subm_conv_f64(feats, nbr, planted, bias), ref) > 1e-2
    planted_t = weight.reshape(3, 3, 3, 3, 4).transpose(0, 3, 2, 1, 4).reshape(3, 27, 4).copy()
    assert orc.rel_err(orc.subm_conv_f64(feats, nbr, planted_t, bias), ref) > 1e-2


def test_conv_golden(orc, golden):
    g = golden("conv_rand800_c32.npz")
    nbr = orc.neighbor_table(g["coords"])
    out = orc.subm_conv_f64(g["feats"], nbr, g["weight"], g["bias"])
    assert np.allclose(out, g["out"], rtol=1e-12, atol=1e-12)
    assert orc.rel_err(orc.subm_conv_f32(g["feats"], nbr, g["weight"], g["bias"]), g["out"]) < 1e-5


def test_conv_invariants(orc, shells):
    rng = np.random.default_rng(7)
    coords = shells.sphere_shell(20, 10.0, 5.0, 7.0)
    n = len(coords)
    f1 = rng.standard_normal((n, 16)).astype(np.float32)
    f2 = rng.standard_normal((n, 16)).astype(np.float32)
    w = rng.standard_normal((8, 27, 16)).astype(np.float32)
    b0 = np.zeros(8, np.float32)
    nbr = orc.neighbor_table(coords)
    y1, y2 = orc.subm_conv_f64(f1, nbr, w, b0), orc.subm_conv_f64(f2, nbr, w, b0)
    y12 = orc.subm_conv_f64((2 * f1 + f2).astype(np.float32), nbr, w, b0)
    # (2*f1 + f2 is rounded to f32 before the conv, hence the 1e-5 tolerance)
    assert np.allclose(y12, 2 * y1 + y2, rtol=1e-5, atol=1e-5)          # linear in features
    w2 = rng.standard_normal((8, 27, 16)).astype(np.float32)
    yw = orc.subm_conv_f64(f1, nbr, (w + w2).astype(np.float32), b0)
    assert np.allclose(yw, y1 + orc.subm_conv_f64(f1, nbr, w2, b0), rtol=1e-5, atol=1e-5)
    shifted = coords + np.array([7, 3, 11], np.int32)                  # translation invariance
    assert np.array_equal(orc.neighbor_table(shifted), nbr)
    perm = rng.permutation(n)                                           # row relabelling
    nbr_p = orc.neighbor_table(coords[perm])
    yp = orc.subm_conv_f64(f1[perm], nbr_p, w, b0)
    assert np.allclose(yp, y1[perm], atol=1e-12)
    bias = rng.standard_normal(8).astype(np.float32)                    # bias added once
    assert np.allclose(orc.subm_conv_f64(f1, nbr, w, bias), y1 + bias, atol=1e-12)



def test_conv_sentinel_row(orc, shells):
    """The padding row absent taps read is 0 * feats[0] (submconv_pad, sparse.cpp:81-85), not a
    zero row: with finite features it contributes nothing, so changing row 0 moves only the
    outputs of row 0's neighbours; with an Inf or a NaN in row 0 every output row that has an
    absent tap is NaN in every channel (0 * Inf = NaN, and NaN * w = NaN), and the rows whose 27
    taps are all present stay finite. A zero sentinel row would leave them all finite."""
    rng = np.random.default_rng(17)
    coords = np.concatenate([shells.sphere_shell(20, 10.0, 5.0, 7.0),
                             np.stack(np.meshgrid(*[np.arange(30, 34)] * 3, indexing="ij"), -1).reshape(-1, 3)])
    coords = np.ascontiguousarray(coords, np.int32)
    n = len(coords)
    f = rng.standard_normal((n, 16)).astype(np.float32)
    w = rng.standard_normal((8, 27, 16)).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float32)
    nbr = orc.neighbor_table(coords)
    absent = (nbr.reshape(27, n) == n).any(axis=0)
    assert absent.any() and (~absent).any()             # the 4^3 block's interior has all 27
    near0 = (nbr.reshape(27, n) == 0).any(axis=0)
    f2 = f.copy()
    f2[0] = rng.standard_normal(16).astype(np.float32) * 100
    for conv in (orc.subm_conv_f64, orc.subm_conv_f32):
        y, y2 = conv(f, nbr, w, b), conv(f2, nbr, w, b)
        assert np.array_equal(y[~near0], y2[~near0])    # finite row 0: the padding adds +-0
        for bad in (np.inf, -np.inf, np.nan):
            f3 = f.copy()
            f3[0, 5] = bad
            y3 = conv(f3, nbr, w, b)
            assert np.isnan(y3[absent]).all()
            assert np.isfinite(y3[~absent & ~near0]).all()


def test_conv_rows_variants(orc, golden):
    g = golden("conv_rand800_c32.npz")
    nbr = orc.neighbor_table(g["coords"])
    rows = np.array([0, 5, 799, 400], np.int64)
    r64 = orc.subm_conv_f64_rows(g["feats"], nbr, g["weight"], g["bias"], rows)
    assert np.allclose(r64, g["out"][rows], rtol=0, atol=1e-12)
    r32 = orc.subm_conv_f32_rows(g["feats"], nbr, g["weight"], g["bias"], 100, 200)
    full = orc.subm_conv_f32(g["feats"], nbr, g["weight"], g["bias"])
    assert np.array_equal(r32[100:200], full[100:200])


# ------------------------------------------------------------------------------------------
# Subdivision
# ------------------------------------------------------------------------------------------
def test_subdivide_golden(orc, golden):
    g = golden("subdivide_rand600.npz")
    ch, gi, ms = orc.subdivide(g["mask"], g["coords"])
    assert np.array_equal(ch, g["child"]) and np.array_equal(gi, g["gidx"])
    assert np.array_equal(ms, g["mstart"])


def test_subdivide_properties(orc, shells):
    rng = np.random.default_rng(8)
    coords = shells.random_distinct_voxels(300, 12, 8)
    for p in (0.0, 0.2, 1.0):
        mask = (rng.random(8 * 300) < p).astype(np.uint8) * rng.integers(1, 255, 8 * 300).astype(np.uint8)
        ch, gi, ms = orc.subdivide(mask, coords)
        ch2, gi2, ms2 = orc.subdivide_vectorised(mask, coords)
        assert np.array_equal(ch, ch2) and np.array_equal(gi, gi2) and np.array_equal(ms, ms2)
        m = len(ch)
        assert m == int((mask != 0).sum()) and ms[-1] == m
        parent, octant = gi // 8, gi % 8
        assert np.array_equal(ch >> 1, coords[parent])                   # child / 2 = parent
        bits = np.stack([(octant >> a) & 1 for a in range(3)], 1)
        assert np.array_equal(ch & 1, bits)                              # bit0->x,1->y,2->z
        assert np.all(np.diff(gi) > 0)                                   # parent-major order
        assert len(np.unique(ch, axis=0)) == m                           # children distinct


def test_subdivide_planted(orc, golden):
    g = golden("subdivide_rand600.npz")
    ch, _, _ = orc.subdivide(g["mask"], g["coords"])
    planted = orc.subdivide(g["mask"].reshape(-1, 8)[:, ::-1].reshape(-1).copy(), g["coords"])[0]
    assert not np.array_equal(ch, planted)     # reversed octant bit order is caught


# ------------------------------------------------------------------------------------------
# Block arithmetic against torch library routines
# ------------------------------------------------------------------------------------------
def test_layer_norm_and_silu(orc):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((50, 24))
    w, b = rng.standard_normal(24), rng.standard_normal(24)
    ref = F.layer_norm(torch.from_numpy(x), (24,), torch.from_numpy(w), torch.from_numpy(b), 1e-6)
    assert np.allclose(orc.layer_norm(x, w, b, 1e-6), ref.numpy(), atol=1e-12)
    assert np.allclose(orc.silu(x), F.silu(torch.from_numpy(x)).numpy(), atol=1e-14)


def _block_params(rng, c, cout=None):
    p = {}
    s = lambda *shape: (rng.standard_normal(shape) * 0.05).astype(np.float32)
    pre = "blk"
    p[pre + ".conv.weight"], p[pre + ".conv.bias"] = s(c, 27, c), s(c)
    p[pre + ".norm.weight"], p[pre + ".norm.bias"] = (1 + s(c)), s(c)
    p[pre + ".mlp.0.weight"], p[pre + ".mlp.0.bias"] = s(4 * c, c), s(4 * c)
    p[pre + ".mlp.2.weight"], p[pre + ".mlp.2.bias"] = s(c, 4 * c), s(c)
    if cout:
        p["c2s.to_subdiv.weight"], p["c2s.to_subdiv.bias"] = s(8, c) * 20, s(8)
        p["c2s.norm1.weight"], p["c2s.norm1.bias"] = (1 + s(c)), s(c)
        p["c2s.conv1.weight"], p["c2s.conv1.bias"] = s(8 * cout, 27, c), s(8 * cout)
        p["c2s.conv2.weight"], p["c2s.conv2.bias"] = s(cout, 27, cout), s(cout)
    return p


def test_convnext_block_vs_torch(orc, shells):
    """sparse.cpp:102-137 restated with torch's layer_norm / linear / silu."""
    rng = np.random.default_rng(10)
    coords = shells.random_distinct_voxels(200, 8, 10)
    c = 16
    x = rng.standard_normal((200, c)).astype(np.float32)
    p = _block_params(rng, c)
    nbr = orc.neighbor_table(coords)
    out = orc.convnext_block(x, nbr, p, "blk")
    T = lambda a: torch.from_numpy(np.asarray(a)).double()
    h = T(orc.subm_conv_f64(x, nbr, p["blk.conv.weight"], p["blk.conv.bias"]))
    h = F.layer_norm(h, (c,), T(p["blk.norm.weight"]), T(p["blk.norm.bias"]), 1e-6)
    h = F.silu(F.linear(h, T(p["blk.mlp.0.weight"]), T(p["blk.mlp.0.bias"])))
    h = F.linear(h, T(p["blk.mlp.2.weight"]), T(p["blk.mlp.2.bias"])) + T(x)
    assert np.allclose(out, h.numpy(), atol=1e-10)


def test_convnext_block_rows_vs_whole_block(orc, shells):
    """convnext_block_rows equals the rows of convnext_block (a row's block output depends on its
    conv row and its own input only), with and without product-input rounding; a planted mistake
    (the rows' block read from the neighbouring rows) must differ."""
    rng = np.random.default_rng(14)
    coords = shells.random_distinct_voxels(300, 9, 14)
    c = 16
    x = rng.standard_normal((300, c)).astype(np.float32)
    p = _block_params(rng, c)
    nbr = orc.neighbor_table(coords)
    rows = np.array([0, 1, 7, 150, 298, 299, 42])
    for wt in (None, {k: ("bf16" if v.ndim >= 2 else "f32") for k, v in p.items()}):
        whole = orc.convnext_block(x, nbr, p, "blk", wt)
        part = orc.convnext_block_rows(x, nbr, p, "blk", rows, wt)
        assert np.allclose(part, whole[rows], rtol=1e-12, atol=1e-12)
        assert not np.allclose(part, whole[(rows + 1) % 300], rtol=1e-6, atol=1e-6)


def test_c2s_block_vs_loops(orc, shells):
    """sparse.cpp:172-336 against a per-(parent, octant) loop statement of SparseResBlockC2S3d
    (the formulation of tools/ref_c2s.py:59-79)."""
    rng = np.random.default_rng(12)
    n, cin, cout = 120, 16, 8
    coords = shells.random_distinct_voxels(n, 8, 12)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    p = _block_params(rng, cin, cout)
    out, child, mask = orc.c2s_block(x, coords, p, "c2s", cout)
    T = lambda a: torch.from_numpy(np.asarray(a)).double()
    logits = F.linear(T(x), T(p["c2s.to_subdiv.weight"]), T(p["c2s.to_subdiv.bias"]))
    sub = (logits > 0).numpy()
    assert np.array_equal(mask.reshape(n, 8) != 0, sub)
    h = F.silu(F.layer_norm(T(x), (cin,), T(p["c2s.norm1.weight"]), T(p["c2s.norm1.bias"]), 1e-6))
    nbr = orc.neighbor_table(coords)
    h = orc.subm_conv_f64(h.numpy().astype(np.float32), nbr, p["c2s.conv1.weight"], p["c2s.conv1.bias"])
    rows, kids, skips = [], [], []
    k = cin // 8
    for i in range(n):
        for o in range(8):
            if sub[i, o]:
                xx, yy, zz = coords[i]
                kids.append((2 * xx + (o & 1), 2 * yy + ((o >> 1) & 1), 2 * zz + ((o >> 2) & 1)))
                rows.append(h[i, o * cout:(o + 1) * cout])
                skips.append(np.repeat(x[i, o * k:(o + 1) * k].astype(np.float64), cout // k))
    kids = np.array(kids, np.int32)
    assert np.array_equal(kids, child)
    hn = F.silu(F.layer_norm(T(np.array(rows)), (cout,), None, None, 1e-6)).numpy()
    nbr2 = orc.neighbor_table(kids).reshape(27, -1)
    # conv2 as the reference states it: hn with its zero padding column M appended
    # (silu(norm(0)) = 0, sparse.cpp:289-306), gathered per tap and multiplied
    m = len(kids)
    hn_pad = np.concatenate([hn.astype(np.float32).astype(np.float64), np.zeros((1, cout))])
    w2 = p["c2s.conv2.weight"].astype(np.float64)
    h2 = p["c2s.conv2.bias"].astype(np.float64) + sum(hn_pad[nbr2[t]] @ w2[:, t, :].T for t in range(27))
    assert nbr2.shape[1] == m
    assert np.allclose(out, h2 + np.array(skips), atol=1e-9)


def test_rounding_matches_library_conversions(orc):
    """round_f16 / round_bf16 against numpy's float16 and torch's bfloat16 conversions of the
    float32 values (round to nearest even), including ties, overflow, subnormals and NaN."""
    rng = np.random.default_rng(21)
    x = np.concatenate([rng.standard_normal(5000) * 10.0 ** rng.integers(-8, 6, 5000),
                        [0.0, -0.0, 65504.0, 65520.0, 1e5, -1e5, 6e-8, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                         1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, np.inf, -np.inf, np.nan]]).astype(np.float32)
    f16 = orc.round_f16(x)
    ref16 = x.astype(np.float16).astype(np.float64)
    bad = np.nonzero(~((f16 == ref16) | (np.isnan(f16) & np.isnan(ref16))))[0]
    assert bad.size == 0, [(float(x[i]), float(f16[i]), float(ref16[i])) for i in bad[:8]]
    bf = orc.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float64).numpy()
    assert np.array_equal(bf, ref, equal_nan=True)
    assert orc.round_f16(np.float32(1.0 + 2.0 ** -11)) == 1.0              # tie to even
    assert orc.round_bf16(np.float32(1.0 + 3 * 2.0 ** -8)) == 1.0 + 2.0 ** -6


def test_act_round_rule(orc):
    """ggml's mul_mat input rounding: F16/BF16 weights round to their type, F32 weights do not;
    g_sparse_cast_f32 lifts it for F16 conv weights only (w32 casts F16, sparse.cpp:16-19)."""
    x = np.float32(1.0 + 2.0 ** -10 + 2.0 ** -13)   # not representable in F16 or BF16
    assert orc.act_round(x, "f16") == orc.round_f16(x) != x
    assert orc.act_round(x, "bf16") == orc.round_bf16(x) != x
    assert orc.act_round(x, "f32") == x and orc.act_round(x, None) == x
    assert orc.act_round(x, "f16", conv_weight=True, cast_f32=True) == x
    assert orc.act_round(x, "f16", conv_weight=False, cast_f32=True) == orc.round_f16(x)
    assert orc.act_round(x, "bf16", conv_weight=True, cast_f32=True) == orc.round_bf16(x)


def test_convnext_block_rounds_each_product_input(orc, shells):
    """With wt, the block equals the same block on inputs rounded at the three products: the conv
    (feats), mlp.0 (the LN + affine output) and mlp.2 (the SiLU output)."""
    rng = np.random.default_rng(14)
    coords = shells.random_distinct_voxels(150, 7, 14)
    c = 16
    x = rng.standard_normal((150, c)).astype(np.float32)
    p = _block_params(rng, c)
    wt = {k: ("f16" if v.ndim >= 2 else "f32") for k, v in p.items()}
    nbr = orc.neighbor_table(coords)
    out = orc.convnext_block(x, nbr, p, "blk", wt)
    T = lambda a: torch.from_numpy(np.asarray(a)).double()
    r16 = lambda a: T(np.asarray(a, np.float64).astype(np.float32).astype(np.float16).astype(np.float64))
    h = T(orc.subm_conv_f64(r16(x).numpy().astype(np.float32), nbr, p["blk.conv.weight"], p["blk.conv.bias"]))
    h = F.layer_norm(h, (c,), T(p["blk.norm.weight"]), T(p["blk.norm.bias"]), 1e-6)
    h = F.silu(F.linear(r16(h), T(p["blk.mlp.0.weight"]), T(p["blk.mlp.0.bias"])))
    h = F.linear(r16(h), T(p["blk.mlp.2.weight"]), T(p["blk.mlp.2.bias"])) + T(x)
    assert np.allclose(out, h.numpy(), atol=1e-10)
    assert not np.allclose(out, orc.convnext_block(x, nbr, p, "blk"), atol=1e-6)   # the rounding shows


def test_decode_unet_zero_weight_closed_form(orc, shells):
    """decode_unet pinned by the closed form its zero-weight case reduces to: the stage loop (2 and
    1 blocks), the C2S skip's octant slice and repeat, the guide masks' routing and child order,
    and the head's LayerNorm (eps 1e-5, no affine). A planted eps of 1e-6, a dropped block or a
    swapped octant slice moves the closed form far beyond the bar."""
    rng = np.random.default_rng(31)
    coords = shells.random_distinct_voxels(60, 6, 31)
    latent = rng.standard_normal((60, 8)).astype(np.float32)
    p, stages = zero_weight_decoder(rng, (32, 16, 8), (2, 1))
    guide, n = [], 60
    for _ in stages:
        guide.append((rng.random(8 * n) < 0.4).astype(np.uint8))
        n = int(guide[-1].sum())
    out, coords_out, masks = orc.decode_unet(latent, coords, p, stages, 6, guide)
    ref, rc = decode_closed_form(latent, coords, p, stages, guide)
    assert np.array_equal(coords_out, rc)
    assert all(np.array_equal(m, g) for m, g in zip(masks, guide))
    scale = np.abs(ref).max()
    assert np.abs(out - ref).max() < 1e-5 * scale
    far = lambda r: np.abs(r[0] - ref).max() > 1e-3 * scale
    # (an earlier stage's block bias reaches the head as a constant per child, which the head's
    # LayerNorm removes: the skip of the later stage repeats each element of its slice)
    q = dict(p)
    q[stages[1][0][0] + ".mlp.2.bias"] = np.zeros_like(p[stages[1][0][0] + ".mlp.2.bias"])
    assert far(decode_closed_form(latent, coords, q, stages, guide))                 # a block dropped
    assert far(decode_closed_form(latent, coords, p, stages, guide, eps=1e-6))       # the head's eps
    assert far(decode_closed_form(latent, coords, p, stages, guide, octant_shift=1))  # the skip's slice


def test_rounding_noise_floor_helper(orc, shells):
    """The decoder tests' noise floor: nonzero where products round (flips appear), zero where
    nothing rounds, and the oracle's rounding rule restored afterwards."""
    from host_cases import rounding_noise_floor
    rng = np.random.default_rng(15)
    coords = shells.random_distinct_voxels(150, 7, 15)
    x = rng.standard_normal((150, 16)).astype(np.float32)
    p = _block_params(rng, 16)
    nbr = orc.neighbor_table(coords)
    wt = {k: ("bf16" if v.ndim >= 2 else "f32") for k, v in p.items()}
    exact = orc.act_round
    out, floor = rounding_noise_floor(orc, lambda: orc.convnext_block(x, nbr, p, "blk", wt), rel=1e-4)
    assert orc.act_round is exact
    assert np.array_equal(out, orc.convnext_block(x, nbr, p, "blk", wt))
    assert 0 < floor < 1e-2
    _, none = rounding_noise_floor(orc, lambda: orc.convnext_block(x, nbr, p, "blk"), rel=1e-4)
    assert none == 0


@pytest.mark.parametrize("wtype", ["bf16", "f16"])
def test_block_bar_catches_planted_mistakes(orc, shells, wtype):
    """The block tests' bar, max(2e-4, 1.5 x the rounding noise floor), on the ConvNeXt block at
    C = 128 (the composite test's case): the floor itself stays below the bar, while plausible
    mistakes in the rounding of the product inputs -- none at all, the other 16-bit type,
    truncation instead of round-to-nearest-even, or a systematic relative error of 3e-4 in every
    product input -- move the block by more than the bar."""
    from host_cases import rounding_noise_floor
    c = 128
    rng = np.random.default_rng(c + len(wtype))
    coords = np.ascontiguousarray(shells.sphere_shell(20, 10.0, 6.0, 7.5), np.int32)
    x = rng.standard_normal((len(coords), c)).astype(np.float32)
    shapes = {"conv.weight": ((c, 27, c), 1 / np.sqrt(27 * c), 0), "conv.bias": ((c,), 0.1, 0),
              "norm.weight": ((c,), 0.1, 1), "norm.bias": ((c,), 0.1, 0),
              "mlp.0.weight": ((4 * c, c), 1 / np.sqrt(c), 0), "mlp.0.bias": ((4 * c,), 0.1, 0),
              "mlp.2.weight": ((c, 4 * c), 1 / np.sqrt(4 * c), 0), "mlp.2.bias": ((c,), 0.1, 0)}
    q, wt = {}, {}
    for k, (shape, scale, off) in shapes.items():
        v = (rng.standard_normal(shape) * scale + off).astype(np.float32)
        q["blk." + k] = shells.round_to(v, wtype) if len(shape) >= 2 else v
        wt["blk." + k] = wtype if len(shape) >= 2 else "f32"
    tab = orc.neighbor_table(coords)
    ref, floor = rounding_noise_floor(orc, lambda: orc.convnext_block(x, tab, q, "blk", wt), runs=3)
    bar = max(2e-4, 1.5 * floor)
    assert 0 < floor < bar
    exact = orc.act_round
    other = "f16" if wtype == "bf16" else "bf16"
    keep = 16 if wtype == "bf16" else 13   # mantissa bits dropped by truncation to the 16-bit type

    def truncate(v, wtype_, conv_weight=False, cast_f32=False):
        u = np.asarray(v, np.float32).view(np.uint32) & np.uint32((0xffffffff >> keep) << keep)
        return exact(u.view(np.float32), wtype_, conv_weight, cast_f32)

    planted = {
        "no rounding": lambda v, w_, cw=False, cf=False: np.asarray(v, np.float64),
        "other type": lambda v, w_, cw=False, cf=False: exact(v, other if w_ == wtype else w_, cw, cf),
        "truncation": truncate,
        "relative 3e-4": lambda v, w_, cw=False, cf=False: exact(np.asarray(v, np.float64) * (1 + 3e-4), w_, cw, cf),
    }
    for name, fn in planted.items():
        orc.act_round = fn
        try:
            moved = orc.rel_err(orc.convnext_block(x, tab, q, "blk", wt), ref)
        finally:
            orc.act_round = exact
        assert moved > bar, (name, moved, bar)


@pytest.mark.parametrize("wtype", ["bf16", "f32"])
def test_c2s_block_rows_equals_block(orc, shells, wtype):
    """c2s_block_rows (the C2S block on sampled child rows, for sets too large to run whole)
    equals the whole block's rows exactly, including the first and last child and parents whose
    octants are all pruned; decoder_head_rows equals decode_unet's head on a one-stage decoder."""
    rng = np.random.default_rng(17)
    coords = shells.sphere_shell(20, 10.0, 6.0, 7.5)
    n, cin, cout = len(coords), 32, 16
    x = rng.standard_normal((n, cin)).astype(np.float32)
    rnd = (lambda v: shells.round_to(v, wtype)) if wtype != "f32" else (lambda v: v)
    p = {"c.norm1.weight": (1 + 0.1 * rng.standard_normal(cin)).astype(np.float32),
         "c.norm1.bias": (0.1 * rng.standard_normal(cin)).astype(np.float32),
         "c.conv1.weight": rnd((rng.standard_normal((8 * cout, 27, cin)) / 30).astype(np.float32)),
         "c.conv1.bias": (0.1 * rng.standard_normal(8 * cout)).astype(np.float32),
         "c.conv2.weight": rnd((rng.standard_normal((cout, 27, cout)) / 20).astype(np.float32)),
         "c.conv2.bias": (0.1 * rng.standard_normal(cout)).astype(np.float32)}
    wt = {k: (wtype if v.ndim >= 2 else "f32") for k, v in p.items()}
    mask = (rng.random(8 * n) < 0.4).astype(np.uint8)
    mask[:8 * 5] = 0                                   # the first parents keep no child
    full, child, _ = orc.c2s_block(x, coords, p, "c", cout, mask, wt)
    rows = np.unique(np.concatenate([[0, 1, len(child) - 1], rng.integers(0, len(child), 60)]))
    part, child2 = orc.c2s_block_rows(x, coords, p, "c", cout, mask, rows, wt)
    assert np.array_equal(child, child2)
    assert np.abs(part - full[rows]).max() <= 1e-12 * np.abs(full).max()
    # the head: one stage of decode_unet with no ConvNeXt block
    q = dict(p)
    q.update({"from_latent.weight": rnd((rng.standard_normal((cin, 8)) / 3).astype(np.float32)),
              "from_latent.bias": np.zeros(cin, np.float32),
              "output_layer.weight": rnd((rng.standard_normal((6, cout)) / 4).astype(np.float32)),
              "output_layer.bias": (0.1 * rng.standard_normal(6)).astype(np.float32)})
    wq = {k: (wtype if v.ndim >= 2 else "f32") for k, v in q.items()}
    latent = rng.standard_normal((n, 8)).astype(np.float32)
    out, _, _ = orc.decode_unet(latent, coords, q, [([], ("c", cin, cout))], 6, [mask], wt=wq)
    h0 = orc.linear(orc._rounder(wq, False)(latent, "from_latent.weight"), q["from_latent.weight"],
                    q["from_latent.bias"])
    last, _ = orc.c2s_block_rows(h0.astype(np.float32), coords, q, "c", cout, mask, rows, wq)
    assert np.abs(orc.decoder_head_rows(last, q, wq) - out[rows]).max() <= 1e-12 * np.abs(out).max()
