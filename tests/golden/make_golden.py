"""Writes the committed golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

The reference ships no golden vectors for its sparse path (its parity scripts write .npy
dumps to an external disk and load checkpoint weights, tools/ref_sparse_conv.py:14-15,82-85).
These fixtures are computed by the CPU oracle (oracle/) and, before they are written, each is
cross-checked against an independent statement of the same result:

  rulebook_rand800.npz   800 distinct voxels of [0,16)^3 drawn exactly as the reference's
                         conv parity script draws them (tools/ref_sparse_conv.py:38-44,
                         seed 3). Table checked three ways: hash restatement, dense-grid
                         brute force, sorted-key binary search.
  rulebook_edges.npz     duplicates (largest row wins), voxels on the 0 faces, an isolated
                         voxel and a full 3x3x3 block; the same three-way check.
  conv_rand800_c32.npz   the rand800 voxels with torch.randn(800, 32) features (seed 3, as
                         the reference script draws its features), synthetic weights and bias;
                         output of the fp64 oracle, checked against the fp32 tap-sequential
                         oracle and, for the isolated-voxel rows, against W_13 . f + b.
  subdivide_rand600.npz  600 distinct voxels of [0,16)^3 drawn as tools/ref_c2s.py:30-36
                         (seed 5) with a random octant mask; child coords, gidx and mstart from
                         the C restatement, checked against the nonzero/repeat_interleave
                         formulation.
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def _load(name, path, pkg_dir=None):
    spec = importlib.util.spec_from_file_location(
        name, path, submodule_search_locations=[pkg_dir] if pkg_dir else None)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def main():
    orc = _load("trellis_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    pkg_dir = os.path.join(ROOT, "trellis.cpp_amd")
    _load("trellis_cpp_amd", os.path.join(pkg_dir, "__init__.py"), pkg_dir)
    import trellis_cpp_amd.shells as shells
    import torch

    def three_way(coords):
        a = orc.neighbor_table(coords)
        b = orc.neighbor_table_grid(coords)
        c = orc.neighbor_table_sorted(coords)
        assert np.array_equal(a, b) and np.array_equal(a, c), "rulebook statements disagree"
        return a

    # ---- rulebook on the reference's parity voxels
    coords = shells.random_distinct_voxels(800, 16, 3)
    nbr = three_way(coords)
    np.savez_compressed(os.path.join(HERE, "rulebook_rand800.npz"), coords=coords, nbr=nbr)

    # ---- rulebook edge cases
    block = np.array([(x, y, z) for x in range(5, 8) for y in range(5, 8) for z in range(5, 8)],
                     np.int32)
    edge = np.concatenate([
        np.array([[0, 0, 0], [0, 0, 1], [1, 0, 0], [0, 1, 0], [40, 40, 40]], np.int32),
        block,
        np.array([[0, 0, 1], [6, 6, 6], [0, 0, 0]], np.int32),   # duplicates, appended last
    ])
    enbr = three_way(edge)
    np.savez_compressed(os.path.join(HERE, "rulebook_edges.npz"), coords=edge, nbr=enbr)

    # ---- conv on the parity voxels
    n, c = 800, 32
    feats = torch.randn(n, c, generator=torch.Generator().manual_seed(3)).numpy()
    rng = np.random.default_rng(3)
    weight = (rng.standard_normal((c, 27, c)) / np.sqrt(27 * c)).astype(np.float32)
    bias = (rng.standard_normal(c) * 0.1).astype(np.float32)
    out64 = orc.subm_conv_f64(feats, nbr, weight, bias)
    out32 = orc.subm_conv_f32(feats, nbr, weight, bias)
    assert orc.rel_err(out32, out64) < 1e-5
    iso = [i for i in range(n) if all(nbr[t * n + i] == n for t in range(27) if t != 13)]
    for i in iso:
        ref = weight[:, 13, :].astype(np.float64) @ feats[i].astype(np.float64) + bias
        assert np.allclose(out64[i], ref, rtol=0, atol=1e-12)
    np.savez_compressed(os.path.join(HERE, "conv_rand800_c32.npz"), coords=coords, feats=feats,
                        weight=weight, bias=bias, out=out64)

    # ---- subdivision index math
    coords6 = shells.random_distinct_voxels(600, 16, 5)
    mrng = np.random.default_rng(5)
    mask = (mrng.random(8 * 600) < 0.3).astype(np.uint8)
    mask[8 * 7:8 * 8] = 0                     # a parent with no children
    mask[8 * 9:8 * 10] = 1                    # a parent with all eight
    ch, gi, ms = orc.subdivide(mask, coords6)
    ch2, gi2, ms2 = orc.subdivide_vectorised(mask, coords6)
    assert np.array_equal(ch, ch2) and np.array_equal(gi, gi2) and np.array_equal(ms, ms2)
    np.savez_compressed(os.path.join(HERE, "subdivide_rand600.npz"), coords=coords6, mask=mask,
                        child=ch, gidx=gi, mstart=ms)
    print("wrote fixtures to", HERE, "isolated voxels in rand800:", len(iso))


if __name__ == "__main__":
    main()
