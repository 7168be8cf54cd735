"""GPU parity of the 2x subdivision index math: bit-exact against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[subdivide] {name}", flush=True)


def _gpu(pkg, mask, coords):
    import torch
    m = torch.from_numpy(np.ascontiguousarray(mask, np.uint8)).cuda()
    c = torch.from_numpy(np.ascontiguousarray(coords, np.int32)).cuda()
    ch, gi, ms = pkg.subdivide(m, c)
    torch.cuda.synchronize()
    return ch.cpu().numpy(), gi.cpu().numpy(), ms.cpu().numpy()


def test_golden(gpu_lib, golden):
    _case("subdivide_rand600")
    g = golden("subdivide_rand600.npz")
    ch, gi, ms = _gpu(gpu_lib, g["mask"], g["coords"])
    assert np.array_equal(ch, g["child"]) and np.array_equal(gi, g["gidx"])
    assert np.array_equal(ms, g["mstart"])


@pytest.mark.parametrize("n,p", [(0, 0.5), (1, 1.0), (1023, 0.3), (1024, 0.0), (1025, 1.0),
                                 (70000, 0.45)])
def test_random(gpu_lib, orc, n, p):
    _case(f"n={n} p={p}")
    rng = np.random.default_rng(n)
    coords = rng.integers(0, 1000, size=(n, 3)).astype(np.int32)
    mask = ((rng.random(8 * n) < p) * rng.integers(1, 256, 8 * n)).astype(np.uint8)
    ch, gi, ms = _gpu(gpu_lib, mask, coords)
    rch, rgi, rms = orc.subdivide(mask, coords)
    assert np.array_equal(ch, rch) and np.array_equal(gi, rgi) and np.array_equal(ms, rms)


def test_band_pipeline(gpu_lib, orc, shells):
    """2x subdivision pruned to a surface band, then the rulebook of the children: the
    band512 workload's construction, checked at a 64^3 parent grid."""
    _case("band pipeline")
    import torch
    rng = np.random.default_rng(3)
    shapes = shells.random_shapes(rng, 64, 3, 10, 28, boxes=True)
    parents = shells.band_voxels(shapes, 64, 2.0)
    mask = shells.subdivision_band_mask(parents, shapes, 2.0)
    ch, gi, ms = _gpu(gpu_lib, mask, parents)
    assert np.array_equal(ch, shells.children(mask, parents))
    nbr = gpu_lib.rulebook_build(torch.from_numpy(ch).cuda()).cpu().numpy()
    assert np.array_equal(nbr, orc.neighbor_table(ch))
