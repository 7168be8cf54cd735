"""GPU parity of the coordinate hash / neighbour table: bit-exact against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _gpu_table(pkg, coords):
    import torch
    c = torch.from_numpy(np.ascontiguousarray(coords, np.int32)).cuda()
    nbr = pkg.rulebook_build(c)
    torch.cuda.synchronize()
    return nbr.cpu().numpy()


def _case(name):
    print(f"[rulebook] {name}", flush=True)


@pytest.mark.parametrize("fixture", ["rulebook_rand800.npz", "rulebook_edges.npz"])
def test_golden(gpu_lib, golden, fixture):
    _case(fixture)
    g = golden(fixture)
    assert np.array_equal(_gpu_table(gpu_lib, g["coords"]), g["nbr"])


def test_edge_cases(gpu_lib, orc, shells):
    rng = np.random.default_rng(21)
    big = (1 << 21) - 3
    cases = {
        "single": np.array([[0, 0, 0]], np.int32),
        "duplicates": rng.integers(0, 12, size=(3000, 3)).astype(np.int32),
        "corners": np.array([[0, 0, 0], [big, big, big], [big, 0, big], [1, 0, 0],
                             [big - 1, big, big]], np.int32),
        "sparse-huge": rng.integers(0, big + 1, size=(5000, 3)).astype(np.int32),
        "dense-cube": np.array([(x, y, z) for x in range(10) for y in range(10)
                                for z in range(10)], np.int32),
        "shell-255": shells.sphere_shell(40, 20.0, 10.0, 11.0)[:255],
        "shell-257": shells.sphere_shell(40, 20.0, 10.0, 11.0)[:257],
        "unsorted": rng.permutation(shells.sphere_shell(40, 20.0, 12.0, 14.0)),
        # a cell directory fits the workspace but the occupied cells' blocks do not: the hash
        "scattered-box": rng.integers(0, 400, size=(20000, 3)).astype(np.int32),
        # duplicates spread over many cells of the grid
        "shell-duplicates": np.concatenate([shells.sphere_shell(40, 20.0, 12.0, 14.0)] * 2)[::-1].copy(),
        # rows in (x, y, z) order with repeats next to each other (the grid's duplicate fix is
        # skipped only for strictly ascending rows): every row twice, and one repeat whose two rows
        # fall in different workgroups of the ascending check
        "sorted-repeats": np.repeat(shells.sphere_shell(40, 20.0, 12.0, 14.0), 2, axis=0),
        "sorted-one-repeat": np.insert(shells.sphere_shell(40, 20.0, 12.0, 14.0), 256,
                                       shells.sphere_shell(40, 20.0, 12.0, 14.0)[255], axis=0),
    }
    import torch
    for name, c in cases.items():
        _case(name)
        ref = orc.neighbor_table_sorted(c)
        assert np.array_equal(_gpu_table(gpu_lib, c), ref), name
        # pair count, also of a copy of the table that starts 1-3 elements past a 16-byte boundary
        n, want = len(c), int((ref != len(c)).sum())
        for off in range(4):
            buf = torch.zeros(27 * n + off, dtype=torch.int32, device="cuda")
            buf[off:] = torch.from_numpy(ref).cuda()
            view = buf[off:]
            assert view.data_ptr() % 16 == 4 * off
            assert gpu_lib.count_pairs(view, n) == want, (name, off)


def test_empty(gpu_lib):
    import torch
    nbr = gpu_lib.rulebook_build(torch.zeros((0, 3), dtype=torch.int32, device="cuda"))
    assert nbr.numel() == 0


def test_out_of_range_reported(gpu_lib):
    import torch
    for bad in ([-1, 0, 0], [0, (1 << 21) - 2, 0]):
        c = torch.tensor([[1, 1, 1], bad], dtype=torch.int32, device="cuda")
        with pytest.raises(gpu_lib.TspError):
            gpu_lib.rulebook_build(c)


@pytest.mark.parametrize("name", ["shell64-c64-f32", "shells256-c128-bf16"])
def test_workload_bit_exact(gpu_lib, orc, shells, name):
    _case(name)
    import torch
    w = shells.workload(name)
    c = torch.from_numpy(w.coords).cuda()
    nbr = gpu_lib.rulebook_build(c)
    again = gpu_lib.rulebook_build(c)
    got = nbr.cpu().numpy()
    ref = orc.neighbor_table(w.coords)
    assert np.array_equal(got, ref)
    assert torch.equal(nbr, again)                                   # deterministic
    assert gpu_lib.count_pairs(nbr, w.n) == orc.count_pairs(ref, w.n)


def test_one_voxel_per_brick_bit_exact(gpu_lib, orc):
    """Every voxel in a 2x2x2 brick of its own: the table holds N bricks in 1.5 N + 1024 buckets,
    the fullest it gets, so probe sequences run longest. 10^6 voxels on a 100^3 brick grid, each
    at a random octant, so neighbouring bricks still give neighbours."""
    _case("one-voxel-per-brick 100^3")
    rng = np.random.default_rng(5)
    a = np.stack(np.meshgrid(*(np.arange(100, dtype=np.int32),) * 3, indexing="ij"), -1)
    # voxel x lies in brick (x + 1) >> 1: x = 2a + 1 + e with e in {0, 1} gives brick a + 1
    c = (2 * a.reshape(-1, 3) + rng.integers(0, 2, size=(a.size // 3, 3)) + 1).astype(np.int32)
    c = c[rng.permutation(len(c))]
    ref = orc.neighbor_table(c)
    assert np.array_equal(_gpu_table(gpu_lib, c), ref)
    assert (ref[13 * len(c):14 * len(c)] == np.arange(len(c))).all()   # centre tap: itself
