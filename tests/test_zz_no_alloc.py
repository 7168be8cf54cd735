"""tsp_subdivide_noalloc (the subdivision with its block counts in the library's static device
array instead of a workspace) against tsp_subdivide, both called through the C ABI: two calls
in a row, the second on a smaller input, so that the array still holds the first call's
counts when the second runs. Output buffers start filled with -7 so an unwritten entry shows."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _subdivide_both(pkg, torch, mask, coords):
    L = pkg.lib()
    n = coords.shape[0]
    dev = coords.device
    outs = []
    for noalloc in (False, True):
        mstart = torch.full((n + 1,), -7, dtype=torch.int32, device=dev)
        child = torch.full((max(8 * n, 1), 3), -7, dtype=torch.int32, device=dev)
        gidx = torch.full((max(8 * n, 1),), -7, dtype=torch.int32, device=dev)
        m = torch.full((1,), -7, dtype=torch.int64, device=dev)
        args = [pkg._ptr(mask), pkg._ptr(coords), n, pkg._ptr(mstart), pkg._ptr(child),
                pkg._ptr(gidx), pkg._ptr(m)]
        if noalloc:
            st = L.tsp_subdivide_noalloc(*args, None)
            pkg._check("tsp_subdivide_noalloc", st)
        else:
            ws_bytes = L.tsp_subdivide_workspace_bytes(n)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
            pkg._check("tsp_subdivide", L.tsp_subdivide(*args, pkg._ptr(ws), ws_bytes, None))
        torch.cuda.synchronize()
        mm = int(m.item())
        outs.append((mm, mstart.cpu().numpy(), child[:mm].cpu().numpy(), gidx[:mm].cpu().numpy()))
    return outs


@pytest.mark.parametrize("sizes", [(300_000, 70_001), (5000, 1)])
def test_noalloc_matches_workspace_entry(gpu_lib, sizes):
    import torch
    pkg = gpu_lib
    rng = np.random.default_rng(11)
    for n in sizes:
        print(f"[no_alloc] n={n}", flush=True)
        coords = torch.from_numpy(rng.integers(0, 1 << 20, (n, 3), dtype=np.int32)).cuda()
        mask = torch.from_numpy((rng.random(8 * n) < 0.4).astype(np.uint8)).cuda()
        (m0, ms0, c0, g0), (m1, ms1, c1, g1) = _subdivide_both(pkg, torch, mask, coords)
        assert m1 == m0 and m0 > 0
        assert np.array_equal(ms1, ms0)
        assert np.array_equal(c1, c0)
        assert np.array_equal(g1, g0)


def test_noalloc_empty_input(gpu_lib):
    import torch
    pkg = gpu_lib
    coords = torch.zeros((0, 3), dtype=torch.int32, device="cuda")
    mask = torch.zeros(0, dtype=torch.uint8, device="cuda")
    (m0, ms0, _, _), (m1, ms1, _, _) = _subdivide_both(pkg, torch, mask, coords)
    assert m0 == m1 == 0
    assert np.array_equal(ms0, ms1) and ms1.tolist() == [0]

