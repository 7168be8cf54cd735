"""CPU checks of the synthetic workload generators the benchmark and the GPU tests run on."""
from __future__ import annotations

import numpy as np


def test_decoder_workload_levels(shells):
    """Each level is the previous one's children under its band mask, in subdivision order
    (parent-major, octant ascending), and every level is a set of distinct voxels."""
    w = shells.decoder_workload("decoder-shells16-c64")
    assert len(w.masks) == len(w.channels) - 1 == len(w.level_coords) - 1
    assert w.latent.shape == (w.counts[0], 32) and w.latent.dtype == np.float32
    for s, m in enumerate(w.masks):
        parents, kids = w.level_coords[s], w.level_coords[s + 1]
        assert m.shape == (8 * len(parents),) and m.dtype == np.uint8
        assert int(m.sum()) == len(kids) == w.counts[s + 1]
        p, o = np.nonzero(m.reshape(-1, 8))
        expect = 2 * parents[p] + np.stack([o & 1, (o >> 1) & 1, (o >> 2) & 1], 1)
        assert np.array_equal(kids, expect)
        assert len(np.unique(kids, axis=0)) == len(kids)
    # the thickness-2 band grows about 4x per 2x subdivision
    for a, b in zip(w.counts[:-1], w.counts[1:]):
        assert 3.0 < b / a < 5.5, w.counts


def test_decoder_params_names_and_shapes(shells):
    """Key names and shapes as the host decoder reads them (shape_decoder.cpp:79-117): conv
    weights [Co, 27, Ci], C2S conv1 to 8*Cout channels, linears [out, in]."""
    ch = (64, 32, 16)
    p = shells.decoder_params(ch, 2, 32, 6, 0.02, 4)
    assert p["from_latent.weight"].shape == (64, 32)
    for s, (ci, co) in enumerate(zip(ch[:-1], ch[1:])):
        for j in range(2):
            q = f"blocks.{s}.{j}"
            assert p[f"{q}.conv.weight"].shape == (ci, 27, ci)
            assert p[f"{q}.mlp.0.weight"].shape == (4 * ci, ci) and p[f"{q}.mlp.2.weight"].shape == (ci, 4 * ci)
            assert np.all(p[f"{q}.norm.weight"] == 1) and np.all(p[f"{q}.conv.bias"] == 0)
        q = f"blocks.{s}.2"
        assert p[f"{q}.conv1.weight"].shape == (8 * co, 27, ci)
        assert p[f"{q}.conv2.weight"].shape == (co, 27, co)
        assert p[f"{q}.to_subdiv.weight"].shape == (8, ci)
    assert p["output_layer.weight"].shape == (6, 16)
    w = p["blocks.0.0.conv.weight"]
    assert abs(float(w.std()) - 0.02) < 0.002
    # seeded: the same arguments give the same weights
    assert np.array_equal(shells.decoder_params(ch, 2, 32, 6, 0.02, 4)["blocks.1.2.conv1.weight"],
                          p["blocks.1.2.conv1.weight"])
