"""Inputs and expected outputs for the C++ host check programs (tests/host/*.cpp): a GGUF of
synthetic weights under the reference's key names (sparse.cpp:89, 104, 125-128, 188, 260,
278, 305) and .npy files computed by the oracle."""
from __future__ import annotations

import os

import numpy as np

from trellis_cpp_amd.gguf_writer import write as write_gguf


def _f16(a):
    """Values as the GGUF stores them (F16), back in float32 for the oracle."""
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def _save(d, **arrays):
    for k, v in arrays.items():
        np.save(os.path.join(d, k + ".npy"), v, allow_pickle=False)


def convnext_params(rng, c, prefix="blocks.3.0"):
    s = lambda scale, *shape: (rng.standard_normal(shape) * scale).astype(np.float32)
    return {f"{prefix}.conv.weight": s(1 / np.sqrt(27 * c), c, 27, c),
            f"{prefix}.conv.bias": s(0.1, c),
            f"{prefix}.norm.weight": 1 + s(0.1, c), f"{prefix}.norm.bias": s(0.1, c),
            f"{prefix}.mlp.0.weight": s(1 / np.sqrt(c), 4 * c, c), f"{prefix}.mlp.0.bias": s(0.1, 4 * c),
            f"{prefix}.mlp.2.weight": s(1 / np.sqrt(4 * c), c, 4 * c), f"{prefix}.mlp.2.bias": s(0.1, c)}


def c2s_params(rng, cin, cout, prefix="blocks.3.4"):
    s = lambda scale, *shape: (rng.standard_normal(shape) * scale).astype(np.float32)
    return {f"{prefix}.to_subdiv.weight": s(1.0, 8, cin), f"{prefix}.to_subdiv.bias": s(0.1, 8),
            f"{prefix}.norm1.weight": 1 + s(0.1, cin), f"{prefix}.norm1.bias": s(0.1, cin),
            f"{prefix}.conv1.weight": s(1 / np.sqrt(27 * cin), 8 * cout, 27, cin),
            f"{prefix}.conv1.bias": s(0.1, 8 * cout),
            f"{prefix}.conv2.weight": s(1 / np.sqrt(27 * cout), cout, 27, cout),
            f"{prefix}.conv2.bias": s(0.1, cout)}


def decoder_params(rng, channels=(128, 64, 32, 16), blocks=(1, 1, 1), latent=32, out_ch=7):
    """A small SparseUnetVaeDecoder under the reference's key names (shape_decoder.cpp:79-117):
    from_latent, per stage `blocks` ConvNeXt blocks then a C2S block, output_layer. Returns the
    parameters and the stage list the oracle decoder takes."""
    s = lambda scale, *shape: (rng.standard_normal(shape) * scale).astype(np.float32)
    p = {"from_latent.weight": s(1 / np.sqrt(latent), channels[0], latent),
         "from_latent.bias": s(0.1, channels[0])}
    stages = []
    for si, (cin, cout) in enumerate(zip(channels[:-1], channels[1:])):
        names = []
        for j in range(blocks[si]):
            p.update(convnext_params(rng, cin, f"blocks.{si}.{j}"))
            names.append(f"blocks.{si}.{j}")
        c2s = f"blocks.{si}.{blocks[si]}"
        p.update(c2s_params(rng, cin, cout, c2s))
        stages.append((names, (c2s, cin, cout)))
    p["output_layer.weight"] = s(1 / np.sqrt(channels[-1]), out_ch, channels[-1])
    p["output_layer.bias"] = s(0.1, out_ch)
    return p, stages


def stored(params):
    """The parameters as the host program will see them: 2-D+ weights through F16."""
    return {k: (_f16(v) if v.ndim >= 2 else v) for k, v in params.items()}


def write_conv_case(d, orc, coords, c, seed):
    """ConvNeXt block `blocks.3.0` with c channels on `coords` (the reference's
    test_sparse_conv.cpp inputs: coords, feats_in, conv_out, block_out) plus the table and
    conv_out16 (the conv of the F16-rounded features, what the matrix-core path computes)."""
    rng = np.random.default_rng(seed)
    n = len(coords)
    x = rng.standard_normal((n, c)).astype(np.float32)
    p = convnext_params(rng, c)
    write_gguf(os.path.join(d, "model.gguf"), p)
    q = stored(p)
    nbr = orc.neighbor_table(coords)
    w, b = q["blocks.3.0.conv.weight"], q["blocks.3.0.conv.bias"]
    _save(d, coords=np.ascontiguousarray(coords, np.int32), feats_in=x, nbr=nbr,
          conv_out=orc.subm_conv_f64(x, nbr, w, b).astype(np.float32),
          conv_out16=orc.subm_conv_f64(_f16(x), nbr, w, b).astype(np.float32),
          block_out=orc.convnext_block(x, nbr, q, "blocks.3.0").astype(np.float32))


def write_c2s_case(d, orc, coords, cin, cout, seed, ext=False):
    """C2S up-block `blocks.3.4` (the reference's test_c2s.cpp inputs) with the expected
    children, mask and features; with ext, a random ext_mask.npy drives the subdivision."""
    rng = np.random.default_rng(seed)
    n = len(coords)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    p = c2s_params(rng, cin, cout)
    write_gguf(os.path.join(d, "model.gguf"), p)
    q = stored(p)
    ext_mask = (rng.random(8 * n) < 0.3).astype(np.uint8) if ext else None
    out, child, mask = orc.c2s_block(x, coords, q, "blocks.3.4", cout, ext_mask)
    _save(d, coords=np.ascontiguousarray(coords, np.int32), feats_in=x,
          new_coords=np.ascontiguousarray(child, np.int32), out=np.asarray(out, np.float32),
          subdiv=np.asarray(mask, np.uint8))
    if ext:
        _save(d, ext_mask=ext_mask)
