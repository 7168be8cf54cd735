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


def stored_types(params, wtype="f16"):
    """Weight name -> the type the GGUF stores it in (the oracle's rounding rule reads it)."""
    return {k: (wtype if np.asarray(v).ndim >= 2 else "f32") for k, v in params.items()}


def write_conv_case(d, orc, coords, c, seed, cast_f32=False):
    """ConvNeXt block `blocks.3.0` with c channels on `coords` (the reference's
    test_sparse_conv.cpp inputs: coords, feats_in, conv_out, block_out) plus the table. The
    expected outputs round every product's input as ggml's mul_mat does (F16 weights; under
    cast_f32, the reference's g_sparse_cast_f32, the conv weights are cast and its input is not
    rounded)."""
    rng = np.random.default_rng(seed)
    n = len(coords)
    x = rng.standard_normal((n, c)).astype(np.float32)
    p = convnext_params(rng, c)
    write_gguf(os.path.join(d, "model.gguf"), p)
    q, wt = stored(p), stored_types(p)
    nbr = orc.neighbor_table(coords)
    w, b = q["blocks.3.0.conv.weight"], q["blocks.3.0.conv.bias"]
    xc = orc.act_round(x, "f16", True, cast_f32).astype(np.float32)
    _save(d, coords=np.ascontiguousarray(coords, np.int32), feats_in=x, nbr=nbr,
          conv_out=orc.subm_conv_f64(xc, nbr, w, b, row0=x[0]).astype(np.float32),
          block_out=orc.convnext_block(x, nbr, q, "blocks.3.0", wt, cast_f32).astype(np.float32))


def write_c2s_case(d, orc, coords, cin, cout, seed, ext=False, cast_f32=False):
    """C2S up-block `blocks.3.4` (the reference's test_c2s.cpp inputs) with the expected
    children, mask and features (rounded as in write_conv_case); with ext, a random ext_mask.npy
    drives the subdivision."""
    rng = np.random.default_rng(seed)
    n = len(coords)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    p = c2s_params(rng, cin, cout)
    write_gguf(os.path.join(d, "model.gguf"), p)
    q, wt = stored(p), stored_types(p)
    ext_mask = (rng.random(8 * n) < 0.3).astype(np.uint8) if ext else None
    out, child, mask = orc.c2s_block(x, coords, q, "blocks.3.4", cout, ext_mask, wt, cast_f32)
    _save(d, coords=np.ascontiguousarray(coords, np.int32), feats_in=x,
          new_coords=np.ascontiguousarray(child, np.int32), out=np.asarray(out, np.float32),
          subdiv=np.asarray(mask, np.uint8))
    if ext:
        _save(d, ext_mask=ext_mask)


def zero_weight_decoder(rng, channels, blocks):
    """decoder parameters (f32) whose conv and MLP weights are zero: every ConvNeXt block adds its
    mlp.2 bias, every C2S block gives a child conv2's bias + the skip, so the decoder reduces to
    from_latent, the routing of the skips and the head."""
    p, stages = decoder_params(rng, channels, blocks, latent=8, out_ch=6)
    for k in p:
        if k.endswith((".conv.weight", ".mlp.0.weight", ".mlp.2.weight", ".conv1.weight", ".conv2.weight")):
            p[k] = np.zeros_like(p[k])
    p["from_latent.weight"] = p["from_latent.weight"] * 0.01   # features ~ 0.01: the head's eps matters
    p["from_latent.bias"] = p["from_latent.bias"] * 0.01
    for k in p:
        if k.endswith((".mlp.2.bias", ".conv2.bias")):
            p[k] = p[k] * 0.05
    return p, stages


def decode_closed_form(latent, coords, p, stages, guide, eps=1e-5, octant_shift=0):
    """The zero-weight decoder by explicit loops: h = latent W^T + b; each ConvNeXt block adds
    mlp.2.bias; child (parent i, octant o, in parent order and ascending octant) of a C2S block is
    conv2.bias + repeat(h[i, o k:(o+1) k], cout / k) at (2x + (o&1), 2y + (o>>1 & 1), 2z + (o>>2 & 1));
    then LayerNorm with eps 1e-5 and no affine, and output_layer. eps and octant_shift (the skip
    read from slice o ^ shift) plant mistakes."""
    h = [np.asarray(latent[i], np.float64) @ p["from_latent.weight"].T.astype(np.float64) + p["from_latent.bias"]
         for i in range(len(latent))]
    c = [tuple(int(v) for v in row) for row in coords]
    for si, (blocks, (c2s, cin, cout)) in enumerate(stages):
        for b in blocks:
            h = [hi + p[b + ".mlp.2.bias"] for hi in h]
        k = cin // 8
        nh, nc = [], []
        for i, (x, y, z) in enumerate(c):
            for o in range(8):
                if guide[si][8 * i + o]:
                    nc.append((2 * x + (o & 1), 2 * y + ((o >> 1) & 1), 2 * z + ((o >> 2) & 1)))
                    os_ = o ^ octant_shift
                    nh.append(p[c2s + ".conv2.bias"] + np.repeat(h[i][os_ * k:(os_ + 1) * k], cout // k))
        h, c = nh, nc
    out = []
    for hi in h:
        mu = hi.mean()
        var = ((hi - mu) ** 2).mean()
        y = (hi - mu) / np.sqrt(var + eps)
        out.append(y @ p["output_layer.weight"].T.astype(np.float64) + p["output_layer.bias"])
    return np.array(out), np.array(c, np.int32)


def rounding_noise_floor(orc, run, runs=2, rel=1e-7, seed=0):
    """How far two correct evaluations of the rounding semantics fall apart: the largest
    max|d|/max|ref| between run() (an oracle computation returning an array) and run() again with
    every matrix product's input perturbed by a relative `rel` before its rounding, as another
    float32 evaluation order of what produced it would perturb it. A rounding step then falls on
    the other side for some elements, as it does between the device and the oracle. run() returns
    the array, or a tuple whose first item is it; the first result is returned with the floor."""
    first = run()
    pick = lambda r: np.asarray(r[0] if isinstance(r, tuple) else r, np.float64)
    ref = pick(first)
    exact = orc.act_round
    rng = np.random.default_rng(seed)

    def jittered(x, wtype, conv_weight=False, cast_f32=False):
        x = np.asarray(x, np.float64)
        return exact(x * (1 + rel * rng.uniform(-1, 1, x.shape)), wtype, conv_weight, cast_f32)

    worst = 0.0
    orc.act_round = jittered
    try:
        for _ in range(runs):
            worst = max(worst, orc.rel_err(pick(run()), ref))
    finally:
        orc.act_round = exact
    return first, worst
