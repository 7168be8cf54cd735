"""GPU parity of the C++ host side: the check programs (tests/host/*.cpp) load a GGUF of
synthetic weights through Model::load and run trellis::build_neighbor_table, sparse_submconv and
sparse_convnext in a ggml graph, sparse_c2s, and the device-resident decoders (shape_decode,
shape_upsample, tex_decode), against the oracle's outputs.

The oracle rounds the input of every matrix product to the weights' stored type where ggml's
mul_mat does (oracle.act_round: F16 / BF16 weights; under --f32, the reference's
g_sparse_cast_f32, the conv weights are cast to F32 and their input stays F32, the linears still
round). Bars: table, children and masks exact. Features max|d|/max|ref|: <= 2e-5 for a conv (fp32
accumulation against fp64 on the same rounded inputs); 2e-4 for a block, whose later products
take inputs that both sides round from float32 values computed in another order, where one
rounding step (2^-11 for F16) can fall on either side. Over a whole decoder such flips compound:
its bar is 1.5x the oracle's own noise floor (host_cases.rounding_noise_floor: the oracle against
itself with every product input perturbed by 1e-7 before rounding), measured in the test."""
from __future__ import annotations

import dataclasses

import os
import re
import subprocess

import numpy as np
import pytest

from host_cases import rounding_noise_floor, write_c2s_case, write_conv_case

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "trellis.cpp_amd", "host", "bin")


@pytest.fixture(scope="module")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    for b in ("sparse_conv_check", "c2s_check"):
        if not os.path.exists(os.path.join(BIN, b)):
            pytest.fail(f"{b} is not built")


def _run(args):
    print("[host]", " ".join(os.path.basename(a) for a in args), flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    return r.stdout


def _val(out, key):
    m = re.search(rf"{key}\s*(?:rel=)?([-+0-9.eE]+)", out)
    assert m, (key, out)
    return float(m.group(1))


TOL_CONV = 2e-5
TOL_BLOCK_F16 = 2e-4


@pytest.mark.parametrize("c,f32", [(64, False), (64, True), (128, False), (48, False), (48, True)])
def test_conv_and_convnext(gpu, orc, shells, tmp_path, c, f32):
    """sparse_submconv and sparse_convnext in a ggml graph: C = 64 and 128 on the matrix cores, 48
    on the VALU kernel (on F16-rounded input too), and --f32."""
    coords = shells.sphere_shell(40, 20.0, 12.0, 14.0)
    write_conv_case(str(tmp_path), orc, coords, c, seed=c, cast_f32=f32)
    args = [os.path.join(BIN, "sparse_conv_check"), str(tmp_path / "model.gguf"), str(tmp_path), "0"]
    out = _run(args + (["--f32"] if f32 else []))
    assert _val(out, "nbr_exact") == 1
    conv, block = _val(out, "conv_out"), _val(out, "block_out")
    print(f"c={c} f32={f32} conv rel={conv:.3e} block rel={block:.3e}", flush=True)
    assert conv < TOL_CONV and block < TOL_BLOCK_F16, (conv, block)


@pytest.mark.parametrize("cin,cout,ext,f32", [(64, 32, False, False), (64, 32, True, False),
                                              (128, 64, False, False), (128, 64, True, True)])
def test_c2s(gpu, orc, shells, tmp_path, cin, cout, ext, f32):
    coords = shells.random_distinct_voxels(700, 14, cin + cout)
    write_c2s_case(str(tmp_path), orc, coords, cin, cout, seed=cin + cout, ext=ext, cast_f32=f32)
    args = [os.path.join(BIN, "c2s_check"), str(tmp_path / "model.gguf"), str(tmp_path), "0"]
    out = _run(args + (["--ext"] if ext else []) + (["--f32"] if f32 else []))
    assert _val(out, "coords_exact") == 1
    assert _val(out, "mask_exact") == 1
    err = _val(out, "feats")
    print(f"c2s {cin}->{cout} ext={ext} f32={f32} rel={err:.3e}", flush=True)
    assert err < TOL_BLOCK_F16


# ---- the device-resident decoders (shape_decode, shape_upsample, tex_decode) ----------------------
def _decoder_case(tmp_path, orc, shells, out_ch, seed):
    from trellis_cpp_amd.gguf_writer import write as write_gguf
    from host_cases import decoder_params, stored, stored_types
    rng = np.random.default_rng(seed)
    coords = shells.random_distinct_voxels(200, 10, seed)
    latent = rng.standard_normal((len(coords), 32)).astype(np.float32)
    p, stages = decoder_params(rng, out_ch=out_ch)
    write_gguf(str(tmp_path / f"model{out_ch}.gguf"), p)
    np.save(tmp_path / "latent.npy", latent)
    np.save(tmp_path / "coords.npy", np.ascontiguousarray(coords, np.int32))
    return coords, latent, stored(p), stages, stored_types(p)


def test_shape_decode_fp32(gpu, orc, shells, tmp_path):
    """Predicted masks, fp32 paths: masks, children and output against the oracle decoder. A
    predicted mask bit is the sign of a to_subdiv logit, computed after whole stages of float32
    sums whose order differs from the oracle's (the device's differs from the fp64 oracle by
    ~1e-5 of the logits' range by the third stage), so a logit that close to zero may land on
    either side. The oracle therefore runs on the device's masks, recording its own logits: every
    device bit must equal logit > 0 except where |logit| <= 1e-3 of the stage's largest |logit|,
    and at most 1 in 10^4 bits of a stage may disagree (a systematic error flips far more); the
    unguided oracle must reproduce the device's masks outright when no bit disagrees."""
    coords, latent, q, stages, wt = _decoder_case(tmp_path, orc, shells, 7, seed=11)
    _run([os.path.join(BIN, "decoder_check"), str(tmp_path / "model7.gguf"), str(tmp_path), "0", "--f32"])
    dmasks = [np.load(tmp_path / f"subs_out_{s}.npy") for s in range(len(stages))]
    logits = []
    (ref, rcoords, rmasks), floor = rounding_noise_floor(
        orc, lambda: orc.decode_unet(latent, coords, q, stages, 7, guide=dmasks, wt=wt, cast_f32=True,
                                     logits_out=logits if not logits else None))
    flips = 0
    for s, (dm, lg) in enumerate(zip(dmasks, logits)):
        lg = np.asarray(lg).reshape(-1)
        diff = dm != (lg > 0).astype(np.uint8)
        if diff.any():
            rel = np.abs(lg[diff]).max() / np.abs(lg).max()
            print(f"stage {s}: {int(diff.sum())} of {diff.size} mask bits on the other side of a logit "
                  f"within {rel:.2e} of the largest |logit| from zero", flush=True)
            assert rel <= 1e-3 and diff.sum() <= max(1, diff.size // 10000), s
        flips += int(diff.sum())
    if flips == 0:
        (_, pcoords, pmasks) = orc.decode_unet(latent, coords, q, stages, 7, wt=wt, cast_f32=True)
        assert all(np.array_equal(a, b) for a, b in zip(pmasks, dmasks))
        assert np.array_equal(pcoords, rcoords)
    assert np.array_equal(np.load(tmp_path / "coords_out.npy"), rcoords)
    err = orc.rel_err(np.load(tmp_path / "out.npy"), ref)
    print(f"shape_decode fp32 rel={err:.3e} floor={floor:.3e} M={len(rcoords)}", flush=True)
    assert err < max(TOL_BLOCK_F16, 1.5 * floor)
    _run([os.path.join(BIN, "decoder_check"), str(tmp_path / "model7.gguf"), str(tmp_path), "0", "--f32",
          "--upsample"])
    assert np.array_equal(np.load(tmp_path / "coords_out.npy"), rcoords)


def test_tex_decode_guided(gpu, orc, shells, tmp_path):
    """Masks given (the texture decoder's route), matrix-core paths with 16-bit activations."""
    coords, latent, q, stages, wt = _decoder_case(tmp_path, orc, shells, 6, seed=12)
    rng = np.random.default_rng(5)
    guide, n = [], len(coords)
    for _ in stages:
        guide.append((rng.random(8 * n) < 0.4).astype(np.uint8))
        n = int(guide[-1].sum())
    for s, g in enumerate(guide):
        np.save(tmp_path / f"subs_{s}.npy", g)
    _run([os.path.join(BIN, "decoder_check"), str(tmp_path / "model6.gguf"), str(tmp_path), "0", "--tex"])
    (ref, rcoords, _), floor = rounding_noise_floor(
        orc, lambda: orc.decode_unet(latent, coords, q, stages, 6, guide, wt=wt))
    out = np.load(tmp_path / "out.npy")
    assert out.shape == ref.shape
    err = orc.rel_err(out, ref)
    print(f"tex_decode 16-bit rel={err:.3e} floor={floor:.3e} M={len(rcoords)}", flush=True)
    assert err < max(TOL_BLOCK_F16, 1.5 * floor)


@pytest.mark.parametrize("channels", [None, (128, 64)])
def test_tex_decode_bf16_decoder_workload(gpu, orc, shells, tmp_path, channels):
    """The decoder benchmark's model format on its miniature workload: bf16 weights ~ N(0, 0.02)
    under the reference's key names, band masks driving the texture route. Against the oracle
    decoder fed the same bf16-rounded weights; every conv and linear rounds its input to bf16 (a
    2^-8 relative step, so the bar is looser than the F16 case's). channels (128, 64): one stage
    whose C2S conv1 stores its octants into the children and whose conv2 adds the skip as it
    stores, and the fused LayerNorm + output head over 64 channels. The oracle rounds every
    product's input to bf16 where the device does; with bf16's 2^-8 step the flips between two
    correct evaluation orders reach 3e-3 (one stage) to 8e-3 (three stages), so the bar is 1.5x
    that floor, measured here."""
    from trellis_cpp_amd.gguf_writer import write as write_gguf
    w = shells.decoder_workload("decoder-shells16-c64")
    if channels is not None:
        w = dataclasses.replace(w, channels=channels, masks=w.masks[:len(channels) - 1],
                                counts=w.counts[:len(channels)])
    p = shells.decoder_params(w.channels, w.blocks, 32, w.out_ch, w.std, w.seed)
    write_gguf(str(tmp_path / "model.gguf"), p, dtypes={k: ("bf16" if v.ndim >= 2 else "f32") for k, v in p.items()})
    np.save(tmp_path / "latent.npy", w.latent)
    np.save(tmp_path / "coords.npy", np.ascontiguousarray(w.coords, np.int32))
    for s, m in enumerate(w.masks):
        np.save(tmp_path / f"subs_{s}.npy", m)
    # three decodes in one process: the later ones run on device blocks the first released
    _run([os.path.join(BIN, "decoder_check"), str(tmp_path / "model.gguf"), str(tmp_path), "0", "--tex",
          "--repeat", "3"])
    q = {k: (shells.round_to(v, "bf16") if v.ndim >= 2 else v) for k, v in p.items()}
    stages = [([f"blocks.{s}.{j}" for j in range(w.blocks)], (f"blocks.{s}.{w.blocks}", ci, co))
              for s, (ci, co) in enumerate(zip(w.channels[:-1], w.channels[1:]))]
    wt = {k: ("bf16" if v.ndim >= 2 else "f32") for k, v in p.items()}
    (ref, rcoords, _), floor = rounding_noise_floor(
        orc, lambda: orc.decode_unet(w.latent, w.coords, q, stages, w.out_ch, w.masks, wt=wt))
    assert len(rcoords) == w.counts[-1]
    out = np.load(tmp_path / "out.npy")
    assert out.shape == ref.shape
    err = orc.rel_err(out, ref)
    print(f"tex_decode bf16 rel={err:.3e} floor={floor:.3e} M={len(rcoords)}", flush=True)
    assert err < 1.5 * floor


def test_decoder_zero_weight_closed_form(gpu, shells, tmp_path):
    """tex_decode on a model whose conv and MLP weights are zero (F32), against the closed form
    that case reduces to (host_cases.decode_closed_form: from_latent, each block's mlp.2 bias, the
    C2S skip's octant slices and child order, the head's LayerNorm with eps 1e-5 and no affine):
    the decoder's stage structure checked without the oracle decoder."""
    from trellis_cpp_amd.gguf_writer import write as write_gguf
    from host_cases import decode_closed_form, zero_weight_decoder
    rng = np.random.default_rng(31)
    coords = shells.random_distinct_voxels(300, 10, 31)
    latent = rng.standard_normal((300, 8)).astype(np.float32)
    p, stages = zero_weight_decoder(rng, (32, 16, 8), (2, 1))
    write_gguf(str(tmp_path / "model.gguf"), p, dtypes={k: "f32" for k in p})
    np.save(tmp_path / "latent.npy", latent)
    np.save(tmp_path / "coords.npy", np.ascontiguousarray(coords, np.int32))
    guide, n = [], len(coords)
    for s, _ in enumerate(stages):
        guide.append((rng.random(8 * n) < 0.4).astype(np.uint8))
        np.save(tmp_path / f"subs_{s}.npy", guide[-1])
        n = int(guide[-1].sum())
    _run([os.path.join(BIN, "decoder_check"), str(tmp_path / "model.gguf"), str(tmp_path), "0", "--tex"])
    ref, rc = decode_closed_form(latent, coords, p, stages, guide)
    out = np.load(tmp_path / "out.npy")     # the children's rows in the closed form's order
    assert out.shape == ref.shape
    err = np.abs(out - ref).max() / np.abs(ref).max()
    print(f"zero-weight decoder rel={err:.3e} M={len(rc)}", flush=True)
    assert err < 1e-5


def test_decoder_full_size_properties(gpu, orc, shells, tmp_path):
    """The decoder stack at the benchmark's widths and size (decoder-shells64-c1024: 33,543 ->
    9,881,361 voxels, 1024 -> 512 -> 256 -> 128 -> 64 channels, bf16 weights ~ N(0, 0.02)),
    where the oracle cannot run whole: the coordinates of every level (read back through
    TRELLIS_DECODER_DUMP) equal the oracle's chained subdivision of the input by the masks; the
    output has one row per final voxel, all finite, and is the same bits on a repeat; and a row
    sample of the output -- the first and last rows and random ones -- equals the oracle's last
    C2S block (conv1 with its octant stores and child norm at Cout = 64, conv2 with the skip) and
    head on those rows, fed the device's own input to that stage, within 1.5x the sample's rounding
    noise floor (at least 2e-4)."""
    import torch
    from trellis_cpp_amd.gguf_writer import write as write_gguf
    w = shells.decoder_workload("decoder-shells64-c1024")
    p = shells.decoder_params(w.channels, w.blocks, w.latent.shape[1], w.out_ch, w.std, w.seed)
    dtypes = {k: ("bf16" if v.ndim >= 2 else "f32") for k, v in p.items()}
    write_gguf(str(tmp_path / "model.gguf"), p, dtypes=dtypes, arch="trellis2-tex-dec")
    np.save(tmp_path / "latent.npy", w.latent)
    np.save(tmp_path / "coords.npy", np.ascontiguousarray(w.coords, np.int32))
    for s, m in enumerate(w.masks):
        np.save(tmp_path / f"subs_{s}.npy", np.ascontiguousarray(m, np.uint8))
    dump = tmp_path / "dump"
    dump.mkdir()
    env = dict(os.environ, TRELLIS_DECODER_DUMP=str(dump))
    args = [os.path.join(BIN, "decoder_check"), str(tmp_path / "model.gguf"), str(tmp_path), "0", "--tex",
            "--repeat", "2"]
    print("[host] decoder_check full size, with the level dump", flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=600, env=env)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stderr
    # every level's coordinates: the oracle's subdivision chain
    c = np.ascontiguousarray(w.coords, np.int32)
    nst = len(w.channels) - 1
    for s in range(nst + 1):
        got = np.load(dump / f"level{s}_coords.npy")
        assert np.array_equal(got, c), s
        if s < nst:
            c, _, _ = orc.subdivide(w.masks[s], c)
    out = np.load(tmp_path / "out.npy")
    assert out.shape == (w.counts[-1], w.out_ch) and np.isfinite(out).all()
    # the last stage and the head on sampled rows, from the device's input to that stage
    x = np.load(dump / f"level{nst - 1}_in.npy")
    pc = np.load(dump / f"level{nst - 1}_coords.npy")
    assert x.shape == (w.counts[nst - 1], w.channels[nst - 1]) and np.isfinite(x).all()
    q = {k: (shells.round_to(v, "bf16") if v.ndim >= 2 else v) for k, v in p.items()}
    rng = np.random.default_rng(4)
    m = w.counts[-1]
    rows = np.unique(np.concatenate([np.arange(8), np.arange(m - 8, m), rng.integers(0, m, 48)]))
    pre = f"blocks.{nst - 1}.{w.blocks}"

    def sample():
        h, _ = orc.c2s_block_rows(x, pc, q, pre, w.channels[-1], w.masks[nst - 1], rows, wt=dtypes)
        return orc.decoder_head_rows(h, q, wt=dtypes)
    ref, floor = rounding_noise_floor(orc, sample, runs=2)
    err = orc.rel_err(out[rows], ref)
    print(f"decoder full size: M={m} sampled rows {len(rows)} rel={err:.3e} floor={floor:.3e}", flush=True)
    assert err < max(2e-4, 1.5 * floor)
