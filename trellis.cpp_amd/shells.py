"""Synthetic surface-shell voxel sets and seeded conv inputs.

Active voxel sets in the shape the sparse path sees in a decoder: thin surface bands of
closed shapes, coordinates sorted lexicographically with x slowest and z fastest (the order
ss_coords emits, ss_decoder.cpp:114-129). Voxel p of a G^3 grid is the unit cube [p, p+1)^3
and belongs to a band when the signed distance of its centre p + 0.5 to some shape's
surface satisfies |d| < thickness / 2.

Shapes are rotated ellipsoids (distance: first-order estimate (F-1)/|grad F| of the
normalised radius F) and rotated boxes (exact box distance). A 2x subdivision keeps child
q of parent p (q = 2p + octant) when its centre (q + 0.5) / 2 lies in the band of the same
shapes with the same thickness in child-voxel units.

Everything is seeded numpy; the generated arrays are the single input to both the HIP
library and the CPU oracle.
"""
from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass
class Shape:
    kind: str          # "ellipsoid" | "box"
    center: np.ndarray  # (3,) float64, continuous coordinates of the grid it was drawn in
    semi: np.ndarray    # (3,) semi-axes / half extents
    rot: np.ndarray     # (3,3) rotation, local = (p - center) @ rot


def _random_rotation(rng) -> np.ndarray:
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([[a*a + b*b - c*c - d*d, 2*(b*c - a*d), 2*(b*d + a*c)],
                     [2*(b*c + a*d), a*a - b*b + c*c - d*d, 2*(c*d - a*b)],
                     [2*(b*d - a*c), 2*(c*d + a*b), a*a - b*b - c*c + d*d]])


def _distance(shape: Shape, px, py, pz) -> np.ndarray:
    """Signed distance estimate of points (float32 arrays, continuous coords) to the surface."""
    R = shape.rot.astype(np.float32)
    cx, cy, cz = (np.float32(v) for v in shape.center)
    x, y, z = px - cx, py - cy, pz - cz
    q = [x * R[0, j] + y * R[1, j] + z * R[2, j] for j in range(3)]
    a = [np.float32(v) for v in shape.semi]
    if shape.kind == "box":
        e = [np.abs(q[j]) - a[j] for j in range(3)]
        outside = np.sqrt(np.maximum(e[0], 0) ** 2 + np.maximum(e[1], 0) ** 2 +
                          np.maximum(e[2], 0) ** 2)
        inside = np.minimum(np.maximum(np.maximum(e[0], e[1]), e[2]), 0)
        return outside + inside
    u = [q[j] / a[j] for j in range(3)]
    F = np.sqrt(u[0] ** 2 + u[1] ** 2 + u[2] ** 2)
    g = np.sqrt((u[0] / a[0]) ** 2 + (u[1] / a[1]) ** 2 + (u[2] / a[2]) ** 2)
    g = g / np.maximum(F, np.float32(1e-12))
    return (F - 1) / np.maximum(g, np.float32(1e-12))


def random_shapes(rng, grid: int, count: int, semi_lo: float, semi_hi: float,
                  boxes: bool) -> list:
    """`count` shapes with semi-axes U[semi_lo, semi_hi]; with boxes=True every second shape
    is a box. Centres are uniform in the range that keeps the shape inside the grid (the grid
    centre when the shape is larger than that)."""
    shapes = []
    for s in range(count):
        semi = rng.uniform(semi_lo, semi_hi, 3)
        m = semi.max() + 2
        lo, hi = min(m, grid / 2), max(grid - m, grid / 2)
        center = rng.uniform(lo, hi, 3)
        rot = _random_rotation(rng)
        kind = "box" if (boxes and s % 2 == 1) else "ellipsoid"
        shapes.append(Shape(kind, center, semi, rot))
    return shapes


def band_voxels(shapes: list, grid: int, thickness: float = 2.0) -> np.ndarray:
    """int32 [N,3] voxels of a grid^3 grid within thickness/2 of any shape surface, sorted."""
    occ = np.zeros((grid, grid, grid), bool)
    half = np.float32(thickness / 2)
    for sh in shapes:
        ext = (np.sqrt(3.0) if sh.kind == "box" else 1.0) * sh.semi.max() + thickness + 1
        lo = np.maximum(np.floor(sh.center - ext), 0).astype(int)
        hi = np.minimum(np.ceil(sh.center + ext) + 1, grid).astype(int)
        if np.any(hi <= lo):
            continue
        ax = [np.arange(lo[k], hi[k], dtype=np.float32) + np.float32(0.5) for k in range(3)]
        # slabs along x keep the temporaries small
        for x0 in range(0, hi[0] - lo[0], 32):
            xs = ax[0][x0:x0 + 32]
            X, Y, Z = np.meshgrid(xs, ax[1], ax[2], indexing="ij")
            d = _distance(sh, X, Y, Z)
            sl = occ[lo[0] + x0:lo[0] + x0 + len(xs), lo[1]:hi[1], lo[2]:hi[2]]
            sl |= np.abs(d) < half
    return np.argwhere(occ).astype(np.int32)


def sphere_shell(grid: int = 64, center: float = 32.0, r_in: float = 23.0,
                 r_out: float = 25.0) -> np.ndarray:
    """All integer points p of [0,grid)^3 with r_in <= |p - center| <= r_out, sorted."""
    ax = np.arange(grid, dtype=np.float64)
    X, Y, Z = np.meshgrid(ax, ax, ax, indexing="ij")
    r = np.sqrt((X - center) ** 2 + (Y - center) ** 2 + (Z - center) ** 2)
    return np.argwhere((r >= r_in) & (r <= r_out)).astype(np.int32)


def subdivision_band_mask(coords: np.ndarray, shapes: list, thickness: float = 2.0) -> np.ndarray:
    """uint8 [8N] subdivision mask: octant o of parent p is kept when the child's centre
    (2p + o + 0.5) / 2 (parent-grid units) is within thickness/2 child voxels of a surface."""
    c = np.asarray(coords, np.int64)
    n = c.shape[0]
    mask = np.zeros((n, 8), bool)
    half = np.float32(thickness / 4)      # thickness/2 child voxels = thickness/4 parent units
    for o in range(8):
        off = np.array([(o & 1), (o >> 1) & 1, (o >> 2) & 1], np.float32)
        p = (2 * c + off).astype(np.float32)
        px, py, pz = ((p[:, k] + np.float32(0.5)) / np.float32(2) for k in range(3))
        best = np.full(n, np.inf, np.float32)
        for sh in shapes:
            best = np.minimum(best, np.abs(_distance(sh, px, py, pz)))
        mask[:, o] = best < half
    return mask.astype(np.uint8).reshape(-1)


def children(mask: np.ndarray, coords: np.ndarray) -> np.ndarray:
    """Child coordinates in parent-major, octant-ascending order (the subdivision order)."""
    c = np.asarray(coords, np.int64)
    sub = np.asarray(mask).reshape(-1, 8) != 0
    parent, octant = np.nonzero(sub)
    ch = 2 * c[parent]
    for a in range(3):
        ch[:, a] += (octant >> a) & 1
    return ch.astype(np.int32)


# ------------------------------------------------------------------------------------------
# Named conv workloads
# ------------------------------------------------------------------------------------------
@dataclasses.dataclass
class ConvWorkload:
    name: str
    coords: np.ndarray        # int32 [N,3]
    feats: np.ndarray         # float32 [N,Ci] (already rounded to `dtype`)
    weight: np.ndarray        # float32 [Co,27,Ci] (already rounded to `dtype`)
    bias: np.ndarray          # float32 [Co]
    dtype: str                # "f32" | "bf16" | "f16"
    grid: int
    description: str

    @property
    def n(self) -> int:
        return int(self.coords.shape[0])

    @property
    def ci(self) -> int:
        return int(self.feats.shape[1])

    @property
    def co(self) -> int:
        return int(self.weight.shape[0])


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to bf16 / f16 (nearest even) and widen back to float32."""
    x = np.ascontiguousarray(x, np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        import torch
        return torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    raise ValueError(dtype)


_CHUNK_ROWS = 1 << 16


def standard_normal_rows(rng, rows: int, cols: int) -> np.ndarray:
    """float32 [rows, cols] ~ N(0,1). Rows are filled in chunks of 65536, each from its own
    generator spawned from one draw of `rng`, on a thread pool; the result depends only on
    the state of `rng`, not on the thread count."""
    from concurrent.futures import ThreadPoolExecutor
    out = np.empty((rows, cols), np.float32)
    nchunk = (rows + _CHUNK_ROWS - 1) // _CHUNK_ROWS
    seeds = np.random.SeedSequence(int(rng.integers(0, 2**63 - 1))).spawn(max(nchunk, 1))

    def fill(k):
        r0 = k * _CHUNK_ROWS
        np.random.default_rng(seeds[k]).standard_normal(
            (min(_CHUNK_ROWS, rows - r0), cols), dtype=np.float32, out=out[r0:r0 + _CHUNK_ROWS])

    with ThreadPoolExecutor(max_workers=8) as ex:
        list(ex.map(fill, range(nchunk)))
    return out


def conv_inputs(rng, n, ci, co, std, dtype, bias_std):
    """Seeded conv inputs: feats [n, ci] ~ N(0,1), W [co, 27, ci] ~ N(0, std), bias ~ N(0, bias_std)
    (zeros when bias_std is 0), feats and W rounded to dtype."""
    feats = round_to(standard_normal_rows(rng, n, ci), dtype)
    weight = round_to(rng.standard_normal((co, 27, ci), dtype=np.float32) * np.float32(std), dtype)
    bias = (rng.standard_normal(co, dtype=np.float32) * np.float32(bias_std)
            if bias_std else np.zeros(co, np.float32))
    return feats, weight, bias


def workload(name: str) -> ConvWorkload:
    """The benchmark / parity conv workloads, by name:

    shell64-c64-f32          sphere shell 23<=r<=25 at centre 32 of 64^3 (~14.5K voxels),
                             C=64 fp32, W ~ N(0, 1/sqrt(27*64)), bias 0, seed 0
    ellipsoids128-c256-bf16  4 random ellipsoid shells, semi-axes U[20,50], thickness 2, in
                             128^3; C=256 bf16, W ~ N(0, 1/sqrt(27*256)), seed 1
    shells256-c128-bf16      8 random ellipsoid/box shells, semi-axes U[40,110], thickness 2,
                             in 256^3; C=128 bf16, Kaiming W ~ N(0, sqrt(2/(27*128))), seed 2
    band512-c64-bf16         the seed-3 256^3 shell set subdivided 2x and pruned to the
                             thickness-2 band at 512^3; C=64 bf16, W ~ N(0, 1/sqrt(27*64))
    shells600k-c128-bf16     shells256-c128-bf16 with the semi-axes drawn from U[24,66] (0.6x),
                             so the set has ~640K voxels, the size the 256^3 C=128 target names
    shells256-c8-bf16        the shells256 voxel set with C=8 bf16 (a thin layer: the VALU path),
                             W ~ N(0, 1/sqrt(27*8)), seed 2
    """
    if name == "shell64-c64-f32":
        rng = np.random.default_rng(0)
        coords = sphere_shell(64, 32.0, 23.0, 25.0)
        f, w, b = conv_inputs(rng, len(coords), 64, 64, 1 / np.sqrt(27 * 64), "f32", 0.0)
        return ConvWorkload(name, coords, f, w, b, "f32", 64, workload.__doc__)
    if name == "ellipsoids128-c256-bf16":
        rng = np.random.default_rng(1)
        coords = band_voxels(random_shapes(rng, 128, 4, 20, 50, boxes=False), 128, 2.0)
        f, w, b = conv_inputs(rng, len(coords), 256, 256, 1 / np.sqrt(27 * 256), "bf16", 0.1)
        return ConvWorkload(name, coords, f, w, b, "bf16", 128, workload.__doc__)
    if name == "shells256-c128-bf16":
        rng = np.random.default_rng(2)
        coords = band_voxels(random_shapes(rng, 256, 8, 40, 110, boxes=True), 256, 2.0)
        f, w, b = conv_inputs(rng, len(coords), 128, 128, np.sqrt(2 / (27 * 128)), "bf16", 0.1)
        return ConvWorkload(name, coords, f, w, b, "bf16", 256, workload.__doc__)
    if name == "shells256-c8-bf16":
        rng = np.random.default_rng(2)
        coords = band_voxels(random_shapes(rng, 256, 8, 40, 110, boxes=True), 256, 2.0)
        f, w, b = conv_inputs(rng, len(coords), 8, 8, 1 / np.sqrt(27 * 8), "bf16", 0.1)
        return ConvWorkload(name, coords, f, w, b, "bf16", 256, workload.__doc__)
    if name == "shells600k-c128-bf16":
        rng = np.random.default_rng(2)
        coords = band_voxels(random_shapes(rng, 256, 8, 24, 66, boxes=True), 256, 2.0)
        f, w, b = conv_inputs(rng, len(coords), 128, 128, np.sqrt(2 / (27 * 128)), "bf16", 0.1)
        return ConvWorkload(name, coords, f, w, b, "bf16", 256, workload.__doc__)
    if name == "band512-c64-bf16":
        rng, parents, mask = band512_parents()
        coords = children(mask, parents)
        f, w, b = conv_inputs(rng, len(coords), 64, 64, 1 / np.sqrt(27 * 64), "bf16", 0.1)
        return ConvWorkload(name, coords, f, w, b, "bf16", 512, workload.__doc__)
    raise KeyError(name)


def band512_parents():
    """The band512 workload's parents and subdivision: 8 random ellipsoid/box shells (semi-axes
    U[40,110], thickness 2, seed 3) voxelised at 256^3, and the mask [8N] that keeps each child
    whose centre lies in the thickness-2 band at 512^3. Returns (rng after the draws, parents,
    mask); the children are children(mask, parents)."""
    rng = np.random.default_rng(3)
    shapes = random_shapes(rng, 256, 8, 40, 110, boxes=True)
    parents = band_voxels(shapes, 256, 2.0)
    mask = subdivision_band_mask(parents, shapes, 2.0)
    return rng, parents, mask


WORKLOADS = ("shell64-c64-f32", "ellipsoids128-c256-bf16", "shells256-c128-bf16",
             "band512-c64-bf16", "shells600k-c128-bf16", "shells256-c8-bf16")


def random_distinct_voxels(n: int, extent: int, seed: int) -> np.ndarray:
    """n distinct voxels drawn uniformly from [0, extent)^3 in draw order, with
    numpy default_rng(seed) integers(0, extent, 3) per draw -- the sampling of the reference's
    parity scripts (tools/ref_sparse_conv.py:38-44, tools/ref_c2s.py:30-36)."""
    rng = np.random.default_rng(seed)
    seen, rows = set(), []
    while len(rows) < n:
        p = tuple(int(x) for x in rng.integers(0, extent, 3))
        if p not in seen:
            seen.add(p)
            rows.append(p)
    return np.asarray(rows, np.int32).reshape(-1, 3)


# ------------------------------------------------------------------------------------------
# The decoder-stack workload
# ------------------------------------------------------------------------------------------
@dataclasses.dataclass
class DecoderWorkload:
    name: str
    coords: np.ndarray        # int32 [N0,3] at the latent resolution
    latent: np.ndarray        # float32 [N0, latent_ch]
    masks: list               # uint8 [8 N_s] subdivision mask of each stage
    counts: list              # voxels at each level (N0 .. N_stages)
    level_coords: list        # int32 [N_s,3] of each level (N0 .. N_stages)
    channels: tuple           # stage widths, e.g. (1024, 512, 256, 128, 64)
    blocks: int               # ConvNeXt blocks per stage
    out_ch: int
    std: float                # weight init
    seed: int
    description: str


def decoder_workload(name: str = "decoder-shells64-c1024") -> DecoderWorkload:
    """The full decoder stack on a 64^3 latent:

    decoder-shells64-c1024   4 random ellipsoid/box shells at 64^3, semi-axes U[8,20],
                             thickness 2 (~34K voxels, 32 latent channels ~ N(0,1)); 4 stages
                             1024 -> 512 -> 256 -> 128 -> 64 channels, each 2 ConvNeXt blocks
                             and a 2x subdivision pruned to the thickness-2 band of the same
                             shapes (the mask drives the texture decoder's route), ending at
                             1024^3; 6 output channels; every weight ~ N(0, 0.02); seed 4
    decoder-shells16-c64     a 16^3 miniature for tests: 2 shells, semi-axes U[3,6], 2 stages
                             64 -> 32 -> 16
    """
    if name == "decoder-shells64-c1024":
        grid, count, lo, hi, ch = 64, 4, 8.0, 20.0, (1024, 512, 256, 128, 64)
    elif name == "decoder-shells16-c64":
        grid, count, lo, hi, ch = 16, 2, 3.0, 6.0, (64, 32, 16)
    else:
        raise KeyError(name)
    rng = np.random.default_rng(4)
    shapes = random_shapes(rng, grid, count, lo, hi, boxes=True)
    coords = band_voxels(shapes, grid, 2.0)
    latent = standard_normal_rows(rng, len(coords), 32)
    masks, levels = [], [coords]
    c = coords
    for _ in range(len(ch) - 1):
        m = subdivision_band_mask(c, shapes, 2.0)
        c = children(m, c)
        masks.append(m)
        levels.append(c)
        shapes = [Shape(sh.kind, sh.center * 2, sh.semi * 2, sh.rot) for sh in shapes]
    return DecoderWorkload(name, coords, latent, masks, [len(x) for x in levels], levels, ch, 2, 6,
                           0.02, 4, decoder_workload.__doc__)


def decoder_params(channels: tuple, blocks: int, latent_ch: int, out_ch: int, std: float,
                   seed: int) -> dict:
    """Random-init weights of the sparse U-Net decoder under the reference's key names
    (shape_decoder.cpp:79-117, sparse.cpp:104, 125-128, 188, 260, 278, 305): from_latent, per stage
    `blocks` ConvNeXt blocks `blocks.s.j` then the C2S block `blocks.s.<blocks>`, output_layer.
    Weights ~ N(0, std); LayerNorm weights 1; biases 0. Conv weights are [Co, 27, Ci]."""
    rng = np.random.default_rng(seed)

    def w(*shape):
        return rng.standard_normal(shape, dtype=np.float32) * np.float32(std)

    z = lambda n: np.zeros(n, np.float32)
    one = lambda n: np.ones(n, np.float32)
    p = {"from_latent.weight": w(channels[0], latent_ch), "from_latent.bias": z(channels[0])}
    for s, (ci, co) in enumerate(zip(channels[:-1], channels[1:])):
        for j in range(blocks):
            q = f"blocks.{s}.{j}"
            p.update({f"{q}.conv.weight": w(ci, 27, ci), f"{q}.conv.bias": z(ci),
                      f"{q}.norm.weight": one(ci), f"{q}.norm.bias": z(ci),
                      f"{q}.mlp.0.weight": w(4 * ci, ci), f"{q}.mlp.0.bias": z(4 * ci),
                      f"{q}.mlp.2.weight": w(ci, 4 * ci), f"{q}.mlp.2.bias": z(ci)})
        q = f"blocks.{s}.{blocks}"
        p.update({f"{q}.to_subdiv.weight": w(8, ci), f"{q}.to_subdiv.bias": z(8),
                  f"{q}.norm1.weight": one(ci), f"{q}.norm1.bias": z(ci),
                  f"{q}.conv1.weight": w(8 * co, 27, ci), f"{q}.conv1.bias": z(8 * co),
                  f"{q}.conv2.weight": w(co, 27, co), f"{q}.conv2.bias": z(co)})
    p["output_layer.weight"] = w(out_ch, channels[-1])
    p["output_layer.bias"] = z(out_ch)
    return p
