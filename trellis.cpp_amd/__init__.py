"""Python binding of libtrellis_sparse.so, the MI355X sparse-voxel conv library.

The library's interface is the C ABI declared in include/trellis_sparse.h; this module loads
it with ctypes and wraps each entry point for torch device tensors (torch supplies device
memory and the current HIP stream; all compute happens in the library's HIP kernels).

There is no fallback: if the shared library is missing or a call fails, an exception is
raised.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtrellis_sparse.so")

TSP_F32, TSP_F16, TSP_BF16 = 0, 1, 2
ALGO = {"auto": 0, "mfma": 1, "narrow": 2, "mfma_gather": 3, "thin": 4, "thin_mfma": 5, "f32_mfma": 6}
STATUS = {0: "OK", 1: "INVALID", 2: "HIP", 3: "RANGE", 4: "UNSUPPORTED", 5: "WORKSPACE"}

# Every extern "C" entry point the header declares (checked by the CPU test suite).
EXPORTS = (
    "tsp_last_error", "tsp_version",
    "tsp_rulebook_workspace_bytes", "tsp_rulebook_build", "tsp_rulebook_build_planned", "tsp_rulebook_count_pairs",
    "tsp_convnext_mlp_packed_bytes", "tsp_convnext_mlp_pack", "tsp_convnext_mlp",
    "tsp_subm_conv3x3", "tsp_subm_conv3x3_ex",
    "tsp_conv_plan_bytes", "tsp_conv_plan_build", "tsp_conv_plan_build_ordered",
    "tsp_conv_weight_pack", "tsp_conv_weight_packed_bytes", "tsp_subm_conv3x3_planned_ln",
    "tsp_subm_conv3x3_planned", "tsp_subm_conv3x3_planned_ex", "tsp_subm_conv3x3_planned_octants",
    "tsp_subm_conv3x3_planned_skip",
    "tsp_subdivide_workspace_bytes", "tsp_subdivide", "tsp_subdivide_noalloc",
    "tsp_linear", "tsp_linear_ex", "tsp_linear_rows_per_call", "tsp_layer_norm", "tsp_c2s_gather", "tsp_c2s_skip_add",
    "tsp_mask_positive",
    "tsp_convnext_workspace_bytes", "tsp_convnext", "tsp_convnext_ex", "tsp_c2s_workspace_bytes", "tsp_c2s",
    "tsp_c2s_ex", "tsp_c2s_part",
)

BLOCK_CAST_F32 = 2


class ConvNextWeights(ctypes.Structure):
    """tsp_convnext_weights: device pointers, dtypes as tsp_dtype codes."""
    _fields_ = [("conv_weight", ctypes.c_void_p), ("conv_dtype", ctypes.c_int), ("conv_bias", ctypes.c_void_p),
                ("conv_packed", ctypes.c_void_p), ("norm_weight", ctypes.c_void_p),
                ("norm_bias", ctypes.c_void_p), ("mlp0_weight", ctypes.c_void_p), ("mlp0_dtype", ctypes.c_int),
                ("mlp0_bias", ctypes.c_void_p), ("mlp2_weight", ctypes.c_void_p), ("mlp2_dtype", ctypes.c_int),
                ("mlp2_bias", ctypes.c_void_p), ("mlp_packed", ctypes.c_void_p)]


class C2SWeights(ctypes.Structure):
    """tsp_c2s_weights: device pointers, dtypes as tsp_dtype codes."""
    _fields_ = [("norm1_weight", ctypes.c_void_p), ("norm1_bias", ctypes.c_void_p),
                ("conv1_weight", ctypes.c_void_p), ("conv1_dtype", ctypes.c_int), ("conv1_bias", ctypes.c_void_p),
                ("conv1_packed", ctypes.c_void_p), ("conv2_weight", ctypes.c_void_p), ("conv2_dtype", ctypes.c_int),
                ("conv2_bias", ctypes.c_void_p), ("conv2_packed", ctypes.c_void_p)]


class TspError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} -> {STATUS.get(code, code)}: {msg}")
        self.code = code


_lib = None


def build(jobs: int = 8) -> str:
    """Compile libtrellis_sparse.so for gfx950 (hipcc through trellis.cpp_amd/Makefile)."""
    subprocess.run(["make", "-s", "-C", HERE, f"-j{jobs}"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(
            f"{LIB_PATH} is not built; run `make -C {HERE}` (or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    c_i64, c_int, c_sz, c_vp = ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
    L.tsp_last_error.restype = ctypes.c_char_p
    L.tsp_last_error.argtypes = []
    L.tsp_version.restype = c_int
    L.tsp_rulebook_workspace_bytes.restype = c_sz
    L.tsp_rulebook_workspace_bytes.argtypes = [c_i64]
    L.tsp_rulebook_build.restype = c_int
    L.tsp_rulebook_build.argtypes = [c_vp, c_i64, c_vp, c_vp, c_sz, c_vp, c_vp]
    L.tsp_convnext_mlp_packed_bytes.restype = c_sz
    L.tsp_convnext_mlp_packed_bytes.argtypes = [c_int]
    L.tsp_convnext_mlp_pack.restype = c_int
    L.tsp_convnext_mlp_pack.argtypes = [c_vp, c_vp, c_int, c_int, c_vp, c_vp]
    L.tsp_convnext_mlp.restype = c_int
    L.tsp_convnext_mlp.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]
    L.tsp_rulebook_build_planned.restype = c_int
    L.tsp_rulebook_build_planned.argtypes = [c_vp, c_i64, c_vp, c_vp, c_sz, c_vp, c_vp, c_sz, c_vp]
    L.tsp_rulebook_count_pairs.restype = c_int
    L.tsp_rulebook_count_pairs.argtypes = [c_vp, c_i64, c_vp, c_vp]
    L.tsp_subm_conv3x3.restype = c_int
    L.tsp_subm_conv3x3.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, c_int, c_vp, c_int,
                                   c_vp, c_int, c_int, c_vp]
    L.tsp_subm_conv3x3_ex.restype = c_int
    L.tsp_subm_conv3x3_ex.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, c_int, c_vp, c_int,
                                      c_vp, c_int, c_int, c_int, c_vp, c_vp]
    L.tsp_conv_plan_bytes.restype = c_sz
    L.tsp_conv_plan_bytes.argtypes = [c_i64]
    L.tsp_conv_plan_build.restype = c_int
    L.tsp_conv_plan_build.argtypes = [c_vp, c_i64, c_vp, c_sz, c_vp]
    L.tsp_conv_plan_build_ordered.restype = c_int
    L.tsp_conv_plan_build_ordered.argtypes = [c_vp, c_vp, c_i64, c_vp, c_sz, c_vp]
    L.tsp_conv_weight_pack.restype = c_int
    L.tsp_conv_weight_pack.argtypes = [c_vp, c_int, c_int, c_int, c_vp, c_vp]
    L.tsp_conv_weight_packed_bytes.restype = c_sz
    L.tsp_conv_weight_packed_bytes.argtypes = [c_int, c_int]
    L.tsp_subm_conv3x3_planned_ln.restype = c_int
    L.tsp_subm_conv3x3_planned_ln.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, c_vp, c_vp, c_int, c_vp, c_vp,
                                              ctypes.c_float, c_vp, c_vp, c_vp]
    L.tsp_subm_conv3x3_planned.restype = c_int
    L.tsp_subm_conv3x3_planned.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, c_vp, c_vp,
                                           c_int, c_vp, c_int, c_vp]
    L.tsp_subm_conv3x3_planned_ex.restype = c_int
    L.tsp_subm_conv3x3_planned_ex.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, c_vp, c_vp,
                                              c_int, c_vp, c_int, c_int, c_vp, c_vp]
    L.tsp_subm_conv3x3_planned_octants.restype = c_int
    L.tsp_subm_conv3x3_planned_octants.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, c_vp,
                                                   c_vp, c_int, c_vp, c_vp, c_vp, c_vp]
    L.tsp_subm_conv3x3_planned_skip.restype = c_int
    L.tsp_subm_conv3x3_planned_skip.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, c_vp, c_vp,
                                                c_int, c_vp, c_int, c_vp, c_vp, c_vp]
    L.tsp_linear.restype = c_int
    L.tsp_linear.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_int, c_vp, c_int, c_vp, c_int,
                             c_vp]
    L.tsp_linear_ex.restype = c_int
    L.tsp_linear_ex.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_int, c_vp, c_int, c_int, c_vp,
                                c_vp, c_int, c_vp]
    L.tsp_linear_rows_per_call.restype = c_i64
    L.tsp_linear_rows_per_call.argtypes = [c_int, c_int, c_int, c_int, c_int]
    L.tsp_layer_norm.restype = c_int
    L.tsp_layer_norm.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, ctypes.c_float, c_int,
                                 c_vp, c_int, c_vp]
    L.tsp_c2s_gather.restype = c_int
    L.tsp_c2s_gather.argtypes = [c_vp, c_int, c_vp, c_i64, c_int, c_vp, c_vp]
    L.tsp_c2s_skip_add.restype = c_int
    L.tsp_c2s_skip_add.argtypes = [c_vp, c_int, c_vp, c_i64, c_int, c_int, c_vp, c_int, c_vp]
    L.tsp_mask_positive.restype = c_int
    L.tsp_mask_positive.argtypes = [c_vp, c_i64, c_vp, c_vp]
    L.tsp_subdivide_workspace_bytes.restype = c_sz
    L.tsp_subdivide_workspace_bytes.argtypes = [c_i64]
    L.tsp_subdivide.restype = c_int
    L.tsp_subdivide.argtypes = [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp]
    L.tsp_subdivide_noalloc.restype = c_int
    L.tsp_subdivide_noalloc.argtypes = [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp]
    cnw, c2w = ctypes.POINTER(ConvNextWeights), ctypes.POINTER(C2SWeights)
    L.tsp_convnext_workspace_bytes.restype = c_sz
    L.tsp_convnext_workspace_bytes.argtypes = [c_i64, c_int, c_int, cnw, c_int, c_int]
    L.tsp_convnext.restype = c_int
    L.tsp_convnext.argtypes = [c_vp, c_int, c_i64, c_int, c_vp, c_vp, cnw, c_vp, c_vp, c_sz, c_int, c_vp]
    L.tsp_convnext_ex.restype = c_int
    L.tsp_convnext_ex.argtypes = [c_vp, c_int, c_vp, c_i64, c_int, c_vp, c_vp, cnw, c_vp, c_vp, c_int, c_vp, c_sz,
                                  c_int, c_vp]
    L.tsp_c2s_workspace_bytes.restype = c_sz
    L.tsp_c2s_workspace_bytes.argtypes = [c_i64, c_i64, c_int, c_int, c2w, c_int, c_int, c_int]
    L.tsp_c2s.restype = c_int
    L.tsp_c2s.argtypes = [c_vp, c_i64, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_int, c_vp, c_vp, c2w,
                          c_vp, c_vp, c_sz, c_int, c_vp]
    L.tsp_c2s_ex.restype = c_int
    L.tsp_c2s_ex.argtypes = [c_vp, c_i64, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_int, c_vp, c_vp, c2w,
                             c_vp, c_vp, c_int, c_vp, c_sz, c_int, c_vp]
    L.tsp_c2s_part.restype = c_int
    L.tsp_c2s_part.argtypes = [c_vp, c_i64, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_int, c_vp, c_vp, c2w,
                               c_vp, c_vp, c_int, c_vp, c_sz, c_int, c_int, c_i64, c_i64, c_vp]
    _lib = L
    return L


def _check(fn: str, code: int) -> None:
    if code != 0:
        raise TspError(fn, code, lib().tsp_last_error().decode(errors="replace"))


# --------------------------------------------------------------------------------------------
# torch conveniences (device memory + stream plumbing only)
# --------------------------------------------------------------------------------------------
def _torch():
    import torch
    return torch


def dtype_code(dt) -> int:
    torch = _torch()
    return {torch.float32: TSP_F32, torch.float16: TSP_F16, torch.bfloat16: TSP_BF16}[dt]


def _stream(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("tensors must live on the GPU")


def _table_buffers(c, n, nbr, workspace):
    torch = _torch()
    ws_bytes = lib().tsp_rulebook_workspace_bytes(n)
    if nbr is None:
        nbr = torch.empty(27 * n, dtype=torch.int32, device=c.device)
    elif nbr.dtype != torch.int32 or nbr.numel() != 27 * n or not nbr.is_contiguous():
        raise ValueError("nbr must be a contiguous int32 buffer of 27*N")
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=c.device)
    elif workspace.dtype != torch.uint8 or workspace.numel() < ws_bytes:
        raise ValueError("workspace must be a uint8 buffer of tsp_rulebook_workspace_bytes(N)")
    return nbr, workspace, ws_bytes


def rulebook_build(coords, check: bool = True, nbr=None, workspace=None, stream=None):
    """coords int32 [N,3] on the GPU -> tap-major int32 neighbour table [27*N] (sentinel N).
    nbr and workspace (uint8, tsp_rulebook_workspace_bytes(N)) may be given to reuse buffers;
    check=False skips the range check's read-back."""
    torch = _torch()
    _require_cuda(coords)
    c = coords.contiguous()
    if c.dtype != torch.int32 or c.dim() != 2 or c.shape[1] != 3:
        raise ValueError("coords must be int32 [N, 3]")
    n = c.shape[0]
    nbr, ws, ws_bytes = _table_buffers(c, n, nbr, workspace)
    status = torch.zeros(1, dtype=torch.int32, device=c.device) if check else None
    _check("tsp_rulebook_build",
           lib().tsp_rulebook_build(_ptr(c), n, _ptr(nbr), _ptr(ws), ws_bytes, _ptr(status),
                                    _stream(stream)))
    if check and n and int(status.item()) != 0:
        raise TspError("tsp_rulebook_build", 3, "coordinate outside [0, 2^21-3]")
    return nbr


def rulebook_build_planned(coords, check: bool = True, nbr=None, workspace=None, plan=None, stream=None):
    """coords int32 [N,3] on the GPU -> (neighbour table int32 [27*N], Morton-ordered conv plan
    uint8 buffer): rulebook_build and conv_plan_build(coords=...) in one call on one cell grid.
    nbr, workspace (uint8, tsp_rulebook_workspace_bytes(N)) and plan (uint8, tsp_conv_plan_bytes(N))
    may be given to reuse buffers."""
    torch = _torch()
    _require_cuda(coords)
    c = coords.contiguous()
    if c.dtype != torch.int32 or c.dim() != 2 or c.shape[1] != 3:
        raise ValueError("coords must be int32 [N, 3]")
    n = c.shape[0]
    nbr, workspace, ws_bytes = _table_buffers(c, n, nbr, workspace)
    nb = lib().tsp_conv_plan_bytes(n)
    if plan is None:
        plan = torch.empty(max(nb, 1), dtype=torch.uint8, device=c.device)
    elif plan.dtype != torch.uint8 or plan.numel() < nb:
        raise ValueError("plan must be a uint8 buffer of tsp_conv_plan_bytes(N)")
    status = torch.zeros(1, dtype=torch.int32, device=c.device) if check else None
    _check("tsp_rulebook_build_planned",
           lib().tsp_rulebook_build_planned(_ptr(c), n, _ptr(nbr), _ptr(workspace), ws_bytes,
                                            _ptr(status), _ptr(plan), nb,
                                            _stream(stream)))
    if check and n and int(status.item()) != 0:
        raise TspError("tsp_rulebook_build_planned", 3, "coordinate outside [0, 2^21-3]")
    return nbr, plan


def convnext_mlp_pack(w0, w2, stream=None):
    """w0 [4C, C], w2 [C, 4C] of one 16-bit dtype -> the packed buffer tsp_convnext_mlp reads."""
    torch = _torch()
    _require_cuda(w0, w2)
    c = w0.shape[1]
    if w2.dtype != w0.dtype or tuple(w0.shape) != (4 * c, c) or tuple(w2.shape) != (c, 4 * c):
        raise ValueError("w0 [4C, C] and w2 [C, 4C] of one dtype")
    w0, w2 = w0.contiguous(), w2.contiguous()
    packed = torch.empty(lib().tsp_convnext_mlp_packed_bytes(c) // 2, dtype=w0.dtype, device=w0.device)
    _check("tsp_convnext_mlp_pack",
           lib().tsp_convnext_mlp_pack(_ptr(w0), _ptr(w2), dtype_code(w0.dtype), c, _ptr(packed), _stream(stream)))
    return packed


def convnext_mlp(xn, packed, b0, b2, x, out=None, stream=None):
    """The ConvNeXt MLP in one kernel: out f32 [N, C] = x + b2 + w2 . silu(w0 . xn + b0) for xn
    [N, C] (16-bit), the weights packed by convnext_mlp_pack, x f32 [N, C], C = 128; out may be x."""
    torch = _torch()
    _require_cuda(xn, packed, x)
    n, c = xn.shape
    if packed.dtype != xn.dtype or packed.numel() * 2 != lib().tsp_convnext_mlp_packed_bytes(c):
        raise ValueError("packed must come from convnext_mlp_pack with xn's dtype and C")
    if x.dtype != torch.float32 or tuple(x.shape) != (n, c):
        raise ValueError("x must be float32 [N, C]")
    for name, b, size in (("b0", b0, 4 * c), ("b2", b2, c)):
        if b is not None and (b.dtype != torch.float32 or b.numel() != size or not b.is_contiguous()
                              or b.device != xn.device):
            raise ValueError(f"{name} must be a contiguous float32 vector of {size} on xn's device")
    if out is None:
        out = torch.empty((n, c), dtype=torch.float32, device=xn.device)
    elif (out.dtype != torch.float32 or tuple(out.shape) != (n, c) or not out.is_contiguous()
          or out.device != xn.device):
        raise ValueError("out must be a contiguous float32 [N, C] tensor on xn's device")
    xn, x = xn.contiguous(), x.contiguous()
    _check("tsp_convnext_mlp",
           lib().tsp_convnext_mlp(_ptr(xn), dtype_code(xn.dtype), n, c, _ptr(packed), _ptr(b0), _ptr(b2),
                                  _ptr(x), _ptr(out), _stream(stream)))
    return out


def count_pairs(nbr, n: int, stream=None) -> int:
    torch = _torch()
    _require_cuda(nbr)
    cnt = torch.zeros(1, dtype=torch.int64, device=nbr.device)
    _check("tsp_rulebook_count_pairs",
           lib().tsp_rulebook_count_pairs(_ptr(nbr), n, _ptr(cnt), _stream(stream)))
    return int(cnt.item())


def _check_out(out, n: int, co: int, dtype, device):
    """A caller's out= must be a contiguous [n, co] tensor of the output dtype on the device the
    inputs are on: the kernels write n * co elements through its raw pointer."""
    if tuple(out.shape) != (n, co):
        raise ValueError(f"out must have shape ({n}, {co}), got {tuple(out.shape)}")
    if out.dtype != dtype:
        raise ValueError(f"out must be {dtype}, got {out.dtype}")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")
    if out.device != device:
        raise ValueError(f"out must live on {device}, got {out.device}")


def _check_nbr(nbr, n: int, device):
    torch = _torch()
    if nbr.dtype != torch.int32 or nbr.numel() != 27 * n or not nbr.is_contiguous():
        raise ValueError(f"nbr must be a contiguous int32 table of 27*N = {27 * n} entries")
    if nbr.device != device:
        raise ValueError("nbr must live on the features' device")


def subm_conv3x3(feats, nbr, weight, bias, out_dtype=None, algo: str = "auto", out=None,
                 zero_pad: bool = False, row0=None, stream=None):
    """feats [N,Ci], nbr int32 [27*N], weight [Co,27,Ci], bias f32 [Co] -> out [N,Co].
    zero_pad: absent taps read an exact zero row instead of 0 * feats[0]; row0 (float32 [Ci]):
    the unrounded row 0 the features were rounded from, whose 0 * row0 is the padding row."""
    torch = _torch()
    if feats.dim() != 2:
        raise ValueError("feats must be [N, Ci]")
    n, ci = feats.shape
    co = weight.shape[0]
    if weight.shape != (co, 27, ci):
        raise ValueError(f"weight must be [Co,27,Ci]=[{co},27,{ci}], got {tuple(weight.shape)}")
    _check_nbr(nbr, n, feats.device)
    if bias.dtype != torch.float32 or bias.numel() != co:
        raise ValueError("bias must be float32 [Co]")
    if row0 is not None and (row0.dtype != torch.float32 or row0.numel() != ci):
        raise ValueError("row0 must be float32 [Ci]")
    odt = out_dtype or feats.dtype
    if out is None:
        out = torch.empty((n, co), dtype=odt, device=feats.device)
    else:
        _check_out(out, n, co, odt, feats.device)
    _require_cuda(feats, nbr, weight, bias, out, row0)
    f, w, b = feats.contiguous(), weight.contiguous(), bias.contiguous()
    r0 = row0.contiguous() if row0 is not None else None
    _check("tsp_subm_conv3x3_ex",
           lib().tsp_subm_conv3x3_ex(_ptr(f), dtype_code(f.dtype), n, ci, _ptr(nbr), _ptr(w),
                                     dtype_code(w.dtype), _ptr(b), co, _ptr(out),
                                     dtype_code(out.dtype), ALGO[algo], 1 if zero_pad else 0,
                                     _ptr(r0), _stream(stream)))
    return out


def conv_plan_build(nbr, n: int, coords=None, plan=None, stream=None):
    """Plan of neighbour table nbr (int32 [27*N]) for the planned convs -> uint8 buffer (plan, of
    tsp_conv_plan_bytes(N), may be given to reuse it). With coords (int32 [N, 3], the coordinates
    the table was built from) tiles follow the Morton order of the voxels' 8^3 cells; without,
    tiles are consecutive rows."""
    torch = _torch()
    _require_cuda(nbr, coords)
    _check_nbr(nbr, n, nbr.device)
    nb = lib().tsp_conv_plan_bytes(n)
    if plan is None:
        plan = torch.empty(max(nb, 1), dtype=torch.uint8, device=nbr.device)
    elif plan.dtype != torch.uint8 or plan.numel() < nb:
        raise ValueError("plan must be a uint8 buffer of tsp_conv_plan_bytes(N)")
    if coords is None:
        _check("tsp_conv_plan_build",
               lib().tsp_conv_plan_build(_ptr(nbr), n, _ptr(plan), nb, _stream(stream)))
    else:
        c = coords.contiguous()
        if c.dtype != torch.int32 or tuple(c.shape) != (n, 3):
            raise ValueError("coords must be int32 [N, 3]")
        _check("tsp_conv_plan_build_ordered",
               lib().tsp_conv_plan_build_ordered(_ptr(nbr), _ptr(c), n, _ptr(plan), nb, _stream(stream)))
    return plan


def conv_weight_pack(weight, stream=None):
    """W [Co,27,Ci] f16/bf16 -> packed copy (same dtype, flat): the values in operand order, then
    the 256-byte trailer (tsp_conv_weight_packed_bytes(Ci, Co) bytes in all)."""
    torch = _torch()
    _require_cuda(weight)
    w = weight.contiguous()
    co, _, ci = w.shape
    packed = torch.empty(lib().tsp_conv_weight_packed_bytes(ci, co) // 2, dtype=w.dtype, device=w.device)
    _check("tsp_conv_weight_pack",
           lib().tsp_conv_weight_pack(_ptr(w), dtype_code(w.dtype), ci, co, _ptr(packed),
                                      _stream(stream)))
    return packed


def _check_planned(feats, nbr, plan, packed_weight, ci: int, co: int):
    n = feats.shape[0]
    _check_nbr(nbr, n, feats.device)
    need = lib().tsp_conv_plan_bytes(n)
    if plan.numel() * plan.element_size() < need:
        raise ValueError(f"plan holds {plan.numel() * plan.element_size()} bytes; a table of {n} "
                         f"voxels needs {need}")
    if packed_weight.dtype != feats.dtype:
        raise ValueError(f"packed weight is {packed_weight.dtype}, features are {feats.dtype}")
    if packed_weight.numel() * packed_weight.element_size() != lib().tsp_conv_weight_packed_bytes(ci, co):
        raise ValueError("packed weight size does not match [Co,27,Ci] (see conv_weight_pack)")
    if not packed_weight.is_contiguous():
        raise ValueError("packed weight must be contiguous")


def subm_conv3x3_planned(feats, nbr, plan, packed_weight, bias, co: int, out_dtype=None, out=None,
                         zero_pad: bool = False, row0=None, stream=None):
    """The MFMA conv with a plan (conv_plan_build) and packed weights (conv_weight_pack).
    zero_pad: absent taps read an exact zero row; row0 (float32 [Ci]): the unrounded row 0 the
    features were rounded from, whose 0 * row0 is the padding row."""
    torch = _torch()
    if feats.dim() != 2:
        raise ValueError("feats must be [N, Ci]")
    n, ci = feats.shape
    _check_planned(feats, nbr, plan, packed_weight, ci, co)
    if bias.dtype != torch.float32 or bias.numel() != co:
        raise ValueError("bias must be float32 [Co]")
    if row0 is not None and (row0.dtype != torch.float32 or row0.numel() != ci):
        raise ValueError("row0 must be float32 [Ci]")
    odt = out_dtype or feats.dtype
    if out is None:
        out = torch.empty((n, co), dtype=odt, device=feats.device)
    else:
        _check_out(out, n, co, odt, feats.device)
    _require_cuda(feats, nbr, plan, packed_weight, bias, out, row0)
    f = feats.contiguous()
    r0 = row0.contiguous() if row0 is not None else None
    _check("tsp_subm_conv3x3_planned_ex",
           lib().tsp_subm_conv3x3_planned_ex(_ptr(f), dtype_code(f.dtype), n, ci, _ptr(nbr),
                                             _ptr(plan), _ptr(packed_weight), _ptr(bias), co,
                                             _ptr(out), dtype_code(out.dtype),
                                             1 if zero_pad else 0, _ptr(r0), _stream(stream)))
    return out


def subm_conv3x3_planned_ln(feats, nbr, plan, packed_weight, bias, co: int, norm_weight, norm_bias,
                            eps: float = 1e-6, out=None, row0=None, stream=None):
    """The planned conv with each output row layer-normalised by its stores (co = 64 or 128):
    (h - mean) / sqrt(var + eps) * norm_weight + norm_bias for h = conv + bias, in the feature
    dtype."""
    torch = _torch()
    if feats.dim() != 2:
        raise ValueError("feats must be [N, Ci]")
    n, ci = feats.shape
    _check_planned(feats, nbr, plan, packed_weight, ci, co)
    for name, t in (("bias", bias), ("norm_weight", norm_weight), ("norm_bias", norm_bias)):
        if t.dtype != torch.float32 or t.numel() != co:
            raise ValueError(f"{name} must be float32 [Co]")
    if row0 is not None and (row0.dtype != torch.float32 or row0.numel() != ci):
        raise ValueError("row0 must be float32 [Ci]")
    if out is None:
        out = torch.empty((n, co), dtype=feats.dtype, device=feats.device)
    else:
        _check_out(out, n, co, feats.dtype, feats.device)
    _require_cuda(feats, nbr, plan, packed_weight, bias, norm_weight, norm_bias, out, row0)
    f = feats.contiguous()
    r0 = row0.contiguous() if row0 is not None else None
    _check("tsp_subm_conv3x3_planned_ln",
           lib().tsp_subm_conv3x3_planned_ln(_ptr(f), dtype_code(f.dtype), n, ci, _ptr(nbr), _ptr(plan),
                                             _ptr(packed_weight), _ptr(bias), co, _ptr(norm_weight),
                                             _ptr(norm_bias), float(eps), _ptr(out), _ptr(r0), _stream(stream)))
    return out


def subm_conv3x3_planned_octants(feats, nbr, plan, packed_weight, bias, cout: int, mask, mstart,
                                 m: int, stream=None):
    """The C2S conv1 with its octant gather in the stores: the planned conv to 8*cout channels,
    parent i's channels [o*cout, +cout) written to its child of octant o (mask and mstart as
    given to / returned by subdivide) -> float32 [M, cout]."""
    torch = _torch()
    n, ci = feats.shape
    co = 8 * cout
    _check_planned(feats, nbr, plan, packed_weight, ci, co)
    if bias.dtype != torch.float32 or bias.numel() != co:
        raise ValueError("bias must be float32 [8*cout]")
    m8 = mask.reshape(-1).contiguous()
    if m8.dtype != torch.uint8 or m8.numel() != 8 * n:
        raise ValueError("mask must be uint8 with 8*N entries")
    if mstart.dtype != torch.int32 or mstart.numel() != n + 1:
        raise ValueError("mstart must be int32 [N+1]")
    _require_cuda(feats, nbr, plan, packed_weight, bias, mask, mstart)
    # the kernel writes rows up to mstart[N] - 1: the output must hold exactly that many
    if n and int(mstart[-1].item()) != m:
        raise ValueError(f"m={m} but the subdivision has mstart[N]={int(mstart[-1].item())} children")
    out = torch.empty((m, cout), dtype=torch.float32, device=feats.device)
    f = feats.contiguous()
    _check("tsp_subm_conv3x3_planned_octants",
           lib().tsp_subm_conv3x3_planned_octants(_ptr(f), dtype_code(f.dtype), n, ci, _ptr(nbr),
                                                  _ptr(plan), _ptr(packed_weight), _ptr(bias), cout,
                                                  _ptr(m8), _ptr(mstart), _ptr(out),
                                                  _stream(stream)))
    return out


def subm_conv3x3_planned_skip(feats, nbr, plan, packed_weight, bias, co: int, x, gidx, stream=None):
    """The C2S conv2 with the block's skip added by its stores: the planned conv (f32 out) over
    the M children plus repeat_interleave of x's octant blocks (x float32 [N, cin], gidx from
    subdivide) -> float32 [M, co]."""
    torch = _torch()
    m, ci = feats.shape
    _check_planned(feats, nbr, plan, packed_weight, ci, co)
    if bias.dtype != torch.float32 or bias.numel() != co:
        raise ValueError("bias must be float32 [Co]")
    xc = x.contiguous()
    if xc.dtype != torch.float32 or xc.dim() != 2:
        raise ValueError("x must be float32 [N, cin]")
    if gidx.dtype != torch.int32 or gidx.numel() != m:
        raise ValueError("gidx must be int32 [M]")
    _require_cuda(feats, nbr, plan, packed_weight, bias, x, gidx)
    # the stores read x[gidx // 8]: every gidx must name an octant of a row of x
    if m and not (0 <= int(gidx.min().item()) and int(gidx.max().item()) < 8 * xc.shape[0]):
        raise ValueError("gidx holds an octant outside x's rows")
    out = torch.empty((m, co), dtype=torch.float32, device=feats.device)
    f = feats.contiguous()
    _check("tsp_subm_conv3x3_planned_skip",
           lib().tsp_subm_conv3x3_planned_skip(_ptr(f), dtype_code(f.dtype), m, ci, _ptr(nbr),
                                               _ptr(plan), _ptr(packed_weight), _ptr(bias), co,
                                               _ptr(xc), xc.shape[1], _ptr(gidx), _ptr(out),
                                               _stream(stream)))
    return out


def subdivide(mask, coords, stream=None):
    """mask uint8 [8N] (or [N,8]), coords int32 [N,3] -> (child coords [M,3], gidx [M],
    mstart [N+1])."""
    torch = _torch()
    _require_cuda(mask, coords)
    c = coords.contiguous()
    n = c.shape[0]
    m8 = mask.reshape(-1).contiguous()
    if m8.dtype != torch.uint8 or m8.numel() != 8 * n:
        raise ValueError("mask must be uint8 with 8*N entries")
    mstart = torch.empty(n + 1, dtype=torch.int32, device=c.device)
    child = torch.empty((max(8 * n, 1), 3), dtype=torch.int32, device=c.device)
    gidx = torch.empty(max(8 * n, 1), dtype=torch.int32, device=c.device)
    m_dev = torch.empty(1, dtype=torch.int64, device=c.device)
    ws_bytes = lib().tsp_subdivide_workspace_bytes(n)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=c.device)
    _check("tsp_subdivide",
           lib().tsp_subdivide(_ptr(m8), _ptr(c), n, _ptr(mstart), _ptr(child), _ptr(gidx),
                               _ptr(m_dev), _ptr(ws), ws_bytes, _stream(stream)))
    m = int(m_dev.item())
    return child[:m], gidx[:m], mstart


def linear(x, weight, bias=None, out_dtype=None, stream=None):
    """x [N,Ci] . W^T + bias for W [Co,Ci] -> [N,Co] (fp32 accumulation)."""
    torch = _torch()
    _require_cuda(x, weight, bias)
    n, ci = x.shape
    co = weight.shape[0]
    if weight.shape != (co, ci):
        raise ValueError("weight must be [Co, Ci]")
    out = torch.empty((n, co), dtype=out_dtype or x.dtype, device=x.device)
    xc, wc = x.contiguous(), weight.contiguous()
    _check("tsp_linear",
           lib().tsp_linear(_ptr(xc), dtype_code(xc.dtype), n, ci, _ptr(wc), dtype_code(wc.dtype),
                            _ptr(bias), co, _ptr(out), dtype_code(out.dtype), _stream(stream)))
    return out


ACT = {"none": 0, "silu": 1}


def linear_ex(x, weight, bias=None, act: str = "none", residual=None, out_dtype=None, stream=None):
    """act(x [N,Ci] . W^T + bias) + residual for W [Co,Ci] -> [N,Co], one library GEMM with the
    bias, activation and residual in its epilogue (16-bit x and W of one dtype; raises
    TspError UNSUPPORTED otherwise)."""
    torch = _torch()
    _require_cuda(x, weight, bias, residual)
    n, ci = x.shape
    co = weight.shape[0]
    if weight.shape != (co, ci):
        raise ValueError("weight must be [Co, Ci]")
    if residual is not None and (residual.dtype != torch.float32 or residual.shape != (n, co)):
        raise ValueError("residual must be float32 [N, Co]")
    out = torch.empty((n, co), dtype=out_dtype or x.dtype, device=x.device)
    xc, wc = x.contiguous(), weight.contiguous()
    rc = residual.contiguous() if residual is not None else None
    _check("tsp_linear_ex",
           lib().tsp_linear_ex(_ptr(xc), dtype_code(xc.dtype), n, ci, _ptr(wc), dtype_code(wc.dtype),
                               _ptr(bias), co, ACT[act], _ptr(rc), _ptr(out), dtype_code(out.dtype),
                               _stream(stream)))
    return out


def layer_norm(x, gamma=None, beta=None, eps: float = 1e-6, silu: bool = False, out_dtype=None,
               stream=None):
    """Row LayerNorm over channels (biased variance) [* gamma + beta] [then SiLU]."""
    torch = _torch()
    _require_cuda(x, gamma, beta)
    xc = x.contiguous()
    n, c = xc.shape
    out = torch.empty((n, c), dtype=out_dtype or x.dtype, device=x.device)
    _check("tsp_layer_norm",
           lib().tsp_layer_norm(_ptr(xc), dtype_code(xc.dtype), n, c, _ptr(gamma), _ptr(beta),
                                eps, 1 if silu else 0, _ptr(out), dtype_code(out.dtype),
                                _stream(stream)))
    return out


def c2s_gather(h, gidx, cout: int, stream=None):
    """h [N, 8*cout] -> [M, cout]: child m takes block gidx[m] % 8 of parent gidx[m] // 8."""
    torch = _torch()
    _require_cuda(h, gidx)
    m = gidx.numel()
    out = torch.empty((m, cout), dtype=h.dtype, device=h.device)
    hc = h.contiguous()
    _check("tsp_c2s_gather",
           lib().tsp_c2s_gather(_ptr(hc), dtype_code(hc.dtype), _ptr(gidx), m, cout, _ptr(out),
                                _stream(stream)))
    return out


def c2s_skip_add(x, gidx, acc, stream=None):
    """acc [M, Cout] += repeat_interleave(x.reshape(8N, Cin/8)[gidx], Cout/(Cin/8)) in place."""
    _require_cuda(x, gidx, acc)
    xc = x.contiguous()
    m, cout = acc.shape
    _check("tsp_c2s_skip_add",
           lib().tsp_c2s_skip_add(_ptr(xc), dtype_code(xc.dtype), _ptr(gidx), m, xc.shape[1],
                                  cout, _ptr(acc), dtype_code(acc.dtype), _stream(stream)))
    return acc


def mask_positive(logits, stream=None):
    """uint8 mask of logits > 0 (float32 input, any shape)."""
    torch = _torch()
    _require_cuda(logits)
    lc = logits.contiguous()
    mask = torch.empty(lc.shape, dtype=torch.uint8, device=lc.device)
    _check("tsp_mask_positive",
           lib().tsp_mask_positive(_ptr(lc), lc.numel(), _ptr(mask), _stream(stream)))
    return mask


def _vec(t, n: int, name: str):
    torch = _torch()
    if t.dtype != torch.float32 or t.numel() != n:
        raise ValueError(f"{name} must be float32 [{n}]")
    return t.contiguous()


def _mat(t, shape, name: str):
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {list(shape)}, got {list(t.shape)}")
    return t.contiguous()


def convnext(x, nbr, p: dict, plan=None, cast_f32: bool = False, stream=None, x16=None, out16_dtype=None):
    """SparseConvNeXtBlock3d through tsp_convnext_ex: x [N, C] (f32, or 16-bit of the conv input's
    type), p the block's tensors by their reference names without the prefix ("conv.weight"
    [C,27,C], "conv.bias", "norm.weight", "norm.bias", "mlp.0.weight" [4C,C], "mlp.0.bias",
    "mlp.2.weight" [C,4C], "mlp.2.bias"); optional "conv.packed" (conv_weight_pack) and
    "mlp.packed" (convnext_mlp_pack of mlp.0 and mlp.2). x16, optional with f32 x: x already
    rounded to the conv input's 16-bit type. -> f32 [N, C], or (out, out rounded to out16_dtype)
    when out16_dtype (torch.bfloat16 / torch.float16) is given."""
    torch = _torch()
    n, c = x.shape
    _check_nbr(nbr, n, x.device)
    t = {"conv.weight": _mat(p["conv.weight"], (c, 27, c), "conv.weight"),
         "mlp.0.weight": _mat(p["mlp.0.weight"], (4 * c, c), "mlp.0.weight"),
         "mlp.2.weight": _mat(p["mlp.2.weight"], (c, 4 * c), "mlp.2.weight")}
    for k, m in (("conv.bias", c), ("norm.weight", c), ("norm.bias", c), ("mlp.0.bias", 4 * c), ("mlp.2.bias", c)):
        t[k] = _vec(p[k], m, k)
    packed = p.get("conv.packed")
    if packed is not None and (packed.numel() * packed.element_size() != lib().tsp_conv_weight_packed_bytes(c, c)):
        raise ValueError("conv.packed must be conv.weight packed by conv_weight_pack")
    mpacked = p.get("mlp.packed")
    if mpacked is not None and mpacked.numel() * mpacked.element_size() != lib().tsp_convnext_mlp_packed_bytes(c):
        raise ValueError("mlp.packed must be mlp.0 and mlp.2 packed by convnext_mlp_pack")
    if plan is not None and (plan.dtype != torch.uint8 or plan.numel() < lib().tsp_conv_plan_bytes(n)):
        raise ValueError("plan must be a uint8 buffer of tsp_conv_plan_bytes(N)")
    _require_cuda(x, nbr, plan, packed, mpacked, *t.values())
    w = ConvNextWeights(_ptr(t["conv.weight"]), dtype_code(t["conv.weight"].dtype), _ptr(t["conv.bias"]),
                        _ptr(packed), _ptr(t["norm.weight"]), _ptr(t["norm.bias"]), _ptr(t["mlp.0.weight"]),
                        dtype_code(t["mlp.0.weight"].dtype), _ptr(t["mlp.0.bias"]), _ptr(t["mlp.2.weight"]),
                        dtype_code(t["mlp.2.weight"].dtype), _ptr(t["mlp.2.bias"]), _ptr(mpacked))
    flags = BLOCK_CAST_F32 if cast_f32 else 0
    xc = x.contiguous()
    if x16 is not None:
        x16 = x16.contiguous()
        if tuple(x16.shape) != (n, c) or x16.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("x16 must be a 16-bit [N, C] tensor")
        _require_cuda(x16)
    out = torch.empty((n, c), dtype=torch.float32, device=x.device)
    out16 = None if out16_dtype is None else torch.empty((n, c), dtype=out16_dtype, device=x.device)
    nb = lib().tsp_convnext_workspace_bytes(n, c, dtype_code(xc.dtype), ctypes.byref(w), int(plan is not None), flags)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=x.device)
    _check("tsp_convnext_ex", lib().tsp_convnext_ex(
        _ptr(xc), dtype_code(xc.dtype), _ptr(x16), n, c, _ptr(nbr), _ptr(plan), ctypes.byref(w), _ptr(out),
        _ptr(out16), dtype_code(out16_dtype) if out16 is not None else 2, _ptr(ws), nb, flags, _stream(stream)))
    return out if out16 is None else (out, out16)


def c2s(x, nbr, mask, mstart, gidx, m: int, cout: int, child_nbr, p: dict, plan=None, child_plan=None,
        cast_f32: bool = False, stream=None, out16_dtype=None, conv2_tiles=None):
    """The C2S block's features through tsp_c2s_ex, after its subdivision (mask uint8 [8N], mstart
    and gidx from subdivide, child_nbr the children's table): x f32 [N, Cin], p by reference
    names without the prefix ("norm1.weight", "norm1.bias", "conv1.weight" [8 Cout,27,Cin],
    "conv1.bias", "conv2.weight" [Cout,27,Cout], "conv2.bias"; optional "conv1.packed",
    "conv2.packed"). -> f32 [M, Cout], or (out, out rounded to out16_dtype) when out16_dtype is
    given. conv2_tiles, a list of (t0, nt) child-plan tile ranges: through tsp_c2s_part instead,
    the front part once, then conv2 over each range in turn."""
    torch = _torch()
    n, cin = x.shape
    if x.dtype != torch.float32:
        raise ValueError("x must be float32")
    _check_nbr(nbr, n, x.device)
    _check_nbr(child_nbr, m, x.device)
    if mask.dtype != torch.uint8 or mask.numel() != 8 * n:
        raise ValueError("mask must be uint8 with 8*N entries")
    if mstart.dtype != torch.int32 or mstart.numel() != n + 1 or gidx.dtype != torch.int32 or gidx.numel() < m:
        raise ValueError("mstart must be int32 [N+1] and gidx int32 [>= M]")
    t = {"conv1.weight": _mat(p["conv1.weight"], (8 * cout, 27, cin), "conv1.weight"),
         "conv2.weight": _mat(p["conv2.weight"], (cout, 27, cout), "conv2.weight")}
    for k, k_n in (("norm1.weight", cin), ("norm1.bias", cin), ("conv1.bias", 8 * cout), ("conv2.bias", cout)):
        t[k] = _vec(p[k], k_n, k)
    p1, p2 = p.get("conv1.packed"), p.get("conv2.packed")
    for pk, (ci_, co_), name in ((p1, (cin, 8 * cout), "conv1.packed"), (p2, (cout, cout), "conv2.packed")):
        if pk is not None and pk.numel() * pk.element_size() != lib().tsp_conv_weight_packed_bytes(ci_, co_):
            raise ValueError(f"{name} must hold the weight packed by conv_weight_pack")
    for pl, rows, name in ((plan, n, "plan"), (child_plan, m, "child_plan")):
        if pl is not None and (pl.dtype != torch.uint8 or pl.numel() < lib().tsp_conv_plan_bytes(rows)):
            raise ValueError(f"{name} must be a uint8 buffer of tsp_conv_plan_bytes")
    _require_cuda(x, nbr, mask, mstart, gidx, child_nbr, plan, child_plan, p1, p2, *t.values())
    w = C2SWeights(_ptr(t["norm1.weight"]), _ptr(t["norm1.bias"]), _ptr(t["conv1.weight"]),
                   dtype_code(t["conv1.weight"].dtype), _ptr(t["conv1.bias"]), _ptr(p1), _ptr(t["conv2.weight"]),
                   dtype_code(t["conv2.weight"].dtype), _ptr(t["conv2.bias"]), _ptr(p2))
    flags = BLOCK_CAST_F32 if cast_f32 else 0
    xc = x.contiguous()
    out = torch.empty((m, cout), dtype=torch.float32, device=x.device)
    out16 = None if out16_dtype is None else torch.empty((m, cout), dtype=out16_dtype, device=x.device)
    nb = lib().tsp_c2s_workspace_bytes(n, m, cin, cout, ctypes.byref(w), int(plan is not None),
                                       int(child_plan is not None), flags)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=x.device)
    mk = mask.reshape(-1).contiguous()
    args = (_ptr(xc), n, cin, _ptr(nbr), _ptr(plan), _ptr(mk), _ptr(mstart), _ptr(gidx), m, cout, _ptr(child_nbr),
            _ptr(child_plan), ctypes.byref(w), _ptr(out), _ptr(out16), dtype_code(out16_dtype) if out16 is not None
            else 2, _ptr(ws), nb, flags)
    if conv2_tiles is None:
        _check("tsp_c2s_ex", lib().tsp_c2s_ex(*args, _stream(stream)))
    else:
        _check("tsp_c2s_part", lib().tsp_c2s_part(*args, 1, 0, -1, _stream(stream)))
        for t0, nt in conv2_tiles:
            _check("tsp_c2s_part", lib().tsp_c2s_part(*args, 2, t0, nt, _stream(stream)))
    return out if out16 is None else (out, out16)
