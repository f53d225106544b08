"""ctypes binding of libnatten_amd.so (the C ABI in include/natten_amd.h).

The library is built in-tree by ``natten-mlx_amd/build_lib.py``.  It must be
loaded after ``import torch`` so that it shares torch's HIP runtime (both
link ``libamdhip64.so.7``) and therefore torch's streams and allocations.
Nothing here falls back to another implementation: a missing library or a
failing call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libnatten_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), LIB_NAME)
# The fused op as a torch custom operator (csrc/na_torch.cpp): its autograd
# node runs in C++ over this library
OP_LIB_PATH = os.path.join(os.path.dirname(LIB_PATH), "libnatten_amd_torch.so")

NA_F32, NA_F16, NA_BF16 = 0, 1, 2
NA_FLAG_DENSE = 1
NA_FLAG_GENERIC = 2
NA_FLAG_NO_LEAN = 4
NA_FLAG_VARLEN_CLAMPED = 8
ABI_VERSION = 2

_STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported", 3: "launch failure",
           4: "workspace"}

_I32x3 = ctypes.c_int32 * 3


class NaParams(ctypes.Structure):
    """Mirror of ``na_params`` (include/natten_amd.h)."""

    _fields_ = [
        ("rank", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("extent", _I32x3),
        ("kernel", _I32x3),
        ("dilation", _I32x3),
        ("stride", _I32x3),
        ("causal", _I32x3),
        ("scale", ctypes.c_float),
        ("n_extra", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("sample_extent", ctypes.c_void_p),
    ]


class NaRpbParams(ctypes.Structure):
    """Mirror of ``na_rpb_params`` (include/natten_amd.h)."""

    _fields_ = [
        ("rank", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("extent", ctypes.c_int32 * 2),
        ("kernel", ctypes.c_int32 * 2),
        ("dilation", ctypes.c_int32 * 2),
        ("heads_first", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("has_scale", ctypes.c_int32),
    ]


class NaPlan(ctypes.Structure):
    """Mirror of ``na_plan`` (include/natten_amd.h)."""

    _fields_ = [
        ("path", ctypes.c_int32),
        ("tile", _I32x3),
        ("waves", ctypes.c_int32),
        ("box", _I32x3),
        ("slabs", ctypes.c_int32),
        ("grouped_heads", ctypes.c_int32),
        ("workgroups", ctypes.c_int32),
        ("lds_bytes", ctypes.c_int32),
        ("extra_reduction", ctypes.c_int32),
    ]


class NaRpbPlan(ctypes.Structure):
    """Mirror of ``na_rpb_plan`` (include/natten_amd.h)."""

    _fields_ = [
        ("qk", ctypes.c_int32),
        ("av", ctypes.c_int32),
        ("dq", ctypes.c_int32),
        ("dk", ctypes.c_int32),
        ("dattn", ctypes.c_int32),
        ("dv", ctypes.c_int32),
        ("fused_bias", ctypes.c_int32),
        ("block", ctypes.c_int32),
    ]


RPB_GENERIC, RPB_STAGED, RPB_PHASE = 0, 1, 2


class NaMergeParams(ctypes.Structure):
    """Mirror of ``na_merge_params`` (include/natten_amd.h)."""

    _fields_ = [
        ("n_parts", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rows", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
    ]


MERGE_MAX_PARTS = 8

_P = ctypes.POINTER(NaParams)
_R = ctypes.POINTER(NaRpbParams)
_M = ctypes.POINTER(NaMergeParams)
_PP = ctypes.POINTER(ctypes.c_void_p)  # host array of device pointers
_V = ctypes.c_void_p
_I = ctypes.c_int32

# name -> (restype, argtypes)
SIGNATURES = {
    "na_abi_version": (ctypes.c_int, []),
    "na_last_error": (ctypes.c_char_p, []),
    "na_window_start": (_I, [_I, _I, _I, _I, _I]),
    "na_window_end": (_I, [_I, _I, _I, _I]),
    "na_pb_start": (_I, [_I, _I, _I, _I, _I]),
    "na_window_start_partition": (_I, [_I, _I, _I, _I, _I]),
    "na_neighbor_table": (ctypes.c_int, [_P, _V, _V, _V]),
    "na_mfma_selftest": (ctypes.c_int, [_I, _V, _V]),
    "na_kernel_path": (ctypes.c_int, [_P, _I]),
    "na_kernel_plan": (ctypes.c_int, [_P, _I, ctypes.POINTER(NaPlan)]),
    "na_fwd": (ctypes.c_int, [_P, _V, _V, _V, _V, _V, _V, _V, _V]),
    "na_bwd_workspace_bytes": (ctypes.c_size_t, [_P]),
    "na_bwd": (ctypes.c_int, [_P] + [_V] * 15 + [ctypes.c_size_t, _V]),
    "na_bwd_noalloc_max_workspace": (ctypes.c_size_t, []),
    "na_bwd_noalloc": (ctypes.c_int, [_P] + [_V] * 15),
    "na_qk_fwd": (ctypes.c_int, [_P, _V, _V, _V, _V]),
    "na_av_fwd": (ctypes.c_int, [_P, _V, _V, _V, _V]),
    "na_qk_bwd": (ctypes.c_int, [_P, _V, _V, _V, _V, _V, _V]),
    "na_av_bwd": (ctypes.c_int, [_P, _V, _V, _V, _V, _V, _V]),
    "na_rpb_qk_fwd": (ctypes.c_int, [_R, _V, _V, _V, _V, _V]),
    "na_rpb_av_fwd": (ctypes.c_int, [_R, _V, _V, _V, _I, _V]),
    "na_rpb_bwd_workspace_bytes": (ctypes.c_size_t, [_R]),
    "na_rpb_qk_bwd": (ctypes.c_int, [_R, _V, _V, _V, _V, _V, _V, _V, ctypes.c_size_t, _V]),
    "na_rpb_av_bwd": (ctypes.c_int, [_R, _V, _V, _V, _I, _V, _V, _V]),
    "na_rpb_kernel_plan": (ctypes.c_int, [_R, ctypes.POINTER(NaRpbPlan)]),
    "na_merge_fwd": (ctypes.c_int, [_M, _PP, _PP, _V, _V, _V]),
    "na_merge_bwd": (ctypes.c_int, [_M, _PP, _PP, _V, _V, _PP, _PP, _V]),
}

_lib = None
_lock = threading.Lock()
_load_error: str | None = None
_fused_op = None


def load():
    """Load (once) and return the library; raise if it is unavailable."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            _load_error = (f"{LIB_NAME} is not built (expected at {LIB_PATH}); "
                           "run `python natten-mlx_amd/build_lib.py`")
            raise RuntimeError(_load_error)
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.na_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI {lib.na_abi_version()} != {ABI_VERSION}")
        _load_fused_op()
        _lib = lib
        return lib


def _load_fused_op() -> None:
    """Register natten_amd::na_fused from libnatten_amd_torch.so (built
    beside the library; it links this library, which the loader then shares
    with the ctypes handle)."""
    global _fused_op
    if not os.path.exists(OP_LIB_PATH):
        return
    torch.ops.load_library(OP_LIB_PATH)
    _fused_op = torch.ops.natten_amd.na_fused


def fused_op():
    """torch.ops.natten_amd.na_fused, or None where the operator library is
    not built (the fused op then runs through the Python autograd Function
    over the same kernels)."""
    if _lib is None:
        load()
    return _fused_op


def available() -> bool:
    try:
        load()
    except Exception:
        return False
    return True


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().na_last_error().decode(errors="replace")
        raise RuntimeError(f"natten_amd {what} failed ({_STATUS.get(rc, rc)}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return NA_F32
    if dt == torch.float16:
        return NA_F16
    if dt == torch.bfloat16:
        return NA_BF16
    raise TypeError(f"natten_amd supports float32/float16/bfloat16 tensors, got {dt}")


def ptr(t: torch.Tensor | None):
    """Device address of a tensor as a Python int (None for NULL); the
    c_void_p argtypes take ints directly."""
    return None if t is None else t.data_ptr()


def ptr_array(tensors):
    """Host array of device pointers (NULL for None entries)."""
    arr = (ctypes.c_void_p * len(tensors))()
    for i, t in enumerate(tensors):
        arr[i] = None if t is None else t.data_ptr()
    return arr


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor):
    """torch's current HIP stream on the tensor's device (the handle the
    library launches on), as an int."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def make_params(rank: int, batch: int, heads: int, kv_heads: int, head_dim: int, dtype: int,
                extent, kernel, dilation, stride, causal, scale: float, n_extra: int = 0,
                flags: int = 0, sample_extent: torch.Tensor | None = None) -> NaParams:
    p = NaParams()
    p.rank, p.batch, p.heads, p.kv_heads, p.head_dim, p.dtype = (
        rank, batch, heads, kv_heads, head_dim, dtype)
    for arr, vals in ((p.extent, extent), (p.kernel, kernel), (p.dilation, dilation),
                      (p.stride, stride), (p.causal, causal)):
        for i in range(3):
            arr[i] = int(vals[i]) if i < len(vals) else 1
    p.scale = float(scale)
    p.n_extra = int(n_extra)
    p.flags = int(flags)
    p.sample_extent = None if sample_extent is None else sample_extent.data_ptr()
    return p


def make_rpb_params(rank: int, batch: int, heads: int, head_dim: int, extent, kernel,
                    dilation, heads_first: bool, dtype: int,
                    scale: float | None) -> NaRpbParams:
    """``kernel`` / ``dilation``: an int (every axis) or one value per axis."""
    p = NaRpbParams()
    p.rank, p.batch, p.heads, p.head_dim = rank, batch, heads, head_dim
    p.extent[0] = int(extent[0])
    p.extent[1] = int(extent[1]) if rank == 2 else 1
    ks = (kernel,) * rank if isinstance(kernel, int) else tuple(kernel)
    ds = (dilation,) * rank if isinstance(dilation, int) else tuple(dilation)
    for a in range(2):
        p.kernel[a] = int(ks[a]) if a < rank else 1
        p.dilation[a] = int(ds[a]) if a < rank else 1
    p.heads_first = 1 if heads_first else 0
    p.dtype = dtype
    p.scale = 1.0 if scale is None else float(scale)
    p.has_scale = 0 if scale is None else 1
    return p
