"""The ``hip`` backend: natten-mlx's backend-module interface on PyTorch-ROCm
tensors, executed by libnatten_amd.so.

It exposes the eighteen entry points every reference backend module has
(``src/natten_mlx/_core/ops.py:49-135``: ``na{1,2,3}d_forward``,
``na{1,2,3}d_backward``, ``na{1,2,3}d_{qk,av}_{forward,backward}``) with the
same argument order and meaning (normalised tuples; ``scale`` may be None),
plus the hooks the autograd layer calls directly (reference
``autograd/na2d.py:34-53`` calls ``fast_metal.na2d_fused_simd_backward``
with the forward output; ``autograd/na1d.py:76-80`` calls the varlen
forward).  Tensors must live on a HIP device; there is no CPU path.
"""

from __future__ import annotations

import contextlib
import os
from typing import Optional, Sequence

import torch

from . import _lib

# NATTEN_AMD_GENERIC=1 (or the generic_kernels() context) runs the fused op on
# the generic vector-ALU kernels even where the matrix-core kernels apply.
_force_generic = os.environ.get("NATTEN_AMD_GENERIC", "0") == "1"
_no_lean = False


@contextlib.contextmanager
def generic_kernels(enabled: bool = True):
    """Temporarily route the fused op to the generic kernels."""
    global _force_generic
    prev = _force_generic
    _force_generic = enabled
    try:
        yield
    finally:
        _force_generic = prev


@contextlib.contextmanager
def no_lean_kernels(enabled: bool = True):
    """Temporarily route the fused op to the 32-query matrix-core kernels
    where the lean workgroup kernels would run (A/B comparison)."""
    global _no_lean
    prev = _no_lean
    _no_lean = enabled
    try:
        yield
    finally:
        _no_lean = prev


def is_available() -> bool:
    return torch.cuda.is_available() and _lib.available()


def _require_device(*tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "natten_amd's hip backend runs on MI355X (HIP) tensors only; got a tensor on "
                f"{t.device}. There is no CPU implementation.")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors are on different devices: {dev} and {t.device}")
    return dev


def _c(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.contiguous()


def _scale(scale, head_dim: int) -> float:
    return head_dim ** -0.5 if scale is None else float(scale)


# Built parameter blocks (and their backward workspace sizes) by problem:
# a training loop calls with the same few shapes every step, and building the
# ctypes struct costs more than the launch itself.  Entries are never
# mutated; the cache is cleared when it grows past _PARAMS_MAX.
_params_cache: dict = {}
_PARAMS_MAX = 256


def _params_entry(q: torch.Tensor, k: torch.Tensor, kernel_size, stride, dilation, is_causal,
                  scale, n_extra: int = 0, dense: bool = False,
                  sample_extent: Optional[torch.Tensor] = None, varlen_clamped: bool = False):
    flags = ((_lib.NA_FLAG_DENSE if dense else 0) | (_lib.NA_FLAG_GENERIC if _force_generic else 0)
             | (_lib.NA_FLAG_NO_LEAN if _no_lean else 0)
             | (_lib.NA_FLAG_VARLEN_CLAMPED if varlen_clamped and sample_extent is not None
                else 0))
    se_ptr = None if sample_extent is None else sample_extent.data_ptr()
    key = (tuple(q.shape), k.shape[-2], q.dtype, tuple(kernel_size), tuple(stride),
           tuple(dilation), tuple(is_causal), scale, n_extra, flags, se_ptr)
    hit = _params_cache.get(key)
    if hit is not None:
        return hit
    rank = q.dim() - 3
    p = _lib.make_params(
        rank, q.shape[0], q.shape[-2], k.shape[-2], q.shape[-1], _lib.dtype_code(q.dtype),
        tuple(q.shape[1:-2]), tuple(kernel_size), tuple(dilation), tuple(stride),
        tuple(int(bool(c)) for c in is_causal), _scale(scale, q.shape[-1]), n_extra, flags,
        sample_extent)
    entry = [p, None]  # [params, backward workspace bytes (filled on first use)]
    if len(_params_cache) >= _PARAMS_MAX:
        _params_cache.clear()
    _params_cache[key] = entry
    return entry


def _params(q: torch.Tensor, k: torch.Tensor, kernel_size, stride, dilation, is_causal, scale,
            n_extra: int = 0, dense: bool = False,
            sample_extent: Optional[torch.Tensor] = None,
            varlen_clamped: bool = False) -> _lib.NaParams:
    return _params_entry(q, k, kernel_size, stride, dilation, is_causal, scale, n_extra, dense,
                         sample_extent, varlen_clamped)[0]


def _out_spatial(spatial: Sequence[int], stride: Sequence[int]) -> tuple[int, ...]:
    return tuple((s + st - 1) // st for s, st in zip(spatial, stride))


# ---------------------------------------------------------------------------
# fused op (with LSE, additional tokens, varlen and the dense FMHA mode)

def fused_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale,
                  extra_k=None, extra_v=None, sample_extent=None, dense=False,
                  want_lse=True, varlen_clamped=False):
    """Returns ``(out, lse)``; lse is float32 ``[B, *O, H]`` (or None).
    ``varlen_clamped``: the caller has checked that every sample extent is at
    least dilation * kernel_size on each non-causal axis."""
    _require_device(q, k, v, extra_k, extra_v, sample_extent)
    q, k, v, extra_k, extra_v = map(_c, (q, k, v, extra_k, extra_v))
    lib = _lib.load()
    n_extra = 0 if extra_k is None else extra_k.shape[1]
    p = _params(q, k, kernel_size, stride, dilation, is_causal, scale, n_extra, dense,
                sample_extent, varlen_clamped)
    osp = _out_spatial(q.shape[1:-2], stride)
    B, H, D = q.shape[0], q.shape[-2], q.shape[-1]
    out = torch.empty((B, *osp, H, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, *osp, H), dtype=torch.float32, device=q.device) if want_lse else None
    _lib.check(lib.na_fwd(p, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(extra_k),
                          _lib.ptr(extra_v), _lib.ptr(out), _lib.ptr(lse), _lib.stream_of(q)),
               "na_fwd")
    return out, lse


KERNEL_PATHS = {0: "generic", 1: "mfma", 2: "lean", 3: "dense"}


def kernel_path(q, k, kernel_size, stride, dilation, is_causal, scale=None, n_extra=0,
                dense=False, sample_extent=None, backward=False, varlen_clamped=False,
                split=False):
    """Name of the kernel family na_fwd (or na_bwd; or with ``split`` the
    split ops qk/av forward and backward) runs for this problem: "generic",
    "mfma" or "lean" (a diagnostic; launches nothing)."""
    lib = _lib.load()
    p = _params(q, k, kernel_size, stride, dilation, is_causal, scale, n_extra, dense,
                sample_extent, varlen_clamped)
    r = int(lib.na_kernel_path(p, 2 if split else 1 if backward else 0))
    if r < 0:
        _lib.check(-r, "na_kernel_path")
    return KERNEL_PATHS[r]


def kernel_plan(q, k, kernel_size, stride, dilation, is_causal, scale=None, n_extra=0,
                dense=False, sample_extent=None, backward=False, varlen_clamped=False):
    """How na_fwd (or na_bwd) launches for this problem (a diagnostic;
    launches nothing): a dict with the kernel family and, on the lean
    kernels, the wave tile, waves per workgroup, staged box, axis-0 slabs,
    grouped query heads (and how many per workgroup), workgroups, LDS bytes;
    with additional tokens in
    the backward, which unit reduces their gradients."""
    lib = _lib.load()
    p = _params(q, k, kernel_size, stride, dilation, is_causal, scale, n_extra, dense,
                sample_extent, varlen_clamped)
    plan = _lib.NaPlan()
    _lib.check(lib.na_kernel_plan(p, 1 if backward else 0, plan), "na_kernel_plan")
    return {"path": KERNEL_PATHS[plan.path], "tile": tuple(plan.tile), "waves": plan.waves,
            "box": tuple(plan.box), "slabs": plan.slabs,
            "grouped_heads": bool(plan.grouped_heads),
            "heads_per_workgroup": max(int(plan.grouped_heads), 1), "workgroups": plan.workgroups,
            "lds_bytes": plan.lds_bytes,
            "extra_reduction": {0: None, 1: "valu", 2: "matrix"}[plan.extra_reduction]}


def fused_backward(q, k, v, out, lse, grad_out, grad_lse, kernel_size, stride, dilation,
                   is_causal, scale, extra_k=None, extra_v=None, sample_extent=None,
                   dense=False, varlen_clamped=False):
    """Returns ``(dq, dk, dv, d_extra_k, d_extra_v)``; ``varlen_clamped`` as
    in ``fused_forward``."""
    _require_device(q, k, v, out, lse, grad_out, grad_lse, extra_k, extra_v)
    q, k, v, out, lse, grad_out, grad_lse, extra_k, extra_v = map(
        _c, (q, k, v, out, lse, grad_out, grad_lse, extra_k, extra_v))
    if grad_out.dtype != q.dtype:
        grad_out = grad_out.to(q.dtype)
    if grad_lse is not None and grad_lse.dtype != torch.float32:
        grad_lse = grad_lse.float()
    lib = _lib.load()
    n_extra = 0 if extra_k is None else extra_k.shape[1]
    entry = _params_entry(q, k, kernel_size, stride, dilation, is_causal, scale, n_extra, dense,
                          sample_extent, varlen_clamped)
    p = entry[0]
    if entry[1] is None:
        entry[1] = int(lib.na_bwd_workspace_bytes(p))
    ws_bytes = entry[1]
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dek = torch.empty_like(extra_k) if n_extra else None
    dev = torch.empty_like(extra_v) if n_extra else None
    # the lean backward without additional tokens needs no workspace
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    _lib.check(lib.na_bwd(p, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(extra_k),
                          _lib.ptr(extra_v), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(grad_out),
                          _lib.ptr(grad_lse), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
                          _lib.ptr(dek), _lib.ptr(dev), _lib.ptr(ws), ws_bytes,
                          _lib.stream_of(q)), "na_bwd")
    return dq, dk, dv, dek, dev


# ---------------------------------------------------------------------------
# split ops

def qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale):
    _require_device(q, k)
    q, k = _c(q), _c(k)
    if k.dtype != q.dtype:
        k = k.to(q.dtype)
    lib = _lib.load()
    p = _params(q, k, kernel_size, stride, dilation, is_causal, scale)
    osp = _out_spatial(q.shape[1:-2], stride)
    kprod = 1
    for x in kernel_size:
        kprod *= int(x)
    logits = torch.empty((q.shape[0], *osp, q.shape[-2], kprod), dtype=q.dtype, device=q.device)
    _lib.check(lib.na_qk_fwd(p, _lib.ptr(q), _lib.ptr(k), _lib.ptr(logits), _lib.stream_of(q)),
               "na_qk_fwd")
    return logits


def _av_params(attn, v, kernel_size, stride, dilation, is_causal):
    rank = v.dim() - 3
    return _lib.make_params(
        rank, v.shape[0], attn.shape[-2], v.shape[-2], v.shape[-1], _lib.dtype_code(v.dtype),
        tuple(v.shape[1:-2]), tuple(kernel_size), tuple(dilation), tuple(stride),
        tuple(int(bool(c)) for c in is_causal), 1.0)


def _check_attn_shape(attn, v, kernel_size, stride):
    osp = _out_spatial(v.shape[1:-2], stride)
    kprod = 1
    for x in kernel_size:
        kprod *= int(x)
    if tuple(attn.shape[1:-2]) != osp or attn.shape[-1] != kprod or attn.shape[0] != v.shape[0]:
        raise ValueError(
            f"attn shape {tuple(attn.shape)} must be [B, *ceil(input/stride), heads, {kprod}] "
            f"for value shape {tuple(v.shape)}")


def av_forward(attn, v, kernel_size, stride, dilation, is_causal):
    _require_device(attn, v)
    _check_attn_shape(attn, v, kernel_size, stride)
    dt = torch.promote_types(attn.dtype, v.dtype)
    attn, v = _c(attn.to(dt)), _c(v.to(dt))
    lib = _lib.load()
    p = _av_params(attn, v, kernel_size, stride, dilation, is_causal)
    out = torch.empty((*attn.shape[:-1], v.shape[-1]), dtype=dt, device=v.device)
    _lib.check(lib.na_av_fwd(p, _lib.ptr(attn), _lib.ptr(v), _lib.ptr(out), _lib.stream_of(v)),
               "na_av_fwd")
    return out


def qk_backward(q, k, grad_attn, kernel_size, stride, dilation, is_causal, scale):
    _require_device(q, k, grad_attn)
    q, k = _c(q), _c(k)
    kd = k.dtype
    if k.dtype != q.dtype:
        k = k.to(q.dtype)
    g = _c(grad_attn.to(q.dtype))
    lib = _lib.load()
    p = _params(q, k, kernel_size, stride, dilation, is_causal, scale)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    _lib.check(lib.na_qk_bwd(p, _lib.ptr(q), _lib.ptr(k), _lib.ptr(g), _lib.ptr(dq),
                             _lib.ptr(dk), _lib.stream_of(q)), "na_qk_bwd")
    return dq, dk.to(kd)


def av_backward(attn, v, grad_out, kernel_size, stride, dilation, is_causal):
    _require_device(attn, v, grad_out)
    dt = torch.promote_types(attn.dtype, v.dtype)
    ad, vd = attn.dtype, v.dtype
    attn, v = _c(attn.to(dt)), _c(v.to(dt))
    g = _c(grad_out.to(dt))
    lib = _lib.load()
    p = _av_params(attn, v, kernel_size, stride, dilation, is_causal)
    dattn = torch.empty_like(attn)
    dv = torch.empty_like(v)
    _lib.check(lib.na_av_bwd(p, _lib.ptr(attn), _lib.ptr(v), _lib.ptr(g), _lib.ptr(dattn),
                             _lib.ptr(dv), _lib.stream_of(v)), "na_av_bwd")
    return dattn.to(ad), dv.to(vd)


# ---------------------------------------------------------------------------
# the reference backend-module interface (ops.py:49-135)

def na1d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    return fused_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale,
                         want_lse=False)[0]


na2d_forward = na1d_forward
na3d_forward = na1d_forward


def na1d_backward(q, k, v, grad_out, kernel_size, stride, dilation, is_causal, scale):
    out, lse = fused_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)
    dq, dk, dv, _, _ = fused_backward(q, k, v, out, lse, grad_out, None, kernel_size, stride,
                                      dilation, is_causal, scale)
    return dq, dk, dv


na2d_backward = na1d_backward
na3d_backward = na1d_backward


def na1d_qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale):
    return qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale)


na2d_qk_forward = na1d_qk_forward
na3d_qk_forward = na1d_qk_forward


def na1d_av_forward(attn, v, kernel_size, stride, dilation, is_causal):
    return av_forward(attn, v, kernel_size, stride, dilation, is_causal)


na2d_av_forward = na1d_av_forward
na3d_av_forward = na1d_av_forward


def na1d_qk_backward(q, k, grad_attn, kernel_size, stride, dilation, is_causal, scale):
    return qk_backward(q, k, grad_attn, kernel_size, stride, dilation, is_causal, scale)


na2d_qk_backward = na1d_qk_backward
na3d_qk_backward = na1d_qk_backward


def na1d_av_backward(attn, v, grad_out, kernel_size, stride, dilation, is_causal):
    return av_backward(attn, v, grad_out, kernel_size, stride, dilation, is_causal)


na2d_av_backward = na1d_av_backward
na3d_av_backward = na1d_av_backward


def na1d_fused_backward(q, k, v, grad_out, fwd_out, kernel_size, stride, dilation, is_causal,
                        scale, lse=None, grad_lse=None):
    """Backward from a saved forward, with the positional signature of the
    reference's ``fast_metal.na{n}d_fused_simd_backward(q, k, v, grad_out,
    fwd_out, kernel_size, stride, dilation, is_causal, scale)``
    (``fast_metal.py:2390-2521``), which the VJPs call with the forward output
    only (``autograd/na2d.py:39-46``).  ``lse`` (float32 ``[B, *O, H]``) is
    the forward's log-sum-exp when the caller kept it; when None it is
    recomputed by one forward launch."""
    if lse is None:
        _, lse = fused_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)
    dq, dk, dv, _, _ = fused_backward(q, k, v, fwd_out, lse, grad_out, grad_lse, kernel_size,
                                      stride, dilation, is_causal, scale)
    return dq, dk, dv


na2d_fused_backward = na1d_fused_backward
na3d_fused_backward = na1d_fused_backward


def varlen_forward(q, k, v, sample_extent, kernel_size, dilation, scale):
    """Varlen fused forward (reference ``fast_metal.na1d_varlen_forward``)."""
    rank = q.dim() - 3
    return fused_forward(q, k, v, kernel_size, (1,) * rank, dilation, (False,) * rank, scale,
                         sample_extent=sample_extent)


# ---------------------------------------------------------------------------
# DiNAT all-in-one operators (rank 1 and 2, square window, one dilation)

def _rpb_geometry(x: torch.Tensor, heads_first: bool):
    """(rank, batch, heads, extent, last) of a [B, *L, H, X] (or heads-first
    [B, H, *L, X]) tensor."""
    rank = x.dim() - 3
    if rank not in (1, 2):
        raise ValueError(f"allin1 ops take rank-1 or rank-2 tensors, got {x.dim()}D")
    if heads_first:
        return rank, x.shape[0], x.shape[1], tuple(x.shape[2:-1]), x.shape[-1]
    return rank, x.shape[0], x.shape[-2], tuple(x.shape[1:-2]), x.shape[-1]


def _per_axis(v, rank):
    """An int (every axis) or a per-axis tuple, as a rank-long int tuple."""
    if isinstance(v, (tuple, list)):
        if len(v) != rank:
            raise ValueError(f"expected {rank} per-axis values, got {tuple(v)}")
        return tuple(int(x) for x in v)
    return (int(v),) * rank


def _rpb_params(x, kernel_size, dilation, heads_first, scale=None):
    rank, B, H, ext, D = _rpb_geometry(x, heads_first)
    return _lib.make_rpb_params(rank, B, H, D, ext, _per_axis(kernel_size, rank),
                                _per_axis(dilation, rank), heads_first,
                                _lib.dtype_code(x.dtype), scale)


def _slots_shape(x, kernel_size, heads_first):
    rank = x.dim() - 3
    n = 1
    for k in _per_axis(kernel_size, rank):
        n *= k
    return tuple(x.shape[:-1]) + (n,)


def _check_same_layout(a, b, what):
    if tuple(a.shape) != tuple(b.shape):
        raise ValueError(f"{what} must have identical shapes, got {tuple(a.shape)} and "
                         f"{tuple(b.shape)}")


def _bias_shape(rank, heads, kernel_size):
    return (heads,) + tuple(2 * k - 1 for k in _per_axis(kernel_size, rank))


def rpb_qk_forward(q, k, rpb, kernel_size, dilation, scale=None, heads_first=False):
    """float32 logits ``[.., K^rank]``: <round(q*scale), key_nbr> + bias, -inf
    outside the window (C ABI ``na_rpb_qk_fwd``)."""
    _require_device(q, k, rpb)
    q, k = _c(q), _c(k)
    if k.dtype != q.dtype:
        k = k.to(q.dtype)
    _check_same_layout(q, k, "query and key")
    p = _rpb_params(q, kernel_size, dilation, heads_first, scale)
    rp = None
    if rpb is not None:
        rp = _c(rpb.to(torch.float32))
        want = _bias_shape(p.rank, p.heads, kernel_size)
        if tuple(rp.shape) != want:
            raise ValueError(f"rpb must have shape {list(want)}, got {tuple(rp.shape)}")
    out = torch.empty(_slots_shape(q, kernel_size, heads_first), dtype=torch.float32,
                      device=q.device)
    lib = _lib.load()
    _lib.check(lib.na_rpb_qk_fwd(p, _lib.ptr(q), _lib.ptr(k), _lib.ptr(rp), _lib.ptr(out),
                                 _lib.stream_of(q)), "na_rpb_qk_fwd")
    return out


def rpb_av_forward(attn, v, kernel_size, dilation, heads_first=False, out_dtype=torch.float32):
    """out = sum attn * value_nbr in ``out_dtype`` (float32 or v.dtype)
    (C ABI ``na_rpb_av_fwd``)."""
    _require_device(attn, v)
    v = _c(v)
    a = _c(attn.to(torch.float32))
    want = _slots_shape(v, kernel_size, heads_first)
    if tuple(a.shape) != want:
        raise ValueError(f"attn must have shape {want}, got {tuple(a.shape)}")
    if out_dtype not in (torch.float32, v.dtype):
        raise ValueError("out_dtype must be float32 or the value dtype")
    p = _rpb_params(v, kernel_size, dilation, heads_first)
    out = torch.empty(v.shape, dtype=out_dtype, device=v.device)
    lib = _lib.load()
    _lib.check(lib.na_rpb_av_fwd(p, _lib.ptr(a), _lib.ptr(v), _lib.ptr(out),
                                 _lib.dtype_code(out_dtype), _lib.stream_of(v)), "na_rpb_av_fwd")
    return out


def rpb_qk_backward(q, k, d_logits, kernel_size, dilation, scale=None, heads_first=False,
                    need_q=True, need_k=True, need_rpb=True):
    """(dq, dk, drpb) of ``rpb_qk_forward``; drpb is float32 (C ABI
    ``na_rpb_qk_bwd``).  Unrequested gradients come back as None."""
    _require_device(q, k, d_logits)
    q, k = _c(q), _c(k)
    if k.dtype != q.dtype:
        k = k.to(q.dtype)
    dl = _c(d_logits.to(torch.float32))
    if tuple(dl.shape) != _slots_shape(q, kernel_size, heads_first):
        raise ValueError(f"d_logits must have shape {_slots_shape(q, kernel_size, heads_first)}")
    p = _rpb_params(q, kernel_size, dilation, heads_first, scale)
    dq = torch.empty_like(q) if need_q else None
    dk = torch.empty_like(k) if need_k else None
    drpb = ws = None
    lib = _lib.load()
    nbytes = 0
    if need_rpb:
        drpb = torch.empty(_bias_shape(p.rank, p.heads, kernel_size), dtype=torch.float32,
                           device=q.device)
        nbytes = lib.na_rpb_bwd_workspace_bytes(p)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    _lib.check(lib.na_rpb_qk_bwd(p, _lib.ptr(q), _lib.ptr(k), _lib.ptr(dl), _lib.ptr(dq),
                                 _lib.ptr(dk), _lib.ptr(drpb), _lib.ptr(ws), nbytes,
                                 _lib.stream_of(q)), "na_rpb_qk_bwd")
    return dq, dk, drpb


def rpb_av_backward(attn, v, d_out, kernel_size, dilation, heads_first=False, need_attn=True,
                    need_v=True):
    """(dattn float32, dv) of ``rpb_av_forward``; ``d_out`` has the forward's
    output dtype (C ABI ``na_rpb_av_bwd``)."""
    _require_device(attn, v, d_out)
    v = _c(v)
    a = _c(attn.to(torch.float32))
    do = _c(d_out if d_out.dtype in (torch.float32, v.dtype) else d_out.to(torch.float32))
    _check_same_layout(v, do, "value and d_out")
    p = _rpb_params(v, kernel_size, dilation, heads_first)
    da = torch.empty(a.shape, dtype=torch.float32, device=v.device) if need_attn else None
    dv = torch.empty_like(v) if need_v else None
    lib = _lib.load()
    _lib.check(lib.na_rpb_av_bwd(p, _lib.ptr(a), _lib.ptr(v), _lib.ptr(do),
                                 _lib.dtype_code(do.dtype), _lib.ptr(da), _lib.ptr(dv),
                                 _lib.stream_of(v)), "na_rpb_av_bwd")
    return da, dv


# ---------------------------------------------------------------------------
# merge of attention outputs (C ABI na_merge_fwd / na_merge_bwd)

def _merge_params(outs, lses):
    n = len(outs)
    if not 2 <= n <= _lib.MERGE_MAX_PARTS:
        raise ValueError(f"a merge call takes 2..{_lib.MERGE_MAX_PARTS} parts, got {n}")
    o0 = outs[0]
    for o, l in zip(outs, lses):
        if o.dtype != o0.dtype or tuple(o.shape) != tuple(o0.shape):
            raise ValueError("merge parts must share shape and dtype")
        if l.dtype != torch.float32 or tuple(l.shape) != tuple(o0.shape[:-1]):
            raise ValueError("merge LSEs must be float32 with the outputs' leading shape")
    p = _lib.NaMergeParams()
    p.n_parts = n
    p.head_dim = int(o0.shape[-1])
    p.rows = int(o0.numel() // max(int(o0.shape[-1]), 1))
    p.dtype = _lib.dtype_code(o0.dtype)
    return p


def merge_forward(outs, lses):
    """(out, lse float32) of the concatenated-keys merge, one kernel pass."""
    _require_device(*outs, *lses)
    outs = [_c(o) for o in outs]
    lses = [_c(l) for l in lses]
    p = _merge_params(outs, lses)
    out = torch.empty_like(outs[0])
    lse = torch.empty(outs[0].shape[:-1], dtype=torch.float32, device=outs[0].device)
    lib = _lib.load()
    _lib.check(lib.na_merge_fwd(p, _lib.ptr_array(outs), _lib.ptr_array(lses), _lib.ptr(out),
                                _lib.ptr(lse), _lib.stream_of(out)), "na_merge_fwd")
    return out, lse


def merge_backward(outs, lses, d_out, d_lse, need_outs, need_lses):
    """Per-part gradients of ``merge_forward``: d_outs in the parts' dtype,
    d_lses float32; entries not needed come back as None."""
    _require_device(*outs, *lses, d_out, d_lse)
    outs = [_c(o) for o in outs]
    lses = [_c(l) for l in lses]
    p = _merge_params(outs, lses)
    do = _c(d_out.to(outs[0].dtype))
    dl = None if d_lse is None else _c(d_lse.to(torch.float32))
    d_outs = [torch.empty_like(o) if need else None for o, need in zip(outs, need_outs)]
    d_lses = [torch.empty_like(l) if need else None for l, need in zip(lses, need_lses)]
    lib = _lib.load()
    _lib.check(lib.na_merge_bwd(p, _lib.ptr_array(outs), _lib.ptr_array(lses), _lib.ptr(do),
                                _lib.ptr(dl), _lib.ptr_array(d_outs), _lib.ptr_array(d_lses),
                                _lib.stream_of(do)), "na_merge_bwd")
    return d_outs, d_lses
