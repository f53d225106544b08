"""Autograd for the fused op (reference ``autograd/na{1,2,3}d.py``).

One op covers every rank, GQA, additional tokens, varlen and the dense
(FMHA) mode.  Its forward returns ``(out, lse)``; the backward takes
gradients for both (the LSE gradient enters as ``delta - dlse``), so a loss
that uses the returned LSE differentiates correctly
(reference ``tests/test_new_features.py:1177-1192``).

With the built-in ``hip`` backend the op is ``torch.ops.natten_amd.na_fused``
(``csrc/na_torch.cpp``): its autograd node runs in C++ over the C ABI, so
neither direction passes through Python or ctypes per call.  ``_FusedNA``
below is the same op as a Python ``autograd.Function`` over the backend
module's hooks; it runs for other registered backends, where the operator
library is not built, and under ``python_autograd()`` /
``NATTEN_AMD_PY_AUTOGRAD=1`` (A/B checks: both launch the same kernels).
"""

from __future__ import annotations

import contextlib
import os
from typing import NamedTuple, Optional

import torch

from .._core import _lib, ops
from .._core import hip as _hip

_py_autograd = os.environ.get("NATTEN_AMD_PY_AUTOGRAD", "0") == "1"


@contextlib.contextmanager
def python_autograd(enabled: bool = True):
    """Temporarily run the fused op through the Python autograd Function."""
    global _py_autograd
    prev = _py_autograd
    _py_autograd = enabled
    try:
        yield
    finally:
        _py_autograd = prev


class FusedSpec(NamedTuple):
    kernel_size: tuple
    stride: tuple
    dilation: tuple
    is_causal: tuple
    scale: Optional[float]
    dense: bool = False
    # every per-sample extent satisfies dilation * kernel_size <= extent on
    # each non-causal axis (checked by the caller on the host)
    varlen_clamped: bool = False


class _FusedNA(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, extra_k, extra_v, sample_extent, spec: FusedSpec):
        be = ops.backend_module()
        out, lse = be.fused_forward(q, k, v, spec.kernel_size, spec.stride, spec.dilation,
                                    spec.is_causal, spec.scale, extra_k, extra_v,
                                    sample_extent, spec.dense,
                                    varlen_clamped=spec.varlen_clamped)
        ctx.save_for_backward(q, k, v, extra_k, extra_v, out, lse, sample_extent)
        ctx.spec = spec
        ctx.set_materialize_grads(False)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        q, k, v, extra_k, extra_v, out, lse, sample_extent = ctx.saved_tensors
        spec = ctx.spec
        if grad_out is None:
            grad_out = torch.zeros_like(out)
        be = ops.backend_module()
        dq, dk, dv, dek, dev = be.fused_backward(
            q, k, v, out, lse, grad_out, grad_lse, spec.kernel_size, spec.stride, spec.dilation,
            spec.is_causal, spec.scale, extra_k, extra_v, sample_extent, spec.dense,
            varlen_clamped=spec.varlen_clamped)
        return dq, dk, dv, dek, dev, None, None


def _op_flags(spec: FusedSpec, sample_extent) -> int:
    return ((_lib.NA_FLAG_DENSE if spec.dense else 0)
            | (_lib.NA_FLAG_GENERIC if _hip._force_generic else 0)
            | (_lib.NA_FLAG_NO_LEAN if _hip._no_lean else 0)
            | (_lib.NA_FLAG_VARLEN_CLAMPED if spec.varlen_clamped and sample_extent is not None
               else 0))


def na_fused_with_grad(q, k, v, spec: FusedSpec, extra_k=None, extra_v=None,
                       sample_extent=None):
    """Differentiable fused op; returns ``(out, lse_float32)``."""
    if not _py_autograd and q.is_cuda:
        op = _lib.fused_op()
        if op is not None and ops.backend_module() is _hip:
            scale = q.shape[-1] ** -0.5 if spec.scale is None else float(spec.scale)
            return op(q, k, v, extra_k, extra_v, sample_extent, spec.kernel_size, spec.stride,
                      spec.dilation, [int(c) for c in spec.is_causal], scale,
                      _op_flags(spec, sample_extent), _lib.stream_of(q))
    return _FusedNA.apply(q, k, v, extra_k, extra_v, sample_extent, spec)


def _plain(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    spec = FusedSpec(tuple(kernel_size), tuple(stride), tuple(dilation),
                     tuple(bool(c) for c in is_causal), scale)
    return na_fused_with_grad(q, k, v, spec)[0]


def na1d_with_grad(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    """Autograd-capable 1D NA (reference ``autograd/na1d.py:56-63``)."""
    return _plain(q, k, v, kernel_size, stride, dilation, is_causal, scale)


def na2d_with_grad(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    """Autograd-capable 2D NA (reference ``autograd/na2d.py:59-64``)."""
    return _plain(q, k, v, kernel_size, stride, dilation, is_causal, scale)


def na3d_with_grad(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    """Autograd-capable 3D NA (reference ``autograd/na3d.py``)."""
    return _plain(q, k, v, kernel_size, stride, dilation, is_causal, scale)


# Device copies of host-side per-sample extents, by content: a training
# loop passes the same few length vectors again and again, and a cached copy
# needs no host-to-device transfer (which would wait for the stream), so the
# call stays asynchronous and can be captured in a HIP graph.  Entries are
# never evicted (a captured graph may hold their addresses); past
# _EXTENTS_MAX distinct vectors, further ones are copied per call.
_extents_cache: dict = {}
_EXTENTS_MAX = 1024


def device_extents(sizes: torch.Tensor, batch: int, rank: int, device) -> torch.Tensor:
    """Per-sample extents as a contiguous int32 ``[batch, rank]`` tensor on
    ``device``; host tensors go through the content-keyed cache."""
    if sizes.device.type != "cpu":
        return sizes.to(device=device, dtype=torch.int32).reshape(batch, rank).contiguous()
    key = (str(device), batch, rank, tuple(int(x) for x in sizes.reshape(-1).tolist()))
    hit = _extents_cache.get(key)
    if hit is not None:
        return hit
    t = sizes.to(torch.int32).reshape(batch, rank).contiguous().to(device)
    if len(_extents_cache) < _EXTENTS_MAX:
        _extents_cache[key] = t
    return t


def _varlen(q, k, v, sizes, kernel_size, dilation, scale):
    rank = q.dim() - 3
    host = sizes.detach().to("cpu", torch.int64).reshape(q.shape[0], rank)
    clamped = bool((host >= torch.tensor([d * kk for d, kk in zip(dilation, kernel_size)])).all())
    se = device_extents(sizes, q.shape[0], rank, q.device)
    spec = FusedSpec(tuple(kernel_size), (1,) * rank, tuple(dilation), (False,) * rank, scale,
                     varlen_clamped=clamped)
    return na_fused_with_grad(q, k, v, spec, sample_extent=se)[0]


def na1d_varlen_with_grad(q, k, v, seq_lens, kernel_size, dilation, scale):
    """Reference ``autograd/na1d.py:73-103``; the backward is the same
    fused HIP backward (the reference runs pure per-sample autodiff)."""
    return _varlen(q, k, v, seq_lens, kernel_size, dilation, scale)


def na2d_varlen_with_grad(q, k, v, spatial_sizes, kernel_size, dilation, scale):
    return _varlen(q, k, v, spatial_sizes, kernel_size, dilation, scale)


def na3d_varlen_with_grad(q, k, v, spatial_sizes, kernel_size, dilation, scale):
    return _varlen(q, k, v, spatial_sizes, kernel_size, dilation, scale)
