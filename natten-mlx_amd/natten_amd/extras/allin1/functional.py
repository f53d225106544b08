"""Heads-first DiNAT functions (mirrors ``extras/allin1/functional.py`` and
``extras/allin1/functional_metal.py``).

Layout ``[B, H, L, D]`` (1D) / ``[B, H, Hh, Hw, D]`` (2D), as the original
DiNAT ``natten{1,2}dqkrpb`` / ``natten{1,2}dav`` functions take it.  The
kernels read this layout directly (no transposes).  As in the reference's
torch path, results come back in the dtype of the tensor the reference
converts against (the query for QK, the attention weights for AV, the
input itself for each gradient), computed in float32.  ``kernel_size *
dilation`` must not exceed an axis (``functional.py:49-54``).
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from ..._core import hip
from ...autograd.allin1 import av_rpb_with_grad, qk_rpb_with_grad


def _check_args_against_dim(length: int, kernel_size: int, dilation: int, axis_name: str) -> None:
    if kernel_size * dilation > length:
        raise ValueError(
            f"Invalid NATTEN args on {axis_name}: kernel_size * dilation must be <= axis length. "
            f"Got kernel_size={kernel_size}, dilation={dilation}, {axis_name}={length}.")


def _square(kernel_size, dilation) -> Tuple[int, int]:
    """Square kernel and uniform dilation (``functional_metal.py:2074-2082``)."""
    if isinstance(kernel_size, (tuple, list)):
        if kernel_size[0] != kernel_size[1]:
            raise ValueError("Only square kernels supported")
        kernel_size = kernel_size[0]
    if isinstance(dilation, (tuple, list)):
        if dilation[0] != dilation[1]:
            raise ValueError("Only uniform dilation supported")
        dilation = dilation[0]
    return int(kernel_size), int(dilation)


def _as(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == like.dtype else t.to(like.dtype)


def natten1dqkrpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor],
                  kernel_size: int, dilation: int) -> torch.Tensor:
    """1D QK + RPB, scores before softmax: ``[B, H, L, K]``
    (``functional.py:372-388``, ``functional_metal.py:2037-2049``)."""
    _check_args_against_dim(int(query.shape[2]), int(kernel_size), int(dilation), "length")
    out = qk_rpb_with_grad(query, key, rpb, int(kernel_size), int(dilation), None,
                           heads_first=True)
    return _as(out, query)


def natten1dav(attention_probs: torch.Tensor, value: torch.Tensor, kernel_size: int,
               dilation: int) -> torch.Tensor:
    """1D AV: ``[B, H, L, D]`` (``functional.py:391-406``)."""
    _check_args_against_dim(int(value.shape[2]), int(kernel_size), int(dilation), "length")
    out = av_rpb_with_grad(attention_probs, value, int(kernel_size), int(dilation),
                           heads_first=True)
    return _as(out, attention_probs)


def natten2dqkrpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor],
                  kernel_size: Union[int, Tuple[int, int]],
                  dilation: Union[int, Tuple[int, int]]) -> torch.Tensor:
    """2D QK + RPB: ``[B, H, Hh, Hw, K*K]`` (``functional.py:409-434``)."""
    K, d = _square(kernel_size, dilation)
    _check_args_against_dim(int(query.shape[2]), K, d, "height")
    _check_args_against_dim(int(query.shape[3]), K, d, "width")
    return _as(qk_rpb_with_grad(query, key, rpb, K, d, None, heads_first=True), query)


def natten2dav(attention_probs: torch.Tensor, value: torch.Tensor,
               kernel_size: Union[int, Tuple[int, int]],
               dilation: Union[int, Tuple[int, int]]) -> torch.Tensor:
    """2D AV: ``[B, H, Hh, Hw, D]`` (``functional.py:437-462``)."""
    K, d = _square(kernel_size, dilation)
    _check_args_against_dim(int(value.shape[2]), K, d, "height")
    _check_args_against_dim(int(value.shape[3]), K, d, "width")
    return _as(av_rpb_with_grad(attention_probs, value, K, d, heads_first=True),
               attention_probs)


def natten2d_qkv_fused(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                       rpb: Optional[torch.Tensor], kernel_size: Union[int, Tuple[int, int]],
                       dilation: Union[int, Tuple[int, int]]) -> torch.Tensor:
    """QK + RPB -> softmax -> AV in one call (``functional_metal.py:2130-2169``;
    its unfused composition).  Output in the query dtype."""
    K, d = _square(kernel_size, dilation)
    _check_args_against_dim(int(query.shape[2]), K, d, "height")
    _check_args_against_dim(int(query.shape[3]), K, d, "width")
    attn = torch.softmax(qk_rpb_with_grad(query, key, rpb, K, d, None, heads_first=True), -1)
    return _as(av_rpb_with_grad(attn, value, K, d, heads_first=True), query)


def _qk_backward(d_attn, query, key, rpb, kernel_size, dilation):
    dq, dk, drpb = hip.rpb_qk_backward(query, key, d_attn, kernel_size, dilation, None,
                                       heads_first=True, need_rpb=rpb is not None)
    return _as(dq, query), _as(dk, query), (None if drpb is None else _as(drpb, rpb))


def _av_backward(d_out, attention_probs, value, kernel_size, dilation):
    da, dv = hip.rpb_av_backward(attention_probs, value, d_out, kernel_size, dilation,
                                 heads_first=True)
    return _as(da, attention_probs), _as(dv, value)


def natten1dqkrpb_backward(d_attn, query, key, rpb, kernel_size: int, dilation: int):
    """(d_query, d_key, d_rpb) of ``natten1dqkrpb`` (``functional_metal.py:2172-2192``)."""
    return _qk_backward(d_attn, query, key, rpb, int(kernel_size), int(dilation))


def natten1dav_backward(d_out, attention_probs, value, kernel_size: int, dilation: int):
    """(d_attn, d_value) of ``natten1dav`` (``functional_metal.py:2195-2213``)."""
    return _av_backward(d_out, attention_probs, value, int(kernel_size), int(dilation))


def natten2dqkrpb_backward(d_attn, query, key, rpb, kernel_size, dilation):
    """(d_query, d_key, d_rpb) of ``natten2dqkrpb`` (``functional_metal.py:2216-2244``)."""
    K, d = _square(kernel_size, dilation)
    return _qk_backward(d_attn, query, key, rpb, K, d)


def natten2dav_backward(d_out, attention_probs, value, kernel_size, dilation):
    """(d_attn, d_value) of ``natten2dav`` (``functional_metal.py:2247-2274``)."""
    K, d = _square(kernel_size, dilation)
    return _av_backward(d_out, attention_probs, value, K, d)


__all__ = [
    "natten1dqkrpb", "natten1dav", "natten2dqkrpb", "natten2dav",
    "natten1dqkrpb_backward", "natten1dav_backward",
    "natten2dqkrpb_backward", "natten2dav_backward",
    "natten2d_qkv_fused",
]
