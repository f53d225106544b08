"""DiNAT all-in-one operators (mirrors ``extras/allin1/__init__.py``).

``na{1,2}d_qk_rpb`` fuse the QK product with the relative-position-bias
add; ``na{1,2}d_av_fused`` apply softmaxed weights.  Square window of side
``kernel_size`` with one dilation, dilation-partition window (reference
``extras/allin1/reference_impl.py:13-45``), float32 results as the
reference's Metal kernels return.  Layout: spatial-first ``[B, *L, H, D]``.
Unlike the reference's forward-only functions these are differentiable
(q, k, rpb; attn, v) through the library's backward kernels.

Example::

    logits = na1d_qk_rpb(q, k, rpb, kernel_size=5, dilation=2, scale=0.288)
    attn = torch.softmax(logits, dim=-1)
    out = na1d_av_fused(attn, v, kernel_size=5, dilation=2)
"""

from __future__ import annotations

from typing import Optional

import torch

from ...autograd.allin1 import av_rpb_with_grad, qk_rpb_with_grad


def _square(value, name):
    if isinstance(value, (tuple, list)):
        if len(set(int(v) for v in value)) != 1:
            raise ValueError(f"Only square {name} is supported")
        value = value[0]
    return int(value)


def na1d_qk_rpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor],
                kernel_size: int, dilation: int = 1, *,
                scale: Optional[float] = None) -> torch.Tensor:
    """Fused 1D QK + RPB (reference ``__init__.py:40-79``): ``[B, L, H, K]``
    float32 logits before softmax.  The query is scaled in its own dtype
    before the dot; ``rpb`` ``[H, 2K-1]`` or None (zero bias)."""
    if query.ndim != 4:
        raise ValueError(f"query must be 4D [B, L, H, D], got shape {tuple(query.shape)}")
    return qk_rpb_with_grad(query, key, rpb, int(kernel_size), int(dilation), scale)


def na1d_av_fused(attn: torch.Tensor, value: torch.Tensor, kernel_size: int,
                  dilation: int = 1) -> torch.Tensor:
    """Fused 1D AV (reference ``__init__.py:82-109``): ``[B, L, H, D]`` float32."""
    if attn.ndim != 4 or value.ndim != 4:
        raise ValueError("attn and value must be 4D for na1d_av_fused")
    return av_rpb_with_grad(attn, value, int(kernel_size), int(dilation))


def na2d_qk_rpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor],
                kernel_size: int, dilation: int = 1, *,
                scale: Optional[float] = None) -> torch.Tensor:
    """Fused 2D QK + RPB (reference ``__init__.py:112-150``): query
    ``[B, Hh, Hw, H, D]`` -> ``[B, Hh, Hw, H, K*K]`` float32; ``rpb``
    ``[H, 2K-1, 2K-1]`` or None."""
    if query.ndim != 5:
        raise ValueError(f"query must be 5D [B, Hh, Hw, H, D], got shape {tuple(query.shape)}")
    return qk_rpb_with_grad(query, key, rpb, _square(kernel_size, "kernel_size"),
                            _square(dilation, "dilation"), scale)


def na2d_av_fused(attn: torch.Tensor, value: torch.Tensor, kernel_size: int,
                  dilation: int = 1) -> torch.Tensor:
    """Fused 2D AV (reference ``__init__.py:153-180``): ``[B, Hh, Hw, H, D]``
    float32."""
    if attn.ndim != 5 or value.ndim != 5:
        raise ValueError("attn and value must be 5D for na2d_av_fused")
    return av_rpb_with_grad(attn, value, _square(kernel_size, "kernel_size"),
                            _square(dilation, "dilation"))


__all__ = ["na1d_qk_rpb", "na1d_av_fused", "na2d_qk_rpb", "na2d_av_fused"]
