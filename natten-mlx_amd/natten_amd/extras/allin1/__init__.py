"""DiNAT all-in-one 1D operators (mirrors ``extras/allin1/__init__.py:40-109``).

``na1d_qk_rpb`` fuses the QK product with the relative-position-bias add and
``na1d_av_fused`` applies softmaxed weights; both use the dilation-partition
window (``extras/allin1/reference_impl.py:13-45``) and return float32, as the
reference's Metal kernels do.  Layout: spatial-first ``[B, L, H, D]``.

Example::

    logits = na1d_qk_rpb(q, k, rpb, kernel_size=5, dilation=2, scale=0.288)
    attn = torch.softmax(logits, dim=-1)
    out = na1d_av_fused(attn, v, kernel_size=5, dilation=2)
"""

from __future__ import annotations

from typing import Optional

import torch

from ..._core import hip


def na1d_qk_rpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor],
                kernel_size: int, dilation: int = 1, *,
                scale: Optional[float] = None) -> torch.Tensor:
    """Fused 1D QK + RPB: ``[B, L, H, K]`` float32 logits (before softmax).
    The query is scaled in its own dtype before the dot product; ``rpb``
    ``[H, 2K-1]`` or None (zeros)."""
    if query.ndim != 4:
        raise ValueError(f"query must be 4D [B, L, H, D], got shape {tuple(query.shape)}")
    return hip.qk_rpb_1d(query, key, rpb, int(kernel_size), int(dilation), scale)


def na1d_av_fused(attn: torch.Tensor, value: torch.Tensor, kernel_size: int,
                  dilation: int = 1) -> torch.Tensor:
    """Fused 1D AV: ``[B, L, H, D]`` float32."""
    if attn.ndim != 4 or value.ndim != 4:
        raise ValueError("attn and value must be 4D for na1d_av_fused")
    return hip.av_rpb_1d(attn, value, int(kernel_size), int(dilation))


__all__ = ["na1d_qk_rpb", "na1d_av_fused"]
