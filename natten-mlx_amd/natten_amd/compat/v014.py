"""NATTEN v0.14 API (mirrors ``compat/v014.py``).

* ``NeighborhoodAttention{1,2}D(dim, kernel_size, dilation, num_heads, ...)``:
  the v0.14 layers (no stride, no causal masking), parameters ``qkv`` and
  ``proj`` as in ``compat/v014.py:52-189``.
* ``natten{1,2}dqkrpb`` / ``natten{1,2}dav``: heads-first ``[B, H, *L, D]``
  QK with relative position bias and AV (``compat/v014.py:192-313``).  The
  QK logits are the plain dot products (no query scale: the reference
  divides its default-scaled logits by that scale again) plus
  ``rpb[h, clip(pb_start + k, 0, 2K-2)]`` per axis, pair index
  ``r_h * (2*K_w - 1) + r_w`` in 2D.  Windows are the NATTEN ones (the
  dilation-partition rule, identical to the core windows while
  ``kernel_size * dilation <= length``, which is checked).  Both run on the
  library's all-in-one kernels (``na_rpb_qk_fwd`` / ``na_rpb_av_fwd``) in
  the heads-first layout directly, with non-square kernels and per-axis
  dilation, and are differentiable (q, k, rpb; attn, value).

Result dtypes follow MLX's promotion in the reference: logits in the
promotion of the query and bias dtypes, AV output in that of attn and
value; arithmetic is float32.
"""

from __future__ import annotations

from typing import Optional

import torch

from ..autograd.allin1 import av_rpb_with_grad, qk_rpb_with_grad
from ..nn import _NeighborhoodAttention
from ..utils.params import (
    check_dilation_kernel_vs_input,
    check_kernel_size_vs_input,
    normalize_tuple_param,
)


class _V014Layer(_NeighborhoodAttention):
    """v0.14 constructor and input check over the modern layer body (no
    stride, non-causal; ``qk_scale`` falls back to ``head_dim**-0.5`` when
    falsy, as ``qk_scale or ...`` does in the reference)."""

    def __init__(self, dim, kernel_size, dilation=1, num_heads=1, qkv_bias=True,
                 qk_scale=None, attn_drop=0.0, proj_drop=0.0):
        if num_heads <= 0 or dim % num_heads != 0:
            raise ValueError("dim must be divisible by num_heads")
        super().__init__(embed_dim=dim, num_heads=num_heads, kernel_size=kernel_size,
                         stride=1, dilation=dilation, is_causal=False, qkv_bias=qkv_bias,
                         qk_scale=qk_scale or None, attn_drop=attn_drop,
                         proj_drop=proj_drop)
        self.dim = int(dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.ndim != self.rank + 2:
            raise ValueError(f"Expected a rank-{self.rank + 2} input, got {tuple(x.shape)}")
        if x.shape[-1] != self.dim:
            raise ValueError(f"Expected dim={self.dim}, got channels={x.shape[-1]}")
        return self._attend(x, None)


class NeighborhoodAttention1D(_V014Layer):
    """v0.14 1D layer: ``[B, L, dim]`` -> ``[B, L, dim]`` (``compat/v014.py:52-117``)."""

    rank = 1


class NeighborhoodAttention2D(_V014Layer):
    """v0.14 2D layer: ``[B, H, W, dim]`` -> same (``compat/v014.py:120-189``)."""

    rank = 2


def _qkrpb(rank, query, key, rpb, kernel_size, dilation):
    nd = rank + 3
    if query.ndim != nd or key.ndim != nd:
        shape = "[B, H, L, D]" if rank == 1 else "[B, H, Hh, Hw, D]"
        raise ValueError(f"query and key must be {shape}")
    ks = normalize_tuple_param(kernel_size, rank, "kernel_size")
    dil = normalize_tuple_param(dilation, rank, "dilation")
    spatial = tuple(int(n) for n in query.shape[2:-1])
    check_kernel_size_vs_input(ks, spatial)
    check_dilation_kernel_vs_input(dil, ks, spatial)
    want = tuple(2 * k - 1 for k in ks)
    if rpb.ndim != rank + 1 or tuple(rpb.shape[1:]) != want:
        if rank == 1:
            raise ValueError(f"rpb must be [heads, {want[0]}] for kernel_size={ks[0]}, "
                             f"got {tuple(rpb.shape)}")
        raise ValueError("rpb must be [heads, 2*Kh-1, 2*Kw-1] for the provided kernel_size; "
                         f"got {tuple(rpb.shape)}")
    logits = qk_rpb_with_grad(query, key, rpb, ks, dil, None, heads_first=True)
    return logits.to(torch.promote_types(query.dtype, rpb.dtype))


def _av(rank, attn, value, kernel_size, dilation):
    ks = normalize_tuple_param(kernel_size, rank, "kernel_size")
    dil = normalize_tuple_param(dilation, rank, "dilation")
    spatial = tuple(int(n) for n in value.shape[2:-1])
    check_kernel_size_vs_input(ks, spatial)
    check_dilation_kernel_vs_input(dil, ks, spatial)
    want = torch.promote_types(attn.dtype, value.dtype)
    out_dtype = want if want in (torch.float32, value.dtype) else torch.float32
    out = av_rpb_with_grad(attn, value, ks, dil, heads_first=True, out_dtype=out_dtype)
    return out if out.dtype == want else out.to(want)


def natten1dqkrpb(query, key, rpb, kernel_size, dilation):
    """query/key ``[B, H, L, D]``, rpb ``[H, 2K-1]`` -> logits ``[B, H, L, K]``
    (``compat/v014.py:192-227``)."""
    return _qkrpb(1, query, key, rpb, kernel_size, dilation)


def natten1dav(attn, value, kernel_size, dilation):
    """attn ``[B, H, L, K]``, value ``[B, H, L, D]`` -> ``[B, H, L, D]``
    (``compat/v014.py:230-248``)."""
    return _av(1, attn, value, kernel_size, dilation)


def natten2dqkrpb(query, key, rpb, kernel_size, dilation):
    """query/key ``[B, H, Hh, Hw, D]``, rpb ``[H, 2Kh-1, 2Kw-1]`` -> logits
    ``[B, H, Hh, Hw, Kh*Kw]`` (``compat/v014.py:251-290``)."""
    return _qkrpb(2, query, key, rpb, kernel_size, dilation)


def natten2dav(attn, value, kernel_size, dilation):
    """attn ``[B, H, Hh, Hw, Kh*Kw]``, value ``[B, H, Hh, Hw, D]``
    (``compat/v014.py:293-313``)."""
    return _av(2, attn, value, kernel_size, dilation)


def add_natten_handle(flop_counter):
    """fvcore flop-counter hook; returned unchanged (``compat/v014.py:316-318``)."""
    return flop_counter


__all__ = [
    "NeighborhoodAttention1D",
    "NeighborhoodAttention2D",
    "natten1dqkrpb",
    "natten1dav",
    "natten2dqkrpb",
    "natten2dav",
    "add_natten_handle",
]
