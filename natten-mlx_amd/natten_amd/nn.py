"""Neighborhood-attention layers as ``torch.nn.Module`` s (mirrors
``src/natten_mlx/nn/na{1,2,3}d.py``).

A layer projects channels-last input ``[B, *spatial, C]`` to per-head
queries, keys and values, runs the neighborhood attention of its rank and
projects back to ``C`` channels.  Parameter names (``qkv``; or ``q_proj`` +
``kv_proj`` when ``num_kv_heads`` differs from ``num_heads``; ``proj``) and
their layouts match the reference, so a state dict converted from an MLX
checkpoint loads unchanged.

Routing follows the reference layer (``nn/na2d.py:80-154``):

* per-sample extents given (``seq_lens`` / ``spatial_sizes``) -> the varlen op
  (kernel size, dilation and scale only, as there);
* ``attn_drop > 0`` -> split path ``na*_qk`` -> softmax -> dropout -> ``na*_av``,
  so dropout acts on the attention probabilities;
* otherwise the fused op.

Key/value heads for GQA are not repeated: the kernels map query head ``h``
to key/value head ``h // (num_heads // num_kv_heads)`` directly.
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch
from torch import nn as _nn

from . import functional as F
from .utils.params import normalize_tuple_param

IntOrTuple = Union[int, Tuple[int, ...]]
BoolOrTuple = Union[bool, Tuple[bool, ...]]

_FUSED = {1: F.na1d, 2: F.na2d, 3: F.na3d}
_QK = {1: F.na1d_qk, 2: F.na2d_qk, 3: F.na3d_qk}
_AV = {1: F.na1d_av, 2: F.na2d_av, 3: F.na3d_av}
_VARLEN = {1: F.na1d_varlen, 2: F.na2d_varlen, 3: F.na3d_varlen}
_INPUT = {1: "[B, L, C]", 2: "[B, H, W, C]", 3: "[B, D, H, W, C]"}


class _NeighborhoodAttention(_nn.Module):
    """Rank-generic body of the three layers (``rank`` is set by each
    subclass).  Construction-time checks and messages follow
    ``nn/na2d.py:29-78``."""

    rank: int = 0

    def __init__(
        self,
        embed_dim: int,
        num_heads: int,
        kernel_size: IntOrTuple,
        stride: IntOrTuple = 1,
        dilation: IntOrTuple = 1,
        is_causal: BoolOrTuple = False,
        num_kv_heads: Optional[int] = None,
        qkv_bias: bool = True,
        qk_scale: Optional[float] = None,
        attn_drop: float = 0.0,
        proj_drop: float = 0.0,
    ):
        super().__init__()
        if embed_dim <= 0:
            raise ValueError(f"embed_dim must be positive, got {embed_dim}")
        if num_heads <= 0:
            raise ValueError(f"num_heads must be positive, got {num_heads}")
        if embed_dim % num_heads != 0:
            raise ValueError("embed_dim must be divisible by num_heads")
        self.embed_dim = int(embed_dim)
        self.num_heads = int(num_heads)
        self.head_dim = self.embed_dim // self.num_heads
        self.num_kv_heads = self.num_heads if num_kv_heads is None else int(num_kv_heads)
        if self.num_kv_heads <= 0 or self.num_heads % self.num_kv_heads != 0:
            raise ValueError(
                f"num_heads ({self.num_heads}) must be divisible by "
                f"num_kv_heads ({self.num_kv_heads})")

        r = self.rank
        self.kernel_size = normalize_tuple_param(kernel_size, r, "kernel_size")
        self.stride = normalize_tuple_param(stride, r, "stride")
        self.dilation = normalize_tuple_param(dilation, r, "dilation")
        self.is_causal = normalize_tuple_param(is_causal, r, "is_causal")
        self.scale = self.head_dim ** -0.5 if qk_scale is None else float(qk_scale)

        self._use_gqa = self.num_kv_heads != self.num_heads
        kv_width = self.num_kv_heads * self.head_dim
        if self._use_gqa:
            self.q_proj = _nn.Linear(self.embed_dim, self.embed_dim, bias=qkv_bias)
            self.kv_proj = _nn.Linear(self.embed_dim, 2 * kv_width, bias=qkv_bias)
        else:
            self.qkv = _nn.Linear(self.embed_dim, 3 * self.embed_dim, bias=qkv_bias)
        self.attn_drop_rate = float(attn_drop)
        self.attn_drop = _nn.Dropout(self.attn_drop_rate) if self.attn_drop_rate > 0.0 else None
        self.proj = _nn.Linear(self.embed_dim, self.embed_dim)
        self.proj_drop_rate = float(proj_drop)
        self.proj_drop = _nn.Dropout(self.proj_drop_rate) if self.proj_drop_rate > 0.0 else None

    def extra_repr(self) -> str:
        return (f"embed_dim={self.embed_dim}, num_heads={self.num_heads}, "
                f"num_kv_heads={self.num_kv_heads}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}, dilation={self.dilation}, is_causal={self.is_causal}")

    def _project(self, x: torch.Tensor):
        """``[B, *S, C]`` -> q ``[B, *S, H, D]``, k/v ``[B, *S, H_kv, D]`` (views
        into the projection output; the ops make them contiguous)."""
        lead = x.shape[:-1]
        if self._use_gqa:
            q = self.q_proj(x).reshape(*lead, self.num_heads, self.head_dim)
            kv = self.kv_proj(x).reshape(*lead, 2, self.num_kv_heads, self.head_dim)
            k, v = kv.unbind(dim=-3)
        else:
            qkv = self.qkv(x).reshape(*lead, 3, self.num_heads, self.head_dim)
            q, k, v = qkv.unbind(dim=-3)
        return q, k, v

    def _attend(self, x: torch.Tensor, sizes: Optional[torch.Tensor]) -> torch.Tensor:
        r = self.rank
        if x.ndim != r + 2:
            raise ValueError(f"Expected input shape {_INPUT[r]}, got {tuple(x.shape)}")
        if x.shape[-1] != self.embed_dim:
            raise ValueError(
                f"Input channel dim ({x.shape[-1]}) must match embed_dim ({self.embed_dim})")
        q, k, v = self._project(x)
        if sizes is not None:
            out = _VARLEN[r](q, k, v, sizes, kernel_size=self.kernel_size,
                             dilation=self.dilation, scale=self.scale)
        elif self.attn_drop_rate > 0.0:
            logits = _QK[r](q, k, kernel_size=self.kernel_size, dilation=self.dilation,
                            stride=self.stride, is_causal=self.is_causal, scale=self.scale)
            attn = torch.softmax(logits, dim=-1)
            if self.attn_drop is not None:
                attn = self.attn_drop(attn)
            out = _AV[r](attn, v, kernel_size=self.kernel_size, dilation=self.dilation,
                         stride=self.stride, is_causal=self.is_causal)
        else:
            out = _FUSED[r](q, k, v, kernel_size=self.kernel_size, stride=self.stride,
                            dilation=self.dilation, is_causal=self.is_causal, scale=self.scale)
        out = self.proj(out.reshape(*out.shape[:-2], self.embed_dim))
        if self.proj_drop is not None:
            out = self.proj_drop(out)
        return out


class NeighborhoodAttention1D(_NeighborhoodAttention):
    """1D layer (``nn/na1d.py``).  Input ``[B, L, C]`` -> ``[B, ceil(L/stride), C]``."""

    rank = 1

    def forward(self, x: torch.Tensor, seq_lens: Optional[torch.Tensor] = None) -> torch.Tensor:
        return self._attend(x, seq_lens)


class NeighborhoodAttention2D(_NeighborhoodAttention):
    """2D layer (``nn/na2d.py``).  Input ``[B, H, W, C]`` ->
    ``[B, ceil(H/s_h), ceil(W/s_w), C]``; ``spatial_sizes`` ``[B, 2]`` selects
    the varlen op."""

    rank = 2

    def forward(self, x: torch.Tensor,
                spatial_sizes: Optional[torch.Tensor] = None) -> torch.Tensor:
        return self._attend(x, spatial_sizes)


class NeighborhoodAttention3D(_NeighborhoodAttention):
    """3D layer (``nn/na3d.py``).  Input ``[B, D, H, W, C]``; ``spatial_sizes``
    ``[B, 3]`` selects the varlen op."""

    rank = 3

    def forward(self, x: torch.Tensor,
                spatial_sizes: Optional[torch.Tensor] = None) -> torch.Tensor:
        return self._attend(x, spatial_sizes)


__all__ = ["NeighborhoodAttention1D", "NeighborhoodAttention2D", "NeighborhoodAttention3D"]
