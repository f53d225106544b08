"""NATTEN v0.15 API (mirrors ``compat/v015.py``): everything of v0.14 plus
the fused ``na{1,2,3}d(query, key, value, kernel_size, dilation, is_causal,
scale)`` without stride, the split ops, a v0.15-style 3D layer and the
feature probes."""

from __future__ import annotations

import torch

from .. import functional as _F
from ..functional import na1d_av, na1d_qk, na2d_av, na2d_qk
from ..nn import NeighborhoodAttention3D as _Modern3D
from .v014 import *  # noqa: F401,F403
from .v014 import __all__ as _v014_all


def na1d(query, key, value, kernel_size, dilation=1, is_causal=False, scale=None):
    """Fused 1D neighborhood attention, stride 1 (``compat/v015.py:14-24``)."""
    return _F.na1d(query, key, value, kernel_size=kernel_size, stride=1, dilation=dilation,
                   is_causal=is_causal, scale=scale)


def na2d(query, key, value, kernel_size, dilation=1, is_causal=False, scale=None):
    """Fused 2D neighborhood attention, stride 1 (``compat/v015.py:27-37``)."""
    return _F.na2d(query, key, value, kernel_size=kernel_size, stride=1, dilation=dilation,
                   is_causal=is_causal, scale=scale)


def na3d(query, key, value, kernel_size, dilation=1, is_causal=False, scale=None):
    """Fused 3D neighborhood attention, stride 1 (``compat/v015.py:40-50``)."""
    return _F.na3d(query, key, value, kernel_size=kernel_size, stride=1, dilation=dilation,
                   is_causal=is_causal, scale=scale)


class NeighborhoodAttention3D(torch.nn.Module):
    """v0.15 3D layer (``compat/v015.py:53-84``): ``dim``, no stride; the
    modern layer sits under ``_impl`` (so parameters are ``_impl.qkv.*`` and
    ``_impl.proj.*``, as in the reference)."""

    def __init__(self, dim, kernel_size, dilation=1, is_causal=False, num_heads=1,
                 qkv_bias=True, qk_scale=None, attn_drop=0.0, proj_drop=0.0):
        super().__init__()
        self._impl = _Modern3D(embed_dim=dim, num_heads=num_heads, kernel_size=kernel_size,
                               stride=1, dilation=dilation, is_causal=is_causal,
                               qkv_bias=qkv_bias, qk_scale=qk_scale, attn_drop=attn_drop,
                               proj_drop=proj_drop)

    def forward(self, x):
        return self._impl(x)


def has_cuda() -> bool:
    """No CUDA NATTEN kernels here (the library runs on HIP)."""
    return False


def has_mps() -> bool:
    return False


def has_mlx() -> bool:
    """No MLX here; ``natten_amd.has_hip()`` reports this package's backend."""
    return False


def has_gemm() -> bool:
    return False


def has_fna() -> bool:
    return False


__all__ = list(_v014_all) + [
    "na1d", "na2d", "na3d", "na1d_qk", "na1d_av", "na2d_qk", "na2d_av",
    "NeighborhoodAttention3D", "has_cuda", "has_mps", "has_mlx", "has_gemm", "has_fna",
]
