"""natten_amd — MI355X-native neighborhood attention.

The functional and module API of natten-mlx (``na1d``/``na2d``/``na3d``, the
split ``*_qk``/``*_av`` ops, varlen, ``merge_attentions``, backend
selection) on PyTorch-ROCm tensors, executed by hand-written HIP kernels for
gfx950 in ``libnatten_amd.so``.
"""

from __future__ import annotations

from ._core import hip as _hip
from ._core import ops
from .functional import (
    na1d,
    na1d_av,
    na1d_qk,
    na1d_varlen,
    na1d_varlen_gqa,
    na2d,
    na2d_av,
    na2d_qk,
    na2d_varlen,
    na3d,
    na3d_av,
    na3d_qk,
    na3d_varlen,
)
from .merge import merge_attentions
from .support_matrix import get_support_matrix
from .version import __version__


def has_hip() -> bool:
    """True when libnatten_amd.so is built and a HIP device is visible."""
    return _hip.is_available()


def has_metal() -> bool:
    """The reference's Metal-tier probe (``natten_mlx/__init__.py:23-24``):
    there is no Metal tier on this platform, so always False."""
    return False


def has_nanobind() -> bool:
    """The reference's nanobind-tier probe (``natten_mlx/__init__.py:27-28``):
    always False here (the native tier is the HIP library, see has_hip)."""
    return False


def get_backend() -> str:
    return ops.get_backend()


def set_backend(name: str) -> None:
    ops.set_backend(name)


def __getattr__(name):
    if name in ("NeighborhoodAttention1D", "NeighborhoodAttention2D", "NeighborhoodAttention3D"):
        from . import nn
        return getattr(nn, name)
    raise AttributeError(name)


__all__ = [
    "__version__", "na1d", "na1d_varlen", "na1d_varlen_gqa", "na2d", "na2d_varlen", "na1d_qk",
    "na1d_av", "na2d_qk", "na2d_av", "na3d", "na3d_varlen", "na3d_qk", "na3d_av",
    "merge_attentions", "NeighborhoodAttention1D", "NeighborhoodAttention2D",
    "NeighborhoodAttention3D", "has_hip", "has_metal", "has_nanobind", "get_backend", "set_backend", "get_support_matrix",
]
