"""NATTEN v0.20+ API (mirrors ``compat/v020.py``): the modern functional
ops and layers under their v0.20 names, plus the feature probes."""

from ..functional import na1d, na1d_av, na1d_qk, na2d, na2d_av, na2d_qk, na3d, na3d_av, na3d_qk
from ..nn import NeighborhoodAttention1D, NeighborhoodAttention2D, NeighborhoodAttention3D
from .v015 import has_cuda, has_fna, has_mlx, has_mps

__all__ = [
    "na1d", "na2d", "na1d_qk", "na1d_av", "na2d_qk", "na2d_av", "na3d", "na3d_qk", "na3d_av",
    "NeighborhoodAttention1D", "NeighborhoodAttention2D", "NeighborhoodAttention3D",
    "has_cuda", "has_mps", "has_mlx", "has_fna",
]
