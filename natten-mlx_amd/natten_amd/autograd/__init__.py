"""torch.autograd wrappers (mirrors ``src/natten_mlx/autograd``).

The reference wraps each op in ``mx.custom_function`` with a VJP; here each
is a ``torch.autograd.Function`` whose backward calls the backend's
deterministic HIP backward with the saved forward output and LSE.
"""

from .fused import (
    device_extents,
    FusedSpec,
    na1d_varlen_with_grad,
    na1d_with_grad,
    na2d_varlen_with_grad,
    na2d_with_grad,
    na3d_varlen_with_grad,
    na3d_with_grad,
    na_fused_with_grad,
)
from .split import (
    na1d_av_with_grad,
    na1d_qk_with_grad,
    na2d_av_with_grad,
    na2d_qk_with_grad,
    na3d_av_with_grad,
    na3d_qk_with_grad,
)

__all__ = [
    "device_extents",
    "FusedSpec",
    "na_fused_with_grad",
    "na1d_with_grad",
    "na1d_varlen_with_grad",
    "na2d_with_grad",
    "na2d_varlen_with_grad",
    "na3d_with_grad",
    "na3d_varlen_with_grad",
    "na1d_qk_with_grad",
    "na1d_av_with_grad",
    "na2d_qk_with_grad",
    "na2d_av_with_grad",
    "na3d_qk_with_grad",
    "na3d_av_with_grad",
]
