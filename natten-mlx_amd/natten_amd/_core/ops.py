"""Backend registry and dispatch (mirrors ``src/natten_mlx/_core/ops.py``).

Backends are modules exposing ``is_available()`` and the eighteen entry
points below.  This package registers one: ``hip`` (libnatten_amd.so on
MI355X).  ``auto`` resolves to ``hip``; there is deliberately no CPU backend
to fall back to, so an unavailable library fails loudly at call time.
``NATTEN_BACKEND`` selects the initial backend as in the reference
(``ops.py:11``).
"""

from __future__ import annotations

import os
from typing import Any

from . import hip

_BACKEND_REGISTRY: dict[str, Any] = {}
_ACTIVE_BACKEND = os.environ.get("NATTEN_BACKEND", "auto")


def register_backend(name: str, module: Any) -> None:
    _BACKEND_REGISTRY[name] = module


def _resolve_backend() -> str:
    if _ACTIVE_BACKEND != "auto":
        return _ACTIVE_BACKEND
    return "hip"


def get_backend() -> str:
    return _resolve_backend()


def set_backend(name: str) -> None:
    global _ACTIVE_BACKEND
    valid = {"auto", *_BACKEND_REGISTRY.keys()}
    if name not in valid:
        raise ValueError(f"Unknown backend {name!r}. Expected one of {sorted(valid)}")
    _ACTIVE_BACKEND = name


def _backend_module() -> Any:
    name = _resolve_backend()
    try:
        return _BACKEND_REGISTRY[name]
    except KeyError as exc:
        raise RuntimeError(f"Backend {name!r} is not registered") from exc


def na1d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    return _backend_module().na1d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)


def na2d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    return _backend_module().na2d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)


def na3d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    return _backend_module().na3d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)


def na1d_qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale):
    return _backend_module().na1d_qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale)


def na1d_av_forward(attn, v, kernel_size, stride, dilation, is_causal):
    return _backend_module().na1d_av_forward(attn, v, kernel_size, stride, dilation, is_causal)


def na2d_qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale):
    return _backend_module().na2d_qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale)


def na2d_av_forward(attn, v, kernel_size, stride, dilation, is_causal):
    return _backend_module().na2d_av_forward(attn, v, kernel_size, stride, dilation, is_causal)


def na3d_qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale):
    return _backend_module().na3d_qk_forward(q, k, kernel_size, stride, dilation, is_causal, scale)


def na3d_av_forward(attn, v, kernel_size, stride, dilation, is_causal):
    return _backend_module().na3d_av_forward(attn, v, kernel_size, stride, dilation, is_causal)


def _backend_fn(name: str):
    fn = getattr(_backend_module(), name, None)
    if fn is None:
        raise NotImplementedError(f"backend {get_backend()!r} has no {name}")
    return fn


def na1d_backward(q, k, v, grad_out, kernel_size, stride, dilation, is_causal, scale):
    return _backend_fn("na1d_backward")(q, k, v, grad_out, kernel_size, stride, dilation,
                                        is_causal, scale)


def na2d_backward(q, k, v, grad_out, kernel_size, stride, dilation, is_causal, scale):
    return _backend_fn("na2d_backward")(q, k, v, grad_out, kernel_size, stride, dilation,
                                        is_causal, scale)


def na3d_backward(q, k, v, grad_out, kernel_size, stride, dilation, is_causal, scale):
    return _backend_fn("na3d_backward")(q, k, v, grad_out, kernel_size, stride, dilation,
                                        is_causal, scale)


def na1d_qk_backward(q, k, grad_attn, kernel_size, stride, dilation, is_causal, scale):
    return _backend_fn("na1d_qk_backward")(q, k, grad_attn, kernel_size, stride, dilation,
                                           is_causal, scale)


def na1d_av_backward(attn, v, grad_out, kernel_size, stride, dilation, is_causal):
    return _backend_fn("na1d_av_backward")(attn, v, grad_out, kernel_size, stride, dilation,
                                           is_causal)


def na2d_qk_backward(q, k, grad_attn, kernel_size, stride, dilation, is_causal, scale):
    return _backend_fn("na2d_qk_backward")(q, k, grad_attn, kernel_size, stride, dilation,
                                           is_causal, scale)


def na2d_av_backward(attn, v, grad_out, kernel_size, stride, dilation, is_causal):
    return _backend_fn("na2d_av_backward")(attn, v, grad_out, kernel_size, stride, dilation,
                                           is_causal)


def na3d_qk_backward(q, k, grad_attn, kernel_size, stride, dilation, is_causal, scale):
    return _backend_fn("na3d_qk_backward")(q, k, grad_attn, kernel_size, stride, dilation,
                                           is_causal, scale)


def na3d_av_backward(attn, v, grad_out, kernel_size, stride, dilation, is_causal):
    return _backend_fn("na3d_av_backward")(attn, v, grad_out, kernel_size, stride, dilation,
                                           is_causal)


def backend_module():
    """The resolved backend module (used by the autograd layer for the
    fused-forward/backward hooks)."""
    return _backend_module()


register_backend("hip", hip)

if _ACTIVE_BACKEND not in {"auto", *_BACKEND_REGISTRY.keys()}:
    _ACTIVE_BACKEND = "auto"
