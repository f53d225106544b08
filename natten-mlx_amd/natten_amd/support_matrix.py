"""Backend capability matrix (mirrors ``src/natten_mlx/support_matrix.py``)."""

from __future__ import annotations

from ._core import hip


def get_support_matrix() -> dict[str, dict]:
    return {
        "hip": {
            "available": hip.is_available(),
            "forward": {"na1d": True, "na2d": True, "na3d": True, "split_qk_av": True},
            "backward": {"na1d": True, "na2d": True, "na3d": True, "split_qk_av": True},
            "varlen": {"na1d": True, "na2d": True, "na3d": True},
            "fusion": {"na1d": True, "na2d": True, "na3d": True},
            "constraints": [
                "MI355X (gfx950) via libnatten_amd.so; tensors must be on a HIP device.",
                "Any kernel size / dilation / stride / causal mask per axis, GQA, "
                "return_lse and additional tokens in the fused kernels.",
                "float32 / float16 / bfloat16; fp32 accumulation.",
                "No CPU fallback: an unavailable library raises.",
            ],
        },
    }
