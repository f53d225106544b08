"""Attention merging (mirrors ``src/natten_mlx/merge.py:20-68``).

Merges attention outputs that share a query as if their key/value contexts
had been concatenated, with the numerically stable sigmoid form.  Math runs
in float32; the merged output keeps ``outputs[0]``'s dtype and the merged
LSE is float32, as in the reference.
"""

from __future__ import annotations

from typing import List, Tuple

import torch
import torch.nn.functional as F


def merge_attentions(outputs: List[torch.Tensor],
                     lse_tensors: List[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    if len(outputs) < 2:
        raise ValueError("merge_attentions expects at least two outputs.")
    if len(outputs) != len(lse_tensors):
        raise ValueError("Number of outputs and LSE tensors must match.")
    ref_shape = tuple(outputs[0].shape)
    for i, (o, l) in enumerate(zip(outputs, lse_tensors)):
        if tuple(o.shape) != ref_shape:
            raise ValueError(
                f"Output {i} shape {tuple(o.shape)} does not match output 0 shape {ref_shape}.")
        if tuple(l.shape) != ref_shape[:-1]:
            raise ValueError(
                f"LSE {i} shape {tuple(l.shape)} does not match expected {ref_shape[:-1]}.")
    lse = [l.to(torch.float32).unsqueeze(-1) for l in lse_tensors]
    outs = [o.to(torch.float32) for o in outputs]
    out = outs[0] - torch.sigmoid(lse[1] - lse[0]) * (outs[0] - outs[1])
    acc = lse[0] - F.logsigmoid(lse[0] - lse[1])
    for i in range(2, len(outs)):
        out = out - torch.sigmoid(lse[i] - acc) * (out - outs[i])
        acc = acc - F.logsigmoid(acc - lse[i])
    return out.to(outputs[0].dtype), acc.squeeze(-1)


__all__ = ["merge_attentions"]
