"""Attention merging (mirrors ``src/natten_mlx/merge.py:20-68``).

Merges attention outputs that share a query as if their key/value contexts
had been concatenated.  One HIP kernel pass (``na_merge_fwd``) computes the
closed form of the reference's sequential sigmoid merge,
``L = logsumexp_i lse_i`` and ``out = sum_i exp(lse_i - L) * out_i``, in
float32; its gradient is a second kernel (``na_merge_bwd``).  The merged
output keeps ``outputs[0]``'s dtype and the merged LSE is float32, as in the
reference.  Up to 8 parts of one dtype merge in one call; more parts, or
parts of different dtypes, merge in float32 in chunks of 8 (the merge is
associative) and round once at the end.
"""

from __future__ import annotations

from typing import List, Tuple

import torch

from ._core import _lib
from ._core import hip


class _Merge(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, *tensors):
        outs, lses = tensors[:n], tensors[n:]
        out, lse = hip.merge_forward(outs, lses)
        ctx.n = n
        ctx.save_for_backward(*outs, *lses)
        return out, lse

    @staticmethod
    def backward(ctx, d_out, d_lse):
        n = ctx.n
        saved = ctx.saved_tensors
        outs, lses = saved[:n], saved[n:]
        need = ctx.needs_input_grad[1:]
        if d_out is None:
            d_out = torch.zeros_like(outs[0])
        d_outs, d_lses = hip.merge_backward(outs, lses, d_out, d_lse, need[:n], need[n:])
        return (None, *d_outs, *d_lses)


def _merge(outs, lses):
    return _Merge.apply(len(outs), *outs, *lses)


def merge_attentions(outputs: List[torch.Tensor],
                     lse_tensors: List[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(merged_output, merged_lse)`` of outputs ``[B, *spatial, H, D]`` and
    their LSEs ``[B, *spatial, H]`` (``merge.py:20-68``)."""
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
    lses = [l.to(torch.float32) for l in lse_tensors]
    dt = outputs[0].dtype
    if len(outputs) <= _lib.MERGE_MAX_PARTS and all(o.dtype == dt for o in outputs):
        return _merge(list(outputs), lses)
    outs = [o.to(torch.float32) for o in outputs]
    step = _lib.MERGE_MAX_PARTS
    out, lse = _merge(outs[:step], lses[:step])
    i = step
    while i < len(outs):
        j = min(len(outs), i + step - 1)
        out, lse = _merge([out] + outs[i:j], [lse] + lses[i:j])
        i = j
    return out.to(dt), lse


__all__ = ["merge_attentions"]
