"""Autograd for the DiNAT all-in-one operators.

The reference's public ``na{1,2}d_qk_rpb`` / ``na{1,2}d_av_fused`` are
forward-only; its Metal backward lives in separate functions
(``extras/allin1/functional_metal.py:1206-1918``: dq, dk, drpb and dattn,
dvalue).  Here both directions are joined in ``torch.autograd.Function`` s
whose backward calls the library's deterministic gather kernels.
"""

from __future__ import annotations

import torch

from .._core import hip


class _QKRPB(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, rpb, kernel_size, dilation, scale, heads_first):
        ctx.save_for_backward(q, k)
        ctx.args = (kernel_size, dilation, scale, heads_first)
        ctx.rpb_dtype = None if rpb is None else rpb.dtype
        return hip.rpb_qk_forward(q, k, rpb, kernel_size, dilation, scale, heads_first)

    @staticmethod
    def backward(ctx, d_logits):
        q, k = ctx.saved_tensors
        need_q, need_k, need_rpb = ctx.needs_input_grad[:3]
        dq, dk, drpb = hip.rpb_qk_backward(q, k, d_logits, *ctx.args, need_q=need_q,
                                           need_k=need_k,
                                           need_rpb=need_rpb and ctx.rpb_dtype is not None)
        if dk is not None and dk.dtype != k.dtype:
            dk = dk.to(k.dtype)
        if drpb is not None and drpb.dtype != ctx.rpb_dtype:
            drpb = drpb.to(ctx.rpb_dtype)
        return dq, dk, drpb, None, None, None, None


class _AVRPB(torch.autograd.Function):
    @staticmethod
    def forward(ctx, attn, v, kernel_size, dilation, heads_first, out_dtype):
        ctx.save_for_backward(attn, v)
        ctx.args = (kernel_size, dilation, heads_first)
        return hip.rpb_av_forward(attn, v, kernel_size, dilation, heads_first, out_dtype)

    @staticmethod
    def backward(ctx, d_out):
        attn, v = ctx.saved_tensors
        need_a, need_v = ctx.needs_input_grad[:2]
        da, dv = hip.rpb_av_backward(attn, v, d_out, *ctx.args, need_attn=need_a, need_v=need_v)
        if da is not None and da.dtype != attn.dtype:
            da = da.to(attn.dtype)
        return da, dv, None, None, None, None


def _axes(v):
    """An int, or a per-axis tuple of ints (non-square windows)."""
    return tuple(int(x) for x in v) if isinstance(v, (tuple, list)) else int(v)


def qk_rpb_with_grad(q, k, rpb, kernel_size, dilation, scale=None, heads_first=False):
    """float32 logits of the fused QK + RPB op, differentiable in q, k, rpb.
    kernel_size / dilation: an int or one value per axis."""
    return _QKRPB.apply(q, k, rpb, _axes(kernel_size), _axes(dilation), scale,
                        bool(heads_first))


def av_rpb_with_grad(attn, v, kernel_size, dilation, heads_first=False,
                     out_dtype=torch.float32):
    """AV op output, differentiable in attn and v."""
    return _AVRPB.apply(attn, v, _axes(kernel_size), _axes(dilation), bool(heads_first),
                        out_dtype)


__all__ = ["qk_rpb_with_grad", "av_rpb_with_grad"]
