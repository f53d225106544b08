"""Autograd for the split QK / AV ops (reference ``autograd/split.py``)."""

from __future__ import annotations

import torch

from .._core import ops

_QK_FWD = {1: ops.na1d_qk_forward, 2: ops.na2d_qk_forward, 3: ops.na3d_qk_forward}
_QK_BWD = {1: ops.na1d_qk_backward, 2: ops.na2d_qk_backward, 3: ops.na3d_qk_backward}
_AV_FWD = {1: ops.na1d_av_forward, 2: ops.na2d_av_forward, 3: ops.na3d_av_forward}
_AV_BWD = {1: ops.na1d_av_backward, 2: ops.na2d_av_backward, 3: ops.na3d_av_backward}


class _QK(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, kernel_size, stride, dilation, is_causal, scale):
        rank = q.dim() - 3
        ctx.save_for_backward(q, k)
        ctx.args = (kernel_size, stride, dilation, is_causal, scale)
        return _QK_FWD[rank](q, k, kernel_size, stride, dilation, is_causal, scale)

    @staticmethod
    def backward(ctx, grad_attn):
        q, k = ctx.saved_tensors
        rank = q.dim() - 3
        dq, dk = _QK_BWD[rank](q, k, grad_attn, *ctx.args)
        return dq, dk, None, None, None, None, None


class _AV(torch.autograd.Function):
    @staticmethod
    def forward(ctx, attn, v, kernel_size, stride, dilation, is_causal):
        rank = v.dim() - 3
        ctx.save_for_backward(attn, v)
        ctx.args = (kernel_size, stride, dilation, is_causal)
        return _AV_FWD[rank](attn, v, kernel_size, stride, dilation, is_causal)

    @staticmethod
    def backward(ctx, grad_out):
        attn, v = ctx.saved_tensors
        rank = v.dim() - 3
        dattn, dv = _AV_BWD[rank](attn, v, grad_out, *ctx.args)
        return dattn, dv, None, None, None, None


def _qk(q, k, kernel_size, stride, dilation, is_causal, scale):
    return _QK.apply(q, k, tuple(kernel_size), tuple(stride), tuple(dilation),
                     tuple(bool(c) for c in is_causal), scale)


def _av(attn, v, kernel_size, stride, dilation, is_causal):
    return _AV.apply(attn, v, tuple(kernel_size), tuple(stride), tuple(dilation),
                     tuple(bool(c) for c in is_causal))


na1d_qk_with_grad = na2d_qk_with_grad = na3d_qk_with_grad = _qk
na1d_av_with_grad = na2d_av_with_grad = na3d_av_with_grad = _av
