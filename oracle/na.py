"""Neighborhood attention restated on the CPU with torch (test oracle).

All functions take spatial-first tensors ``[B, *spatial, H, D]`` (the
reference layout) and compute in ``compute_dtype`` (float64 by default; the
``cpu_baseline`` leg of bench.py passes the input dtype, as the reference's
``pure`` backend computes in the input dtype).  Backward is torch autograd of
these forwards.

Reference code followed:
* ``na_qk`` / ``na_av`` / ``na_forward``: ``_core/pure.py:155-494``
  (gather neighbors, masked logits = -inf, softmax, masked weighted sum);
  3D fused = qk -> softmax -> av (``pure.py:251-255``).
* ``na_functional``: ``functional.py:207-473`` composition (GQA repeat
  ``:29-33``, FMHA ``:141-187``, return_lse / additional KV ``:277-292``).
* ``full_attn_with_lse``: ``functional.py:71-104``.
* ``merge_attentions``: ``merge.py:20-68`` (sigmoid form, float32 inside).
* ``na_varlen``: ``pure.py:497-688`` (per-sample calls, zero padding).
* ``qk_rpb`` / ``av_rpb`` (rank 1 and 2): ``extras/allin1/__init__.py:40-180``
  with the MLX fallbacks ``extras/allin1/functional.py:57-368`` (query scaled
  in its own dtype first; partition window, equal to the legacy window when
  d*K <= L; rpb index clip(pb + k, 0, 2K-2) per axis, 2D pair index
  i*(2K-1)+j).

Pinned by (tests/test_oracle_na.py): scalar brute-force loops
(``oracle.brute``), the global-attention special case against a plain
softmax(QK^T)V, causal first-token / linearity KATs, logsumexp identity,
merge == attention over concatenated keys, GQA == explicit repeat, varlen ==
per-sample calls, allin1 == split qk + relative-offset bias, and
``torch.autograd.gradcheck`` (finite differences) for the backward.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

from . import window as W


def _tup(x, rank):
    if isinstance(x, (tuple, list)):
        assert len(x) == rank
        return tuple(x)
    return (x,) * rank


def _repeat_kv(x: torch.Tensor, rep: int) -> torch.Tensor:
    """``functional.py:29-33`` (``mx.repeat`` on the head axis)."""
    return x if rep == 1 else torch.repeat_interleave(x, rep, dim=-2)


def _query_select(q: torch.Tensor, stride) -> torch.Tensor:
    idx = (slice(None),) + tuple(slice(None, None, s) for s in stride)
    return q[idx]


def na_qk(q, k, kernel_size, stride=1, dilation=1, is_causal=False, scale=None,
          compute_dtype=torch.float64):
    """Split QK (``pure.py:258-283,320-359,404-449``): ``[B, *O, H, Kprod]``."""
    rank = q.dim() - 3
    ks, st, dil, caus = (_tup(kernel_size, rank), _tup(stride, rank),
                         _tup(dilation, rank), _tup(is_causal, rank))
    spatial = tuple(q.shape[1:-2])
    B, H, D = q.shape[0], q.shape[-2], q.shape[-1]
    rep = H // k.shape[-2]
    scale = D ** -0.5 if scale is None else float(scale)
    lin, valid = W.neighbor_table(spatial, ks, dil, caus, st)
    qs = _query_select(q.to(compute_dtype), st)
    kf = _repeat_kv(k.to(compute_dtype), rep).reshape(B, -1, H, D)
    out_sp = lin.shape[:-1]
    kp = lin.shape[-1]
    kn = kf[:, torch.from_numpy(lin.reshape(-1))].reshape(B, *out_sp, kp, H, D)
    logits = torch.einsum("b...hd,b...khd->b...hk", qs, kn) * scale
    mask = torch.from_numpy(valid).reshape(1, *out_sp, 1, kp)
    return torch.where(mask, logits, torch.full_like(logits, -math.inf))


def na_av(attn, v, kernel_size, stride=1, dilation=1, is_causal=False,
          compute_dtype=torch.float64):
    """Split AV (``pure.py:286-317,362-401,452-494``): ``[B, *O, H, D]``."""
    rank = v.dim() - 3
    ks, st, dil, caus = (_tup(kernel_size, rank), _tup(stride, rank),
                         _tup(dilation, rank), _tup(is_causal, rank))
    spatial = tuple(v.shape[1:-2])
    B, D = v.shape[0], v.shape[-1]
    H = attn.shape[-2]
    rep = H // v.shape[-2]
    lin, valid = W.neighbor_table(spatial, ks, dil, caus, st)
    out_sp = lin.shape[:-1]
    kp = lin.shape[-1]
    if tuple(attn.shape[1:-2]) != tuple(out_sp) or attn.shape[-1] != kp:
        raise ValueError("attn shape does not match ceil(input/stride) x kernel volume")
    vf = _repeat_kv(v.to(compute_dtype), rep).reshape(B, -1, H, D)
    vn = vf[:, torch.from_numpy(lin.reshape(-1))].reshape(B, *out_sp, kp, H, D)
    mask = torch.from_numpy(valid).reshape(1, *out_sp, 1, kp)
    a = torch.where(mask, attn.to(compute_dtype), torch.zeros((), dtype=compute_dtype))
    return torch.einsum("b...hk,b...khd->b...hd", a, vn)


def na_forward(q, k, v, kernel_size, stride=1, dilation=1, is_causal=False, scale=None,
               compute_dtype=torch.float64, return_lse=False):
    """Fused forward = softmax(qk) -> av (``pure.py:155-255``)."""
    logits = na_qk(q, k, kernel_size, stride, dilation, is_causal, scale, compute_dtype)
    attn = torch.softmax(logits, dim=-1)
    out = na_av(attn, v, kernel_size, stride, dilation, is_causal, compute_dtype)
    if return_lse:
        return out, torch.logsumexp(logits, dim=-1)
    return out


def full_attn_with_lse(q, k, v, scale, compute_dtype=torch.float64):
    """``functional.py:71-104``: every query against N extra tokens."""
    B, H, D = q.shape[0], q.shape[-2], q.shape[-1]
    sp = tuple(q.shape[1:-2])
    qf = q.to(compute_dtype).reshape(B, -1, H, D)
    logits = torch.einsum("bshd,bnhd->bhsn", qf, k.to(compute_dtype)) * scale
    lse = torch.logsumexp(logits, dim=-1)
    out = torch.einsum("bhsn,bnhd->bshd", torch.softmax(logits, dim=-1), v.to(compute_dtype))
    return out.reshape(B, *sp, H, D), lse.transpose(1, 2).reshape(B, *sp, H)


def merge_attentions(outputs: Sequence[torch.Tensor], lses: Sequence[torch.Tensor]):
    """``merge.py:20-68``: sigmoid-form LSE merge computed in float32 (or
    wider when the inputs are wider); output in outputs[0]'s dtype, lse float."""
    if len(outputs) < 2:
        raise ValueError("merge_attentions expects at least two outputs.")
    wide = torch.float64 if outputs[0].dtype == torch.float64 else torch.float32
    lse = [x.to(wide).unsqueeze(-1) for x in lses]
    outs = [o.to(wide) for o in outputs]
    out = outs[0] - torch.sigmoid(lse[1] - lse[0]) * (outs[0] - outs[1])
    acc = lse[0] - torch.nn.functional.logsigmoid(lse[0] - lse[1])
    for i in range(2, len(outs)):
        out = out - torch.sigmoid(lse[i] - acc) * (out - outs[i])
        acc = acc - torch.nn.functional.logsigmoid(acc - lse[i])
    return out.to(outputs[0].dtype), acc.squeeze(-1)


def na_functional(q, k, v, kernel_size, stride=1, dilation=1, is_causal=False, scale=None,
                  return_lse=False, additional_keys=None, additional_values=None,
                  compute_dtype=torch.float64):
    """``functional.na{1,2,3}d`` (``functional.py:207-473``) semantics."""
    rank = q.dim() - 3
    ks, st, dil, caus = (_tup(kernel_size, rank), _tup(stride, rank),
                         _tup(dilation, rank), _tup(is_causal, rank))
    H, D = q.shape[-2], q.shape[-1]
    rep = H // k.shape[-2]
    k = _repeat_kv(k, rep)
    v = _repeat_kv(v, rep)
    ak = _repeat_kv(additional_keys, rep) if additional_keys is not None else None
    av = _repeat_kv(additional_values, rep) if additional_values is not None else None
    spatial = tuple(q.shape[1:-2])
    sc = D ** -0.5 if scale is None else float(scale)
    if all(kk >= s for kk, s in zip(ks, spatial)) and all(s == 1 for s in st) and not any(caus):
        return dense_attention(q, k, v, sc, return_lse, ak, av, compute_dtype)
    if ak is not None or return_lse:
        logits = na_qk(q, k, ks, st, dil, caus, sc, compute_dtype)
        lse = torch.logsumexp(logits, dim=-1)
        out = na_av(torch.softmax(logits, dim=-1), v, ks, st, dil, caus, compute_dtype)
        if ak is not None:
            # the reference attends the extra tokens from every input position,
            # so its merge only lines up at stride 1; the strided queries are
            # the ones that have outputs, which is what is used here
            oe, le = full_attn_with_lse(_query_select(q, st), ak, av, sc, compute_dtype)
            out, lse = merge_attentions([out, oe], [lse, le])
        return (out, lse) if return_lse else out
    return na_forward(q, k, v, ks, st, dil, caus, sc, compute_dtype)


def dense_attention(q, k, v, scale, return_lse=False, ak=None, av=None,
                    compute_dtype=torch.float64):
    """FMHA fast path (``functional.py:146-187``): all tokens (+ extra)."""
    B, H, D = q.shape[0], q.shape[-2], q.shape[-1]
    sp = tuple(q.shape[1:-2])
    kf = k.to(compute_dtype).reshape(B, -1, H, D)
    vf = v.to(compute_dtype).reshape(B, -1, H, D)
    if ak is not None:
        kf = torch.cat([kf, ak.to(compute_dtype)], dim=1)
        vf = torch.cat([vf, av.to(compute_dtype)], dim=1)
    out, lse = full_attn_with_lse(q, kf, vf, scale, compute_dtype)
    return (out, lse) if return_lse else out


def na_varlen(q, k, v, sizes, kernel_size, dilation=1, scale=None,
              compute_dtype=torch.float64):
    """``pure.py:497-688``: per-sample call on the leading ``sizes[b]``
    extent, zero padding elsewhere.  ``sizes``: ``[B]`` (1D) or ``[B, rank]``."""
    rank = q.dim() - 3
    sizes = torch.as_tensor(sizes).reshape(q.shape[0], -1)
    out = torch.zeros(q.shape, dtype=compute_dtype)
    for b in range(q.shape[0]):
        ext = tuple(int(x) for x in sizes[b])
        sl = (slice(b, b + 1),) + tuple(slice(0, e) for e in ext)
        out[sl] = na_forward(q[sl], k[sl], v[sl], kernel_size, 1, dilation, False, scale,
                             compute_dtype)
    return out


def _allin1_axis(L, K, d):
    """Per-axis partition windows: slot positions [L, K], validity [L, K] and
    clipped bias rows [L, K] (``extras/allin1/reference_impl.py:13-45``,
    ``compat/v014.py:18-23``)."""
    nh = K // 2
    ni = np.array([W.window_start_partition(i, L, K, nh, d) for i in range(L)])
    ei = np.minimum(L, ni + K * d)
    pi = np.array([W.pb_start(i, L, K, nh, d) for i in range(L)])
    pos = ni[:, None] + np.arange(K)[None, :] * d
    valid = (pos >= 0) & (pos < ei[:, None])
    bias = np.clip(pi[:, None] + np.arange(K)[None, :], 0, 2 * K - 2)
    return np.clip(pos, 0, L - 1), valid, bias


def _axes_param(v, rank):
    return tuple(int(x) for x in v) if isinstance(v, (tuple, list)) else (int(v),) * rank


def _allin1_tables(spatial, K, d):
    """Flattened neighbor index, validity and bias index over all query
    positions of a rank-1/2 grid: arrays [prod(spatial), K0*K1].  K and d are
    ints (every axis) or per-axis tuples; the 2D bias index is
    r0 * (2*K1 - 1) + r1 (``compat/v014.py:26-49``)."""
    Ks, ds = _axes_param(K, len(spatial)), _axes_param(d, len(spatial))
    axes = [_allin1_axis(L, k, dd) for L, k, dd in zip(spatial, Ks, ds)]
    if len(spatial) == 1:
        pos, valid, bias = axes[0]
        return pos, valid, bias
    (p0, v0, b0), (p1, v1, b1) = axes
    L0, L1 = spatial
    K0, K1 = Ks
    R1 = 2 * K1 - 1
    lin = (p0[:, None, :, None] * L1 + p1[None, :, None, :]).reshape(L0 * L1, K0 * K1)
    val = (v0[:, None, :, None] & v1[None, :, None, :]).reshape(L0 * L1, K0 * K1)
    bia = (b0[:, None, :, None] * R1 + b1[None, :, None, :]).reshape(L0 * L1, K0 * K1)
    return lin, val, bia


def qk_rpb(q, k, rpb, kernel_size, dilation=1, scale=None, compute_dtype=torch.float64):
    """allin1 ``na{1,2}d_qk_rpb``: q ``[B, *L, H, D]`` -> logits
    ``[B, *L, H, K^rank]``; rpb ``[H, 2K-1]`` or ``[H, 2K0-1, 2K1-1]``.
    kernel_size / dilation: int or per-axis tuple; scale None = no scaling."""
    if scale is not None:
        q = q * scale  # in the storage dtype, before the dot (``__init__.py:61-62``)
    B, H, D = q.shape[0], q.shape[-2], q.shape[-1]
    sp = tuple(q.shape[1:-2])
    lin, valid, bidx = _allin1_tables(sp, kernel_size, dilation)
    n, kk = lin.shape
    qf = q.to(compute_dtype).reshape(B, n, H, D)
    kn = k.to(compute_dtype).reshape(B, n, H, D)[:, torch.from_numpy(lin.reshape(-1))]
    kn = kn.reshape(B, n, kk, H, D)
    logits = torch.einsum("bnhd,bnkhd->bnhk", qf, kn)
    if rpb is not None:
        flat = rpb.to(compute_dtype).reshape(H, -1)
        bias = flat[:, torch.from_numpy(bidx)]  # [H, n, kk]
        logits = logits + bias.permute(1, 0, 2).unsqueeze(0)
    logits = torch.where(torch.from_numpy(valid).reshape(1, n, 1, kk), logits,
                         torch.full_like(logits, -math.inf))
    return logits.reshape(B, *sp, H, kk)


def av_rpb(attn, v, kernel_size, dilation=1, compute_dtype=torch.float64):
    """allin1 ``na{1,2}d_av_fused``: attn ``[B, *L, H, K^rank]``, v ``[B, *L, H, D]``."""
    B, H, D = v.shape[0], v.shape[-2], v.shape[-1]
    sp = tuple(v.shape[1:-2])
    lin, valid, _ = _allin1_tables(sp, kernel_size, dilation)
    n, kk = lin.shape
    vn = v.to(compute_dtype).reshape(B, n, H, D)[:, torch.from_numpy(lin.reshape(-1))]
    vn = vn.reshape(B, n, kk, H, D)
    a = torch.where(torch.from_numpy(valid).reshape(1, n, 1, kk),
                    attn.to(compute_dtype).reshape(B, n, H, kk), torch.zeros((), dtype=compute_dtype))
    return torch.einsum("bnhk,bnkhd->bnhd", a, vn).reshape(B, *sp, H, D)


def qk_rpb_1d(q, k, rpb, kernel_size, dilation=1, scale=None, compute_dtype=torch.float64):
    """allin1 ``na1d_qk_rpb``: q ``[B, L, H, D]`` -> logits ``[B, L, H, K]``."""
    return qk_rpb(q, k, rpb, kernel_size, dilation, scale, compute_dtype)


def av_1d(attn, v, kernel_size, dilation=1, compute_dtype=torch.float64):
    """allin1 ``na1d_av_fused``: attn ``[B, L, H, K]``, v ``[B, L, H, D]``."""
    return av_rpb(attn, v, kernel_size, dilation, compute_dtype)


def grads(fn, inputs: Sequence[torch.Tensor], cotangents: Sequence[Optional[torch.Tensor]]):
    """Backward of ``fn`` (float64 autograd): gradients of sum(out_i * cot_i)
    with respect to each input."""
    leaves = [x.detach().to(torch.float64).requires_grad_(True) for x in inputs]
    outs = fn(*leaves)
    if not isinstance(outs, (tuple, list)):
        outs = (outs,)
    total = 0
    for o, c in zip(outs, cotangents):
        if c is not None:
            total = total + (o.to(torch.float64) * c.to(torch.float64)).sum()
    g = torch.autograd.grad(total, leaves, allow_unused=True)
    return [torch.zeros_like(l) if gi is None else gi for gi, l in zip(g, leaves)]
