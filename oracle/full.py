"""Full-size fused neighborhood attention, forward and backward, by query
chunks (test oracle) — TEST INFRASTRUCTURE ONLY.

``oracle.na`` materialises the neighbor gather of every query at once
(``[B, *O, prod(K), H, D]``), which does not fit memory at the benchmark
shapes (config 3: 16,384 positions x 147 slots x 8 heads x 64 in float64 is
9.9 GB per tensor).  This module computes the same quantities exactly, in
float64, a slice of query positions at a time:

* the neighbor indices and validity come from ``oracle.window.neighbor_table``
  over the FULL extent (``pure.py:24-152``), so edge clamping is the
  reference's, never a crop's;
* one chunk's logits are ``scale * <q, k_nbr>`` with invalid slots ``-inf``
  (``pure.py:185-191``), joined by the additional tokens' logits in one
  softmax (the ``merge_attentions`` composition of ``functional.py:277-292``
  equals one softmax over the window and the extra keys);
* GQA reads key/value head ``h // rep`` for query head ``h``
  (``functional.py:29-33``) by viewing the query heads as ``[H_kv, rep]``;
* varlen runs each sample on its leading extent (``pure.py:497-547``) and
  leaves the rows past it zero;
* gradients come from torch autograd of each chunk's forward, with the loss
  ``sum(out * dout) + sum(lse * dlse)``: a query's output depends only on
  its own row, and key/value gradients accumulate over the chunks, so the
  sum over chunks is the full gradient.

Pinned by ``tests/test_oracle_full.py``: equality with ``oracle.na``
(``na_functional`` / ``na_varlen`` and float64 autograd of them, themselves
pinned by brute force and finite differences) on small problems of every
kind (ranks 1-3, causal, stride, dilation, GQA, additional tokens, varlen,
chunk boundaries that split a row block).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import window as W


def _tup(x, rank):
    if isinstance(x, (tuple, list)):
        assert len(x) == rank
        return tuple(int(v) for v in x)
    return (int(x),) * rank


def _one_sample(q, k, v, ek, ev, dout, dlse, ks, st, dil, caus, scale, chunk, need_grad,
                f64=torch.float64, max_rows=None):
    """One sample (leading batch axis of size 1 stripped): q ``[*S, H, D]``,
    k/v ``[*S, Hkv, D]``, ek/ev ``[N, Hkv, D]`` or None, dout ``[*O, H, D]``,
    dlse ``[*O, H]`` or None.  Returns (out, lse, dq, dk, dv, dek, dev).
    ``f64``: the compute dtype; ``max_rows``: stop after that many output
    rows (a bounded sample, for timing only)."""
    spatial = tuple(q.shape[:-2])
    H, D = q.shape[-2], q.shape[-1]
    Hkv = k.shape[-2]
    rep = H // Hkv
    lin, valid = W.neighbor_table(spatial, ks, dil, caus, st)
    out_sp = lin.shape[:-1]
    kp = lin.shape[-1]
    n_out = int(np.prod(out_sp))
    lin = torch.from_numpy(lin.reshape(n_out, kp).astype(np.int64))
    valid = torch.from_numpy(valid.reshape(n_out, kp))
    qsel = q[tuple(slice(None, None, s) for s in st)].to(f64).reshape(n_out, Hkv, rep, D)
    kf = k.to(f64).reshape(-1, Hkv, D).detach().requires_grad_(need_grad)
    vf = v.to(f64).reshape(-1, Hkv, D).detach().requires_grad_(need_grad)
    ekf = evf = None
    if ek is not None:
        ekf = ek.to(f64).detach().requires_grad_(need_grad)
        evf = ev.to(f64).detach().requires_grad_(need_grad)
    do = dout.to(f64).reshape(n_out, Hkv, rep, D) if need_grad else None
    dl = (dlse.to(f64).reshape(n_out, Hkv, rep) if (need_grad and dlse is not None) else None)
    out = torch.zeros((n_out, Hkv, rep, D), dtype=f64)
    lse = torch.zeros((n_out, Hkv, rep), dtype=f64)
    dq_sel = torch.zeros((n_out, Hkv, rep, D), dtype=f64) if need_grad else None
    n_run = n_out if max_rows is None else min(n_out, max_rows)
    for r0 in range(0, n_run, chunk):
        r1 = min(n_run, r0 + chunk)
        qc = qsel[r0:r1].detach().requires_grad_(need_grad)
        idx = lin[r0:r1]
        kn = kf[idx.reshape(-1)].reshape(r1 - r0, kp, Hkv, D)
        vn = vf[idx.reshape(-1)].reshape(r1 - r0, kp, Hkv, D)
        # [n, Hkv, rep, kp]
        s = torch.einsum("nhrd,nkhd->nhrk", qc, kn) * scale
        s = torch.where(valid[r0:r1].reshape(r1 - r0, 1, 1, kp), s,
                        torch.full((), -math.inf, dtype=f64))
        if ekf is not None:
            sx = torch.einsum("nhrd,xhd->nhrx", qc, ekf) * scale
            s = torch.cat([s, sx], dim=-1)
        m = torch.logsumexp(s, dim=-1)
        p = torch.exp(s - m.unsqueeze(-1))
        o = torch.einsum("nhrk,nkhd->nhrd", p[..., :kp], vn)
        if evf is not None:
            o = o + torch.einsum("nhrx,xhd->nhrd", p[..., kp:], evf)
        out[r0:r1] = o.detach()
        lse[r0:r1] = m.detach()
        if need_grad:
            loss = (o * do[r0:r1]).sum()
            if dl is not None:
                loss = loss + (m * dl[r0:r1]).sum()
            loss.backward()
            dq_sel[r0:r1] = qc.grad
    res_out = out.reshape(*out_sp, H, D)
    res_lse = lse.reshape(*out_sp, H)
    if not need_grad:
        return res_out, res_lse, None, None, None, None, None
    dq = torch.zeros(q.shape, dtype=f64)
    dq[tuple(slice(None, None, s) for s in st)] = dq_sel.reshape(*out_sp, H, D)
    dk = kf.grad.reshape(k.shape)
    dv = vf.grad.reshape(v.shape)
    dek = ekf.grad if ekf is not None else None
    dev = evf.grad if evf is not None else None
    return res_out, res_lse, dq, dk, dv, dek, dev


def fused(q, k, v, kernel_size, stride=1, dilation=1, is_causal=False, scale=None,
          dout=None, dlse=None, extra_k=None, extra_v=None, sizes=None, chunk=256,
          compute_dtype=torch.float64, max_rows=None):
    """Fused neighborhood attention over ``[B, *spatial, H, D]`` tensors (k, v
    with ``H_kv`` heads; extra_k / extra_v ``[B, N, H_kv, D]``), exactly in
    float64.  ``sizes``: per-sample extents ``[B]`` / ``[B, rank]`` (varlen,
    stride 1, non-causal); rows past a sample's extent are zero.

    Returns a dict with ``out`` ``[B, *O, H, D]`` and ``lse`` ``[B, *O, H]``
    and, when ``dout`` is given, ``dq``, ``dk``, ``dv`` (and ``dek``,
    ``dev`` with extra tokens): gradients of
    ``sum(out * dout) + sum(lse * dlse)``.

    ``compute_dtype`` other than float64 and ``max_rows`` (compute only the
    first rows of each sample) exist for the benchmark's CPU baseline, which
    times the reference's ``pure`` algorithm in the input dtype on a bounded
    sample; parity checks use the defaults.
    """
    rank = q.dim() - 3
    ks, st, dil, caus = (_tup(kernel_size, rank), _tup(stride, rank),
                         _tup(dilation, rank), _tup(is_causal, rank))
    B, H, D = q.shape[0], q.shape[-2], q.shape[-1]
    sc = D ** -0.5 if scale is None else float(scale)
    need_grad = dout is not None
    f64 = compute_dtype
    out_sp = tuple((s + t - 1) // t for s, t in zip(q.shape[1:-2], st))
    res = {"out": torch.zeros((B, *out_sp, H, D), dtype=f64),
           "lse": torch.zeros((B, *out_sp, H), dtype=f64)}
    if need_grad:
        res["dq"] = torch.zeros(q.shape, dtype=f64)
        res["dk"] = torch.zeros(k.shape, dtype=f64)
        res["dv"] = torch.zeros(v.shape, dtype=f64)
        if extra_k is not None:
            res["dek"] = torch.zeros(extra_k.shape, dtype=f64)
            res["dev"] = torch.zeros(extra_v.shape, dtype=f64)
    if sizes is not None:
        assert all(s == 1 for s in st) and not any(caus), "varlen is stride 1, non-causal"
        sizes = torch.as_tensor(sizes).reshape(B, -1)
    for b in range(B):
        if sizes is None:
            sl = (slice(None),) * rank
        else:
            sl = tuple(slice(0, int(e)) for e in sizes[b])
        osl = sl  # stride 1 under varlen
        if sizes is None:
            osl = (slice(None),) * rank
        qb, kb, vb = q[b][sl], k[b][sl], v[b][sl]
        ekb = extra_k[b] if extra_k is not None else None
        evb = extra_v[b] if extra_v is not None else None
        dob = dout[b][osl] if need_grad else None
        dlb = dlse[b][osl] if (need_grad and dlse is not None) else None
        o, l, dq, dk, dv, dek, dev = _one_sample(qb, kb, vb, ekb, evb, dob, dlb, ks, st, dil,
                                                 caus, sc, chunk, need_grad, f64, max_rows)
        res["out"][b][osl] = o
        res["lse"][b][osl] = l
        if need_grad:
            res["dq"][b][sl] = dq
            res["dk"][b][sl] = dk
            res["dv"][b][sl] = dv
            if dek is not None:
                res["dek"][b] = dek
                res["dev"][b] = dev
    return res

