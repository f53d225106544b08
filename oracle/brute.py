"""Scalar brute-force neighborhood attention for tiny inputs (test oracle).

An independent restatement of the reference semantics written as plain
loops over queries, kernel slots and keys, used to pin ``oracle.na``.  A
query at output index o (position p = o * stride) attends, per axis, to the
key positions raw + k * dilation (k < K) that satisfy the rule of
``_core/pure.py:52-73``; the nd neighborhood is the product of the axis
sets.  Pure Python: keep inputs to a few hundred queries.
"""

from __future__ import annotations

import itertools
import math

import numpy as np

from . import window as W


def axis_keys(p: int, L: int, K: int, d: int, causal: bool) -> list[int | None]:
    """Key position of each kernel slot on one axis, None when invalid."""
    if causal:
        raw = p - (K - 1) * d
        return [raw + k * d if 0 <= raw + k * d <= p else None for k in range(K)]
    start = W.window_start(p, L, K, K // 2, d)
    end = W.window_end(start, L, K, d)
    return [start + k * d if 0 <= start + k * d < end else None for k in range(K)]


def na_forward(q: np.ndarray, k: np.ndarray, v: np.ndarray, ks, st, dil, caus, scale,
               extra_k=None, extra_v=None):
    """q, k, v float64 ``[B, *S, H, D]``; returns out ``[B, *O, H, D]`` and
    lse ``[B, *O, H]`` (one softmax over the window plus extra tokens)."""
    rank = q.ndim - 3
    B, H, D = q.shape[0], q.shape[-2], q.shape[-1]
    Hk = k.shape[-2]
    rep = H // Hk
    S = q.shape[1:-2]
    O = tuple((S[a] + st[a] - 1) // st[a] for a in range(rank))
    out = np.zeros((B, *O, H, D))
    lse = np.zeros((B, *O, H))
    for b in range(B):
        for o in itertools.product(*[range(n) for n in O]):
            pos = tuple(o[a] * st[a] for a in range(rank))
            keys = [axis_keys(pos[a], S[a], ks[a], dil[a], bool(caus[a])) for a in range(rank)]
            for h in range(H):
                hk = h // rep
                qv = q[(b, *pos, h)]
                scores, vals = [], []
                for combo in itertools.product(*keys):
                    if any(c is None for c in combo):
                        continue
                    scores.append(scale * float(qv @ k[(b, *combo, hk)]))
                    vals.append(v[(b, *combo, hk)])
                if extra_k is not None:
                    for n in range(extra_k.shape[1]):
                        scores.append(scale * float(qv @ extra_k[b, n, hk]))
                        vals.append(extra_v[b, n, hk])
                m = max(scores)
                w = [math.exp(s - m) for s in scores]
                z = sum(w)
                out[(b, *o, h)] = sum(wi * vi for wi, vi in zip(w, vals)) / z
                lse[(b, *o, h)] = m + math.log(z)
    return out, lse
