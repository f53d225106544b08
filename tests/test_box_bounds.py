"""The window boxes the lean kernels size their LDS layout by, checked
against the oracle's window rule (`oracle/window.py`, the reference's
`pure.py:52-73`): on a dilation phase's sub-grid, the keys of t consecutive
queries span at most t + K - 1 points, and the queries whose windows hold t
consecutive keys (the backward's inverse box) at most t + 2 (K - 1) on a
non-causal axis (t + K - 1 causal).  With per-sample extents the host
cannot enumerate the boxes of every sample, so these bounds size the
layout; the test also shows that the inverse bound is reached, i.e. that
t + K - 1 + K / 2 would not do."""

import numpy as np
import pytest

from oracle import window as W


def _phase_boxes(L, K, d, causal, t):
    """(forward extent, inverse extent) maxima over tiles of t sub-grid
    points of every phase of an axis of L positions."""
    qpos = np.arange(L)
    idx, valid = W.axis_indices(qpos, L, K, d, causal)
    fwd = inv = 0
    for r in range(min(d, L)):
        pos = np.arange(r, L, d)
        n = len(pos)
        keys = [idx[p][valid[p]] for p in pos]
        for k in keys:  # windows stay in their phase
            assert np.all((k - r) % d == 0)
        sub = [(k - r) // d for k in keys]
        holders = [[] for _ in range(n)]
        for i, s in enumerate(sub):
            for j in s:
                holders[j].append(i)
        for i0 in range(0, n, t):
            i1 = min(i0 + t, n)
            ks = np.concatenate(sub[i0:i1])
            fwd = max(fwd, int(ks.max() - ks.min() + 1))
            qs = [q for j in range(i0, i1) for q in holders[j]]
            if qs:
                inv = max(inv, max(qs) - min(qs) + 1)
    return fwd, inv


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [1, 2])
def test_lean_box_bounds(causal, d):
    reached = False
    for K in (3, 5, 7, 9):
        for L in range(d * K, d * K + 40):
            for t in (1, 2, 4, 8, 16):
                fwd, inv = _phase_boxes(L, K, d, causal, t)
                assert fwd <= t + K - 1, (K, L, t, fwd)
                bound = t + K - 1 if causal else t + 2 * (K - 1)
                assert inv <= bound, (K, L, t, inv)
                if not causal and inv > t + K - 1 + K // 2:
                    reached = True
    assert reached or causal
