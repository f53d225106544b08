"""Pins the oracle's window arithmetic (oracle/window.py) to the reference's
known answers and to properties the definition fixes independently."""

import itertools

import numpy as np
import pytest

from oracle import brute
from oracle import window as W


def test_reference_kats():
    # reference tests/test_shift_semantics.py:53-64
    assert W.window_start(31, 32, 3, 1, 1) == 29
    assert W.pb_start(31, 32, 3, 1, 1) == 0


def test_phase_bounds_and_pb_range():
    # reference tests/test_shift_semantics.py:11-50 (L=64, K=7, d=4)
    L, K, d = 64, 7, 4
    for i in range(L):
        s = W.window_start(i, L, K, K // 2, d)
        e = W.window_end(s, L, K, d)
        assert 0 <= s < L and 0 < e <= L
        for k in range(K):
            if s + k * d < e:
                assert (s + k * d) % d == i % d
        pb = W.pb_start(i, L, K, K // 2, d)
        assert all(0 <= pb + k <= 2 * K - 2 for k in range(K))


def _domain(max_len=60):
    for L in range(1, max_len):
        for K in range(1, L + 1, 2):
            for d in range(1, L // K + 1):
                yield L, K, d


def test_dilation1_closed_form():
    # d = 1, odd K: the window is the K-run centred on i, clamped into [0, L)
    for L in range(1, 80):
        for K in range(1, L + 1, 2):
            for i in range(L):
                assert W.window_start(i, L, K, K // 2, 1) == min(max(i - K // 2, 0), L - K)


def test_legacy_equals_partition_form():
    for L, K, d in _domain(70):
        for i in range(L):
            assert W.window_start(i, L, K, K // 2, d) == W.window_start_partition(i, L, K, K // 2, d)


def test_pb_start_is_relative_offset():
    # bias row of slot k == (key - query) / d + K - 1
    for L, K, d in _domain(50):
        for i in range(L):
            s = W.window_start(i, L, K, K // 2, d)
            pb = W.pb_start(i, L, K, K // 2, d)
            for k in range(K):
                key = s + k * d
                assert (key - i) % d == 0
                assert pb + k == (key - i) // d + K - 1


def test_noncausal_full_window():
    # with d*K <= L every slot of a non-causal window is a valid key
    for L, K, d in _domain(50):
        idx, valid = W.axis_indices(np.arange(L), L, K, d, False)
        assert valid.all()
        assert (idx == W.axis_indices(np.arange(L), L, K, d, False)[0]).all()


def test_causal_axis():
    L, K, d = 20, 4, 3
    idx, valid = W.axis_indices(np.arange(L), L, K, d, True)
    # the last slot is the query itself; the first query sees only itself
    assert (idx[:, -1] == np.arange(L)).all() and valid[:, -1].all()
    assert valid[0].sum() == 1
    for i in range(L):
        assert valid[i].sum() == min(K, i // d + 1)


@pytest.mark.parametrize("spatial,ks,dil,caus,st", [
    ((9,), (3,), (2,), (False,), (1,)),
    ((7, 6), (3, 2), (2, 1), (True, False), (2, 1)),
    ((4, 5, 6), (3, 3, 2), (1, 1, 2), (False, True, False), (1, 2, 3)),
])
def test_neighbor_table_matches_axis_loops(spatial, ks, dil, caus, st):
    lin, valid = W.neighbor_table(spatial, ks, dil, caus, st)
    outs = [range((s + t - 1) // t) for s, t in zip(spatial, st)]
    for o in itertools.product(*outs):
        axes = [brute.axis_keys(o[a] * st[a], spatial[a], ks[a], dil[a], caus[a])
                for a in range(len(spatial))]
        for n, combo in enumerate(itertools.product(*axes)):
            ok = all(c is not None for c in combo)
            assert valid[o][n] == ok
            if ok:
                assert lin[o][n] == np.ravel_multi_index(combo, spatial)


def _phase_windows(L, K, d, r):
    """Sub-grid windows [lo, hi) of every query of phase r (oracle rule)."""
    out = []
    for p in range(r, L, d):
        s = W.window_start(p, L, K, K // 2, d)
        e = W.window_end(s, L, K, d)
        keys = [x for x in (s + k * d for k in range(K)) if 0 <= x < e]
        out.append(((min(keys) - r) // d, (max(keys) - r) // d + 1))
    return out


def test_odd_k_windows_monotone_and_inverse_contiguous():
    """The MFMA backward tiles keys by phase and gathers, per key, the
    queries whose windows contain it as one contiguous run; that needs
    window bounds non-decreasing in the query for odd K (any dilation,
    including d*K > L as varlen allows)."""
    for L in range(1, 44):
        for K in range(1, L + 1, 2):
            for d in range(1, L + 1):
                if d > 8 and d * K > L + 8:
                    break
                for r in range(min(d, L)):
                    wins = _phase_windows(L, K, d, r)
                    los = [w[0] for w in wins]
                    his = [w[1] for w in wins]
                    assert los == sorted(los) and his == sorted(his)
                    for j in range(len(wins)):
                        inv = [i for i, (lo, hi) in enumerate(wins) if lo <= j < hi]
                        assert inv and inv == list(range(inv[0], inv[-1] + 1))


def test_inverse_range_closed_form():
    """Closed form the MFMA backward uses when d*K <= L (odd K): the queries
    of sub-grid key j are [0 if j <= K-1 else j - K//2,
    Lr-1 if j >= Lr-K else j + K//2]."""
    for L in range(1, 60):
        for K in range(1, L + 1, 2):
            for d in range(1, L // K + 1):
                for r in range(d):
                    wins = _phase_windows(L, K, d, r)
                    Lr = len(wins)
                    for j in range(Lr):
                        inv = [i for i, (lo, hi) in enumerate(wins) if lo <= j < hi]
                        qlo = 0 if j <= K - 1 else j - K // 2
                        qhi = Lr - 1 if j >= Lr - K else j + K // 2
                        assert inv == list(range(qlo, qhi + 1)), (L, K, d, r, j)


def test_allin1_interior_keys():
    """The allin1 staged inverse's fast path: with K*d <= L (odd K), a key
    at position j in [K*d, L - 1 - K*d] lies in the partition window of
    exactly the queries j + t*d, |t| <= K//2, at slot K//2 - t (checked
    against every query's window, not derived from the claim)."""
    for L in range(1, 72):
        for K in range(1, L + 1, 2):
            for d in range(1, L // K + 1):
                held = {}
                for i in range(L):
                    s = W.window_start_partition(i, L, K, K // 2, d)
                    for slot in range(K):
                        held.setdefault(s + slot * d, []).append((i, slot))
                for j in range(K * d, L - K * d):
                    want = sorted((j + t * d, K // 2 - t) for t in range(-(K // 2), K // 2 + 1))
                    assert sorted(held.get(j, [])) == want, (L, K, d, j)
