"""Pins the oracle's attention math (oracle/na.py) against independent
computations: scalar brute-force loops, plain dense attention, identities
the reference's own tests state, and finite differences."""

import math

import numpy as np
import pytest
import torch

from oracle import brute
from oracle import na as O


def _r(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64)


CASES = [
    # (B, spatial, H, Hk, D, ks, dil, caus, st, n_extra)
    (2, (9,), 2, 2, 5, (3,), (2,), (False,), (1,), 0),
    (1, (10,), 2, 1, 4, (4,), (1,), (True,), (2,), 2),
    (1, (6, 7), 2, 2, 3, (3, 3), (1, 2), (False, True), (1, 1), 0),
    (1, (5, 6), 4, 2, 4, (3, 2), (1, 1), (True, False), (2, 3), 3),
    (1, (3, 4, 5), 1, 1, 3, (2, 3, 3), (1, 1, 1), (True, False, False), (1, 1, 2), 0),
]


@pytest.mark.parametrize("case", CASES)
def test_forward_matches_brute_force(case):
    B, sp, H, Hk, D, ks, dil, caus, st, ne = case
    q, k, v = _r((B, *sp, H, D), 1), _r((B, *sp, Hk, D), 2), _r((B, *sp, Hk, D), 3)
    ek = _r((B, ne, Hk, D), 4) if ne else None
    ev = _r((B, ne, Hk, D), 5) if ne else None
    scale = 0.7
    ref_out, ref_lse = brute.na_forward(q.numpy(), k.numpy(), v.numpy(), ks, st, dil, caus,
                                        scale, None if ek is None else ek.numpy(),
                                        None if ev is None else ev.numpy())
    out, lse = O.na_functional(q, k, v, ks, st, dil, caus, scale, return_lse=True,
                               additional_keys=ek, additional_values=ev)
    np.testing.assert_allclose(out.numpy(), ref_out, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse.numpy(), ref_lse, rtol=1e-12, atol=1e-12)


def test_global_attention_special_case():
    # kernel == extent: plain softmax(Q K^T * scale) V (reference
    # tests/test_functional.py:122-140)
    B, L, H, D = 2, 9, 3, 4
    q, k, v = _r((B, L, H, D), 1), _r((B, L, H, D), 2), _r((B, L, H, D), 3)
    s = torch.einsum("blhd,bshd->bhls", q, k) * D ** -0.5
    ref = torch.einsum("bhls,bshd->blhd", torch.softmax(s, -1), v)
    torch.testing.assert_close(O.na_forward(q, k, v, L), ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(O.na_functional(q, k, v, L), ref, rtol=1e-12, atol=1e-12)


def test_causal_first_token_attends_to_itself():
    q, k, v = _r((1, 8, 1, 4), 1), _r((1, 8, 1, 4), 2), _r((1, 8, 1, 4), 3)
    out = O.na_forward(q, k, v, 3, is_causal=True)
    torch.testing.assert_close(out[:, 0], v[:, 0])


def test_split_compose_equals_fused_and_lse():
    q, k, v = _r((1, 7, 6, 2, 3), 1), _r((1, 7, 6, 2, 3), 2), _r((1, 7, 6, 2, 3), 3)
    logits = O.na_qk(q, k, (3, 5), 1, (2, 1), (False, True))
    out = O.na_av(torch.softmax(logits, -1), v, (3, 5), 1, (2, 1), (False, True))
    fused, lse = O.na_forward(q, k, v, (3, 5), 1, (2, 1), (False, True), return_lse=True)
    torch.testing.assert_close(out, fused)
    torch.testing.assert_close(lse, torch.logsumexp(logits, -1))


def test_merge_equals_concatenated_keys():
    # reference tests/test_new_features.py:235-309
    q = _r((1, 6, 2, 4), 1)
    ka, va, kb, vb = (_r((1, n, 2, 4), s) for n, s in ((6, 2), (6, 3), (3, 4), (3, 5)))
    oa, la = O.full_attn_with_lse(q, ka, va, 0.5)
    ob, lb = O.full_attn_with_lse(q, kb, vb, 0.5)
    om, lm = O.merge_attentions([oa, ob], [la, lb])
    oc, lc = O.full_attn_with_lse(q, torch.cat([ka, kb], 1), torch.cat([va, vb], 1), 0.5)
    torch.testing.assert_close(om, oc)
    torch.testing.assert_close(lm, lc)


def test_gqa_equals_explicit_repeat():
    q = _r((1, 9, 4, 3), 1)
    k, v = _r((1, 9, 2, 3), 2), _r((1, 9, 2, 3), 3)
    rep = torch.repeat_interleave
    torch.testing.assert_close(O.na_forward(q, k, v, 3),
                               O.na_forward(q, rep(k, 2, -2), rep(v, 2, -2), 3))


def test_varlen_equals_per_sample_calls():
    q, k, v = _r((3, 12, 2, 4), 1), _r((3, 12, 2, 4), 2), _r((3, 12, 2, 4), 3)
    lens = [12, 7, 5]
    out = O.na_varlen(q, k, v, torch.tensor(lens), 5, 1)
    for b, L in enumerate(lens):
        torch.testing.assert_close(out[b, :L], O.na_forward(q[b:b + 1, :L], k[b:b + 1, :L],
                                                            v[b:b + 1, :L], 5)[0])
        assert (out[b, L:] == 0).all()


@pytest.mark.parametrize("K,d", [(3, 1), (5, 2), (7, 4), (5, 8)])
def test_allin1_qk_rpb_relations(K, d):
    B, L, H, D = 2, 64, 3, 12
    q, k = _r((B, L, H, D), 1), _r((B, L, H, D), 2)
    rpb = _r((H, 2 * K - 1), 3)
    got = O.qk_rpb_1d(q, k, rpb, K, d, scale=0.288)
    # == split QK (core window) + bias at the relative offset (key - i)/d + K - 1
    base = O.na_qk(q, k, K, 1, d, False, 0.288)
    starts = np.array([O.W.window_start(i, L, K, K // 2, d) for i in range(L)])
    rel = (starts[:, None] + np.arange(K)[None, :] * d - np.arange(L)[:, None]) // d + K - 1
    bias = rpb[:, torch.from_numpy(rel)].permute(1, 0, 2)
    torch.testing.assert_close(got, base + bias.unsqueeze(0))
    # rpb = arange known answer (reference tests/test_compat_v014.py:78-102)
    zero = torch.zeros((1, L, 1, 4), dtype=torch.float64)
    ar = torch.arange(2 * K - 1, dtype=torch.float64).reshape(1, -1)
    got0 = O.qk_rpb_1d(zero, zero, ar, K, d)
    torch.testing.assert_close(got0[0, :, 0], torch.from_numpy(rel).to(torch.float64))


@pytest.mark.parametrize("K,d", [(3, 1), (7, 2)])
def test_allin1_av_equals_split_av(K, d):
    B, L, H, D = 2, 40, 2, 12
    a = torch.softmax(_r((B, L, H, K), 1), -1)
    v = _r((B, L, H, D), 2)
    torch.testing.assert_close(O.av_1d(a, v, K, d), O.na_av(a, v, K, 1, d, False))


@pytest.mark.parametrize("K,d,shape", [(3, 1, (9, 11)), (5, 2, (12, 10)), (7, 1, (7, 15)),
                                       (3, 3, (10, 9))])
def test_allin1_2d_qk_rpb_relations(K, d, shape):
    """2D QK+RPB == split 2D QK (legacy windows) + the bias at each axis's
    relative offset, pair index r0*(2K-1)+r1 (reference
    tests/test_extras_allin1.py:35-68); rpb = arange known answer."""
    B, H, D = 2, 2, 12
    Hh, Hw = shape
    q, k = _r((B, Hh, Hw, H, D), 1), _r((B, Hh, Hw, H, D), 2)
    R = 2 * K - 1
    rpb = _r((H, R, R), 3)
    got = O.qk_rpb(q, k, rpb, K, d, scale=0.3)
    base = O.na_qk(q, k, K, 1, d, False, 0.3)

    def rel(L):
        st = np.array([O.W.window_start(i, L, K, K // 2, d) for i in range(L)])
        return (st[:, None] + np.arange(K)[None, :] * d - np.arange(L)[:, None]) // d + K - 1

    r0, r1 = rel(Hh), rel(Hw)
    pair = (r0[:, None, :, None] * R + r1[None, :, None, :]).reshape(Hh, Hw, K * K)
    bias = rpb.reshape(H, R * R)[:, torch.from_numpy(pair)].permute(1, 2, 0, 3)
    torch.testing.assert_close(got, base + bias.unsqueeze(0))
    zero = torch.zeros((1, Hh, Hw, 1, 4), dtype=torch.float64)
    ar = torch.arange(R * R, dtype=torch.float64).reshape(1, R, R)
    got0 = O.qk_rpb(zero, zero, ar, K, d)
    torch.testing.assert_close(got0[0, :, :, 0], torch.from_numpy(pair).to(torch.float64))


@pytest.mark.parametrize("K,d", [(3, 1), (5, 2)])
def test_allin1_2d_av_equals_split_av(K, d):
    B, H, D = 2, 2, 12
    a = torch.softmax(_r((B, 11, 10, H, K * K), 1), -1)
    v = _r((B, 11, 10, H, D), 2)
    torch.testing.assert_close(O.av_rpb(a, v, K, d), O.na_av(a, v, K, 1, d, False))


def test_allin1_partition_edges_beyond_d_times_k():
    """Where d*K > L the partition window can start below zero: those slots
    are invalid (-inf), matching a scalar walk of the partition rule."""
    L, K, d, H, D = 9, 5, 3, 1, 2
    q, k = _r((1, L, H, D), 1), _r((1, L, H, D), 2)
    got = O.qk_rpb(q, k, None, K, d)
    for i in range(L):
        s = O.W.window_start_partition(i, L, K, K // 2, d)
        e = min(L, s + K * d)
        for n in range(K):
            j = s + n * d
            if 0 <= j < e:
                assert got[0, i, 0, n] == (q[0, i, 0] * k[0, j, 0]).sum()
            else:
                assert got[0, i, 0, n] == -math.inf


def test_allin1_backward_matches_finite_differences():
    q, k = _r((1, 6, 5, 2, 3), 1), _r((1, 6, 5, 2, 3), 2)
    rpb = _r((2, 5, 5), 3)
    a, v = torch.softmax(_r((1, 6, 5, 2, 9), 4), -1), _r((1, 6, 5, 2, 3), 5)
    for t in (q, k, rpb, a, v):
        t.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda x, y, z: O.qk_rpb(x, y, z, 3, 2, 0.7).clamp_min(-1e9),
                                    (q, k, rpb))
    assert torch.autograd.gradcheck(lambda x, y: O.av_rpb(x, y, 3, 2), (a, v))


def test_backward_matches_finite_differences():
    q, k, v = _r((1, 5, 4, 2, 3), 1), _r((1, 5, 4, 1, 3), 2), _r((1, 5, 4, 1, 3), 3)
    ek, ev = _r((1, 2, 1, 3), 4), _r((1, 2, 1, 3), 5)
    for t in (q, k, v, ek, ev):
        t.requires_grad_(True)

    def f(q, k, v, ek, ev):
        return O.na_functional(q, k, v, (3, 2), (2, 1), (1, 2), (False, True), 0.6,
                               return_lse=True, additional_keys=ek, additional_values=ev)

    assert torch.autograd.gradcheck(f, (q, k, v, ek, ev), eps=1e-6, atol=1e-7)
    # the oracle's gradient helper returns the same numbers as autograd
    go, gl = _r((1, 3, 4, 2, 3), 6), _r((1, 3, 4, 2), 7)
    g = O.grads(f, (q, k, v, ek, ev), (go, gl))
    out, lse = f(q, k, v, ek, ev)
    ref = torch.autograd.grad((out * go).sum() + (lse * gl).sum(), (q, k, v, ek, ev))
    for a, b in zip(g, ref):
        torch.testing.assert_close(a, b)


def test_split_backward_matches_finite_differences():
    q, k = _r((1, 7, 2, 3), 1).requires_grad_(), _r((1, 7, 2, 3), 2).requires_grad_()
    a = torch.softmax(_r((1, 4, 2, 3), 3), -1).requires_grad_()
    v = _r((1, 7, 2, 3), 4).requires_grad_()

    def qk(q, k):
        x = O.na_qk(q, k, 3, 2, 2, True, 0.5)
        return torch.where(torch.isfinite(x), x, torch.zeros_like(x))

    assert torch.autograd.gradcheck(qk, (q, k), eps=1e-6, atol=1e-7)
    assert torch.autograd.gradcheck(lambda a, v: O.na_av(a, v, 3, 2, 2, True), (a, v),
                                    eps=1e-6, atol=1e-7)
