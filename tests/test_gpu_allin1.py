"""DiNAT all-in-one operators on the GPU against the oracle: forward and
backward (q, k, rpb; attn, v), rank 1 and 2, both layouts, even kernel sizes
and windows with d*K > L (reference tests/test_extras_allin1.py; backward
functions extras/allin1/functional_metal.py:2172-2274).  Tolerance: the
fp32 bar (1e-5 relative), bf16/fp16 inputs 2e-2 absolute."""

import sys

import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import na as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _hf(x):
    """spatial-first [B, *L, H, X] -> heads-first [B, H, *L, X]."""
    return x.movedim(-2, 1).contiguous()


def _sf(x):
    return x.movedim(1, -2).contiguous()


def _check_qk_av(q, k, v, rpb, K, d, scale, dtype, tag):
    """Forward and backward of the spatial-first autograd ops vs the oracle."""
    from natten_amd.extras.allin1 import na1d_av_fused, na1d_qk_rpb, na2d_av_fused, na2d_qk_rpb

    rank = q.dim() - 3
    qk_fn, av_fn = (na1d_qk_rpb, na1d_av_fused) if rank == 1 else (na2d_qk_rpb, na2d_av_fused)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k)]
    rp = None if rpb is None else rpb.to(DEV).requires_grad_(True)
    logits = qk_fn(ts[0], ts[1], rp, K, d, scale=scale)
    assert logits.dtype == torch.float32
    ref = O.qk_rpb(q, k, rpb, K, d, scale)
    assert_close(logits, ref, torch.float32 if dtype == torch.float32 else dtype, f"{tag} logits")
    g = randn(logits.shape, torch.float32, 40)
    valid = torch.isfinite(ref)
    g = torch.where(valid, g, torch.zeros_like(g))
    logits.backward(g.to(DEV))
    if rpb is not None:
        refg = O.grads(lambda a, b, c: O.qk_rpb(a, b, c, K, d, scale), (q, k, rpb), (g,))
    else:
        refg = O.grads(lambda a, b: O.qk_rpb(a, b, None, K, d, scale), (q, k), (g,))
    tol_dt = torch.float32 if dtype == torch.float32 else dtype
    assert_close(ts[0].grad, refg[0], tol_dt, f"{tag} dq")
    assert_close(ts[1].grad, refg[1], tol_dt, f"{tag} dk")
    if rpb is not None:
        assert_close(rp.grad, refg[2], torch.float32, f"{tag} drpb")

    attn = torch.softmax(randn(logits.shape, torch.float32, 41), -1)
    a_d = attn.to(DEV).requires_grad_(True)
    v_d = v.to(DEV).requires_grad_(True)
    out = av_fn(a_d, v_d, K, d)
    assert out.dtype == torch.float32
    assert_close(out, O.av_rpb(attn, v, K, d), tol_dt, f"{tag} av")
    go = randn(out.shape, torch.float32, 42)
    out.backward(go.to(DEV))
    ra, rv = O.grads(lambda a, b: O.av_rpb(a, b, K, d), (attn, v), (go,))
    assert_close(a_d.grad, ra, tol_dt, f"{tag} dattn")
    assert_close(v_d.grad, rv, tol_dt, f"{tag} dv")


CASES_1D = [(3, 1), (5, 2), (7, 4), (5, 8), (7, 8), (4, 3), (6, 1), (7, 1)]


@pytest.mark.parametrize("K,d", CASES_1D)
def test_allin1_1d(K, d):
    _say(f"[case] allin1 1d K={K} d={d}")
    B, L, H, D = 2, 256, 12, 12
    q, k, v = (randn((B, L, H, D), torch.float32, s) for s in (1, 2, 3))
    rpb = randn((H, 2 * K - 1), torch.float32, 4, std=0.02)
    _check_qk_av(q, k, v, rpb, K, d, 0.288, torch.float32, f"1d K{K} d{d}")


@pytest.mark.parametrize("B,L,H,D,K,d", [(1, 257, 1, 12, 3, 1), (2, 300, 3, 8, 5, 2),
                                           (1, 129, 1, 4, 3, 1), (3, 77, 5, 16, 7, 1)])
def test_allin1_1d_partial_blocks(B, L, H, D, K, d):
    """Row counts that leave the last block of the rank-1 fp32 kernels
    partly empty, down to a single row (fewer than four weight floats)"""
    _say(f"[case] allin1 1d partial blocks B={B} L={L} H={H} D={D} K={K} d={d}")
    q, k, v = (randn((B, L, H, D), torch.float32, s) for s in (31, 32, 33))
    rpb = randn((H, 2 * K - 1), torch.float32, 34, std=0.02)
    _check_qk_av(q, k, v, rpb, K, d, D ** -0.5, torch.float32, f"1d partial L{L} K{K} d{d}")


# Shapes whose rank-1 blocks of 256, 384 and 512 rows each start inside a
# sequence's clamped first windows with a head above 0 and end inside its
# clamped last windows below the last head (found by enumeration over the
# window rule): a block's staged key rows must then cover the other heads
# of the edge positions, which share those windows.
EDGE_1D = [(2, 86, 9, 12, 7), (3, 109, 7, 12, 5), (3, 29, 9, 8, 7)]


def _plan(B, L, H, D, K, d):
    import ctypes

    from natten_amd._core import _lib

    p = _lib.make_rpb_params(1, B, H, D, (L,), K, d, False, _lib.NA_F32, 0.288)
    plan = _lib.NaRpbPlan()
    assert _lib.load().na_rpb_kernel_plan(ctypes.byref(p), ctypes.byref(plan)) == 0
    return plan


@pytest.mark.parametrize("B,L,H,D,K", EDGE_1D)
def test_allin1_1d_block_edges(B, L, H, D, K):
    from natten_amd._core import _lib

    pl = _plan(B, L, H, D, K, 1)  # the staged kernels and the fused bias partials run
    assert (pl.qk, pl.av, pl.dq, pl.dk, pl.fused_bias) == (_lib.RPB_STAGED,) * 4 + (1,)
    _say(f"[case] allin1 1d block edges B={B} L={L} H={H} D={D} K={K}")
    q, k, v = (randn((B, L, H, D), torch.float32, s) for s in (41, 42, 43))
    rpb = randn((H, 2 * K - 1), torch.float32, 44, std=0.02)
    _check_qk_av(q, k, v, rpb, K, 1, 0.288, torch.float32, f"1d edges L{L} H{H} K{K}")


# Dilations whose contiguous blocks' halos are too wide, so the rows run in
# phase-major order (k_r1p_*): L not a multiple of d (phases of unequal
# length), blocks spanning phases and samples.
PHASE_1D = [(2, 203, 12, 12, 7, 8), (3, 150, 16, 8, 5, 8), (1, 333, 16, 4, 7, 7)]


@pytest.mark.parametrize("B,L,H,D,K,d", PHASE_1D)
def test_allin1_1d_phase_major(B, L, H, D, K, d):
    from natten_amd._core import _lib

    pl = _plan(B, L, H, D, K, d)  # the phase-major kernels run
    assert (pl.qk, pl.av, pl.dq, pl.dattn) == (_lib.RPB_PHASE,) * 4

    _say(f"[case] allin1 1d phase-major B={B} L={L} H={H} D={D} K={K} d={d}")
    q, k, v = (randn((B, L, H, D), torch.float32, s) for s in (51, 52, 53))
    rpb = randn((H, 2 * K - 1), torch.float32, 54, std=0.02)
    _check_qk_av(q, k, v, rpb, K, d, 0.288, torch.float32, f"1d phase L{L} K{K} d{d}")


CASES_2D = [
    # (K, d, Hh, Hw, D)
    (3, 1, 8, 20, 12),
    (5, 1, 8, 36, 12),
    (7, 2, 16, 15, 32),
    (4, 2, 9, 11, 12),
    (5, 3, 11, 16, 64),
]


@pytest.mark.parametrize("K,d,Hh,Hw,D", CASES_2D)
def test_allin1_2d(K, d, Hh, Hw, D):
    _say(f"[case] allin1 2d K={K} d={d} {Hh}x{Hw} D={D}")
    B, H = 2, 3
    q, k, v = (randn((B, Hh, Hw, H, D), torch.float32, s) for s in (5, 6, 7))
    rpb = randn((H, 2 * K - 1, 2 * K - 1), torch.float32, 8, std=0.02)
    _check_qk_av(q, k, v, rpb, K, d, D ** -0.5, torch.float32, f"2d K{K} d{d}")


def test_allin1_no_rpb_and_edge_windows():
    """rpb=None (no bias gradient) and d*K > L, where some slots are invalid."""
    _say("[case] allin1 no rpb / d*K > L")
    q, k, v = (randn((2, 9, 2, 8), torch.float32, s) for s in (9, 10, 11))
    _check_qk_av(q, k, v, None, 5, 3, None, torch.float32, "1d dK>L")
    q2, k2, v2 = (randn((1, 7, 6, 2, 8), torch.float32, s) for s in (12, 13, 14))
    rpb = randn((2, 7, 7), torch.float32, 15)
    _check_qk_av(q2, k2, v2, rpb, 4, 2, 0.5, torch.float32, "2d dK>L")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_allin1_low_precision(dtype):
    _say(f"[case] allin1 {dtype}")
    q, k, v = (randn((2, 64, 4, 32), dtype, s) for s in (16, 17, 18))
    rpb = randn((4, 9), torch.float32, 19, std=0.02)
    _check_qk_av(q, k, v, rpb, 5, 2, 0.2, dtype, f"1d {dtype}")
    q, k, v = (randn((1, 10, 12, 2, 16), dtype, s) for s in (20, 21, 22))
    rpb = randn((2, 5, 5), torch.float32, 23, std=0.02)
    _check_qk_av(q, k, v, rpb, 3, 3, 0.25, dtype, f"2d {dtype}")


def test_allin1_heads_first_functions():
    """natten{1,2}d* (heads-first) and their *_backward against the oracle
    on the permuted tensors; natten2d_qkv_fused == qk -> softmax -> av."""
    from natten_amd.extras.allin1 import functional as F

    _say("[case] allin1 heads-first")
    for rank, sp, K, d in ((1, (40,), 5, 3), (2, (9, 10), 3, 2)):
        q, k, v = (randn((2, *sp, 3, 12), torch.float32, s) for s in (30, 31, 32))
        R = 2 * K - 1
        rpb = randn((3, R) if rank == 1 else (3, R, R), torch.float32, 33)
        qk = F.natten1dqkrpb if rank == 1 else F.natten2dqkrpb
        av = F.natten1dav if rank == 1 else F.natten2dav
        logits = qk(_hf(q).to(DEV), _hf(k).to(DEV), rpb.to(DEV), K, d)
        ref = O.qk_rpb(q, k, rpb, K, d)
        assert_close(_sf(logits), ref, torch.float32, f"hf{rank} logits")
        attn = torch.softmax(ref, -1)
        out = av(_hf(attn).to(DEV), _hf(v).to(DEV), K, d)
        assert_close(_sf(out), O.av_rpb(attn, v, K, d), torch.float32, f"hf{rank} av")
        g = randn(ref.shape, torch.float32, 34)
        qk_b = F.natten1dqkrpb_backward if rank == 1 else F.natten2dqkrpb_backward
        av_b = F.natten1dav_backward if rank == 1 else F.natten2dav_backward
        dq, dk, drpb = qk_b(_hf(g).to(DEV), _hf(q).to(DEV), _hf(k).to(DEV), rpb.to(DEV), K, d)
        rq, rk, rr = O.grads(lambda a, b, c: O.qk_rpb(a, b, c, K, d), (q, k, rpb), (g,))
        assert_close(_sf(dq), rq, torch.float32, f"hf{rank} dq")
        assert_close(_sf(dk), rk, torch.float32, f"hf{rank} dk")
        assert_close(drpb, rr, torch.float32, f"hf{rank} drpb")
        go = randn(v.shape, torch.float32, 35)
        da, dv = av_b(_hf(go).to(DEV), _hf(attn).to(DEV), _hf(v).to(DEV), K, d)
        ra, rv = O.grads(lambda a, b: O.av_rpb(a, b, K, d), (attn, v), (go,))
        assert_close(_sf(da), ra, torch.float32, f"hf{rank} dattn")
        assert_close(_sf(dv), rv, torch.float32, f"hf{rank} dv")
    q, k, v = (randn((1, 8, 9, 2, 12), torch.float32, s) for s in (36, 37, 38))
    rpb = randn((2, 5, 5), torch.float32, 39)
    fused = F.natten2d_qkv_fused(_hf(q).to(DEV), _hf(k).to(DEV), _hf(v).to(DEV), rpb.to(DEV),
                                 3, 1)
    ref = O.av_rpb(torch.softmax(O.qk_rpb(q, k, rpb, 3, 1), -1), v, 3, 1)
    assert_close(_sf(fused), ref, torch.float32, "qkv fused")
    with pytest.raises(ValueError, match="kernel_size \\* dilation"):
        F.natten1dqkrpb(_hf(q[:, 0]).to(DEV), _hf(k[:, 0]).to(DEV), None, 5, 2)


def test_allin1_bias_gradient_deterministic():
    from natten_amd.extras.allin1 import na2d_qk_rpb

    _say("[case] allin1 drpb determinism")
    q, k = (randn((2, 32, 48, 4, 12), torch.float32, s).to(DEV) for s in (50, 51))
    rpb = randn((4, 13, 13), torch.float32, 52).to(DEV)
    g = randn((2, 32, 48, 4, 49), torch.float32, 53).to(DEV)
    res = []
    for _ in range(2):
        r = rpb.clone().requires_grad_(True)
        na2d_qk_rpb(q, k, r, 7, 2, scale=0.3).backward(g)
        res.append(r.grad.clone())
    assert torch.equal(res[0], res[1])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_allin1_1d_low_precision_dilated(dtype):
    """bf16 / fp16 rank-1 at head_dim 12 with d >= 2: the generic kernels
    with the block size the fp32 staged kernels' shapes select (384 rows)."""
    B, L, H, D, K, d = 2, 203, 12, 12, 5, 2
    _say(f"[case] allin1 1d {dtype} B={B} L={L} H={H} D={D} K={K} d={d}")
    q, k, v = (randn((B, L, H, D), dtype, s) for s in (61, 62, 63))
    rpb = randn((H, 2 * K - 1), torch.float32, 64, std=0.02)
    _check_qk_av(q, k, v, rpb, K, d, 0.288, dtype, f"1d {dtype} K{K} d{d}")


@pytest.mark.parametrize("B,L,H,D,K,d", PHASE_1D[:2] + [(2, 2048, 12, 8, 7, 8)])
def test_allin1_backward_pairs_match_separate_launches(B, L, H, D, K, d, monkeypatch):
    """The backward's paired launches (dq with dk and the bias partials,
    dattn with dv) against the same passes as separate launches
    (NATTEN_AMD_RPB_PAIR=0): bit for bit."""
    from natten_amd.extras.allin1 import na1d_av_fused, na1d_qk_rpb

    _say(f"[case] allin1 pairs B={B} L={L} H={H} D={D} K={K} d={d}")
    q, k, v = (randn((B, L, H, D), torch.float32, s).to(DEV) for s in (71, 72, 73))
    rpb = randn((H, 2 * K - 1), torch.float32, 74, std=0.02).to(DEV)
    g = randn((B, L, H, K), torch.float32, 75).to(DEV)
    attn = torch.softmax(randn((B, L, H, K), torch.float32, 76), -1).to(DEV)
    go = randn((B, L, H, D), torch.float32, 77).to(DEV)

    def run():
        ts = [t.detach().clone().requires_grad_(True) for t in (q, k, rpb)]
        gq = torch.autograd.grad(na1d_qk_rpb(ts[0], ts[1], ts[2], K, d, scale=0.3), ts, g)
        a_, v_ = (t.detach().clone().requires_grad_(True) for t in (attn, v))
        ga = torch.autograd.grad(na1d_av_fused(a_, v_, K, d), (a_, v_), go)
        return [*gq, *ga]

    paired = run()
    monkeypatch.setenv("NATTEN_AMD_RPB_PAIR", "0")
    apart = run()
    for a, b, n in zip(paired, apart, ("dq", "dk", "drpb", "dattn", "dv")):
        assert torch.equal(a, b), n
