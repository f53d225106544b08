"""Seeded sweep of the lean workgroup kernels over random problems of their
class (ranks 1-3, odd kernels with d*K <= L on every axis, causal axes,
GQA, head_dim 32/64/128, bf16/fp16), forward + LSE + backward against the
float64 oracle; and the lean forward with per-sample extents and additional
tokens.  Every case asserts it ran on the lean kernels.  Runs on an MI355X.
"""

import random
import sys

import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import na as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _problem(rng):
    rank = rng.choice((1, 1, 2, 2, 2, 3))
    ks, dil, caus, sp = [], [], [], []
    for a in range(rank):
        causal = rng.random() < 0.25
        K = rng.choice((3, 5, 7) if rank < 3 else (3, 5))
        d = rng.choice((1, 1, 2, 3))
        hi = 40 if rank == 1 else 20 if rank == 2 else 10
        L = rng.randint(min(d * K, hi), hi)
        if d * K > L:  # the API requires d * K <= L on every axis
            d = 1
        ks.append(K)
        dil.append(d)
        caus.append(causal)
        sp.append(L)
    if rank == 1:
        sp = [rng.randint(max(ks[0] * dil[0], 20), 300)]
    hkv = rng.choice((1, 2))
    H = hkv * rng.choice((1, 2, 4))
    D = rng.choice((32, 64, 128))
    dtype = rng.choice((torch.bfloat16, torch.float16))
    B = rng.choice((1, 2))
    return B, tuple(sp), H, hkv, D, tuple(ks), tuple(dil), tuple(caus), dtype


CASES = [_problem(random.Random(1000 + i)) for i in range(24)]


@pytest.mark.parametrize("case", CASES, ids=[f"p{i}" for i in range(len(CASES))])
def test_lean_random_problem(case):
    import natten_amd
    from natten_amd._core import hip

    B, sp, H, Hkv, D, ks, dil, caus, dtype = case
    _say(f"[case] lean sweep {case}")
    st = (1,) * len(sp)
    q = randn((B, *sp, H, D), dtype, 51)
    k = randn((B, *sp, Hkv, D), dtype, 52)
    v = randn((B, *sp, Hkv, D), dtype, 53)
    go = randn((B, *sp, H, D), dtype, 54)
    gl = randn((B, *sp, H), dtype, 55)
    if hip.kernel_path(q, k, ks, st, dil, caus) != "lean":
        pytest.skip("outside the lean class (LDS budget)")
    fn = {1: natten_amd.na1d, 2: natten_amd.na2d, 3: natten_amd.na3d}[len(sp)]
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out, lse = fn(*ts, kernel_size=ks, dilation=dil, is_causal=caus, return_lse=True)
    torch.autograd.backward((out, lse), (go.to(DEV), gl.to(DEV)))
    ref_out, ref_lse = O.na_functional(q, k, v, ks, 1, dil, caus, return_lse=True)
    assert_close(out, ref_out, dtype, "out")
    assert_close(lse, ref_lse, dtype, "lse")
    lean_bwd = hip.kernel_path(q, k, ks, st, dil, caus, backward=True) == "lean"
    ref = O.grads(lambda a, b, c: O.na_functional(a, b, c, ks, 1, dil, caus, return_lse=True),
                  (q, k, v), (go, gl))
    for t, r, nm in zip(ts, ref, ("dq", "dk", "dv")):
        assert_close(t.grad, r, dtype, f"{nm} (lean backward: {lean_bwd})")


def _vx_problem(rng):
    rank = rng.choice((1, 1, 2))
    ks, dil, sp = [], [], []
    for a in range(rank):
        K = rng.choice((3, 5, 7, 9))
        d = rng.choice((1, 2))
        L = rng.randint(d * K + 4, 64 if rank == 2 else 200)
        ks.append(K)
        dil.append(d)
        sp.append(L)
    B = rng.choice((2, 3))
    sizes = [[rng.randint(d * K, L) for K, d, L in zip(ks, dil, sp)] for _ in range(B)]
    sizes[0] = list(sp)
    nx = rng.choice((0, 1, 5, 16, 33))
    hkv = rng.choice((1, 2))
    return (B, tuple(sp), hkv * rng.choice((1, 2)), hkv, rng.choice((32, 64)), tuple(ks),
            tuple(dil), sizes, nx, rng.choice((torch.bfloat16, torch.float16)))


VX_CASES = [_vx_problem(random.Random(2000 + i)) for i in range(12)]


@pytest.mark.parametrize("case", VX_CASES, ids=[f"v{i}" for i in range(len(VX_CASES))])
def test_lean_random_varlen_extra_forward(case):
    from natten_amd._core import hip

    B, sp, H, Hkv, D, ks, dil, sizes, nx, dtype = case
    _say(f"[case] lean vx sweep {case}")
    rank = len(sp)
    caus = (False,) * rank
    st = (1,) * rank
    q = randn((B, *sp, H, D), dtype, 61)
    k = randn((B, *sp, Hkv, D), dtype, 62)
    v = randn((B, *sp, Hkv, D), dtype, 63)
    ek = randn((B, nx, Hkv, D), dtype, 64) if nx else None
    ev = randn((B, nx, Hkv, D), dtype, 65) if nx else None
    se = torch.tensor(sizes, dtype=torch.int32)
    assert hip.kernel_path(q, k, ks, st, dil, caus, n_extra=nx, sample_extent=se,
                           varlen_clamped=True) == "lean"
    dev = [None if t is None else t.to(DEV) for t in (q, k, v, ek, ev, se)]
    out, lse = hip.fused_forward(dev[0], dev[1], dev[2], ks, st, dil, caus, None,
                                 extra_k=dev[3], extra_v=dev[4], sample_extent=dev[5],
                                 varlen_clamped=True)
    for b in range(B):
        sl = (slice(b, b + 1),) + tuple(slice(0, e) for e in sizes[b])
        ro, rl = O.na_functional(q[sl], k[sl], v[sl], ks, 1, dil, caus, return_lse=True,
                                 additional_keys=None if ek is None else ek[b:b + 1],
                                 additional_values=None if ev is None else ev[b:b + 1])
        assert_close(out[sl], ro, dtype, f"out b{b}")
        assert_close(lse[sl].to(dtype), rl, dtype, f"lse b{b}")
        pad = torch.ones(sp, dtype=torch.bool)
        pad[tuple(slice(0, e) for e in sizes[b])] = False
        pad = pad.to(DEV)
        assert (out[b][pad] == 0).all() and (lse[b][pad] == 0).all()


SPLIT_CASES = [_problem(random.Random(3000 + i)) for i in range(12)]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[f"s{i}" for i in range(len(SPLIT_CASES))])
def test_lean_random_split_ops(case):
    """Split QK / AV forward and all four gradients on the lean split
    kernels (k_lqk, k_lav, k_linv) against the oracle."""
    import natten_amd
    from natten_amd._core import hip

    B, sp, H, Hkv, D, ks, dil, caus, dtype = case
    _say(f"[case] lean split sweep {case}")
    rank = len(sp)
    q = randn((B, *sp, H, D), dtype, 71)
    k = randn((B, *sp, Hkv, D), dtype, 72)
    v = randn((B, *sp, Hkv, D), dtype, 73)
    if hip.kernel_path(q, k, ks, (1,) * rank, dil, caus, split=True) != "lean":
        pytest.skip("outside the lean split class (LDS budget)")
    qk = {1: natten_amd.na1d_qk, 2: natten_amd.na2d_qk, 3: natten_amd.na3d_qk}[rank]
    av = {1: natten_amd.na1d_av, 2: natten_amd.na2d_av, 3: natten_amd.na3d_av}[rank]
    ref_logits = O.na_qk(q, k, ks, 1, dil, caus, 0.3)
    finite = torch.isfinite(ref_logits)
    attn = torch.softmax(ref_logits, -1).to(dtype)
    gl = randn(ref_logits.shape, dtype, 74)
    go = randn((B, *sp, H, D), dtype, 75)

    def qk_masked(a, b):
        x = O.na_qk(a, b, ks, 1, dil, caus, 0.3)
        return torch.where(finite, x, torch.zeros_like(x))

    rq, rk = O.grads(qk_masked, (q, k), (gl,))
    ra, rv = O.grads(lambda a, b: O.na_av(a, b, ks, 1, dil, caus), (attn, v), (go,))
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    logits = qk(qd, kd, ks, dil, is_causal=caus, scale=0.3)
    assert torch.equal(torch.isinf(logits).cpu(), ~finite), "mask"
    assert_close(logits, ref_logits, dtype, "logits")
    ad = attn.to(DEV).requires_grad_(True)
    out = av(ad, vd, ks, dil, is_causal=caus)
    assert_close(out, O.na_av(attn, v, ks, 1, dil, caus), dtype, "av")
    logits.backward(gl.to(DEV))
    out.backward(go.to(DEV))
    assert_close(qd.grad, rq, dtype, "dq")
    assert_close(kd.grad, rk, dtype, "dk")
    assert_close(ad.grad, ra, dtype, "dattn")
    assert_close(vd.grad, rv, dtype, "dv")


def _vx3_problem(rng):
    # rank 3 (boxes staged in slabs along the first axis), per-sample extents
    ks, dil, sp = [], [], []
    for a in range(3):
        K = rng.choice((3, 5))
        d = rng.choice((1, 1, 2))
        L = rng.randint(d * K + 2, 14)
        ks.append(K)
        dil.append(d)
        sp.append(L)
    B = 2
    sizes = [list(sp), [rng.randint(d * K, L) for K, d, L in zip(ks, dil, sp)]]
    hkv = rng.choice((1, 2))
    return (B, tuple(sp), hkv * rng.choice((1, 2)), hkv, rng.choice((32, 64)), tuple(ks),
            tuple(dil), sizes, rng.choice((0, 3, 17)), rng.choice((torch.bfloat16, torch.float16)))


VXB_CASES = ([_vx_problem(random.Random(4000 + i)) for i in range(12)]
             + [_vx3_problem(random.Random(4100 + i)) for i in range(4)]
             # a rank-3 box beyond the LDS budget: staged in slabs
             + [(2, (8, 24, 24), 4, 2, 64, (3, 7, 7), (1, 1, 1), [[8, 24, 24], [6, 20, 17]], 0,
                 torch.bfloat16)])


@pytest.mark.parametrize("case", VXB_CASES, ids=[f"b{i}" for i in range(len(VXB_CASES))])
def test_lean_random_varlen_extra_backward(case):
    """The lean backward with per-sample extents and additional tokens: dq,
    dk, dv (zero outside each sample) and the additional tokens' gradients,
    against the oracle run per sample, with upstream gradients on out and
    lse."""
    from natten_amd._core import hip

    B, sp, H, Hkv, D, ks, dil, sizes, nx, dtype = case
    _say(f"[case] lean vx backward sweep {case}")
    rank = len(sp)
    caus = (False,) * rank
    st = (1,) * rank
    q = randn((B, *sp, H, D), dtype, 161)
    k = randn((B, *sp, Hkv, D), dtype, 162)
    v = randn((B, *sp, Hkv, D), dtype, 163)
    ek = randn((B, nx, Hkv, D), dtype, 164) if nx else None
    ev = randn((B, nx, Hkv, D), dtype, 165) if nx else None
    go = randn((B, *sp, H, D), dtype, 166)
    gl = randn((B, *sp, H), torch.float32, 167)
    se = torch.tensor(sizes, dtype=torch.int32)
    assert hip.kernel_path(q, k, ks, st, dil, caus, n_extra=nx, sample_extent=se,
                           varlen_clamped=True, backward=True) == "lean"
    dev = [None if t is None else t.to(DEV) for t in (q, k, v, ek, ev, se)]
    out, lse = hip.fused_forward(dev[0], dev[1], dev[2], ks, st, dil, caus, None,
                                 extra_k=dev[3], extra_v=dev[4], sample_extent=dev[5],
                                 varlen_clamped=True)
    dq, dk, dv, dek, dvx = hip.fused_backward(
        dev[0], dev[1], dev[2], out, lse, go.to(DEV), gl.to(DEV), ks, st, dil, caus, None,
        extra_k=dev[3], extra_v=dev[4], sample_extent=dev[5], varlen_clamped=True)
    ref = [torch.zeros(t.shape, dtype=torch.float64) for t in (q, k, v)]
    rx = [torch.zeros((B, nx, Hkv, D), dtype=torch.float64) for _ in range(2)]
    for b in range(B):
        sl = (slice(b, b + 1),) + tuple(slice(0, e) for e in sizes[b])
        ins = (q[sl], k[sl], v[sl]) + ((ek[b:b + 1], ev[b:b + 1]) if nx else ())

        def f(a, c, d, *x):
            return O.na_functional(a, c, d, ks, 1, dil, caus, return_lse=True,
                                   additional_keys=x[0] if x else None,
                                   additional_values=x[1] if x else None)

        g = O.grads(f, ins, (go[sl], gl[sl]))
        for r, gg in zip(ref, g[:3]):
            r[sl] = gg.to(torch.float64)
        if nx:
            rx[0][b:b + 1] = g[3].to(torch.float64)
            rx[1][b:b + 1] = g[4].to(torch.float64)
    for t, r, nm in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert_close(t, r, dtype, nm)
    if nx:
        assert_close(dek, rx[0], dtype, "dek")
        assert_close(dvx, rx[1], dtype, "dev")


@pytest.mark.parametrize("case", [c for c in VX_CASES if c[2] > c[3]],
                         ids=lambda c: f"rep{c[2] // c[3]}")
def test_lean_grouped_heads_forward(case, monkeypatch):
    """The varlen / extra-token forward with every query head of a group run
    over one staged box (NATTEN_AMD_HL=1; chosen automatically for large
    launches) equals the per-head launch bit for bit."""
    from natten_amd._core import hip

    B, sp, H, Hkv, D, ks, dil, sizes, nx, dtype = case
    _say(f"[case] lean grouped heads {case}")
    rank = len(sp)
    q = randn((B, *sp, H, D), dtype, 61).to(DEV)
    k = randn((B, *sp, Hkv, D), dtype, 62).to(DEV)
    v = randn((B, *sp, Hkv, D), dtype, 63).to(DEV)
    ek = randn((B, nx, Hkv, D), dtype, 64).to(DEV) if nx else None
    ev = randn((B, nx, Hkv, D), dtype, 65).to(DEV) if nx else None
    se = torch.tensor(sizes, dtype=torch.int32).to(DEV)
    res = []
    rep = H // Hkv
    # per-head launch, every head of the group per workgroup, and (rep 4) two
    flags = [("0", None), ("1", None)] + ([("1", "2")] if rep % 2 == 0 and rep > 2 else [])
    for flag, heads in flags:
        monkeypatch.setenv("NATTEN_AMD_HL", flag)
        if heads is None:
            monkeypatch.delenv("NATTEN_AMD_HL_HEADS", raising=False)
        else:
            monkeypatch.setenv("NATTEN_AMD_HL_HEADS", heads)
        res.append(hip.fused_forward(q, k, v, ks, (1,) * rank, dil, (False,) * rank, None,
                                     extra_k=ek, extra_v=ev, sample_extent=se,
                                     varlen_clamped=True))
    for r in res[1:]:
        assert torch.equal(res[0][0], r[0]) and torch.equal(res[0][1], r[1])


PAIR_CASES = [
    ((2, 24, 20), 4, 4, 32, 7, 1, torch.bfloat16),   # config-2-like: the pairs apply
    ((2, 30, 18), 4, 2, 64, 5, 2, torch.float16),    # GQA, dilation
    ((3, 70), 4, 4, 32, 9, 3, torch.bfloat16),       # rank 1
]


@pytest.mark.parametrize("case", PAIR_CASES, ids=[f"p{i}" for i in range(len(PAIR_CASES))])
def test_split_backward_pair_matches_separate_launches(case, monkeypatch):
    """The split backward's paired launch (dq + dk, dattn + dv in one
    launch) against the two passes launched separately, bit for bit."""
    from natten_amd._core import hip

    bs, H, Hkv, D, K, d, dtype = case
    _say(f"[case] split pair {case}")
    rank = len(bs) - 1
    sp = bs[1:]
    ks, dil, st, ca = (K,) * rank, (d,) * rank, (1,) * rank, (False,) * rank
    q = randn((bs[0], *sp, H, D), dtype, 81).to(DEV)
    k = randn((bs[0], *sp, Hkv, D), dtype, 82).to(DEV)
    v = randn((bs[0], *sp, Hkv, D), dtype, 83).to(DEV)
    assert hip.kernel_path(q, k, ks, st, dil, ca, split=True) == "lean"
    kp = K ** rank
    dl = randn((bs[0], *sp, H, kp), dtype, 84).to(DEV)
    attn = torch.softmax(randn((bs[0], *sp, H, kp), torch.float32, 85), -1).to(dtype).to(DEV)
    do = randn((bs[0], *sp, H, D), dtype, 86).to(DEV)

    def run():
        a = hip.qk_backward(q, k, dl, ks, st, dil, ca, 0.3)
        b = hip.av_backward(attn, v, do, ks, st, dil, ca)
        torch.cuda.synchronize()
        return [*a, *b]

    paired = run()
    monkeypatch.setenv("NATTEN_AMD_SPLIT_PAIR", "0")
    separate = run()
    for a, b in zip(paired, separate):
        assert torch.equal(a, b)


VQK_CASES = [
    # (B, spatial, H, D, K, dilation, dtype)
    (4, (56, 56), 4, 32, 7, (1, 1), torch.bfloat16),
    (4, (56, 56), 4, 32, 7, (4, 4), torch.bfloat16),
    (2, (19, 23), 2, 64, 5, (3, 2), torch.float16),
    (1, (9, 12), 8, 32, 3, (1, 3), torch.bfloat16),
]


@pytest.mark.parametrize("case", VQK_CASES, ids=[f"v{i}" for i in range(len(VQK_CASES))])
def test_valu_split_qk_against_oracle(case, monkeypatch):
    """The vector-ALU gather kernel for the split QK (k_vqk, opt-in with
    NATTEN_AMD_VSPLIT=1; the matrix-core k_lqh is the default) against the
    oracle, with partial tiles, both dilated axes and head_dim 64."""
    import natten_amd

    B, sp, H, D, K, dil, dtype = case
    _say(f"[case] valu split qk {case}")
    monkeypatch.setenv("NATTEN_AMD_VSPLIT", "1")
    q = randn((B, *sp, H, D), dtype, 81)
    k = randn((B, *sp, H, D), dtype, 82)
    ref = O.na_qk(q, k, (K, K), 1, dil, (False, False), 0.3)
    got = natten_amd.na2d_qk(q.to(DEV), k.to(DEV), K, dil, scale=0.3)
    assert_close(got, ref, dtype, "valu qk logits")
