"""Lean workgroup kernels (na_lean.hip): parity with the float64 oracle on
problems dispatched to them (asserted through na_kernel_path), covering GQA
with 2 and 4 query heads per key/value head, causal and clipped edge tiles,
a key box wider than 16 (several chunks per box row), ranks 1-3, head_dim
32/64/128, fp16 and bf16, a loss on the LSE (non-zero dlse) and bit-for-bit
repeatability of the backward; and the lean forward of varlen problems
(per-sample extents, padded rows zero) and of additional tokens, ranks 1-3,
against the oracle per sample and against the 32-query kernels on the
padded rows.  Runs on an MI355X.
"""

import sys

import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import na as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


CASES = [
    # (name, B, spatial, H, Hkv, D, ks, dil, caus)
    ("2d_gqa_rep2", 2, (19, 23), 4, 2, 32, (5, 7), (1, 2), (False, False)),
    ("2d_causal_edge", 1, (13, 29), 2, 2, 64, (3, 9), (2, 1), (True, False)),
    ("2d_k17_wide", 1, (12, 40), 2, 2, 32, (3, 17), (1, 2), (False, False)),
    ("3d_small", 1, (5, 9, 10), 2, 1, 32, (3, 3, 5), (1, 2, 1), (True, False, False)),
    ("1d_gqa", 2, (150,), 8, 2, 64, (15,), (3,), (False,)),
    ("2d_d128", 1, (14, 18), 2, 2, 128, (5, 5), (1, 1), (False, False)),
    ("2d_d64_gqa4", 1, (24, 20), 8, 2, 64, (7, 5), (2, 3), (False, True)),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_lean_parity(case, dtype):
    import natten_amd
    from natten_amd._core import hip

    name, B, sp, H, Hkv, D, ks, dil, caus = case
    _say(f"[case] lean {name} {dtype}")
    fn = {1: natten_amd.na1d, 2: natten_amd.na2d, 3: natten_amd.na3d}[len(sp)]
    q = randn((B, *sp, H, D), dtype, 11)
    k = randn((B, *sp, Hkv, D), dtype, 12)
    v = randn((B, *sp, Hkv, D), dtype, 13)
    go = randn((B, *sp, H, D), dtype, 14)
    gl = randn((B, *sp, H), dtype, 15)  # the LSE comes back in the input dtype
    st = (1,) * len(sp)
    assert hip.kernel_path(q, k, ks, st, dil, caus) == "lean"
    assert hip.kernel_path(q, k, ks, st, dil, caus, backward=True) == "lean"
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out, lse = fn(*ts, kernel_size=ks, dilation=dil, is_causal=caus, return_lse=True)
    # loss = <out, go> + <lse, gl>: the backward sees a non-zero dlse
    torch.autograd.backward((out, lse), (go.to(DEV), gl.to(DEV)))
    ref_out, ref_lse = O.na_functional(q, k, v, ks, 1, dil, caus, return_lse=True)
    assert_close(out, ref_out, dtype, f"{name} out")
    assert_close(lse, ref_lse, dtype, f"{name} lse")

    def loss_terms(a, b, c):
        o, l = O.na_functional(a, b, c, ks, 1, dil, caus, return_lse=True)
        return o, l

    ref = O.grads(loss_terms, (q, k, v), (go, gl))
    for t, r, nm in zip(ts, ref, ("dq", "dk", "dv")):
        assert_close(t.grad, r, dtype, f"{name} {nm}")


def test_lean_backward_repeatable():
    """Two backward passes give identical bits (no atomics, fixed order)."""
    import natten_amd
    from natten_amd._core import hip

    _say("[case] lean determinism")
    q, k, v = (randn((2, 21, 27, 4, 32), torch.bfloat16, s) for s in (1, 2, 3))
    assert hip.kernel_path(q, k, (7, 5), (1, 1), (1, 2), (False, False), backward=True) == "lean"
    res = []
    for _ in range(2):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
        out = natten_amd.na2d(*ts, (7, 5), dilation=(1, 2))
        out.backward(torch.ones_like(out))
        res.append([t.grad.clone() for t in ts])
    for a, b in zip(*res):
        assert torch.equal(a, b)


VX_CASES = [
    # (name, B, spatial, H, Hkv, D, ks, dil, caus, sizes or None, n_extra)
    ("1d_varlen_gqa_extra", 3, (300,), 8, 2, 64, (15,), (2,), (False,),
     [[300], [137], [30]], 5),
    ("1d_varlen_short", 2, (256,), 4, 4, 32, (9,), (1,), (False,), [[9], [200]], 0),
    ("2d_varlen", 3, (20, 24), 2, 2, 32, (7, 5), (1, 1), (False, False),
     [[20, 24], [13, 17], [7, 9]], 0),
    ("2d_extra_d128", 2, (9, 14), 4, 1, 128, (3, 5), (2, 1), (False, True), None, 40),
    ("2d_extra_causal_gqa", 2, (11, 10), 4, 2, 32, (3, 5), (2, 1), (False, True), None, 21),
    ("3d_varlen_extra", 2, (6, 10, 12), 2, 1, 64, (3, 3, 5), (1, 2, 1), (False, False, False),
     [[6, 10, 12], [3, 7, 5]], 3),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", VX_CASES, ids=[c[0] for c in VX_CASES])
def test_lean_varlen_and_extra_forward(case, dtype):
    from natten_amd._core import hip

    name, B, sp, H, Hkv, D, ks, dil, caus, sizes, nx = case
    _say(f"[case] lean vx {name} {dtype}")
    rank = len(sp)
    q = randn((B, *sp, H, D), dtype, 41)
    k = randn((B, *sp, Hkv, D), dtype, 42)
    v = randn((B, *sp, Hkv, D), dtype, 43)
    ek = randn((B, nx, Hkv, D), dtype, 44) if nx else None
    ev = randn((B, nx, Hkv, D), dtype, 45) if nx else None
    se = None if sizes is None else torch.tensor(sizes, dtype=torch.int32)
    st = (1,) * rank
    assert hip.kernel_path(q, k, ks, st, dil, caus, n_extra=nx, sample_extent=se,
                           varlen_clamped=True) == "lean"
    dev = [None if t is None else t.to(DEV) for t in (q, k, v, ek, ev, se)]

    def run():
        return hip.fused_forward(dev[0], dev[1], dev[2], ks, st, dil, caus, None,
                                 extra_k=dev[3], extra_v=dev[4], sample_extent=dev[5],
                                 varlen_clamped=True)

    out, lse = run()
    with hip.no_lean_kernels():
        out1, lse1 = run()
    for b in range(B):
        ext = sp if sizes is None else tuple(sizes[b])
        sl = (slice(b, b + 1),) + tuple(slice(0, e) for e in ext)
        xk = None if ek is None else ek[b:b + 1]
        xv = None if ev is None else ev[b:b + 1]
        ro, rl = O.na_functional(q[sl], k[sl], v[sl], ks, 1, dil, caus, return_lse=True,
                                 additional_keys=xk, additional_values=xv)
        assert_close(out[sl], ro, dtype, f"{name} out b{b}")
        assert_close(lse[sl].to(dtype), rl, dtype, f"{name} lse b{b}")
    # padded rows: zero output and lse 0, as on the 32-query kernels
    pad = torch.ones((B, *sp), dtype=torch.bool)
    if sizes is not None:
        for b in range(B):
            pad[(b,) + tuple(slice(0, e) for e in sizes[b])] = False
    else:
        pad[:] = False
    pad = pad.to(DEV)
    assert (out[pad] == 0).all() and (lse[pad] == 0).all()
    assert (out1[pad] == 0).all() and (lse1[pad] == 0).all()
    assert_close(out, out1.cpu(), dtype, f"{name} lean vs mfma")
