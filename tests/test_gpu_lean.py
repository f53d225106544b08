"""Lean workgroup kernels (na_lean.hip): parity with the float64 oracle on
problems dispatched to them (asserted through na_kernel_path), covering GQA
with 2 and 4 query heads per key/value head, causal and clipped edge tiles,
a key box wider than 16 (several chunks per box row), ranks 1-3, head_dim
32/64/128, fp16 and bf16, a loss on the LSE (non-zero dlse) and bit-for-bit
repeatability of the backward.  Runs on an MI355X.
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
