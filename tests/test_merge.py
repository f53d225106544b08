"""``merge_attentions`` (reference ``merge.py:20-68``; tests
``tests/test_new_features.py:235-309``).

CPU: argument validation and messages, the loud failure on CPU tensors, and
the closed form the kernel evaluates (logsumexp weights) against the
oracle's sequential sigmoid form.  GPU: the fused merge kernels against the
oracle (forward, gradients of every part's output and LSE, with and without
an LSE cotangent), 2..11 parts (chunked past 8), mixed dtypes, odd head
dims, idempotence at a config-2 size, and the end-to-end identity
merge(NA(q; k, v), Attn(q; extra)) == NA with additional keys.
Tolerance: the fp32 bar (1e-5 relative), bf16/fp16 2e-2 absolute."""

import sys

import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import na as O


def _merge():
    from natten_amd import merge_attentions

    return merge_attentions


# ---------------------------------------------------------------- CPU checks

def test_validation_messages():
    m = _merge()
    o, l = torch.zeros(2, 5, 3, 8), torch.zeros(2, 5, 3)
    with pytest.raises(ValueError, match="at least two outputs"):
        m([o], [l])
    with pytest.raises(ValueError, match="Number of outputs and LSE tensors must match"):
        m([o, o], [l])
    with pytest.raises(ValueError, match="Output 1 shape"):
        m([o, torch.zeros(2, 5, 3, 4)], [l, l])
    with pytest.raises(ValueError, match="LSE 1 shape"):
        m([o, o], [l, torch.zeros(2, 5)])


def test_cpu_tensors_fail_loudly():
    o, l = torch.zeros(2, 5, 3, 8), torch.zeros(2, 5, 3)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        _merge()([o, o], [l, l])


@pytest.mark.parametrize("n", [2, 3, 9])
def test_closed_form_equals_sigmoid_form(n):
    """L = logsumexp(lse_i), out = sum exp(lse_i - L) out_i reproduces the
    reference's sequential sigmoid merge (what the kernels rely on)."""
    outs = [randn((3, 7, 2, 5), torch.float64, s) for s in range(n)]
    lses = [randn((3, 7, 2), torch.float64, 100 + s, std=3.0) for s in range(n)]
    ro, rl = O.merge_attentions(outs, lses)
    L = torch.logsumexp(torch.stack(lses), 0)
    w = torch.exp(torch.stack(lses) - L)
    out = (w.unsqueeze(-1) * torch.stack(outs)).sum(0)
    assert torch.allclose(rl.double(), L, atol=1e-12, rtol=1e-12)
    assert torch.allclose(ro.double(), out, atol=1e-12, rtol=1e-12)


# ---------------------------------------------------------------- GPU parity

def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


MERGE_CASES = [
    # (n parts, shape [B, *sp, H, D], dtype, lse cotangent)
    (2, (2, 9, 4, 32), torch.float32, True),
    (3, (2, 6, 5, 3, 64), torch.bfloat16, True),
    (2, (1, 10, 2, 12), torch.bfloat16, False),   # D=12: scalar path for 2-byte types
    (4, (2, 7, 3, 12), torch.float32, True),      # D=12 with 16-byte fp32 accesses
    (8, (1, 33, 4, 128), torch.float16, True),
    (11, (1, 17, 2, 32), torch.float32, True),    # chunked: 8 + 3
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", MERGE_CASES, ids=lambda c: f"n{c[0]}_{c[2]}".replace("torch.", ""))
def test_merge_matches_oracle(case):
    n, shape, dt, with_dlse = case
    _say(f"[case] merge n={n} shape={shape} {dt}")
    outs = [randn(shape, dt, s) for s in range(n)]
    lses = [randn(shape[:-1], torch.float32, 50 + s, std=2.0) for s in range(n)]
    od = [o.to(DEV).requires_grad_(True) for o in outs]
    ld = [l.to(DEV).requires_grad_(True) for l in lses]
    out, lse = _merge()(od, ld)
    assert out.dtype == dt and lse.dtype == torch.float32
    ro, rl = O.merge_attentions(outs, lses)
    tol = torch.float32 if dt == torch.float32 else dt
    assert_close(out, ro, tol, "out")
    assert_close(lse, rl, torch.float32, "lse")
    go = randn(shape, torch.float32, 7)
    gl = randn(shape[:-1], torch.float32, 8) if with_dlse else None
    if with_dlse:
        torch.autograd.backward((out, lse), (go.to(DEV, dt), gl.to(DEV)))
    else:
        out.backward(go.to(DEV, dt))
    cots = (go.to(dt).double(), gl)
    ref = O.grads(lambda *t: O.merge_attentions(list(t[:n]), list(t[n:])),
                  outs + lses, cots)
    for i in range(n):
        assert od[i].grad.dtype == dt
        assert_close(od[i].grad, ref[i], tol, f"d out {i}")
        assert_close(ld[i].grad, ref[n + i], tol, f"d lse {i}")


@pytest.mark.gpu
def test_merge_mixed_dtypes():
    _say("[case] merge mixed dtypes")
    shape = (2, 8, 3, 32)
    outs = [randn(shape, torch.bfloat16, 1), randn(shape, torch.float32, 2)]
    lses = [randn(shape[:-1], torch.bfloat16, 3), randn(shape[:-1], torch.float32, 4)]
    out, lse = _merge()([o.to(DEV) for o in outs], [l.to(DEV) for l in lses])
    assert out.dtype == torch.bfloat16 and lse.dtype == torch.float32
    ro, rl = O.merge_attentions(outs, lses)
    assert_close(out, ro, torch.bfloat16, "out")
    assert_close(lse, rl, torch.float32, "lse")


@pytest.mark.gpu
def test_merge_idempotent_at_config2_size():
    """Merging n copies of one output returns it and lse + log(n) (config 2
    layout [4, 56, 56, 4, 32] bf16)."""
    _say("[case] merge idempotence cfg2")
    shape = (4, 56, 56, 4, 32)
    o = randn(shape, torch.bfloat16, 1).to(DEV)
    l = randn(shape[:-1], torch.float32, 2).to(DEV)
    for n in (2, 3):
        out, lse = _merge()([o] * n, [l] * n)
        assert_close(out, o.float().cpu().double(), torch.bfloat16, f"n={n} out")
        assert_close(lse, (l + torch.log(torch.tensor(float(n)))).cpu().double(),
                     torch.float32, f"n={n} lse")


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=str)
def test_merge_equals_additional_keys(dt):
    """merge(NA(q; k, v), Attn(q; ek, ev)) == NA with additional keys
    (``functional.py:277-292``; ``tests/test_new_features.py:235-309``)."""
    import natten_amd

    _say(f"[case] merge == additional keys {dt}")
    B, sp, H, D, E = 2, (9, 10), 2, 32, 6
    q, k, v = (randn((B,) + sp + (H, D), dt, s).to(DEV) for s in (1, 2, 3))
    ek, ev = (randn((B, E, H, D), dt, s).to(DEV) for s in (4, 5))
    o_na, l_na = natten_amd.na2d(q, k, v, kernel_size=3, return_lse=True)
    # attention over the extra tokens alone: float32 math on the device
    s = torch.einsum("bxyhd,behd->bxyhe", q.float(), ek.float()) * D ** -0.5
    l_ex = torch.logsumexp(s, -1)
    o_ex = torch.einsum("bxyhe,behd->bxyhd", torch.softmax(s, -1), ev.float()).to(dt)
    out, lse = natten_amd.merge_attentions([o_na, o_ex], [l_na, l_ex])
    ref_o, ref_l = natten_amd.na2d(q, k, v, kernel_size=3, return_lse=True,
                                   additional_keys=ek, additional_values=ev)
    tol = torch.float32 if dt == torch.float32 else dt
    assert_close(out, ref_o.cpu().double(), tol, "out")
    assert_close(lse, ref_l.float().cpu().double(), tol, "lse")
