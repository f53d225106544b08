"""The fused op's C++ autograd node (torch.ops.natten_amd.na_fused) against
the Python autograd Function over the same kernels: outputs, LSE and every
gradient bit for bit, across ranks, dtypes, GQA, additional tokens, varlen,
the dense mode and a strided (generic-kernel) problem; graph capture of a
step through the operator; and a check against the float64 oracle."""

from __future__ import annotations

import pytest
import torch

from _helpers import DEV, assert_close, randn

pytestmark = pytest.mark.gpu


def _run(fn, tensors, grads):
    """fn(*tensors) -> (out, lse); backward of sum(out*g0) + sum(lse*g1)."""
    ts = [t.detach().clone().requires_grad_(True) for t in tensors]
    out, lse = fn(*ts)
    loss = (out.float() * grads[0]).sum() + (lse.float() * grads[1]).sum()
    gs = torch.autograd.grad(loss, ts)
    return out, lse, gs


def _both(fn, tensors, grads):
    import natten_amd.autograd.fused as F

    a = _run(fn, tensors, grads)
    with F.python_autograd():
        b = _run(fn, tensors, grads)
    return a, b


def _node_name(t):
    return t.grad_fn.name() if t.grad_fn is not None else ""


CASES = [
    # rank, batch/spatial, heads, kv heads, dim, dtype, kernel, dilation, causal, extras
    ("2d-bf16-cfg2like", (2, 20, 24), 4, 4, 32, torch.bfloat16, 7, 2, False, 0),
    ("1d-fp16-gqa-extra", (2, 96), 8, 2, 64, torch.float16, 9, 3, False, 5),
    ("3d-bf16-causal", (1, 6, 10, 12), 2, 2, 32, torch.bfloat16, (3, 5, 5), 1, (True, False, False), 0),
    ("2d-fp32", (1, 12, 13), 2, 1, 16, torch.float32, 5, 1, False, 3),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_op_matches_python_function(case):
    import natten_amd

    _, bs, H, Hkv, D, dt, ks, dil, caus, nx = case
    rank = len(bs) - 1
    q = randn((*bs, H, D), dt, 1).to(DEV)
    k = randn((*bs, Hkv, D), dt, 2).to(DEV)
    v = randn((*bs, Hkv, D), dt, 3).to(DEV)
    extra = []
    if nx:
        extra = [randn((bs[0], nx, Hkv, D), dt, s).to(DEV) for s in (4, 5)]
    fn_na = getattr(natten_amd, f"na{rank}d")

    def fn(q_, k_, v_, *ex):
        kw = dict(additional_keys=ex[0], additional_values=ex[1]) if ex else {}
        return fn_na(q_, k_, v_, ks, dilation=dil, is_causal=caus, return_lse=True, **kw)

    out0, lse0 = fn(q, k, v, *extra)
    g = (randn(out0.shape, torch.float32, 6).to(DEV), randn(lse0.shape, torch.float32, 7).to(DEV))
    (o1, l1, g1), (o2, l2, g2) = _both(fn, [q, k, v, *extra], g)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
    # the operator's node runs in C++, the A/B path's in Python
    import natten_amd.autograd.fused as F

    ts = [t.detach().clone().requires_grad_(True) for t in (q, k, v, *extra)]
    assert "CppNode" in _node_name(fn(*ts)[0])
    with F.python_autograd():
        assert "CppNode" not in _node_name(fn(*ts)[0])


def test_op_varlen_and_generic_paths():
    """Varlen (sample extents through the operator) and a strided problem
    (generic kernels), A/B against the Python Function."""
    import natten_amd

    q, k, v = (randn((3, 40, 4, 32), torch.bfloat16, s).to(DEV) for s in (1, 2, 3))
    lens = torch.tensor([40, 23, 31], dtype=torch.int32)
    g = randn((3, 40, 4, 32), torch.float32, 4).to(DEV)

    def run(fn):
        ts = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
        out = fn(*ts)
        return (out, *torch.autograd.grad((out.float() * g[:, :out.shape[1]]).sum(), ts))

    import natten_amd.autograd.fused as F

    for fn in (lambda a, b, c: natten_amd.na1d_varlen(a, b, c, lens, kernel_size=7, dilation=2),
               lambda a, b, c: natten_amd.na1d(a, b, c, kernel_size=5, stride=2)):
        r1 = run(fn)
        with F.python_autograd():
            r2 = run(fn)
        for a, b in zip(r1, r2):
            assert torch.equal(a, b)


def test_op_against_oracle_and_graph_capture():
    """The operator's step against the float64 oracle, then the same step
    captured in a HIP graph and replayed: every replay equals eager."""
    import natten_amd
    from oracle import na as O

    shape = (2, 14, 14, 2, 32)
    qc, kc, vc, gc = (randn(shape, torch.bfloat16, s) for s in (1, 2, 3, 4))
    q, k, v = (t.to(DEV).requires_grad_(True) for t in (qc, kc, vc))
    go = gc.to(DEV)

    def step():
        out = natten_amd.na2d(q, k, v, 7, dilation=2)
        return (out, *torch.autograd.grad(out, (q, k, v), go))

    eager = [t.detach().clone() for t in step()]
    ref = O.na_forward(qc, kc, vc, 7, 1, 2)
    refg = O.grads(lambda a, b, c: O.na_forward(a, b, c, 7, 1, 2), (qc, kc, vc), (gc,))
    assert_close(eager[0], ref, torch.bfloat16, "op out")
    for t, r, n in zip(eager[1:], refg, "qkv"):
        assert_close(t, r, torch.bfloat16, f"op d{n}")

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        step()  # eager work between replays
        torch.cuda.synchronize()
        for a, b in zip(static, eager):
            assert torch.equal(a, b)


def test_operator_library_loaded():
    """The operator library is built beside libnatten_amd.so and registered,
    so the functional API takes it."""
    from natten_amd._core import _lib

    assert _lib.fused_op() is not None


def test_op_edge_cases():
    """Non-contiguous inputs, gradients for some inputs only, a loss on the
    LSE alone (no gradient reaches out) and an empty batch, each through the
    operator against the Python Function."""
    import natten_amd
    import natten_amd.autograd.fused as F

    base = randn((2, 18, 16, 4, 32), torch.bfloat16, 1).to(DEV)
    # a permuted view: [B, X, Y, H, D] seen through a transpose of X and Y
    q = base.transpose(1, 2)
    k = randn((2, 16, 18, 4, 32), torch.bfloat16, 2).to(DEV)
    v = randn((2, 16, 18, 4, 32), torch.bfloat16, 3).to(DEV)
    assert not q.is_contiguous()

    def run(which, lse_only):
        ts = [t.detach().clone() for t in (q, k, v)]
        ts[0] = q.detach()  # keep the non-contiguous view
        for i in which:
            ts[i].requires_grad_(True)
        out, lse = natten_amd.na2d(*ts, 5, dilation=2, return_lse=True)
        loss = lse.float().sum() if lse_only else (out.float() ** 2).sum() + lse.float().sum()
        return (out.detach(), lse.detach(),
                *torch.autograd.grad(loss, [ts[i] for i in which]))

    for which in ((0,), (1, 2), (0, 1, 2)):
        for lse_only in (False, True):
            r1 = run(which, lse_only)
            with F.python_autograd():
                r2 = run(which, lse_only)
            for a, b in zip(r1, r2):
                assert torch.equal(a, b), (which, lse_only)

    # an empty batch: empty outputs and gradients
    e = torch.empty((0, 10, 10, 2, 32), dtype=torch.bfloat16, device=DEV, requires_grad=True)
    out = natten_amd.na2d(e, e, e, 3)
    assert out.shape == e.shape
    (g,) = torch.autograd.grad(out.float().sum(), (e,))
    assert g.shape == e.shape
