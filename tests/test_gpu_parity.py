"""Parity of the HIP library with the CPU oracle (runs on an MI355X).

Every case draws seeded inputs, rounds them to the test dtype, runs the
public API on the device and compares with the float64 oracle on the same
rounded values: fp32 within atol = rtol = 1e-5, fp16/bf16 within 2e-2
absolute of the oracle rounded to that dtype (see tests/_helpers.py).
Indices and masks are compared exactly.
"""

import sys

import numpy as np
import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import na as O
from oracle import window as W

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# (name, B, spatial, H, Hkv, D, ks, dil, caus, st)
CORE = [
    ("1d_cfg1", 2, (64,), 4, 4, 32, (7,), (1,), (False,), (1,)),
    ("1d_causal_stride_dil", 2, (37,), 2, 1, 12, (4,), (3,), (True,), (2,)),
    ("1d_evenK_full", 1, (8,), 2, 2, 16, (8,), (1,), (False,), (1,)),
    ("2d_dil", 1, (20, 18), 4, 2, 32, (7, 5), (2, 3), (False, False), (1, 1)),
    ("2d_causal_stride", 2, (13, 15), 2, 2, 64, (3, 5), (1, 2), (True, False), (2, 3)),
    ("3d_causal_depth", 1, (6, 8, 9), 2, 1, 32, (3, 3, 5), (1, 2, 1), (True, False, False),
     (1, 1, 2)),
    ("3d_odd_dim", 1, (5, 6, 7), 3, 3, 20, (3, 3, 3), (1, 1, 2), (False, True, False),
     (1, 2, 1)),
]


def _inputs(B, sp, H, Hkv, D, dtype, seed=0):
    q = randn((B, *sp, H, D), dtype, seed)
    k = randn((B, *sp, Hkv, D), dtype, seed + 1)
    v = randn((B, *sp, Hkv, D), dtype, seed + 2)
    return q, k, v


def _fns():
    import natten_amd
    return {1: natten_amd.na1d, 2: natten_amd.na2d, 3: natten_amd.na3d}


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", CORE, ids=[c[0] for c in CORE])
def test_fused_forward_backward(case, dtype):
    name, B, sp, H, Hkv, D, ks, dil, caus, st = case
    _say(f"[case] fused {name} {dtype}")
    rank = len(sp)
    q, k, v = _inputs(B, sp, H, Hkv, D, dtype)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out, lse = _fns()[rank](qd, kd, vd, ks, st, dil, caus, return_lse=True)
    ref_out, ref_lse = O.na_functional(q, k, v, ks, st, dil, caus, return_lse=True)
    assert_close(out, ref_out, dtype, f"{name} out")
    assert_close(lse, ref_lse, dtype, f"{name} lse")
    go = randn(out.shape, dtype, 7)
    gl = randn(lse.shape, dtype, 8)
    torch.autograd.backward((out, lse), (go.to(DEV), gl.to(DEV)))
    ref = O.grads(lambda a, b, c: O.na_functional(a, b, c, ks, st, dil, caus, return_lse=True),
                  (q, k, v), (go, gl))
    for g, r, n in zip((qd.grad, kd.grad, vd.grad), ref, "qkv"):
        assert_close(g, r, dtype, f"{name} d{n}")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_additional_tokens_gqa(dtype):
    import natten_amd

    _say(f"[case] extra tokens {dtype}")
    B, sp, H, Hkv, D = 2, (11, 10), 4, 2, 32
    q, k, v = _inputs(B, sp, H, Hkv, D, dtype, 3)
    ek, ev = randn((B, 5, Hkv, D), dtype, 9), randn((B, 5, Hkv, D), dtype, 10)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, ek, ev)]
    out, lse = natten_amd.na2d(ts[0], ts[1], ts[2], (3, 5), dilation=(2, 1),
                               is_causal=(False, True), return_lse=True,
                               additional_keys=ts[3], additional_values=ts[4])
    assert lse.dtype == torch.float32  # merged LSE is float32 (merge.py:53,68)

    def f(a, b, c, d, e):
        return O.na_functional(a, b, c, (3, 5), 1, (2, 1), (False, True), return_lse=True,
                               additional_keys=d, additional_values=e)

    ro, rl = f(q, k, v, ek, ev)
    assert_close(out, ro, dtype, "out")
    assert_close(lse.to(dtype), rl, dtype, "lse")
    go, gl = randn(out.shape, dtype, 11), randn(lse.shape, torch.float32, 12)
    torch.autograd.backward((out, lse), (go.to(DEV), gl.to(DEV)))
    ref = O.grads(f, (q, k, v, ek, ev), (go, gl))
    for t, r, n in zip(ts, ref, ("dq", "dk", "dv", "dek", "dev")):
        assert_close(t.grad, r, dtype, n)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_dense_fmha_path(dtype):
    import natten_amd

    _say(f"[case] dense {dtype}")
    q, k, v = _inputs(2, (6, 7), 2, 1, 32, dtype, 5)
    ek, ev = randn((2, 3, 1, 32), dtype, 6), randn((2, 3, 1, 32), dtype, 7)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, ek, ev)]
    out, lse = natten_amd.na2d(ts[0], ts[1], ts[2], (6, 7), return_lse=True,
                               additional_keys=ts[3], additional_values=ts[4])
    assert lse.dtype == dtype  # FMHA path keeps the query dtype

    def f(a, b, c, d, e):
        return O.na_functional(a, b, c, (6, 7), return_lse=True, additional_keys=d,
                               additional_values=e)

    ro, rl = f(q, k, v, ek, ev)
    assert_close(out, ro, dtype, "out")
    assert_close(lse, rl, dtype, "lse")
    go = randn(out.shape, dtype, 8)
    out.backward(go.to(DEV))
    ref = O.grads(lambda *a: f(*a)[0], (q, k, v, ek, ev), (go,))
    for t, r, n in zip(ts, ref, ("dq", "dk", "dv", "dek", "dev")):
        assert_close(t.grad, r, dtype, n)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", CORE[:6], ids=[c[0] for c in CORE[:6]])
def test_split_ops(case, dtype):
    import natten_amd

    name, B, sp, H, Hkv, D, ks, dil, caus, st = case
    _say(f"[case] split {name} {dtype}")
    rank = len(sp)
    qk = {1: natten_amd.na1d_qk, 2: natten_amd.na2d_qk, 3: natten_amd.na3d_qk}[rank]
    av = {1: natten_amd.na1d_av, 2: natten_amd.na2d_av, 3: natten_amd.na3d_av}[rank]
    q, k, v = _inputs(B, sp, H, H, D, dtype, 2)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    logits = qk(qd, kd, ks, dil, stride=st, is_causal=caus, scale=0.3)
    ref_logits = O.na_qk(q, k, ks, st, dil, caus, 0.3)
    assert logits.dtype == dtype
    assert torch.equal(torch.isinf(logits).cpu(), torch.isinf(ref_logits))  # mask exact
    assert_close(logits, ref_logits, dtype, "logits")
    attn = torch.softmax(logits.float(), -1).to(dtype)
    attn_ref = attn.detach().cpu()
    attn_d = attn.detach().clone().requires_grad_(True)
    out = av(attn_d, vd, ks, dil, stride=st, is_causal=caus)
    assert_close(out, O.na_av(attn_ref, v, ks, st, dil, caus), dtype, "av out")
    gl = randn(logits.shape, dtype, 4)
    go = randn(out.shape, dtype, 5)
    logits.backward(gl.to(DEV))
    out.backward(go.to(DEV))
    finite = torch.isfinite(ref_logits)

    def qk_masked(a, b):
        x = O.na_qk(a, b, ks, st, dil, caus, 0.3)
        return torch.where(finite, x, torch.zeros_like(x))

    rq, rk = O.grads(qk_masked, (q, k), (gl,))
    ra, rv = O.grads(lambda a, b: O.na_av(a, b, ks, st, dil, caus), (attn_ref, v), (go,))
    assert_close(qd.grad, rq, dtype, "dq")
    assert_close(kd.grad, rk, dtype, "dk")
    assert_close(attn_d.grad, ra, dtype, "dattn")
    assert_close(vd.grad, rv, dtype, "dv")


@pytest.mark.parametrize("cfg", [
    ((64,), (7,), (1,), (False,), (1,)),
    ((37,), (4,), (3,), (True,), (2,)),
    ((8,), (8,), (1,), (False,), (1,)),
    ((56, 56), (7, 7), (4, 4), (False, False), (1, 1)),
    ((13, 15), (3, 6), (1, 2), (True, False), (2, 3)),
    ((16, 32, 32), (3, 7, 7), (1, 1, 1), (True, False, False), (1, 1, 1)),
    ((5, 9, 10), (2, 3, 4), (2, 3, 2), (False, True, False), (2, 1, 3)),
])
def test_device_neighbor_table_exact(cfg):
    from natten_amd._core import _lib

    sp, ks, dil, caus, st = cfg
    _say(f"[case] table {cfg}")
    lin, valid = W.neighbor_table(sp, ks, dil, caus, st)
    idx = torch.empty(lin.shape, dtype=torch.int32, device=DEV)
    ok = torch.empty(valid.shape, dtype=torch.uint8, device=DEV)
    p = _lib.make_params(len(sp), 1, 1, 1, 8, _lib.NA_F32, sp, ks, dil, st,
                         [int(c) for c in caus], 1.0)
    lib = _lib.load()
    _lib.check(lib.na_neighbor_table(p, _lib.ptr(idx), _lib.ptr(ok), None), "table")
    torch.cuda.synchronize()
    assert np.array_equal(ok.cpu().numpy().astype(bool), valid)
    assert np.array_equal(idx.cpu().numpy()[valid], lin[valid])


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_varlen(dtype):
    import natten_amd

    _say(f"[case] varlen {dtype}")
    q, k, v = _inputs(3, (40,), 2, 2, 32, dtype, 13)
    lens = torch.tensor([40, 23, 9], dtype=torch.int32)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = natten_amd.na1d_varlen(*ts, lens.to(DEV), kernel_size=7, dilation=1)
    ref = O.na_varlen(q, k, v, lens, 7, 1)
    assert_close(out, ref, dtype, "out")
    go = randn(out.shape, dtype, 14)
    out.backward(go.to(DEV))
    g = O.grads(lambda a, b, c: O.na_varlen(a, b, c, lens, 7, 1), (q, k, v), (go,))
    for t, r, n in zip(ts, g, ("dq", "dk", "dv")):
        assert_close(t.grad, r, dtype, n)
    # 2D varlen
    q, k, v = _inputs(2, (9, 11), 2, 2, 16, dtype, 15)
    sizes = torch.tensor([[9, 11], [6, 8]], dtype=torch.int32)
    out = natten_amd.na2d_varlen(q.to(DEV), k.to(DEV), v.to(DEV), sizes.to(DEV), (3, 5), (2, 1))
    assert_close(out, O.na_varlen(q, k, v, sizes, (3, 5), (2, 1)), dtype, "2d out")


@pytest.mark.parametrize("dtype", [torch.float16], ids=str)
def test_varlen_gqa_extra_cfg4_shape(dtype):
    """Config-4 semantics at a reduced length: varlen + GQA + 16 extra tokens."""
    import natten_amd

    _say(f"[case] varlen gqa extra {dtype}")
    B, L, H, Hkv, D = 3, 300, 8, 2, 64
    q, k, v = _inputs(B, (L,), H, Hkv, D, dtype, 21)
    ek, ev = randn((B, 16, Hkv, D), dtype, 22), randn((B, 16, Hkv, D), dtype, 23)
    lens = torch.tensor([300, 200, 150], dtype=torch.int32)
    out = natten_amd.na1d_varlen_gqa(q.to(DEV), k.to(DEV), v.to(DEV), lens.to(DEV), 63, 2,
                                     additional_keys=ek.to(DEV), additional_values=ev.to(DEV))
    for b in range(B):
        Lb = int(lens[b])
        ref = O.na_functional(q[b:b + 1, :Lb], k[b:b + 1, :Lb], v[b:b + 1, :Lb], 63, 1, 2,
                              False, additional_keys=ek[b:b + 1], additional_values=ev[b:b + 1])
        assert_close(out[b:b + 1, :Lb], ref, dtype, f"sample {b}")
        assert (out[b, Lb:] == 0).all()


def test_backward_is_deterministic():
    import natten_amd

    _say("[case] determinism")
    q, k, v = _inputs(2, (24, 24), 4, 4, 32, torch.bfloat16, 31)
    grads = []
    for _ in range(2):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
        out = natten_amd.na2d(*ts, 7, dilation=2)
        out.backward(torch.ones_like(out))
        grads.append([t.grad.clone() for t in ts])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("generic", [False, True], ids=["matrix", "generic"])
def test_varlen_gqa_extra_gradients(dtype, generic):
    """Gradients of q, k, v and of the additional tokens under varlen + GQA
    (4 query heads per key/value head, 21 tokens: two token tiles), against
    the oracle summed over per-sample calls; the extra-token gradients
    reduce over every query of a sample (matrix-core reduction for bf16 /
    fp16, the vector-ALU one for fp32 and under generic_kernels())."""
    import contextlib

    import natten_amd
    from natten_amd._core import hip

    _say(f"[case] varlen gqa extra gradients {dtype} generic={generic}")
    B, L, H, Hkv, D, nx = 3, 150, 8, 2, 32, 21
    q, k, v = _inputs(B, (L,), H, Hkv, D, dtype, 81)
    ek, ev = randn((B, nx, Hkv, D), dtype, 84), randn((B, nx, Hkv, D), dtype, 85)
    lens = torch.tensor([150, 97, 40], dtype=torch.int32)
    go = randn((B, L, H, D), dtype, 86)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, ek, ev)]
    with hip.generic_kernels() if generic else contextlib.nullcontext():
        out = natten_amd.na1d_varlen_gqa(ts[0], ts[1], ts[2], lens.to(DEV), 7, 2,
                                         additional_keys=ts[3], additional_values=ts[4])
        out.backward(go.to(DEV))
    ref = [torch.zeros(t.shape, dtype=torch.float64) for t in (q, k, v, ek, ev)]
    for b in range(B):
        Lb = int(lens[b])
        sl = (slice(b, b + 1), slice(0, Lb))
        g = O.grads(lambda a, c, d, e, f: O.na_functional(a, c, d, 7, 1, 2, False,
                                                          additional_keys=e,
                                                          additional_values=f),
                    (q[sl], k[sl], v[sl], ek[b:b + 1], ev[b:b + 1]), (go[sl],))
        for r, gg, s in zip(ref, g, (sl, sl, sl, slice(b, b + 1), slice(b, b + 1))):
            r[s] = gg.to(torch.float64)
    for t, r, nm in zip(ts, ref, ("dq", "dk", "dv", "dek", "dev")):
        assert_close(t.grad, r, dtype, nm)


@pytest.mark.parametrize("D", [6, 64, 128, 264, 520, 1024])
def test_extra_gradients_head_dims(D):
    """Extra-token gradients at head_dims that change the reduction's tiling:
    64 and 128 on the matrix-core reduction, not a multiple of 4
    (zero-padded rows) and above 256 (eight, then four tokens per tile) on
    the vector-ALU one, with GQA and a stride, against the oracle."""
    import natten_amd

    dtype = torch.float16
    _say(f"[case] extra gradients head_dim {D}")
    B, L, H, Hkv, nx = 2, 30, 4, 2, 11
    q, k, v = _inputs(B, (L,), H, Hkv, D, dtype, 91)
    ek, ev = randn((B, nx, Hkv, D), dtype, 94), randn((B, nx, Hkv, D), dtype, 95)
    go = randn((B, 15, H, D), dtype, 96)

    def f(a, c, d, e, g):
        return O.na_functional(a, c, d, 5, 2, 1, False, additional_keys=e, additional_values=g)

    ref = O.grads(f, (q, k, v, ek, ev), (go,))
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, ek, ev)]
    out = natten_amd.na1d(ts[0], ts[1], ts[2], 5, stride=2, additional_keys=ts[3],
                          additional_values=ts[4])
    out.backward(go.to(DEV))
    for t, r, nm in zip(ts, ref, ("dq", "dk", "dv", "dek", "dev")):
        assert_close(t.grad, r, dtype, nm)


def test_fused_backward_hook_reference_signature():
    """hip.na2d_fused_backward takes the reference VJP's positional
    arguments (q, k, v, grad_out, fwd_out, kernel_size, stride, dilation,
    is_causal, scale; fast_metal.py:2430) and recomputes the LSE when none is
    passed: same gradients as with the forward's LSE, and as the oracle."""
    from natten_amd._core import hip

    _say("[case] fused backward hook signature")
    dt = torch.bfloat16
    q, k, v = _inputs(2, (20, 18), 4, 4, 32, dt, 61)
    go = randn(q.shape, dt, 62)
    qd, kd, vd, god = (t.to(DEV) for t in (q, k, v, go))
    a = ((7, 5), (1, 1), (2, 1), (False, False), None)
    out, lse = hip.fused_forward(qd, kd, vd, *a)
    g_none = hip.na2d_fused_backward(qd, kd, vd, god, out, *a)
    g_lse = hip.na2d_fused_backward(qd, kd, vd, god, out, *a, lse=lse)
    for x, y in zip(g_none, g_lse):
        assert torch.equal(x, y)
    ref = O.grads(lambda x, y, z: O.na_forward(x, y, z, (7, 5), 1, (2, 1)), (q, k, v), (go,))
    for g, r, n in zip(g_none, ref, "qkv"):
        assert_close(g, r, dt, f"hook d{n}")


def test_varlen_host_lengths_graph_capture():
    """Host-side seq_lens give the same result as device ones, with no
    host-device synchronisation, so the call can be captured in a HIP graph:
    replays (with other work between them) reproduce the eager output."""
    import natten_amd

    _say("[case] varlen host lengths + graph")
    dt = torch.float16
    q, k, v = _inputs(3, (96,), 4, 2, 64, dt, 71)
    qd, kd, vd = (t.to(DEV) for t in (q, k, v))
    lens = torch.tensor([96, 40, 63], dtype=torch.int32)
    ref = natten_amd.na1d_varlen_gqa(qd, kd, vd, lens.to(DEV), 7, 2)
    got = natten_amd.na1d_varlen_gqa(qd, kd, vd, lens, 7, 2)
    assert torch.equal(got, ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        natten_amd.na1d_varlen_gqa(qd, kd, vd, lens, 7, 2)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static = natten_amd.na1d_varlen_gqa(qd, kd, vd, lens, 7, 2)
    for i in range(3):
        torch.zeros(1 << 20, device=DEV).add_(i)  # unrelated eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, ref), f"replay {i}"
