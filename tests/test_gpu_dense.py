"""Dense (FMHA) mode of the fused op beyond the one-shape functional check.

When kernel_size covers every axis (stride 1, no causal mask) the reference
calls its dense attention (``functional.py:141-187``); here the fused
kernels run with the window set to the whole sample (``NA_FLAG_DENSE``).
Each case compares the forward output and LSE, and the backward of both
(dq, dk, dv with a non-zero LSE cotangent), with float64
softmax(q k^T * scale) v (``oracle.na.dense_attention``) on the same
rounded inputs, to the north-star bar of ``tests/_helpers.py``.  Shapes are
ragged (extents not multiples of the 32-query tiles), cover ranks 1-3, GQA,
head_dim 32/64/128 on the matrix-core kernels and an fp32 case on the
vector-ALU kernels; the full-size case is the bench's dense workload,
checked per (sample, head) against the oracle on that head alone (a dense
head's outputs and gradients depend on no other head).
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


def _ref(q, k, v, scale, ek=None, ev=None):
    rep = q.shape[-2] // k.shape[-2]
    r = lambda t: None if t is None else O._repeat_kv(t, rep)  # noqa: E731
    return O.dense_attention(q, r(k), r(v), scale, return_lse=True, ak=r(ek), av=r(ev))


def _run(q, k, v, go, gl, ek=None, ev=None):
    from natten_amd._core import hip

    R = q.dim() - 3
    sp = tuple(q.shape[1:-2])
    a = (sp, (1,) * R, (1,) * R, (False,) * R, q.shape[-1] ** -0.5)
    qd, kd, vd, god, gld = (t.to(DEV) for t in (q, k, v, go, gl))
    ekd, evd = (None if t is None else t.to(DEV) for t in (ek, ev))
    nx = 0 if ek is None else ek.shape[1]
    lowp = q.dtype != torch.float32
    assert hip.kernel_path(qd, kd, *a, n_extra=nx, dense=True) == (
        "dense" if lowp else "generic")
    assert hip.kernel_path(qd, kd, *a, n_extra=nx, dense=True, backward=True) == (
        "dense" if lowp else "generic")
    out, lse = hip.fused_forward(qd, kd, vd, *a, extra_k=ekd, extra_v=evd, dense=True)
    dq, dk, dv, dek, dev = hip.fused_backward(qd, kd, vd, out, lse, god, gld, *a,
                                              extra_k=ekd, extra_v=evd, dense=True)
    torch.cuda.synchronize()
    return out, lse, dq, dk, dv, dek, dev


# (name, B, spatial, H, Hkv, D, dtype)
CASES = [
    ("1d_1000_bf16_d64", 2, (1000,), 4, 4, 64, torch.bfloat16),
    ("1d_777_f16_gqa2_d128", 1, (777,), 4, 2, 128, torch.float16),
    ("2d_33x31_bf16_d32", 1, (33, 31), 2, 2, 32, torch.bfloat16),
    ("3d_9x10x11_f16_gqa2_d64", 1, (9, 10, 11), 2, 1, 64, torch.float16),
    ("1d_300_f32_d48", 1, (300,), 2, 2, 48, torch.float32),
    ("2d_17x19_f32_d32", 2, (17, 19), 2, 1, 32, torch.float32),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_dense_fwd_bwd(case):
    name, B, sp, H, Hkv, D, dt = case
    _say(f"[case] dense {name}")
    q = randn((B, *sp, H, D), dt, 1)
    k = randn((B, *sp, Hkv, D), dt, 2)
    v = randn((B, *sp, Hkv, D), dt, 3)
    go = randn((B, *sp, H, D), dt, 4)
    gl = randn((B, *sp, H), torch.float32, 5)
    out, lse, dq, dk, dv, _, _ = _run(q, k, v, go, gl)
    sc = D ** -0.5
    ro, rl = _ref(q, k, v, sc)
    assert_close(out, ro, dt, "out")
    assert_close(lse.to(dt) if dt != torch.float32 else lse, rl, dt, "lse")
    ref = O.grads(lambda a, b, c: _ref(a, b, c, sc), (q, k, v), (go, gl))
    for t, r, n in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert_close(t, r, dt, n)


# (name, B, spatial, H, Hkv, D, n_extra, dtype): additional tokens join the
# keys of every query (the dense forward appends them after the sample)
XCASES = [
    ("1d_500_bf16_d64_x16", 2, (500,), 4, 2, 64, 16, torch.bfloat16),
    ("2d_20x23_f16_d128_x5", 1, (20, 23), 2, 2, 128, 5, torch.float16),
    ("1d_64_bf16_d32_x70", 1, (64,), 2, 1, 32, 70, torch.bfloat16),
]


@pytest.mark.parametrize("case", XCASES, ids=[c[0] for c in XCASES])
def test_dense_additional_tokens(case):
    name, B, sp, H, Hkv, D, nx, dt = case
    _say(f"[case] dense {name}")
    q = randn((B, *sp, H, D), dt, 1)
    k = randn((B, *sp, Hkv, D), dt, 2)
    v = randn((B, *sp, Hkv, D), dt, 3)
    ek = randn((B, nx, Hkv, D), dt, 6)
    ev = randn((B, nx, Hkv, D), dt, 7)
    go = randn((B, *sp, H, D), dt, 4)
    gl = randn((B, *sp, H), torch.float32, 5)
    out, lse, dq, dk, dv, dek, dev = _run(q, k, v, go, gl, ek, ev)
    sc = D ** -0.5
    ro, rl = _ref(q, k, v, sc, ek, ev)
    assert_close(out, ro, dt, "out")
    assert_close(lse.to(dt), rl, dt, "lse")
    ref = O.grads(lambda a, b, c, d, e: _ref(a, b, c, sc, d, e), (q, k, v, ek, ev), (go, gl))
    for t, r, n in zip((dq, dk, dv, dek, dev), ref, ("dq", "dk", "dv", "dek", "dev")):
        assert_close(t, r, dt, n)


def test_dense_full_size_per_head():
    """The bench's dense workload, [4, 4096, 16, 64] bf16, two (sample, head)
    pairs checked against the oracle on that head alone."""
    B, L, H, D, dt = 4, 4096, 16, 64, torch.bfloat16
    _say(f"[case] dense full size [{B},{L},{H},{D}] bf16")
    q, k, v, go = (randn((B, L, H, D), dt, s) for s in (11, 12, 13, 14))
    gl = randn((B, L, H), torch.float32, 15)
    out, lse, dq, dk, dv, _, _ = _run(q, k, v, go, gl)
    sc = D ** -0.5
    for b, h in ((0, 0), (3, 13)):
        sl = lambda t: t[b:b + 1, ..., h:h + 1, :]  # noqa: E731
        ro, rl = _ref(sl(q), sl(k), sl(v), sc)
        assert_close(sl(out.cpu()), ro, dt, f"out[{b},{h}]")
        assert_close(lse.cpu()[b:b + 1, :, h:h + 1].to(dt), rl, dt, f"lse[{b},{h}]")
        ref = O.grads(lambda x, y, z: _ref(x, y, z, sc), (sl(q), sl(k), sl(v)),
                      (sl(go), gl[b:b + 1, :, h:h + 1]))
        for t, r, n in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
            assert_close(sl(t.cpu()), r, dt, f"{n}[{b},{h}]")
