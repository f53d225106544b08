"""Matrix-core (MFMA) path: lane-layout self-check and parity at the
BASELINE shapes and around the tiling edge cases (runs on an MI355X).

bf16/fp16 problems with head_dim 32/64/128, stride 1 and odd (or causal)
kernels run on the MFMA kernels; each case is compared with the float64
oracle (2e-2 absolute of the dtype-rounded value, see tests/_helpers.py) and
with the generic vector-ALU kernels on the same device.
"""

import contextlib
import sys

import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import na as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_mfma_lane_layout_selftest(dtype):
    from natten_amd._core import _lib

    _say(f"[case] mfma selftest {dtype}")
    m = torch.arange(32).reshape(32, 1)
    kk = torch.arange(16).reshape(1, 16)
    A = ((m + 2 * kk) % 7 - 3).double()
    kk2 = torch.arange(16).reshape(16, 1)
    n = torch.arange(32).reshape(1, 32)
    Bm = ((3 * kk2 + n) % 5 - 2).double()
    out = torch.full((32, 32), float("nan"), dtype=torch.float32, device=DEV)
    lib = _lib.load()
    _lib.check(lib.na_mfma_selftest(_lib.dtype_code(dtype), _lib.ptr(out), None), "selftest")
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().double(), A @ Bm)


def _run(fn, q, k, v, go, **kw):
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out, lse = fn(*ts, return_lse=True, **kw)
    out.backward(go.to(DEV))
    return out.detach(), lse.detach(), [t.grad for t in ts]


CASES = [
    # (name, B, spatial, H, Hkv, D, ks, dil, caus)
    ("cfg2_d1", 4, (56, 56), 4, 4, 32, (7, 7), (1, 1), (False, False)),
    ("cfg2_d4", 4, (56, 56), 4, 4, 32, (7, 7), (4, 4), (False, False)),
    ("cfg3_small", 1, (6, 12, 12), 4, 4, 64, (3, 7, 7), (1, 1, 1), (True, False, False)),
    ("2d_gqa_d128", 1, (10, 13), 4, 2, 128, (5, 3), (1, 2), (False, True)),
    ("1d_long_k63", 2, (300,), 4, 1, 64, (63,), (2,), (False,)),
    ("1d_causal", 2, (70,), 2, 2, 32, (9,), (3,), (True,)),
    ("3d_unit_k", 1, (4, 9, 33), 2, 2, 32, (1, 3, 5), (1, 2, 1), (False, False, True)),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_mfma_parity(case, dtype):
    import natten_amd
    from natten_amd._core import hip

    name, B, sp, H, Hkv, D, ks, dil, caus = case
    _say(f"[case] mfma {name} {dtype}")
    fn = {1: natten_amd.na1d, 2: natten_amd.na2d, 3: natten_amd.na3d}[len(sp)]
    q = randn((B, *sp, H, D), dtype, 1)
    k = randn((B, *sp, Hkv, D), dtype, 2)
    v = randn((B, *sp, Hkv, D), dtype, 3)
    go = randn((B, *sp, H, D), dtype, 4)
    out, lse, grads = _run(fn, q, k, v, go, kernel_size=ks, dilation=dil, is_causal=caus)
    ref_out, ref_lse = O.na_functional(q, k, v, ks, 1, dil, caus, return_lse=True)
    assert_close(out, ref_out, dtype, f"{name} out")
    assert_close(lse, ref_lse, dtype, f"{name} lse")
    ref = O.grads(lambda a, b, c: O.na_functional(a, b, c, ks, 1, dil, caus), (q, k, v), (go,))
    for g, r, nm in zip(grads, ref, ("dq", "dk", "dv")):
        assert_close(g, r, dtype, f"{name} {nm}")
    # the 32-query matrix-core kernels (where the lean ones run by default)
    # and the generic kernels meet the same bar on the same inputs
    with hip.no_lean_kernels():
        out1, lse1, grads1 = _run(fn, q, k, v, go, kernel_size=ks, dilation=dil, is_causal=caus)
    assert_close(out1, ref_out, dtype, f"{name} mfma out")
    assert_close(lse1, ref_lse, dtype, f"{name} mfma lse")
    for g, r, nm in zip(grads1, ref, ("dq", "dk", "dv")):
        assert_close(g, r, dtype, f"{name} mfma {nm}")
    with hip.generic_kernels():
        out2, lse2, grads2 = _run(fn, q, k, v, go, kernel_size=ks, dilation=dil, is_causal=caus)
    assert_close(out2, ref_out, dtype, f"{name} generic out")
    for g, r, nm in zip(grads2, ref, ("dq", "dk", "dv")):
        assert_close(g, r, dtype, f"{name} generic {nm}")


@pytest.mark.parametrize("dtype", [torch.bfloat16], ids=str)
def test_mfma_varlen_2d_and_extra(dtype):
    import natten_amd

    _say(f"[case] mfma varlen 2d {dtype}")
    B, sp, H, D = 3, (20, 24), 2, 32
    q, k, v = (randn((B, *sp, H, D), dtype, s) for s in (5, 6, 7))
    sizes = torch.tensor([[20, 24], [13, 17], [7, 9]], dtype=torch.int32)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = natten_amd.na2d_varlen(*ts, sizes.to(DEV), (7, 5), (1, 1))
    go = randn(out.shape, dtype, 8)
    out.backward(go.to(DEV))
    assert_close(out, O.na_varlen(q, k, v, sizes, (7, 5), (1, 1)), dtype, "out")
    g = O.grads(lambda a, b, c: O.na_varlen(a, b, c, sizes, (7, 5), (1, 1)), (q, k, v), (go,))
    for t, r, nm in zip(ts, g, ("dq", "dk", "dv")):
        assert_close(t.grad, r, dtype, nm)


def test_mfma_backward_deterministic():
    import natten_amd

    _say("[case] mfma determinism")
    q, k, v = (randn((2, 30, 30, 4, 64), torch.bfloat16, s) for s in (1, 2, 3))
    res = []
    for _ in range(2):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
        out = natten_amd.na2d(*ts, (7, 7), dilation=(2, 3))
        out.backward(torch.ones_like(out))
        res.append([t.grad.clone() for t in ts])
    for a, b in zip(*res):
        assert torch.equal(a, b)


SPLIT_CASES = [
    # (name, B, spatial, H, Hkv, D, ks, dil, caus)
    ("cfg2s_d1", 4, (56, 56), 4, 4, 32, (7, 7), (1, 1), (False, False)),
    ("cfg2s_d4", 2, (56, 56), 4, 4, 32, (7, 7), (4, 4), (False, False)),
    ("2d_gqa_d64", 2, (17, 20), 4, 2, 64, (5, 7), (2, 1), (False, False)),
    ("3d_causal", 1, (6, 12, 12), 4, 4, 64, (3, 7, 7), (1, 1, 1), (True, False, False)),
    ("1d_k63_d128", 2, (300,), 2, 1, 128, (63,), (2,), (False,)),
    ("1d_causal", 2, (70,), 2, 2, 32, (9,), (3,), (True,)),
    ("2d_wide_causal_gqa4", 1, (12, 40), 8, 2, 32, (3, 17), (1, 2), (True, False)),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_mfma_split_ops(case, dtype):
    """Split QK / AV forward and backward against the oracle on the lean
    workgroup kernels (where they run by default), the 32-query matrix-core
    kernels and the generic kernels, all on the same inputs."""
    import natten_amd
    from natten_amd._core import hip

    name, B, sp, H, Hkv, D, ks, dil, caus = case
    _say(f"[case] mfma split {name} {dtype}")
    rank = len(sp)
    qk = {1: natten_amd.na1d_qk, 2: natten_amd.na2d_qk, 3: natten_amd.na3d_qk}[rank]
    av = {1: natten_amd.na1d_av, 2: natten_amd.na2d_av, 3: natten_amd.na3d_av}[rank]
    q = randn((B, *sp, H, D), dtype, 11)
    k = randn((B, *sp, Hkv, D), dtype, 12)
    v = randn((B, *sp, Hkv, D), dtype, 13)
    ref_logits = O.na_qk(q, k, ks, 1, dil, caus, 0.25)
    finite = torch.isfinite(ref_logits)
    attn = torch.softmax(ref_logits, -1).to(dtype)
    gl = randn(ref_logits.shape, dtype, 14)
    go = randn((B, *sp, H, D), dtype, 15)

    def qk_masked(a, b):
        x = O.na_qk(a, b, ks, 1, dil, caus, 0.25)
        return torch.where(finite, x, torch.zeros_like(x))

    rq, rk = O.grads(qk_masked, (q, k), (gl,))
    ra, rv = O.grads(lambda a, b: O.na_av(a, b, ks, 1, dil, caus), (attn, v), (go,))
    ref_out = O.na_av(attn, v, ks, 1, dil, caus)
    assert hip.kernel_path(q, k, ks, (1,) * rank, dil, caus, split=True) == "lean"
    with hip.no_lean_kernels():
        assert hip.kernel_path(q, k, ks, (1,) * rank, dil, caus, split=True) == "mfma"
    modes = {"lean": contextlib.nullcontext, "mfma": hip.no_lean_kernels,
             "generic": hip.generic_kernels}
    for mode, ctx in modes.items():
        tag = f"{name} {mode}"
        with ctx():
            qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
            logits = qk(qd, kd, ks, dil, is_causal=caus, scale=0.25)
            assert torch.equal(torch.isinf(logits).cpu(), ~finite), f"{tag} mask"
            assert_close(logits, ref_logits, dtype, f"{tag} logits")
            ad = attn.to(DEV).requires_grad_(True)
            out = av(ad, vd, ks, dil, is_causal=caus)
            assert_close(out, ref_out, dtype, f"{tag} av")
            logits.backward(gl.to(DEV))
            out.backward(go.to(DEV))
            assert_close(qd.grad, rq, dtype, f"{tag} dq")
            assert_close(kd.grad, rk, dtype, f"{tag} dk")
            assert_close(ad.grad, ra, dtype, f"{tag} dattn")
            assert_close(vd.grad, rv, dtype, f"{tag} dv")
