"""Parity at the benchmarked sizes: every configuration the benchmark lines
time, at its full shape and on the kernel path (and launch shape) it
dispatches to, against the float64 oracle on the same dtype-rounded inputs.

* config 1: na1d fp32 [2,64,4,32], k 7 (the README quick-start shape);
* config 2: na2d bf16 [4,56,56,4,32], k 7, dilations 1 and 4, forward and
  backward, and the split qk -> softmax -> av path with its backward;
* config 3: na3d bf16 [1,16,32,32,8,64], k (3,7,7), causal depth, LSE with a
  non-zero LSE gradient: forward, LSE and backward on the lean kernels with
  the key box staged in several depth slabs;
* config 4: na1d varlen GQA fp16 [8,4096,16/4,64], k 63, d 2, 16 additional
  tokens, the benchmark's seq_lens: forward with grouped query heads, LSE,
  and backward including the additional tokens' gradients on matrix cores;
* config 5: allin1 na1d_qk_rpb + na1d_av_fused fp32 [8,2048,12,12] for every
  K in {3,5,7} x d in {1,2,4,8}: forward and backward (dq, dk, dRPB, dattn,
  dv).

The fused configurations are checked against ``oracle.full`` (exact over
every row, in query chunks), the allin1 ones against ``oracle.na``.
Tolerances are the north-star bar (tests/_helpers.py): fp32 1e-5 relative,
fp16 / bf16 2e-2 absolute (or one ulp of the dtype).
"""

import sys

import os

import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import full as F
from oracle import na as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _dev(*ts):
    return [t.to(DEV).requires_grad_(True) for t in ts]


def test_config1_full():
    import natten_amd

    _say("[case] config 1 na1d fp32 [2,64,4,32] k7")
    q, k, v = (randn((2, 64, 4, 32), torch.float32, s) for s in (0, 1, 2))
    qd, kd, vd = _dev(q, k, v)
    out = natten_amd.na1d(qd, kd, vd, 7)
    go = randn(out.shape, torch.float32, 3)
    out.backward(go.to(DEV))
    ref = F.fused(q, k, v, 7, dout=go)
    assert_close(out, ref["out"], torch.float32, "cfg1 out")
    for t, n in zip((qd, kd, vd), ("dq", "dk", "dv")):
        assert_close(t.grad, ref[n], torch.float32, f"cfg1 {n}")


@pytest.mark.parametrize("dil", [1, 4])
def test_config2_full(dil):
    import natten_amd
    from natten_amd._core import hip

    _say(f"[case] config 2 na2d bf16 [4,56,56,4,32] k7 d{dil}")
    dt = torch.bfloat16
    shape = (4, 56, 56, 4, 32)
    q, k, v, go = (randn(shape, dt, s) for s in (10, 11, 12, 13))
    for bwd in (False, True):
        plan = hip.kernel_plan(q, k, (7, 7), (1, 1), (dil, dil), (False, False), backward=bwd)
        assert plan["path"] == "lean", plan
    qd, kd, vd = _dev(q, k, v)
    out = natten_amd.na2d(qd, kd, vd, 7, dilation=dil)
    out.backward(go.to(DEV))
    ref = F.fused(q, k, v, 7, 1, dil, False, None, go)
    assert_close(out, ref["out"], dt, "cfg2 out")
    for t, n in zip((qd, kd, vd), ("dq", "dk", "dv")):
        assert_close(t.grad, ref[n], dt, f"cfg2 {n}")


def test_config2_split_full():
    """na2d_qk -> softmax -> na2d_av and the gradients of both ops at
    config 2 (the split kernels), against the oracle's split ops."""
    import natten_amd

    _say("[case] config 2 split qk/av bf16 full size")
    dt = torch.bfloat16
    shape = (4, 56, 56, 4, 32)
    q, k, v = (randn(shape, dt, s) for s in (20, 21, 22))
    qd, kd, vd = _dev(q, k, v)
    logits = natten_amd.na2d_qk(qd, kd, 7)
    ref_logits = O.na_qk(q, k, 7)
    assert torch.equal(torch.isinf(logits).cpu(), torch.isinf(ref_logits))
    assert_close(logits, ref_logits, dt, "split logits")
    attn = torch.softmax(logits.detach().float(), -1).to(dt)
    ad = attn.clone().requires_grad_(True)
    out = natten_amd.na2d_av(ad, vd, 7)
    assert_close(out, O.na_av(attn.cpu(), v, 7), dt, "split out")
    go = randn(out.shape, dt, 23)
    out.backward(go.to(DEV))
    ra, rv = O.grads(lambda a, b: O.na_av(a, b, 7), (attn.cpu(), v), (go,))
    assert_close(ad.grad, ra, dt, "split dattn")
    assert_close(vd.grad, rv, dt, "split dv")
    gl = randn(logits.shape, dt, 24)
    logits.backward(gl.to(DEV))
    rq, rk = O.grads(lambda a, b: O.na_qk(a, b, 7), (q, k), (gl,))
    assert_close(qd.grad, rq, dt, "split dq")
    assert_close(kd.grad, rk, dt, "split dk")


def test_config3_full():
    import natten_amd
    from natten_amd._core import hip

    _say("[case] config 3 na3d bf16 [1,16,32,32,8,64] k(3,7,7) causal depth, lse")
    dt = torch.bfloat16
    shape = (1, 16, 32, 32, 8, 64)
    ks, caus = (3, 7, 7), (True, False, False)
    q, k, v, go = (randn(shape, dt, s) for s in (30, 31, 32, 33))
    gl = randn(shape[:-1], dt, 34)
    for bwd in (False, True):
        plan = hip.kernel_plan(q, k, ks, (1, 1, 1), (1, 1, 1), caus, backward=bwd)
        assert plan["path"] == "lean" and plan["slabs"] > 1, plan
    qd, kd, vd = _dev(q, k, v)
    out, lse = natten_amd.na3d(qd, kd, vd, ks, is_causal=caus, return_lse=True)
    torch.autograd.backward((out, lse), (go.to(DEV), gl.to(DEV)))
    _say("  device done; oracle ...")
    ref = F.fused(q, k, v, ks, 1, 1, caus, None, go, gl)
    assert_close(out, ref["out"], dt, "cfg3 out")
    assert_close(lse, ref["lse"], dt, "cfg3 lse")
    for t, n in zip((qd, kd, vd), ("dq", "dk", "dv")):
        assert_close(t.grad, ref[n], dt, f"cfg3 {n}")


def test_config4_full():
    import natten_amd
    from natten_amd._core import hip

    _say("[case] config 4 na1d varlen gqa fp16 [8,4096,16/4,64] k63 d2 +16 tokens")
    dt = torch.float16
    B, L, H, Hkv, D, nx = 8, 4096, 16, 4, 64, 16
    q = randn((B, L, H, D), dt, 0)
    k, v = (randn((B, L, Hkv, D), dt, s) for s in (1, 2))
    ek, ev = (randn((B, nx, Hkv, D), dt, s) for s in (3, 4))
    # the benchmark's lengths (bench.py wl_cfg4)
    lens = torch.randint(1024, 4097, (B,), generator=torch.Generator().manual_seed(5),
                         dtype=torch.int32)
    go = randn((B, L, H, D), dt, 6)
    gl = randn((B, L, H), torch.float32, 7)
    se = lens.reshape(B, 1)
    fplan = hip.kernel_plan(q, k, (63,), (1,), (2,), (False,), n_extra=nx, sample_extent=se,
                            varlen_clamped=True)
    bplan = hip.kernel_plan(q, k, (63,), (1,), (2,), (False,), n_extra=nx, sample_extent=se,
                            varlen_clamped=True, backward=True)
    assert fplan["path"] == "lean" and fplan["grouped_heads"], fplan
    assert bplan["path"] == "lean" and bplan["extra_reduction"] == "matrix", bplan
    ts = _dev(q, k, v, ek, ev)
    out, lse = natten_amd.na1d_varlen_gqa(ts[0], ts[1], ts[2], lens.to(DEV), 63, 2,
                                          additional_keys=ts[3], additional_values=ts[4],
                                          return_lse=True)
    torch.autograd.backward((out, lse), (go.to(DEV), gl.to(DEV)))
    _say("  device done; oracle ...")
    ref = F.fused(q, k, v, 63, 1, 2, False, None, go, gl, ek, ev, sizes=lens)
    assert_close(out, ref["out"], dt, "cfg4 out")
    # the LSE comes back in float32, but this is an fp16 problem (the row
    # sums add fp16-rounded probabilities): the fp16 bar applies, as to every
    # fused LSE
    assert_close(lse, ref["lse"], dt, "cfg4 lse")
    for t, n in zip(ts, ("dq", "dk", "dv", "dek", "dev")):
        assert_close(t.grad, ref[n], dt, f"cfg4 {n}")


@pytest.mark.parametrize("K", [3, 5, 7])
@pytest.mark.parametrize("d", [1, 2, 4, 8])
def test_config5_full(K, d):
    from natten_amd.extras.allin1 import na1d_av_fused, na1d_qk_rpb

    import ctypes

    from natten_amd._core import _lib

    _say(f"[case] config 5 allin1 fp32 [8,2048,12,12] K={K} d={d}")
    f32 = torch.float32
    B, L, H, D = 8, 2048, 12, 12
    # the kernels the bench times: staged rank-1 (phase-major at K >= 5,
    # d = 8), and the dq pass (either; phase-major in the QK backward's
    # phase-major pair) forming the bias partials
    pp = _lib.make_rpb_params(1, B, H, D, (L,), K, d, False, _lib.NA_F32, 0.288)
    pl = _lib.NaRpbPlan()
    assert _lib.load().na_rpb_kernel_plan(ctypes.byref(pp), ctypes.byref(pl)) == 0
    want = _lib.RPB_PHASE if (K >= 5 and d == 8) else _lib.RPB_STAGED
    qk_pair = d > 1 and K >= 5 and (K - 1) * d >= 12
    assert (pl.qk, pl.av) == (want,) * 2 and pl.fused_bias == 1
    if "NATTEN_AMD_RPB_PHPAIR" not in os.environ:  # the default rule
        assert pl.dq == (_lib.RPB_PHASE if qk_pair else want)
    q, k, v = (randn((B, L, H, D), f32, s) for s in (40, 41, 42))
    rpb = randn((H, 2 * K - 1), f32, 43, std=0.02)
    qd, kd = _dev(q, k)
    rp = rpb.to(DEV).requires_grad_(True)
    logits = na1d_qk_rpb(qd, kd, rp, K, d, scale=0.288)
    ref = O.qk_rpb(q, k, rpb, K, d, 0.288)
    assert_close(logits, ref, f32, "cfg5 logits")
    gl = randn(logits.shape, f32, 44)
    logits.backward(gl.to(DEV))
    rq, rk, rr = O.grads(lambda a, b, c: O.qk_rpb(a, b, c, K, d, 0.288), (q, k, rpb), (gl,))
    assert_close(qd.grad, rq, f32, "cfg5 dq")
    assert_close(kd.grad, rk, f32, "cfg5 dk")
    assert_close(rp.grad, rr, f32, "cfg5 drpb")
    attn = torch.softmax(ref.float(), -1)
    ad = attn.to(DEV).requires_grad_(True)
    vd = v.to(DEV).requires_grad_(True)
    out = na1d_av_fused(ad, vd, K, d)
    assert_close(out, O.av_rpb(attn, v, K, d), f32, "cfg5 av")
    go = randn(out.shape, f32, 45)
    out.backward(go.to(DEV))
    ra, rv = O.grads(lambda a, b: O.av_rpb(a, b, K, d), (attn, v), (go,))
    assert_close(ad.grad, ra, f32, "cfg5 dattn")
    assert_close(vd.grad, rv, f32, "cfg5 dv")
