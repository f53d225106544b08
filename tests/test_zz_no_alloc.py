"""na_bwd_noalloc: the fused backward with the library's fixed per-GPU
scratch in place of a caller workspace, called through the C ABI and
compared with na_bwd (caller workspace) on the same inputs — bit for bit,
since both run the same deterministic kernels — on two calls in a row, the
second with a smaller problem, for the two workspace users: the additional
tokens' gradient partials (fp16, matrix-core reduction) and the delta rows
of the generic kernels (fp32).  Problems beyond the scratch size are
rejected before anything launches."""

import pytest
import torch

from _helpers import DEV, randn

from natten_amd._core import _lib, hip


def _p(t):
    return _lib.ptr(t)


def _problem(B, sp, H, Hkv, D, nx, dtype, ks, dil, seed):
    q = randn((B, *sp, H, D), dtype, seed).to(DEV)
    k = randn((B, *sp, Hkv, D), dtype, seed + 1).to(DEV)
    v = randn((B, *sp, Hkv, D), dtype, seed + 2).to(DEV)
    ek = randn((B, nx, Hkv, D), dtype, seed + 3).to(DEV) if nx else None
    ev = randn((B, nx, Hkv, D), dtype, seed + 4).to(DEV) if nx else None
    rank = len(sp)
    args = (ks, (1,) * rank, dil, (False,) * rank, None)
    out, lse = hip.fused_forward(q, k, v, *args, extra_k=ek, extra_v=ev)
    do = randn(out.shape, dtype, seed + 5).to(DEV)
    dlse = randn(lse.shape, torch.float32, seed + 6).to(DEV)
    p = hip._params(q, k, ks, (1,) * rank, dil, (False,) * rank, None, nx)
    return p, (q, k, v, ek, ev, out, lse, do, dlse)


def _grads(lib, p, t, noalloc, stream=None):
    q, k, v, ek, ev, out, lse, do, dlse = t
    g = [torch.full_like(x, float("nan")) for x in (q, k, v)]
    gx = [torch.full_like(x, float("nan")) if x is not None else None for x in (ek, ev)]
    torch.cuda.synchronize()
    stream = _lib.stream_of(q) if stream is None else stream
    common = [_p(q), _p(k), _p(v), _p(ek), _p(ev), _p(out), _p(lse), _p(do), _p(dlse),
              _p(g[0]), _p(g[1]), _p(g[2]), _p(gx[0]), _p(gx[1])]
    if noalloc:
        rc = lib.na_bwd_noalloc(p, *common, stream)
    else:
        nbytes = int(lib.na_bwd_workspace_bytes(p))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
        rc = lib.na_bwd(p, *common, _p(ws), nbytes, stream)
    _lib.check(rc, "na_bwd_noalloc" if noalloc else "na_bwd")
    torch.cuda.synchronize()
    return g + [x for x in gx if x is not None]


CASES = [
    # (name, [first problem, second (smaller) problem])
    ("extra_tokens_fp16", [
        dict(B=4, sp=(1024,), H=8, Hkv=2, D=64, nx=16, dtype=torch.float16, ks=(63,),
             dil=(2,)),
        dict(B=2, sp=(300,), H=8, Hkv=2, D=64, nx=5, dtype=torch.float16, ks=(15,),
             dil=(3,)),
    ]),
    ("generic_fp32", [
        dict(B=2, sp=(40, 40), H=4, Hkv=4, D=32, nx=0, dtype=torch.float32, ks=(7, 7),
             dil=(1, 2)),
        dict(B=1, sp=(17, 23), H=2, Hkv=1, D=16, nx=3, dtype=torch.float32, ks=(5, 3),
             dil=(2, 1)),
    ]),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,probs", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_workspace_backward(name, probs):
    lib = _lib.load()
    for i, kw in enumerate(probs):
        print(f"[case] na_bwd_noalloc {name} call {i}: {kw}", flush=True)
        p, t = _problem(seed=10 * i + 1, **kw)
        assert 0 < lib.na_bwd_workspace_bytes(p) <= lib.na_bwd_noalloc_max_workspace()
        ref = _grads(lib, p, t, noalloc=False)
        got = _grads(lib, p, t, noalloc=True)
        for a, b, n in zip(got, ref, ("dq", "dk", "dv", "dek", "dev")):
            assert not torch.isnan(a).any(), f"{name} call {i}: {n} not written"
            assert torch.equal(a, b), f"{name} call {i}: {n} differs from na_bwd"


@pytest.mark.gpu
def test_noalloc_on_a_side_stream():
    """The scratch is the one of the stream's device: a call on a stream other
    than torch's current one (same device here) matches na_bwd."""
    lib = _lib.load()
    kw = CASES[0][1][1]
    print(f"[case] na_bwd_noalloc side stream: {kw}", flush=True)
    p, t = _problem(seed=7, **kw)
    ref = _grads(lib, p, t, noalloc=False)
    side = torch.cuda.Stream()
    got = _grads(lib, p, t, noalloc=True, stream=side.cuda_stream)
    for a, b, n in zip(got, ref, ("dq", "dk", "dv", "dek", "dev")):
        assert torch.equal(a, b), f"side stream: {n} differs from na_bwd"


def test_noalloc_rejects_problems_beyond_the_scratch():
    """Checked on the host before any device call: a problem whose workspace
    exceeds the fixed scratch gets NA_ERR_UNSUPPORTED (no GPU needed)."""
    lib = _lib.load()
    cap = int(lib.na_bwd_noalloc_max_workspace())
    assert cap == 32 << 20
    # fp32 on the generic kernels: one float of delta per (query, head)
    p = _lib.make_params(1, 64, 16, 16, 32, _lib.NA_F32, (16384,), (7,), (1,), (1,), (0,),
                         0.125)
    assert lib.na_bwd_workspace_bytes(p) > cap
    rc = lib.na_bwd_noalloc(p, *([None] * 14), None)
    assert rc == 2  # NA_ERR_UNSUPPORTED
    assert b"fixed maximum" in lib.na_last_error()
