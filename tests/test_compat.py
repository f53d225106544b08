"""NATTEN-version compat layers (reference ``compat/``; tests
``tests/test_compat_for_version.py``, ``test_compat_v014.py``,
``test_compat_v015.py``, ``test_compat_v020.py``, ``test_compat_gradients.py``).

CPU: version routing, constructors, exports, validation, and the oracle's
non-square / per-axis RPB indexing against the pair-index formula of
``compat/v014.py:26-49`` built independently from ``pb_start``.  GPU: the
v0.14 QK+RPB / AV functions (heads-first, non-square kernels, per-axis
dilation) against the oracle, forward and gradients, and the layers against
the modern ones.  Tolerance: the fp32 bar (1e-5 relative), bf16 2e-2."""

import sys

import numpy as np
import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import na as O
from oracle import window as W


def _compat():
    from natten_amd import compat

    return compat


# ---------------------------------------------------------------- CPU checks

@pytest.mark.parametrize("version,name", [
    ("0.14.6", "v014"), ("0.14.0", "v014"), ("0.10.0", "v014"), ("0.15.0", "v015"),
    ("0.15.2", "v015"), ("0.16.0", "v017"), ("0.17.4", "v017"), ("0.20.0", "v020"),
    ("1.0.0", "v020"),
])
def test_for_version_routing(version, name):
    mod = _compat().for_version(version)
    assert mod.__name__ == f"natten_amd.compat.{name}"


def test_for_version_invalid_raises():
    with pytest.raises(Exception):
        _compat().for_version("not_a_version")


def test_exports():
    c = _compat()
    v014, v015, v017, v020 = (c.for_version(v) for v in ("0.14", "0.15", "0.17", "0.20"))
    for mod in (v014, v015, v017, v020):
        for name in mod.__all__:
            assert hasattr(mod, name), (mod.__name__, name)
    assert {"natten1dqkrpb", "natten2dav", "add_natten_handle"} <= set(v014.__all__)
    assert {"na3d", "NeighborhoodAttention3D", "has_fna"} <= set(v017.__all__)
    assert {"na3d_qk", "NeighborhoodAttention1D"} <= set(v020.__all__)
    assert v014.add_natten_handle("counter") == "counter"
    assert not v015.has_cuda() and not v020.has_fna()


def test_v014_layers_construction():
    v014 = _compat().for_version("0.14")
    with pytest.raises(ValueError, match="dim must be divisible by num_heads"):
        v014.NeighborhoodAttention1D(dim=10, kernel_size=3, num_heads=3)
    layer = v014.NeighborhoodAttention2D(dim=32, kernel_size=(3, 5), dilation=(1, 2),
                                         num_heads=4, qk_scale=0)
    assert set(dict(layer.named_parameters())) == {
        "qkv.weight", "qkv.bias", "proj.weight", "proj.bias"}
    assert layer.scale == 8 ** -0.5          # qk_scale=0 falls back, as `or` does
    assert layer.kernel_size == (3, 5) and layer.dilation == (1, 2)
    with pytest.raises(ValueError, match="Expected dim=32, got channels=16"):
        layer(torch.zeros(1, 6, 6, 16))
    v015 = _compat().for_version("0.15")
    l3 = v015.NeighborhoodAttention3D(dim=12, kernel_size=3, num_heads=3, is_causal=True)
    assert set(dict(l3.named_parameters())) == {
        "_impl.qkv.weight", "_impl.qkv.bias", "_impl.proj.weight", "_impl.proj.bias"}


def test_v014_validation_precedes_compute():
    v014 = _compat().for_version("0.14")
    q = torch.zeros(1, 2, 8, 4)
    with pytest.raises(ValueError, match=r"query and key must be \[B, H, L, D\]"):
        v014.natten1dqkrpb(q[0], q[0], torch.zeros(2, 5), 3, 1)
    with pytest.raises(ValueError, match=r"rpb must be \[heads, 5\] for kernel_size=3"):
        v014.natten1dqkrpb(q, q, torch.zeros(2, 7), 3, 1)
    q2 = torch.zeros(1, 2, 6, 7, 4)
    with pytest.raises(ValueError, match=r"rpb must be \[heads, 2\*Kh-1, 2\*Kw-1\]"):
        v014.natten2dqkrpb(q2, q2, torch.zeros(2, 5, 5), (3, 5), 1)
    with pytest.raises(ValueError, match="must be <= input spatial size"):
        v014.natten2dqkrpb(q2, q2, torch.zeros(2, 13, 5), (7, 3), 1)
    with pytest.raises(ValueError, match="dilation"):
        v014.natten1dav(torch.zeros(1, 2, 8, 3), q, 3, 3)


@pytest.mark.parametrize("shape,K,d", [((7, 8), (3, 3), (2, 2)), ((9, 7), (3, 5), (2, 1)),
                                        ((10, 6), (5, 3), (1, 2))])
def test_oracle_rpb_pair_index_per_axis(shape, K, d):
    """rpb = arange, q = k = 0: every logit is its bias entry, whose index is
    clip(pb_h + kh) * (2Kw - 1) + clip(pb_w + kw) (``compat/v014.py:26-49``;
    reference test ``test_compat_v014.py:121-145`` for the square case)."""
    H0, W0 = shape
    (kh, kw), (dh, dw) = K, d
    rpb = torch.arange((2 * kh - 1) * (2 * kw - 1), dtype=torch.float64).reshape(
        1, 2 * kh - 1, 2 * kw - 1)
    z = torch.zeros(1, H0, W0, 1, 4, dtype=torch.float64)
    got = O.qk_rpb(z, z, rpb, K, d)[0, :, :, 0]
    for i in range(H0):
        pi = W.pb_start(i, H0, kh, kh // 2, dh)
        for j in range(W0):
            pj = W.pb_start(j, W0, kw, kw // 2, dw)
            exp = [min(max(pi + a, 0), 2 * kh - 2) * (2 * kw - 1) + min(max(pj + b, 0), 2 * kw - 2)
                   for a in range(kh) for b in range(kw)]
            assert got[i, j].tolist() == [float(e) for e in exp]


def test_oracle_rpb_square_equals_per_axis_tuple():
    q, k = randn((1, 9, 8, 2, 4), torch.float64, 1), randn((1, 9, 8, 2, 4), torch.float64, 2)
    rpb = randn((2, 5, 5), torch.float64, 3)
    a = O.qk_rpb(q, k, rpb, 3, 2)
    b = O.qk_rpb(q, k, rpb, (3, 3), (2, 2))
    assert torch.equal(a, b)


# ---------------------------------------------------------------- GPU parity

def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _sf(x):
    """heads-first [B, H, *L, X] -> spatial-first [B, *L, H, X]."""
    return x.movedim(1, -2).contiguous()


def _hf(x):
    return x.movedim(-2, 1).contiguous()


V014_CASES = [
    # (tag, spatial, K, d, dtype)
    ("1d_k5_d2", (24,), 5, 2, torch.float32),
    ("1d_k7_bf16", (33,), 7, 1, torch.bfloat16),
    ("2d_sq", (9, 10), (3, 3), (2, 2), torch.float32),
    ("2d_nonsq", (11, 9), (3, 5), (2, 1), torch.float32),
    ("2d_nonsq_f16", (8, 12), (5, 3), (1, 3), torch.float16),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", V014_CASES, ids=[c[0] for c in V014_CASES])
def test_v014_qkrpb_av(case):
    tag, sp, K, d, dt = case
    _say(f"[case] compat v014 {tag}")
    v014 = _compat().for_version("0.14")
    rank = len(sp)
    qk_fn = v014.natten1dqkrpb if rank == 1 else v014.natten2dqkrpb
    av_fn = v014.natten1dav if rank == 1 else v014.natten2dav
    B, H, D = 2, 3, 16
    q, k, v = (randn((B, H) + sp + (D,), dt, s) for s in (1, 2, 3))
    Ks = (K,) * rank if isinstance(K, int) else K
    rpb = randn((H,) + tuple(2 * x - 1 for x in Ks), torch.float32, 4, std=0.5)
    tol = torch.float32 if dt == torch.float32 else dt

    qd, kd = q.to(DEV).requires_grad_(True), k.to(DEV).requires_grad_(True)
    rd = rpb.to(DEV).requires_grad_(True)
    logits = qk_fn(qd, kd, rd, K, d)
    assert logits.dtype == torch.promote_types(dt, torch.float32)
    ref = _hf(O.qk_rpb(_sf(q), _sf(k), rpb, K, d))
    assert_close(logits, ref, tol, f"{tag} logits")
    g = randn(logits.shape, torch.float32, 5)
    logits.backward(g.to(DEV))
    rq, rk, rr = O.grads(lambda a, b, c: _hf(O.qk_rpb(_sf(a), _sf(b), c, K, d)),
                         (q, k, rpb), (g,))
    assert_close(qd.grad, rq, tol, f"{tag} dq")
    assert_close(kd.grad, rk, tol, f"{tag} dk")
    assert_close(rd.grad, rr, torch.float32, f"{tag} drpb")

    attn = torch.softmax(ref.to(torch.float32), -1)
    ad, vd = attn.to(DEV).requires_grad_(True), v.to(DEV).requires_grad_(True)
    out = av_fn(ad, vd, K, d)
    assert out.dtype == torch.promote_types(torch.float32, dt)
    assert_close(out, _hf(O.av_rpb(_sf(attn), _sf(v), K, d)), tol, f"{tag} av")
    go = randn(out.shape, torch.float32, 6)
    out.backward(go.to(DEV))
    ra, rv = O.grads(lambda a, b: _hf(O.av_rpb(_sf(a), _sf(b), K, d)), (attn, v), (go,))
    assert_close(ad.grad, ra, tol, f"{tag} dattn")
    assert_close(vd.grad, rv, tol, f"{tag} dv")


@pytest.mark.gpu
def test_v014_rpb_is_added_linearly():
    """Reference test ``test_compat_v014.py:68-81``."""
    _say("[case] compat v014 rpb linearity")
    v014 = _compat().for_version("0.14")
    q, k = (randn((1, 2, 8, 4), torch.float32, s).to(DEV) for s in (7, 8))
    ra, rb = (randn((2, 9), torch.float32, s).to(DEV) for s in (9, 10))
    base = v014.natten1dqkrpb(q, k, torch.zeros_like(ra), 5, 1)
    oa = v014.natten1dqkrpb(q, k, ra, 5, 1)
    ob = v014.natten1dqkrpb(q, k, rb, 5, 1)
    oab = v014.natten1dqkrpb(q, k, ra + rb, 5, 1)
    assert torch.allclose(oab - base, (oa - base) + (ob - base), atol=1e-6, rtol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("rank,attn_drop", [(1, 0.0), (2, 0.0), (2, 0.3)])
def test_v014_layers_match_modern(rank, attn_drop):
    _say(f"[case] compat v014 layer rank {rank} attn_drop {attn_drop}")
    from natten_amd import nn

    v014 = _compat().for_version("0.14")
    old_cls = v014.NeighborhoodAttention1D if rank == 1 else v014.NeighborhoodAttention2D
    new_cls = nn.NeighborhoodAttention1D if rank == 1 else nn.NeighborhoodAttention2D
    torch.manual_seed(4)
    old = old_cls(dim=32, kernel_size=5, dilation=2, num_heads=4, attn_drop=attn_drop).to(DEV)
    new = new_cls(embed_dim=32, num_heads=4, kernel_size=5, dilation=2).to(DEV)
    new.load_state_dict(old.state_dict())
    old.eval()
    shape = (2, 21, 32) if rank == 1 else (2, 11, 12, 32)
    x = randn(shape, torch.float32, 11).to(DEV)
    assert_close(old(x), new(x).cpu().double(), torch.float32, "layer")


@pytest.mark.gpu
@pytest.mark.parametrize("version", ["0.15", "0.17", "0.20"])
def test_fused_compat_functions(version):
    _say(f"[case] compat {version} fused")
    mod = _compat().for_version(version)
    q, k, v = (randn((1, 6, 7, 8, 2, 8), torch.float32, s) for s in (1, 2, 3))
    kw = dict(kernel_size=(3, 3, 3), dilation=(1, 2, 1), is_causal=(True, False, False),
              scale=0.41)
    if version == "0.20":
        kw["stride"] = 1
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = mod.na3d(*ts, **kw)
    ref = O.na_functional(q, k, v, (3, 3, 3), (1, 1, 1), (1, 2, 1), (True, False, False), 0.41)
    assert_close(out, ref, torch.float32, f"{version} na3d")
    go = randn(out.shape, torch.float32, 4)
    out.backward(go.to(DEV))
    refg = O.grads(lambda a, b, c: O.na_functional(a, b, c, (3, 3, 3), (1, 1, 1), (1, 2, 1),
                                                   (True, False, False), 0.41), (q, k, v), (go,))
    for t, r, n in zip(ts, refg, "qkv"):
        assert_close(t.grad, r, torch.float32, f"{version} d{n}")
