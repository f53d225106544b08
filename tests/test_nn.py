"""``natten_amd.nn`` layers: construction rules and parameter layout on the
CPU; on the GPU, the layer output (and input gradient) against an explicit
float64 composition — the projections written out from the state dict and
the oracle's neighborhood attention in between (reference layer
``nn/na2d.py:80-154``; tests ``tests/test_na{1,2,3}d.py``,
``tests/test_nn_module_grad.py``)."""

import sys

import pytest
import torch

from _helpers import DEV, assert_close, randn
from oracle import na as O


def _layers():
    from natten_amd import nn

    return {1: nn.NeighborhoodAttention1D, 2: nn.NeighborhoodAttention2D,
            3: nn.NeighborhoodAttention3D}


# ---------------------------------------------------------------- CPU checks

@pytest.mark.parametrize("kw,msg", [
    (dict(embed_dim=0, num_heads=1), "embed_dim must be positive"),
    (dict(embed_dim=12, num_heads=0), "num_heads must be positive"),
    (dict(embed_dim=10, num_heads=3), "divisible by num_heads"),
    (dict(embed_dim=12, num_heads=4, num_kv_heads=3), r"num_heads \(4\) must be divisible"),
])
def test_construction_errors(kw, msg):
    with pytest.raises(ValueError, match=msg):
        _layers()[2](kernel_size=3, **kw)


def test_parameter_layout_mha_and_gqa():
    L = _layers()
    mha = L[2](embed_dim=32, num_heads=4, kernel_size=3)
    assert set(dict(mha.named_parameters())) == {
        "qkv.weight", "qkv.bias", "proj.weight", "proj.bias"}
    assert mha.qkv.weight.shape == (96, 32) and mha.head_dim == 8
    gqa = L[1](embed_dim=32, num_heads=4, kernel_size=3, num_kv_heads=2, qkv_bias=False)
    names = set(dict(gqa.named_parameters()))
    assert names == {"q_proj.weight", "kv_proj.weight", "proj.weight", "proj.bias"}
    assert gqa.kv_proj.weight.shape == (2 * 2 * 8, 32)
    assert gqa.scale == 8 ** -0.5
    assert L[3](embed_dim=12, num_heads=3, kernel_size=3, qk_scale=0.5).scale == 0.5


def test_tuple_params_and_exports():
    import natten_amd

    layer = natten_amd.NeighborhoodAttention3D(embed_dim=12, num_heads=3, kernel_size=(3, 5, 3),
                                               stride=2, dilation=(1, 2, 1), is_causal=True)
    assert layer.kernel_size == (3, 5, 3) and layer.stride == (2, 2, 2)
    assert layer.dilation == (1, 2, 1) and layer.is_causal == (True, True, True)
    with pytest.raises(ValueError, match="kernel_size must have length 2"):
        natten_amd.NeighborhoodAttention2D(embed_dim=12, num_heads=3, kernel_size=(3, 3, 3))


def test_input_checks_precede_compute():
    layer = _layers()[2](embed_dim=12, num_heads=3, kernel_size=3)
    with pytest.raises(ValueError, match=r"Expected input shape \[B, H, W, C\]"):
        layer(torch.zeros(2, 5, 12))
    with pytest.raises(ValueError, match="must match embed_dim"):
        layer(torch.zeros(2, 5, 5, 8))


# ---------------------------------------------------------------- GPU parity

def _reference(layer, x, sizes=None, round_to=None):
    """float64 composition from the layer's state dict and the oracle.
    ``round_to``: round the projected q / k / v and the attention output to
    that dtype, as a layer running in it stores them between its steps."""
    sd = {k: v.detach().cpu().double() for k, v in layer.state_dict().items()}
    xd = x.to("cpu", torch.float64)
    lead = xd.shape[:-1]
    H, Hkv, D = layer.num_heads, layer.num_kv_heads, layer.head_dim

    def lin(name, t):
        y = t @ sd[name + ".weight"].T
        return y + sd[name + ".bias"] if name + ".bias" in sd else y

    if Hkv != H:
        q = lin("q_proj", xd).reshape(*lead, H, D)
        kv = lin("kv_proj", xd).reshape(*lead, 2, Hkv, D)
        k, v = kv[..., 0, :, :], kv[..., 1, :, :]
    else:
        qkv = lin("qkv", xd).reshape(*lead, 3, H, D)
        q, k, v = qkv[..., 0, :, :], qkv[..., 1, :, :], qkv[..., 2, :, :]
    if round_to is not None:
        q, k, v = (t.to(round_to).double() for t in (q, k, v))
    if sizes is not None:
        a = O.na_varlen(q, k, v, sizes.cpu(), layer.kernel_size, layer.dilation, layer.scale)
    else:
        a = O.na_functional(q, k, v, layer.kernel_size, layer.stride, layer.dilation,
                            layer.is_causal, layer.scale)
    if round_to is not None:
        a = a.to(round_to).double()
    return lin("proj", a.reshape(*a.shape[:-2], H * D))


NN_CASES = [
    # (name, rank, input shape, kwargs)
    ("1d", 1, (2, 19, 32), dict(num_heads=4, kernel_size=5, dilation=2)),
    ("1d_gqa_causal", 1, (2, 24, 64), dict(num_heads=4, num_kv_heads=1, kernel_size=7,
                                           is_causal=True)),
    ("2d", 2, (2, 9, 11, 32), dict(num_heads=2, kernel_size=(3, 5))),
    ("2d_stride", 2, (1, 8, 7, 32), dict(num_heads=2, kernel_size=3, stride=(2, 1))),
    ("2d_gqa", 2, (1, 10, 10, 64), dict(num_heads=4, num_kv_heads=2, kernel_size=5,
                                        dilation=2, qk_scale=0.3)),
    ("3d", 3, (1, 4, 6, 6, 24), dict(num_heads=3, kernel_size=3, is_causal=(True, False,
                                                                             False))),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", NN_CASES, ids=[c[0] for c in NN_CASES])
def test_layer_matches_composition(case):
    name, rank, shape, kw = case
    print(f"[case] nn {name}", flush=True)
    sys.stdout.flush()
    torch.manual_seed(0)
    layer = _layers()[rank](embed_dim=shape[-1], **kw).to(DEV)
    x = randn(shape, torch.float32, 11).to(DEV).requires_grad_(True)
    y = layer(x)
    ref = _reference(layer, x)
    assert_close(y, ref, torch.float32, f"{name} out")
    gy = randn(y.shape, torch.float32, 12)
    y.backward(gy.to(DEV))
    (gx,) = O.grads(lambda t: _reference(layer, t), (x,), (gy,))
    assert_close(x.grad, gx, torch.float32, f"{name} dx")
    for p in layer.parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all()


@pytest.mark.gpu
@pytest.mark.parametrize("rank", [1, 2, 3])
def test_attn_drop_routes_through_split_ops(rank):
    print(f"[case] nn attn_drop rank {rank}", flush=True)
    shapes = {1: (2, 15, 24), 2: (2, 7, 9, 24), 3: (1, 4, 5, 6, 24)}
    torch.manual_seed(1)
    layer = _layers()[rank](embed_dim=24, num_heads=3, kernel_size=3, stride=2,
                            attn_drop=0.25).to(DEV)
    x = randn(shapes[rank], torch.float32, 13).to(DEV)
    layer.eval()                          # dropout off: split path == composition
    assert_close(layer(x), _reference(layer, x), torch.float32, "eval")
    layer.train()
    y = layer(x)
    assert y.shape == _reference(layer, x).shape and torch.isfinite(y).all()


@pytest.mark.gpu
def test_varlen_routing():
    print("[case] nn varlen", flush=True)
    torch.manual_seed(2)
    L = _layers()
    l1 = L[1](embed_dim=32, num_heads=2, kernel_size=5, dilation=2).to(DEV)
    x1 = randn((3, 30, 32), torch.float32, 14).to(DEV)
    lens = torch.tensor([30, 17, 10], dtype=torch.int32)
    y1 = l1(x1, seq_lens=lens.to(DEV))
    assert_close(y1, _reference(l1, x1, lens), torch.float32, "1d varlen")
    l2 = L[2](embed_dim=32, num_heads=2, kernel_size=3).to(DEV)
    x2 = randn((2, 9, 8, 32), torch.float32, 15).to(DEV)
    sizes = torch.tensor([[9, 8], [5, 6]], dtype=torch.int32)
    y2 = l2(x2, spatial_sizes=sizes.to(DEV))
    assert_close(y2, _reference(l2, x2, sizes), torch.float32, "2d varlen")


@pytest.mark.gpu
def test_bf16_layer():
    print("[case] nn bf16", flush=True)
    torch.manual_seed(3)
    layer = _layers()[2](embed_dim=128, num_heads=4, kernel_size=7).to(DEV, torch.bfloat16)
    x = randn((1, 14, 14, 128), torch.bfloat16, 16).to(DEV)
    y = layer(x)
    # the layer stores q / k / v and the attention output in bf16 between
    # its steps: the composition (on the same bf16 weights) rounds them too
    assert_close(y, _reference(layer, x, round_to=torch.bfloat16), torch.bfloat16, "bf16 out")
