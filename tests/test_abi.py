"""CPU checks of the C ABI: the library loads, exports every function the
header declares, and its host window twins (the code the kernels run)
agree bit for bit with the oracle.  No device compute here."""

import os
import re

import numpy as np
import pytest
import torch

from oracle import window as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "natten_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(na[0-9a-z_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    for n in ("na_fwd", "na_bwd", "na_bwd_workspace_bytes", "na_qk_fwd", "na_av_fwd",
              "na_qk_bwd", "na_av_bwd", "na_rpb_qk_fwd", "na_rpb_av_fwd", "na_rpb_qk_bwd",
              "na_rpb_av_bwd", "na_rpb_bwd_workspace_bytes",
              "na_merge_fwd", "na_merge_bwd",
              "na_neighbor_table", "na_last_error", "na_abi_version"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from natten_amd._core import _lib

    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert set(_declared_functions()) == set(_lib.SIGNATURES), \
        "ctypes signature table and header disagree"
    assert lib.na_abi_version() == _lib.ABI_VERSION


def test_host_window_twins_match_oracle_exhaustively():
    from natten_amd._core import _lib

    lib = _lib.load()
    n = 0
    for L in range(1, 72):
        for K in range(1, L + 1):
            nh = K // 2
            for d in range(1, L // K + 1):
                for i in range(L):
                    s = W.window_start(i, L, K, nh, d)
                    assert lib.na_window_start(i, L, K, nh, d) == s
                    assert lib.na_window_end(s, L, K, d) == W.window_end(s, L, K, d)
                    assert lib.na_pb_start(i, L, K, nh, d) == W.pb_start(i, L, K, nh, d)
                    assert lib.na_window_start_partition(i, L, K, nh, d) == \
                        W.window_start_partition(i, L, K, nh, d)
                    n += 1
    assert n > 100000


def test_product_utils_window_api():
    from natten_amd.utils import compute_pb_start, compute_window_start_end, get_window_start

    assert get_window_start(31, 32, 3, 1, 1) == 29
    q = np.arange(64)
    s, e = compute_window_start_end(q, 64, 7, 4)
    rs = np.array([W.window_start(int(i), 64, 7, 3, 4) for i in q])
    assert (s == rs).all() and (e == np.minimum(64, rs + 28)).all()
    assert (compute_pb_start(q, 64, 7, 4) == [W.pb_start(int(i), 64, 7, 3, 4) for i in q]).all()


def test_invalid_params_rejected_without_device():
    """Parameter validation happens on the host before any launch."""
    from natten_amd._core import _lib

    lib = _lib.load()
    p = _lib.make_params(2, 1, 4, 3, 32, _lib.NA_BF16, (8, 8), (3, 3), (1, 1), (1, 1), (0, 0), 1.0)
    rc = lib.na_fwd(p, None, None, None, None, None, None, None, None)
    assert rc == 1 and b"divisible" in lib.na_last_error()
    p = _lib.make_params(4, 1, 4, 4, 32, _lib.NA_BF16, (8, 8), (3, 3), (1, 1), (1, 1), (0, 0), 1.0)
    assert lib.na_fwd(p, None, None, None, None, None, None, None, None) == 1
    p = _lib.make_params(1, 1, 4, 4, 32, _lib.NA_BF16, (8,), (9,), (1,), (1,), (0,), 1.0)
    assert lib.na_qk_fwd(p, None, None, None, None) == 1
    assert b"exceeds" in lib.na_last_error()
    p = _lib.make_params(1, 0, 4, 4, 32, _lib.NA_BF16, (8,), (3,), (1,), (1,), (0,), 1.0)
    assert lib.na_fwd(p, None, None, None, None, None, None, None, None) == 0  # empty batch
    # the workspace is what the chosen kernels read: none for the lean
    # backward, one float of delta per (query, head) on the generic kernels
    p = _lib.make_params(1, 1, 4, 4, 32, _lib.NA_BF16, (8,), (3,), (1,), (1,), (0,), 1.0)
    assert lib.na_bwd_workspace_bytes(p) == 0
    p = _lib.make_params(1, 1, 4, 4, 32, _lib.NA_F32, (8,), (3,), (1,), (1,), (0,), 1.0)
    assert lib.na_bwd_workspace_bytes(p) >= 4 * 8 * 4
    rc = lib.na_bwd(p, *([None] * 15), 0, None)
    assert rc == 1


def test_no_cpu_fallback():
    import natten_amd

    q = torch.randn(1, 16, 2, 8)
    with pytest.raises(RuntimeError, match="HIP"):
        natten_amd.na1d(q, q, q, kernel_size=3)


def test_validation_messages_match_reference():
    import natten_amd

    q = torch.randn(1, 8, 2, 4)
    with pytest.raises(ValueError, match="kernel_size\\[0\\]=9 must be <= input spatial size 8"):
        natten_amd.na1d(q, q, q, kernel_size=9)
    with pytest.raises(ValueError, match="stride\\[0\\]=5 must be <= kernel_size\\[0\\]=3"):
        natten_amd.na1d(q, q, q, kernel_size=3, stride=5)
    with pytest.raises(ValueError, match="exceeds input size 8"):
        natten_amd.na1d(q, q, q, kernel_size=3, dilation=3)
    with pytest.raises(ValueError, match="divisible by heads_kv"):
        natten_amd.na1d(torch.randn(1, 8, 3, 4), q, q, kernel_size=3)
    with pytest.raises(ValueError, match="must both be provided"):
        natten_amd.na1d(q, q, q, kernel_size=3, additional_keys=torch.randn(1, 2, 2, 4))
    with pytest.raises(ValueError, match="seq_lens must be >= kernel_size"):
        natten_amd.na1d_varlen(q, q, q, torch.tensor([2], dtype=torch.int32), kernel_size=3)


def test_backend_registry():
    import natten_amd

    assert natten_amd.get_backend() == "hip"
    natten_amd.set_backend("hip")
    natten_amd.set_backend("auto")
    with pytest.raises(ValueError, match="Unknown backend"):
        natten_amd.set_backend("pure")


def test_reference_tier_probes_exist():
    """natten_mlx's tier probes (``__init__.py:23-28``) exist and report
    that neither the Metal nor the nanobind tier is present."""
    import natten_amd

    assert natten_amd.has_metal() is False
    assert natten_amd.has_nanobind() is False
    assert "has_metal" in natten_amd.__all__ and "has_nanobind" in natten_amd.__all__


def test_fused_operator_registered():
    """libnatten_amd_torch.so registers natten_amd::na_fused (the fused op's
    C++ autograd node); with host tensors it raises like the rest of the
    package (no CPU implementation)."""
    from natten_amd._core import _lib

    op = _lib.fused_op()
    assert op is not None
    q = torch.randn(1, 16, 2, 8, requires_grad=True)
    with pytest.raises(RuntimeError, match="HIP"):
        op(q, q, q, None, None, None, [3], [1], [1], [0], 0.3, 0, 0)
