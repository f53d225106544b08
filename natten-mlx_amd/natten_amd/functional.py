"""Public functional API (mirrors ``src/natten_mlx/functional.py``).

Same functions, arguments, validation rules and error messages as the
reference, on PyTorch-ROCm tensors in the spatial-first layout
``[B, *spatial, heads, dim]``.  Differences are in how the work is done,
not in the result:

* GQA/MQA is handled inside the kernels (query head h reads key/value head
  h // (H_q / H_kv)) instead of materialising ``repeat`` copies
  (reference ``functional.py:29-33,255-256``).
* ``return_lse`` and ``additional_keys/values`` run in the fused kernel,
  which joins the extra tokens to the same online softmax.  That equals the
  reference's composition split QK -> logsumexp -> softmax -> split AV ->
  ``merge_attentions`` (``functional.py:277-292``) in exact arithmetic.
* The FMHA fast path (kernel covers the extent, stride 1, non-causal;
  ``functional.py:141-187``) runs the same kernel in dense mode.
Returned LSE dtypes follow the reference: the query dtype, except after an
additional-token merge on the neighborhood path, where it is float32
(``merge.py:53,68``).
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from .autograd import (
    FusedSpec,
    device_extents,
    na1d_av_with_grad,
    na1d_qk_with_grad,
    na2d_av_with_grad,
    na2d_qk_with_grad,
    na3d_av_with_grad,
    na3d_qk_with_grad,
    na_fused_with_grad,
)
from .utils.params import (
    check_dilation_kernel_vs_input,
    check_kernel_size_vs_input,
    check_stride_vs_kernel,
    normalize_kernel_size,
    normalize_tuple_param,
)

_LAYOUTS = {1: "[B, L, H, D]", 2: "[B, H, W, heads, dim]", 3: "[B, D, H, W, heads, dim]"}


def _validate_qkv(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, rank: int) -> int:
    """Shape checks with GQA (reference ``functional.py:36-68``); returns the
    KV repeat factor."""
    expected_ndim = rank + 3
    if query.ndim != expected_ndim or key.ndim != expected_ndim or value.ndim != expected_ndim:
        raise ValueError(f"na{rank}d expects query/key/value with shape {_LAYOUTS[rank]}.")
    spatial_q, spatial_k, spatial_v = (tuple(query.shape[1:-2]), tuple(key.shape[1:-2]),
                                       tuple(value.shape[1:-2]))
    if spatial_q != spatial_k or spatial_q != spatial_v:
        raise ValueError(
            f"Spatial dimensions must match: Q={spatial_q}, K={spatial_k}, V={spatial_v}.")
    if query.shape[0] != key.shape[0] or query.shape[0] != value.shape[0]:
        raise ValueError("Batch dimensions must match.")
    heads_q, dim_q = query.shape[-2], query.shape[-1]
    heads_kv, dim_k = key.shape[-2], key.shape[-1]
    if dim_q != dim_k:
        raise ValueError(f"Head dim must match: Q has {dim_q}, K has {dim_k}.")
    if key.shape[-2] != value.shape[-2]:
        raise ValueError("K and V must have same number of heads.")
    if key.shape[-1] != value.shape[-1]:
        raise ValueError(f"Head dim must match: K has {dim_k}, V has {value.shape[-1]}.")
    if heads_q % heads_kv != 0:
        raise ValueError(f"heads_q ({heads_q}) must be divisible by heads_kv ({heads_kv}) for GQA.")
    return heads_q // heads_kv


def _validate_additional_kv(query, key, additional_keys, additional_values):
    """Reference ``functional.py:107-138``.  Extra tokens keep the KV head
    count (the kernel maps query heads onto them like onto key/value)."""
    if additional_keys is None and additional_values is None:
        return None, None
    if additional_keys is None or additional_values is None:
        raise ValueError("additional_keys and additional_values must both be provided or both None.")
    if additional_keys.ndim != 4 or additional_values.ndim != 4:
        raise ValueError("additional_keys/additional_values must be 4D: [B, N_extra, heads_kv, dim].")
    if additional_keys.shape[0] != query.shape[0]:
        raise ValueError("additional_keys batch must match query batch.")
    if additional_values.shape[0] != query.shape[0]:
        raise ValueError("additional_values batch must match query batch.")
    if additional_keys.shape[-1] != query.shape[-1]:
        raise ValueError("additional_keys head dim must match query head dim.")
    if additional_values.shape[-1] != query.shape[-1]:
        raise ValueError("additional_values head dim must match query head dim.")
    if additional_keys.shape[-2] != additional_values.shape[-2]:
        raise ValueError("additional_keys and additional_values must have same number of heads.")
    if additional_keys.shape[1] != additional_values.shape[1]:
        raise ValueError("additional_keys and additional_values must have same N_extra.")
    if additional_keys.shape[-2] != key.shape[-2]:
        raise ValueError("additional_keys/additional_values must have heads_kv heads "
                         f"({key.shape[-2]}), got {additional_keys.shape[-2]}.")
    ak, av = additional_keys, additional_values
    if ak.dtype != query.dtype:
        ak = ak.to(query.dtype)
    if av.dtype != query.dtype:
        av = av.to(query.dtype)
    return ak, av


def _is_full_attention(kernel_size: tuple, spatial_shape: tuple) -> bool:
    """Reference ``functional.py:141-143``."""
    return all(ks >= s for ks, s in zip(kernel_size, spatial_shape))


# Validated specs by call signature (shapes, dtypes and the arguments as
# passed): a training loop calls with the same few signatures every step,
# and the checks and tuple normalisation cost more host time than the rest
# of the call.  Only successful validations are stored; unhashable arguments
# (lists) are validated on every call.
_spec_cache: dict = {}
_SPEC_MAX = 512


def _fused_spec(rank, query, key, value, kernel_size, stride, dilation, is_causal, scale,
                additional_keys, additional_values) -> FusedSpec:
    _validate_qkv(query, key, value, rank)
    _validate_additional_kv(query, key, additional_keys, additional_values)
    spatial_shape = tuple(query.shape[1:-2])
    head_dim = query.shape[-1]

    ks = normalize_kernel_size(kernel_size, rank)
    st = normalize_tuple_param(stride, rank, "stride")
    dil = normalize_tuple_param(dilation, rank, "dilation")
    caus = normalize_tuple_param(is_causal, rank, "is_causal")

    check_kernel_size_vs_input(ks, spatial_shape)
    check_stride_vs_kernel(st, ks)
    check_dilation_kernel_vs_input(dil, ks, spatial_shape)

    scale_value = head_dim ** -0.5 if scale is None else float(scale)
    dense = (_is_full_attention(ks, spatial_shape) and all(s == 1 for s in st)
             and not any(caus))
    return FusedSpec(tuple(ks), tuple(st), tuple(dil), tuple(bool(c) for c in caus), scale_value,
                     dense)


def _na(rank, query, key, value, kernel_size, stride, dilation, is_causal, scale, return_lse,
        additional_keys, additional_values):
    add = additional_keys is not None or additional_values is not None
    try:
        ck = (rank, query.shape, key.shape, value.shape, query.dtype, key.dtype, value.dtype,
              kernel_size, stride, dilation, is_causal, scale,
              (None if additional_keys is None else (additional_keys.shape, additional_keys.dtype),
               None if additional_values is None
               else (additional_values.shape, additional_values.dtype)) if add else None)
        spec = _spec_cache.get(ck)
    except TypeError:  # an unhashable argument
        ck = spec = None
    if spec is None:
        spec = _fused_spec(rank, query, key, value, kernel_size, stride, dilation, is_causal,
                           scale, additional_keys, additional_values)
        if ck is not None:
            if len(_spec_cache) >= _SPEC_MAX:
                _spec_cache.clear()
            _spec_cache[ck] = spec
    add_k, add_v = additional_keys, additional_values
    if add:
        if add_k.dtype != query.dtype:
            add_k = add_k.to(query.dtype)
        if add_v.dtype != query.dtype:
            add_v = add_v.to(query.dtype)
    if key.dtype != query.dtype:
        key = key.to(query.dtype)
    if value.dtype != query.dtype:
        value = value.to(query.dtype)
    dense = spec.dense
    out, lse = na_fused_with_grad(query, key, value, spec, add_k, add_v)
    if not return_lse:
        return out
    if add_k is not None and not dense:
        return out, lse
    return out, lse.to(query.dtype)


def na1d(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
         kernel_size: Union[int, Tuple[int]], stride: Union[int, Tuple[int]] = 1,
         dilation: Union[int, Tuple[int]] = 1, is_causal: Union[bool, Tuple[bool]] = False,
         scale: Optional[float] = None, return_lse: bool = False,
         additional_keys: Optional[torch.Tensor] = None,
         additional_values: Optional[torch.Tensor] = None):
    """1D neighborhood attention (reference ``functional.py:207-294``).

    query ``[B, L, H_q, D]``; key/value ``[B, L, H_kv, D]``; optional extra
    tokens ``[B, N_extra, H_kv, D]``.  Returns ``[B, ceil(L/stride), H_q, D]``
    or ``(out, lse)``.
    """
    return _na(1, query, key, value, kernel_size, stride, dilation, is_causal, scale, return_lse,
               additional_keys, additional_values)


def na2d(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
         kernel_size: Union[int, Tuple[int, int]], stride: Union[int, Tuple[int, int]] = 1,
         dilation: Union[int, Tuple[int, int]] = 1,
         is_causal: Union[bool, Tuple[bool, bool]] = False, scale: Optional[float] = None,
         return_lse: bool = False, additional_keys: Optional[torch.Tensor] = None,
         additional_values: Optional[torch.Tensor] = None):
    """2D neighborhood attention (reference ``functional.py:297-383``)."""
    return _na(2, query, key, value, kernel_size, stride, dilation, is_causal, scale, return_lse,
               additional_keys, additional_values)


def na3d(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
         kernel_size: Union[int, Tuple[int, int, int]],
         stride: Union[int, Tuple[int, int, int]] = 1,
         dilation: Union[int, Tuple[int, int, int]] = 1,
         is_causal: Union[bool, Tuple[bool, bool, bool]] = False, scale: Optional[float] = None,
         return_lse: bool = False, additional_keys: Optional[torch.Tensor] = None,
         additional_values: Optional[torch.Tensor] = None):
    """3D neighborhood attention (reference ``functional.py:386-473``)."""
    return _na(3, query, key, value, kernel_size, stride, dilation, is_causal, scale, return_lse,
               additional_keys, additional_values)


# ---------------------------------------------------------------------------
# split ops (reference functional.py:476-634)

def _qk(rank, query, key, kernel_size, dilation, stride, is_causal, scale, fn):
    _validate_qkv(query, key, key, rank)
    spatial = tuple(query.shape[1:-2])
    ks = normalize_kernel_size(kernel_size, rank)
    st = normalize_tuple_param(stride, rank, "stride")
    dil = normalize_tuple_param(dilation, rank, "dilation")
    caus = normalize_tuple_param(is_causal, rank, "is_causal")
    check_kernel_size_vs_input(ks, spatial)
    check_stride_vs_kernel(st, ks)
    check_dilation_kernel_vs_input(dil, ks, spatial)
    return fn(query, key, ks, st, dil, caus, scale)


def _av(rank, attn, value, kernel_size, dilation, stride, is_causal, fn):
    nd = rank + 3
    if attn.ndim != nd or value.ndim != nd:
        raise ValueError(f"attn and value must be {nd}D for na{rank}d_av")
    if attn.shape[0] != value.shape[0] or attn.shape[-2] % value.shape[-2] != 0:
        raise ValueError(
            "attn and value must match batch and heads dimensions; "
            f"got {tuple(attn.shape)} and {tuple(value.shape)}")
    spatial = tuple(value.shape[1:-2])
    ks = normalize_kernel_size(kernel_size, rank)
    st = normalize_tuple_param(stride, rank, "stride")
    dil = normalize_tuple_param(dilation, rank, "dilation")
    caus = normalize_tuple_param(is_causal, rank, "is_causal")
    check_kernel_size_vs_input(ks, spatial)
    check_stride_vs_kernel(st, ks)
    check_dilation_kernel_vs_input(dil, ks, spatial)
    return fn(attn, value, ks, st, dil, caus)


def na1d_qk(query, key, kernel_size, dilation=1, *, stride=1, is_causal=False, scale=None):
    """Separate 1D query-key logits, ``[B, ceil(L/stride), H, K]``; invalid
    slots hold -inf."""
    return _qk(1, query, key, kernel_size, dilation, stride, is_causal, scale, na1d_qk_with_grad)


def na1d_av(attn, value, kernel_size, dilation=1, *, stride=1, is_causal=False):
    """Separate 1D attention-value op; attn ``[B, ceil(L/stride), H, K]``."""
    return _av(1, attn, value, kernel_size, dilation, stride, is_causal, na1d_av_with_grad)


def na2d_qk(query, key, kernel_size, dilation=1, *, stride=1, is_causal=False, scale=None):
    """Separate 2D query-key logits, ``[B, Oh, Ow, heads, Kh*Kw]``."""
    return _qk(2, query, key, kernel_size, dilation, stride, is_causal, scale, na2d_qk_with_grad)


def na2d_av(attn, value, kernel_size, dilation=1, *, stride=1, is_causal=False):
    """Separate 2D attention-value op."""
    return _av(2, attn, value, kernel_size, dilation, stride, is_causal, na2d_av_with_grad)


def na3d_qk(query, key, kernel_size, dilation=1, *, stride=1, is_causal=False, scale=None):
    """Separate 3D query-key logits, ``[B, Od, Oh, Ow, heads, Kd*Kh*Kw]``."""
    return _qk(3, query, key, kernel_size, dilation, stride, is_causal, scale, na3d_qk_with_grad)


def na3d_av(attn, value, kernel_size, dilation=1, *, stride=1, is_causal=False):
    """Separate 3D attention-value op."""
    return _av(3, attn, value, kernel_size, dilation, stride, is_causal, na3d_av_with_grad)


# ---------------------------------------------------------------------------
# varlen (reference functional.py:637-828)

def _validate_spatial_sizes(spatial_sizes, batch_size, max_spatial, kernel_size, rank):
    if spatial_sizes.ndim != 2 or spatial_sizes.shape[0] != batch_size or spatial_sizes.shape[1] != rank:
        raise ValueError(f"spatial_sizes must be a [B, {rank}] array, "
                         f"got shape {tuple(spatial_sizes.shape)}.")
    if spatial_sizes.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"spatial_sizes must be int32 or int64, got {spatial_sizes.dtype}.")
    host = spatial_sizes.detach().cpu()
    for d in range(rank):
        min_dim = int(host[:, d].min())
        max_dim = int(host[:, d].max())
        if min_dim < kernel_size[d]:
            raise ValueError(f"All spatial_sizes[:,{d}] must be >= kernel_size[{d}] "
                             f"({kernel_size[d]}), but min={min_dim}.")
        if max_dim > max_spatial[d]:
            raise ValueError(f"All spatial_sizes[:,{d}] must be <= max_spatial[{d}] "
                             f"({max_spatial[d]}), but max={max_dim}.")


def _validate_seq_lens(seq_lens, batch_size, l_max, kernel_size):
    if seq_lens.ndim != 1 or seq_lens.shape[0] != batch_size:
        raise ValueError(f"seq_lens must be a 1-D array of length B={batch_size}, "
                         f"got shape {tuple(seq_lens.shape)}.")
    if seq_lens.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"seq_lens must be int32 or int64, got {seq_lens.dtype}.")
    host = seq_lens.detach().cpu()
    min_len, max_len = int(host.min()), int(host.max())
    if min_len < kernel_size:
        raise ValueError(f"All seq_lens must be >= kernel_size ({kernel_size}), "
                         f"but min(seq_lens)={min_len}.")
    if max_len > l_max:
        raise ValueError(f"All seq_lens must be <= L_max ({l_max}), but max(seq_lens)={max_len}.")
    return min_len


def na1d_varlen(query, key, value, seq_lens, kernel_size, dilation=1, scale=None):
    """Variable-length 1D NA (reference ``functional.py:697-739``); rows at
    or beyond ``seq_lens[b]`` are zero."""
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("na1d_varlen expects query/key/value with shape [B, L, H, D].")
    if query.shape != key.shape or query.shape != value.shape:
        raise ValueError("query, key, and value must have identical shapes.")
    B, L_max = query.shape[0], query.shape[1]
    ks = normalize_kernel_size(kernel_size, 1)
    dil = normalize_tuple_param(dilation, 1, "dilation")
    _validate_seq_lens(seq_lens, B, L_max, ks[0])
    scale_value = query.shape[-1] ** -0.5 if scale is None else float(scale)
    from .autograd import na1d_varlen_with_grad
    return na1d_varlen_with_grad(query, key, value, seq_lens, ks, dil, scale_value)


def na2d_varlen(query, key, value, spatial_sizes, kernel_size, dilation=1, scale=None):
    """Variable-length 2D NA (reference ``functional.py:742-783``)."""
    if query.ndim != 5 or key.ndim != 5 or value.ndim != 5:
        raise ValueError("na2d_varlen expects query/key/value with shape [B, H, W, heads, D].")
    if query.shape != key.shape or query.shape != value.shape:
        raise ValueError("query, key, and value must have identical shapes.")
    B, H_max, W_max = query.shape[0], query.shape[1], query.shape[2]
    ks = normalize_kernel_size(kernel_size, 2)
    dil = normalize_tuple_param(dilation, 2, "dilation")
    _validate_spatial_sizes(spatial_sizes, B, (H_max, W_max), ks, 2)
    scale_value = query.shape[-1] ** -0.5 if scale is None else float(scale)
    from .autograd import na2d_varlen_with_grad
    return na2d_varlen_with_grad(query, key, value, spatial_sizes, ks, dil, scale_value)


def na3d_varlen(query, key, value, spatial_sizes, kernel_size, dilation=1, scale=None):
    """Variable-length 3D NA (reference ``functional.py:786-828``)."""
    if query.ndim != 6 or key.ndim != 6 or value.ndim != 6:
        raise ValueError(
            "na3d_varlen expects query/key/value with shape [B, D, H, W, heads, dim].")
    if query.shape != key.shape or query.shape != value.shape:
        raise ValueError("query, key, and value must have identical shapes.")
    B = query.shape[0]
    D_max, H_max, W_max = query.shape[1], query.shape[2], query.shape[3]
    ks = normalize_kernel_size(kernel_size, 3)
    dil = normalize_tuple_param(dilation, 3, "dilation")
    _validate_spatial_sizes(spatial_sizes, B, (D_max, H_max, W_max), ks, 3)
    scale_value = query.shape[-1] ** -0.5 if scale is None else float(scale)
    from .autograd import na3d_varlen_with_grad
    return na3d_varlen_with_grad(query, key, value, spatial_sizes, ks, dil, scale_value)


def na1d_varlen_gqa(query, key, value, seq_lens, kernel_size, dilation=1, scale=None,
                    additional_keys=None, additional_values=None, return_lse=False):
    """Variable-length 1D NA with GQA and additional tokens in one fused
    call.  The reference has no single call for this combination; its
    meaning is, per sample b, ``na1d(q[b,:L_b], k[b,:L_b], v[b,:L_b],
    additional_keys=ak[b:b+1], additional_values=av[b:b+1])`` with zero rows
    beyond ``L_b`` (reference ``pure.py:497-518`` + ``functional.py:207-294``).
    """
    if query.ndim != 4:
        raise ValueError("na1d_varlen_gqa expects query/key/value with shape [B, L, H, D].")
    _validate_qkv(query, key, value, 1)
    add_k, add_v = _validate_additional_kv(query, key, additional_keys, additional_values)
    B, L_max = query.shape[0], query.shape[1]
    ks = normalize_kernel_size(kernel_size, 1)
    dil = normalize_tuple_param(dilation, 1, "dilation")
    min_len = _validate_seq_lens(seq_lens, B, L_max, ks[0])
    if min_len < dil[0] * ks[0]:
        raise ValueError(f"All seq_lens must be >= dilation * kernel_size ({dil[0] * ks[0]}).")
    scale_value = query.shape[-1] ** -0.5 if scale is None else float(scale)
    se = device_extents(seq_lens, B, 1, query.device)
    spec = FusedSpec(tuple(ks), (1,), tuple(dil), (False,), scale_value, varlen_clamped=True)
    out, lse = na_fused_with_grad(query, key.to(query.dtype), value.to(query.dtype), spec,
                                  add_k, add_v, sample_extent=se)
    return (out, lse) if return_lse else out


__all__ = [
    "na1d", "na1d_varlen", "na1d_varlen_gqa", "na2d", "na2d_varlen", "na3d", "na3d_varlen",
    "na1d_qk", "na1d_av", "na2d_qk", "na2d_av", "na3d_qk", "na3d_av",
]
