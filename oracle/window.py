"""Window arithmetic of the reference, restated on the CPU (test oracle).

Follows ``src/natten_mlx/utils/window.py`` (legacy NATTEN 0.14 boundary
rule), ``src/natten_mlx/extras/allin1/reference_impl.py:13-45`` (dilation
partition form) and ``src/natten_mlx/_core/pure.py:19-152`` (query positions,
per-axis indices and the row-major nd neighbor tables).

Pinned by (tests/test_oracle_window.py):
* the reference KATs of ``tests/test_shift_semantics.py:53-64``
  (start(31, L=32, K=3, d=1) == 29, pb_start == 0) and its phase / bounds /
  pb-range invariants (``:11-50``);
* the closed form clamp(i - K//2, 0, L - K) for d = 1, odd K;
* agreement of the legacy and partition forms for odd K, d*K <= L;
* pb_start(i) + k == (key_k - i) / d + K - 1 (relative offset identity);
* the non-causal full-window property (all K slots valid when d*K <= L);
* brute-force window membership on tiny axes.
"""

from __future__ import annotations

import numpy as np


def window_start(index: int, length: int, kernel_size: int, nh: int, dilation: int) -> int:
    """``utils/window.py:8-34``."""
    if dilation <= 1:
        s = max(index - nh, 0)
        if index + nh >= length:
            s += length - index - nh - 1
        return s
    if index - nh * dilation < 0:
        return index % dilation
    if index + nh * dilation >= length:
        phase = index % dilation
        whole = (length // dilation) * dilation
        rem = length - whole
        if phase < rem:
            return length - rem + phase - 2 * nh * dilation
        return whole + phase - kernel_size * dilation
    return index - nh * dilation


def window_end(start: int, length: int, kernel_size: int, dilation: int) -> int:
    """``utils/window.py:37-39``."""
    return min(length, start + kernel_size * dilation)


def pb_start(index: int, length: int, kernel_size: int, nh: int, dilation: int) -> int:
    """``utils/window.py:42-62``."""
    if dilation <= 1:
        pb = nh
        if index < nh:
            pb += nh - index
        if index + nh >= length:
            pb += length - index - 1 - nh
        return pb
    if index - nh * dilation < 0:
        return kernel_size - 1 - index // dilation
    if index + nh * dilation >= length:
        return (length - index - 1) // dilation
    return nh


def window_start_partition(index: int, length: int, kernel_size: int, nh: int,
                           dilation: int) -> int:
    """``extras/allin1/reference_impl.py:13-25``: the undilated rule applied
    to the query's dilation phase."""
    phase = index % dilation
    slot = index // dilation
    n_phase = (length + dilation - 1) // dilation
    padded = n_phase * dilation - length
    if phase >= dilation - padded:
        n_phase -= 1
    s = max(slot - nh, 0)
    if slot + nh >= n_phase:
        s += n_phase - slot - nh - 1
    return s * dilation + phase


def query_positions(length: int, stride: int) -> np.ndarray:
    """``pure.py:19-21``: positions o * stride, o < ceil(L / stride)."""
    out_len = (length + stride - 1) // stride
    return np.arange(out_len, dtype=np.int64) * stride


def axis_indices(qpos: np.ndarray, size: int, kernel_size: int, dilation: int,
                 causal: bool) -> tuple[np.ndarray, np.ndarray]:
    """``pure.py:52-73``: clipped key index and validity, ``[n_q, K]``."""
    qpos = np.asarray(qpos, dtype=np.int64)
    steps = np.arange(kernel_size, dtype=np.int64) * dilation
    if causal:
        start = qpos - (kernel_size - 1) * dilation
        raw = start[:, None] + steps[None, :]
        valid = (raw >= 0) & (raw <= qpos[:, None]) & (raw < size)
    else:
        nh = kernel_size // 2
        start = np.array([window_start(int(i), size, kernel_size, nh, dilation) for i in qpos],
                         dtype=np.int64)
        end = np.minimum(size, start + kernel_size * dilation)
        raw = start[:, None] + steps[None, :]
        valid = (raw >= 0) & (raw < end[:, None])
    return np.clip(raw, 0, size - 1), valid


def neighbor_table(spatial, kernel_size, dilation, is_causal, stride):
    """``pure.py:24-152``: linear key index and validity for every output
    position and kernel slot, ``[O0, ..., Kprod]``, slot row-major over the
    kernel axes."""
    rank = len(spatial)
    idx_list, val_list = [], []
    for a in range(rank):
        qpos = query_positions(spatial[a], stride[a])
        i, v = axis_indices(qpos, spatial[a], kernel_size[a], dilation[a], bool(is_causal[a]))
        idx_list.append(i)
        val_list.append(v)
    out_shape = tuple(len(i) for i in idx_list)
    lin = np.zeros(out_shape + tuple(kernel_size), dtype=np.int64)
    valid = np.ones(out_shape + tuple(kernel_size), dtype=bool)
    for a in range(rank):
        shape = [1] * (2 * rank)
        shape[a] = out_shape[a]
        shape[rank + a] = kernel_size[a]
        mult = int(np.prod(spatial[a + 1:], dtype=np.int64)) if a + 1 < rank else 1
        lin = lin + idx_list[a].reshape(shape) * mult
        valid = valid & val_list[a].reshape(shape)
    kprod = int(np.prod(kernel_size))
    return lin.reshape(out_shape + (kprod,)), valid.reshape(out_shape + (kprod,))
