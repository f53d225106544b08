"""Window helpers (the reference's ``utils/window.py`` interface).

These call the host twins exported by libnatten_amd.so, i.e. the very
functions the HIP kernels use, so host and device window arithmetic are the
same code.
"""

from __future__ import annotations

import numpy as np

from .._core import _lib


def get_window_start(index: int, length: int, kernel_size: int, neighborhood_size: int,
                     dilation: int) -> int:
    return int(_lib.load().na_window_start(index, length, kernel_size, neighborhood_size,
                                           dilation))


def get_window_end(start_index: int, length: int, kernel_size: int, dilation: int) -> int:
    return int(_lib.load().na_window_end(start_index, length, kernel_size, dilation))


def get_pb_start(index: int, length: int, kernel_size: int, neighborhood_size: int,
                 dilation: int) -> int:
    return int(_lib.load().na_pb_start(index, length, kernel_size, neighborhood_size, dilation))


def compute_window_start_end(query_positions, length: int, kernel_size: int,
                             dilation: int) -> tuple[np.ndarray, np.ndarray]:
    nh = kernel_size // 2
    starts = np.array([get_window_start(int(i), length, kernel_size, nh, dilation)
                       for i in query_positions], dtype=np.int32)
    ends = np.array([get_window_end(int(s), length, kernel_size, dilation) for s in starts],
                    dtype=np.int32)
    return starts, ends


def compute_pb_start(query_positions, length: int, kernel_size: int, dilation: int) -> np.ndarray:
    nh = kernel_size // 2
    return np.array([get_pb_start(int(i), length, kernel_size, nh, dilation)
                     for i in query_positions], dtype=np.int32)
