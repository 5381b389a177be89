"""The offered task face (host buffers, synchronous): the bodies of the
`Task::offer` arms a topos `Backend::Hip` member would run
(src/backend/task.rs:57-115). `None` means "declined: compute on the
reference path", exactly as the Rust `Option` does."""
from __future__ import annotations

from typing import Optional

import numpy as np

from . import _native as n


def _floats(array: np.ndarray):
    return array.ctypes.data_as(n.FLOAT_P)


def gemm_f32(a: np.ndarray, a_strides: tuple[int, int], b: np.ndarray, b_strides: tuple[int, int],
             m: int, k: int, n_: int, numerics: int = n.FAST) -> Optional[np.ndarray]:
    """GemmTask::new(a, a_strides, b, b_strides, m, k, n) offered to the HIP
    member (src/payload/gemm.rs:57-89). Raises ValueError where GemmTask::new
    panics (a slice that does not span its matrix)."""
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    b = np.ascontiguousarray(b, dtype=np.float32).ravel()
    product = np.empty(m * n_, dtype=np.float32)
    code = n.lib.topos_hip_gemm_f32(_floats(a), a.size, a_strides[0], a_strides[1], _floats(b), b.size,
                                     b_strides[0], b_strides[1], m, k, n_, numerics, _floats(product))
    if code == n.INVALID_ARGUMENT:
        raise ValueError("the gemm task violates its contract (operand slices must span their matrices)")
    return product.reshape(m, n_) if code == n.OK else None


def map_f32(operation: int, elements: np.ndarray, numerics: int = n.FAST) -> Optional[np.ndarray]:
    """MapTask::new(operation, elements) offered to the HIP member."""
    elements = np.ascontiguousarray(elements, dtype=np.float32).ravel()
    out = np.empty_like(elements)
    code = n.lib.topos_hip_map_f32(operation, _floats(elements), elements.size, numerics, _floats(out))
    if code == n.INVALID_ARGUMENT:
        raise ValueError("invalid map task")
    return out if code == n.OK else None
