"""Device-face wrappers over HBM-resident torch tensors: the kernels the plan
executor drives, enqueued on torch's current stream. torch supplies device
memory and the stream only; all arithmetic is the library's."""
from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _native as n


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _f32(t: torch.Tensor) -> None:
    if t.dtype != torch.float32 or not t.is_cuda:
        raise TypeError("expected a float32 CUDA/HIP tensor")


def gemm(a: torch.Tensor, b: torch.Tensor, numerics: int = n.FAST, out: torch.Tensor | None = None) -> torch.Tensor:
    """a @ b for rank-2 views (any non-negative strides) through the library."""
    _f32(a)
    _f32(b)
    (m, k), (k2, n_) = a.shape, b.shape
    if k != k2:
        raise ValueError("inner dimensions differ")
    if out is None:
        out = torch.empty((m, n_), dtype=torch.float32, device=a.device)
    n.checked(n.lib.topos_hip_gemm_f32_device(a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(),
                                              b.stride(0), b.stride(1), m, k, n_, numerics,
                                              out.data_ptr(), out.stride(0), _stream()),
              "gemm")
    return out


def map_(operation: int, x: torch.Tensor) -> torch.Tensor:
    _f32(x)
    x = x.contiguous()
    y = torch.empty_like(x)
    n.checked(n.lib.topos_hip_map_f32_device(operation, x.data_ptr(), x.numel(), y.data_ptr(), _stream()), "map")
    return y


def rows(reduction: int, x: torch.Tensor, numerics: int = n.EXACT) -> torch.Tensor:
    _f32(x)
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("expected a contiguous [rows, columns] tensor")
    r, c = x.shape
    if reduction in (n.ROWS_LOG_SOFTMAX, n.ROWS_SOFTMAX):
        out = torch.empty_like(x)
    else:
        out = torch.empty((r,), dtype=torch.float32, device=x.device)
    n.checked(n.lib.topos_hip_rows_f32_device(reduction, x.data_ptr(), r, c, numerics, out.data_ptr(), _stream()),
              "row reduction")
    return out


def layer_norm(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, epsilon: float,
               numerics: int = n.EXACT) -> torch.Tensor:
    for t in (x, scale, shift):
        _f32(t)
    r, c = x.shape
    out = torch.empty_like(x)
    n.checked(n.lib.topos_hip_layer_norm_f32_device(x.data_ptr(), r, c, scale.contiguous().data_ptr(),
                                                    shift.contiguous().data_ptr(), epsilon, numerics,
                                                    out.data_ptr(), _stream()),
              "layer norm")
    return out


class Chain:
    """One generated elementwise/broadcast chain kernel.

    ``inputs`` are (shape, strides, offset) views over the chain's logical
    ``shape``; ``steps`` are (op, left, right) with references >= 0 naming
    earlier steps and < 0 naming input -ref-1; ``outputs`` are references."""

    def __init__(self, shape: Sequence[int], inputs: Sequence[tuple[Sequence[int], int]],
                 steps: Sequence[tuple[int, int, int]], outputs: Sequence[int]):
        self.shape = tuple(shape)
        rank = len(self.shape)
        layouts = (n.Layout * max(1, len(inputs)))()
        for i, (strides, offset) in enumerate(inputs):
            layouts[i].rank = rank
            for d in range(rank):
                layouts[i].shape[d] = self.shape[d]
                layouts[i].strides[d] = strides[d]
            layouts[i].offset = offset
        step_array = (n.ChainStep * max(1, len(steps)))(*[n.ChainStep(*s) for s in steps])
        out_array = (ctypes.c_int32 * len(outputs))(*outputs)
        desc = n.ChainDesc()
        desc.rank = rank
        for d in range(rank):
            desc.shape[d] = self.shape[d]
        desc.n_inputs, desc.inputs = len(inputs), layouts
        desc.n_steps, desc.steps = len(steps), step_array
        desc.n_outputs, desc.outputs = len(outputs), out_array
        handle = ctypes.c_void_p()
        n.checked(n.lib.topos_hip_chain_create(ctypes.byref(desc), ctypes.byref(handle)), "chain create")
        self._handle = handle
        self.n_inputs, self.n_outputs = len(inputs), len(outputs)

    @property
    def source(self) -> str:
        return n.lib.topos_hip_chain_source(self._handle).decode()

    def __call__(self, *bases: torch.Tensor) -> list[torch.Tensor]:
        if len(bases) != self.n_inputs:
            raise ValueError("wrong number of inputs")
        for t in bases:
            _f32(t)
        device = bases[0].device if bases else torch.device("cuda")
        outs = [torch.empty(self.shape, dtype=torch.float32, device=device) for _ in range(self.n_outputs)]
        ins = (ctypes.c_void_p * max(1, self.n_inputs))(*[t.data_ptr() for t in bases])
        ous = (ctypes.c_void_p * self.n_outputs)(*[t.data_ptr() for t in outs])
        n.checked(n.lib.topos_hip_chain_launch(self._handle, ins, ous, _stream()), "chain launch")
        return outs

    def __del__(self):
        if getattr(self, "_handle", None):
            n.lib.topos_hip_chain_destroy(self._handle)
            self._handle = None
