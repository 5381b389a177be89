"""A device program: a recorded plan executed by libtopos_hip on one GPU.

torch supplies the device memory of parameters and dense inputs (bound by
address) and the stream; planning, the arena and every kernel are the
library's.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

from . import _native as n
from .topos import ProgramTable, Tape, Value


class DeviceProgram:
    """topos_hip_program_*: create once, bind, run many times."""

    def __init__(self, tape: Tape, roots: Sequence[Value], observe: Sequence[Value] = (), numerics: int = n.EXACT,
                 backward: tuple | None = None):
        self.tape = tape
        self.table: ProgramTable = tape.program(roots, observe)
        self.numerics = numerics
        self.handle = self.table.create(numerics) if backward is None else self.table.create_backward(numerics, *backward)
        self._held = {}  # keeps bound tensors alive

    @classmethod
    def engine_backward(cls, tape: Tape, target: Value, wrt: Sequence[Value], observe: Sequence[Value] = (),
                        numerics: int = n.EXACT) -> "DeviceProgram":
        """The engine-backward route (Request::backward() plan, then
        Run::backward(target), src/engine/run.rs:229-318): the tape holds the
        forward graph only, and the library appends the reverse scan itself.
        Read gradients with read_gradient / gradient_pointer."""
        return cls(tape, [target], observe, numerics, backward=(target.id, [v.id for v in wrt]))

    def _gradient_node(self, value: Value) -> int:
        node = ctypes.c_int64()
        n.checked(n.lib.topos_hip_program_gradient(self.handle, value.id, ctypes.byref(node)), "program gradient")
        return node.value

    def read_gradient(self, value: Value) -> np.ndarray:
        """The target's gradient with respect to `value` after a run
        (Gradients::of)."""
        out = np.empty(value.shape, dtype=np.float32)
        n.checked(n.lib.topos_hip_program_read(self.handle, self._gradient_node(value),
                                               out.ctypes.data_as(n.FLOAT_P), out.size), "program read gradient")
        return out

    def gradient_pointer(self, value: Value) -> int:
        p = ctypes.c_void_p()
        n.checked(n.lib.topos_hip_program_output(self.handle, self._gradient_node(value), ctypes.byref(p)),
                  "program gradient output")
        return p.value

    @property
    def describe(self) -> str:
        return n.lib.topos_hip_program_describe(self.handle).decode()

    @property
    def info(self) -> dict:
        arena, launches, groups = ctypes.c_uint64(), ctypes.c_int64(), ctypes.c_int64()
        n.checked(n.lib.topos_hip_program_info(self.handle, ctypes.byref(arena), ctypes.byref(launches),
                                               ctypes.byref(groups)), "program info")
        return {"arena_bytes": arena.value, "launches": launches.value, "generated_kernels": groups.value}

    def bind_parameter(self, slot: int, tensor) -> None:
        self._bind(0, slot, tensor)

    def bind_input(self, slot: int, tensor) -> None:
        self._bind(1, slot, tensor)

    def _bind(self, is_input: int, slot: int, tensor) -> None:
        import torch

        if tensor.dtype != torch.float32 or not tensor.is_cuda or not tensor.is_contiguous():
            raise TypeError("bind a contiguous float32 device tensor")
        shapes = self.tape.input_shapes if is_input else self.tape.parameter_shapes
        if tuple(tensor.shape) != tuple(shapes[slot]):
            raise ValueError(f"slot {slot} records shape {shapes[slot]}, got {tuple(tensor.shape)}")
        n.checked(n.lib.topos_hip_program_bind(self.handle, is_input, slot, tensor.data_ptr()), "program bind")
        self._held[(is_input, slot)] = tensor

    def bind_selection(self, slot: int, indices: np.ndarray, one: float = 1.0) -> None:
        indices = np.ascontiguousarray(indices, dtype=np.int32)
        n.checked(n.lib.topos_hip_program_bind_selection(self.handle, slot, indices.ctypes.data_as(n.INT32_P),
                                                         indices.size, one),
                  "program bind selection")

    def run(self) -> None:
        import torch

        n.checked(n.lib.topos_hip_program_run(self.handle, torch.cuda.current_stream().cuda_stream), "program run")

    def replay(self) -> None:
        """One run as a single HIP graph launch (captured on first use and
        after any bind)."""
        import torch

        n.checked(n.lib.topos_hip_program_replay(self.handle, torch.cuda.current_stream().cuda_stream),
                  "program replay")

    def profile(self) -> list:
        """One run with HIP events around every launch: per launch
        (kind, milliseconds, flops, bytes, description)."""
        import torch

        count = self.info["launches"]
        ms = (ctypes.c_float * count)()
        n.checked(n.lib.topos_hip_program_run_profiled(self.handle, torch.cuda.current_stream().cuda_stream, ms),
                  "program profiled run")
        lines = self.describe.splitlines()[1:]
        out = []
        for i in range(count):
            kind, flops, nbytes = ctypes.c_char_p(), ctypes.c_double(), ctypes.c_double()
            n.checked(n.lib.topos_hip_program_launch(self.handle, i, ctypes.byref(kind), ctypes.byref(flops),
                                                     ctypes.byref(nbytes)), "program launch")
            what = lines[i].split(": ", 1)[1] if i < len(lines) else ""
            out.append((kind.value.decode(), float(ms[i]), flops.value, nbytes.value, what))
        return out

    def pointer(self, value: Value) -> int:
        """Device address of a readable value after a run (contiguous f32)."""
        p = ctypes.c_void_p()
        n.checked(n.lib.topos_hip_program_output(self.handle, value.id, ctypes.byref(p)), "program output")
        return p.value

    def read(self, value: Value) -> np.ndarray:
        out = np.empty(value.shape, dtype=np.float32)
        n.checked(n.lib.topos_hip_program_read(self.handle, value.id, out.ctypes.data_as(n.FLOAT_P), out.size),
                  "program read")
        return out

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle and n is not None and getattr(n, "lib", None) is not None:
            n.lib.topos_hip_program_destroy(handle)
            self.handle = None


def sgd_step(parameter, gradient_pointer: int, rate: float) -> None:
    """Sgd::step on one device-resident parameter (src/neural/optimizer.rs:40-51)."""
    import torch

    n.checked(n.lib.topos_hip_sgd_step_f32(parameter.data_ptr(), gradient_pointer, parameter.numel(), rate,
                                           torch.cuda.current_stream().cuda_stream), "sgd step")


class AdamW:
    """AdamW over device-resident parameters (src/neural/adam.rs:62-171): the
    optimizer's scalar bookkeeping in f32 on the host, the per-element update
    on the device. Moments start at zero, the device stand-in for the absent
    moments whose Constant-zero scaling gives the same bits."""

    def __init__(self, parameters, beta1=0.9, beta2=0.999, epsilon=1e-8, decay=0.01):
        import torch

        f = np.float32
        self.beta1, self.beta2, self.epsilon, self.decay = f(beta1), f(beta2), f(epsilon), f(decay)
        self.first_share = f(1) - self.beta1
        self.second_share = f(1) - self.beta2
        self.beta1_power, self.beta2_power = f(1), f(1)
        self.moments = [(torch.zeros_like(p), torch.zeros_like(p)) for p in parameters]

    def step(self, parameters, gradient_pointers, rate: float) -> None:
        """One AdamW::step over every parameter: the host bookkeeping, then one
        many-parameter launch per 48 parameters (topos_hip_adamw_step_multi_f32,
        the same per-element operations as the single-parameter entry)."""
        import torch

        f = np.float32
        self.beta1_power = f(self.beta1_power * self.beta1)
        self.beta2_power = f(self.beta2_power * self.beta2)
        first_correction = f(1) - self.beta1_power
        second_correction = f(1) - self.beta2_power
        table = (n.AdamwTensor * len(parameters))()
        for j, (p, g, (m, v)) in enumerate(zip(parameters, gradient_pointers, self.moments)):
            table[j] = n.AdamwTensor(p.data_ptr(), g, m.data_ptr(), v.data_ptr(), p.numel(),
                                     1 if p.dim() >= 2 else 0)  # AdamW::step's rank >= 2 policy
        n.checked(n.lib.topos_hip_adamw_step_multi_f32(table, len(parameters), float(self.beta1), float(self.beta2),
                                                       float(self.first_share), float(self.second_share),
                                                       float(first_correction), float(second_correction),
                                                       float(self.epsilon), rate, float(self.decay),
                                                       torch.cuda.current_stream().cuda_stream),
                  "adamw step")
