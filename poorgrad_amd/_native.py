"""ctypes binding of libtopos_hip.so (include/topos_hip.h).

The library is built in-tree by ``python poorgrad_amd/build.py``. Importing
this module without it raises ImportError: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint, c_void_p
from pathlib import Path

# TOPOS_HIP_LIBRARY names another build of the same library (the sanitized
# host build the CPU tests load under the fake runtime).
LIBRARY_PATH = Path(os.environ.get("TOPOS_HIP_LIBRARY", Path(__file__).resolve().parent / "libtopos_hip.so"))

if not LIBRARY_PATH.exists():
    raise ImportError(f"{LIBRARY_PATH} is not built; run `python poorgrad_amd/build.py` "
                      "(the HIP backend has no CPU fallback)")

# One HIP runtime per process. torch carries its own libamdhip64.so.7; the
# library binds to whichever copy of that soname is loaded first, so load
# torch's first. Loading /opt/rocm's first leaves torch a second runtime that
# cannot see the device.
try:
    import torch  # noqa: F401
except ImportError:  # the C ABI itself needs no torch
    pass

lib = ctypes.CDLL(str(LIBRARY_PATH))

# ---- status codes and vocabulary (mirrors include/topos_hip.h) ----
OK, DECLINED, NO_DEVICE, SETUP_FAILED, POISONED, INVALID_ARGUMENT, RUNTIME_ERROR, UNSUPPORTED = range(8)
EXACT, FAST = 0, 1
BIT_IDENTICAL, ENVELOPE = 0, 1
FORMULA_GEMM, FORMULA_MAP, FORMULA_WINDOW_PRODUCT, FORMULA_REDUCE_WINDOW = 0, 1, 2, 3
FORMULA_BATCH_NORM_TRAINING, FORMULA_BATCH_NORM_INFERENCE = 4, 5
PRECISION_F32, PRECISION_F64 = 1, 2
DISPATCH_OFFERED, DISPATCH_ELECTED, DISPATCH_TRANSLATED = 0, 1, 2
MAP_EXP, MAP_LN, MAP_SQRT, MAP_TANH = 0, 1, 2, 3
ROWS_SUM, ROWS_MAX, ROWS_LOG_SOFTMAX, ROWS_SOFTMAX, ROWS_LOG_SUM_EXP = 0, 1, 2, 3, 4
CHAIN_NEG, CHAIN_EXP, CHAIN_LN, CHAIN_SQRT, CHAIN_TANH = 0, 1, 2, 3, 4
CHAIN_ADD, CHAIN_SUB, CHAIN_MUL, CHAIN_DIV, CHAIN_MAX, CHAIN_STEP, CHAIN_POWF = 16, 17, 18, 19, 20, 21, 22
MAX_RANK = 6

FLOAT_P = POINTER(c_float)


class Layout(ctypes.Structure):
    _fields_ = [("rank", c_int32), ("shape", c_int64 * MAX_RANK), ("strides", c_int64 * MAX_RANK),
                ("offset", c_int64)]


class ChainStep(ctypes.Structure):
    _fields_ = [("op", c_int32), ("left", c_int32), ("right", c_int32)]


class ChainDesc(ctypes.Structure):
    _fields_ = [("rank", c_int32), ("shape", c_int64 * MAX_RANK), ("n_inputs", c_int32),
                ("inputs", POINTER(Layout)), ("n_steps", c_int32), ("steps", POINTER(ChainStep)),
                ("n_outputs", c_int32), ("outputs", POINTER(c_int32))]


NODE_READABLE, NODE_SELECTION = 1, 2
LEAF_CONSTANT, LEAF_DENSE, LEAF_SELECTION = 0, 1, 2
INT32_P = POINTER(c_int32)


class Node(ctypes.Structure):
    _fields_ = [("op", c_int32), ("rank", c_int32), ("shape", c_int64 * MAX_RANK), ("operands", c_int32 * 2),
                ("params", c_int64 * MAX_RANK), ("slot", c_int32), ("flags", ctypes.c_uint32)]


class AdamwTensor(ctypes.Structure):
    _fields_ = [("parameter", c_void_p), ("gradient", c_void_p), ("first", c_void_p), ("second", c_void_p),
                ("count", c_int64), ("decayed", c_int32)]


class Leaf(ctypes.Structure):
    _fields_ = [("kind", c_int32), ("value", c_float), ("offset", c_int64), ("count", c_int64)]


# Every symbol the header declares, with its prototype. The CPU tests check
# that each one resolves.
PROTOTYPES = {
    "topos_hip_abi_version": (c_int, []),
    "topos_hip_dispatch": (c_int, []),
    "topos_hip_compiled": (c_int, []),
    "topos_hip_coverage": (c_int, [c_int, POINTER(c_int), POINTER(c_uint)]),
    "topos_hip_status": (c_int, []),
    "topos_hip_status_reason": (c_char_p, []),
    "topos_hip_status_string": (c_char_p, [c_int]),
    "topos_hip_gemm_f32": (c_int, [FLOAT_P, c_size_t, c_size_t, c_size_t, FLOAT_P, c_size_t, c_size_t,
                                   c_size_t, c_size_t, c_size_t, c_size_t, c_int, FLOAT_P]),
    "topos_hip_map_f32": (c_int, [c_int, FLOAT_P, c_size_t, c_int, FLOAT_P]),
    "topos_hip_gemm_f32_device": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64,
                                          c_int64, c_int64, c_int, c_void_p, c_int64, c_void_p]),
    "topos_hip_gemm_f32_device_noalloc": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64,
                                                  c_int64, c_int64, c_int64, c_int, c_void_p, c_int64, c_void_p]),
    "topos_hip_gemm_bf16_device": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                           c_int64, c_int, c_void_p, c_int64, c_void_p]),
    "topos_hip_map_f32_device": (c_int, [c_int, c_void_p, c_int64, c_void_p, c_void_p]),
    "topos_hip_rows_f32_device": (c_int, [c_int, c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "topos_hip_layer_norm_f32_device": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_float,
                                                c_int, c_void_p, c_void_p]),
    "topos_hip_chain_create": (c_int, [POINTER(ChainDesc), POINTER(c_void_p)]),
    "topos_hip_chain_launch": (c_int, [c_void_p, POINTER(c_void_p), POINTER(c_void_p), c_void_p]),
    "topos_hip_chain_source": (c_char_p, [c_void_p]),
    "topos_hip_chain_destroy": (None, [c_void_p]),
    "topos_hip_fake_runtime": (c_int, [c_int]),
    "topos_hip_workspace_bytes": (c_int64, []),
    "topos_hip_program_create": (c_int, [POINTER(Node), c_int64, POINTER(Leaf), c_int64, FLOAT_P, c_int64,
                                         INT32_P, c_int64, c_int, POINTER(c_void_p)]),
    "topos_hip_program_create_backward": (c_int, [POINTER(Node), c_int64, POINTER(Leaf), c_int64, FLOAT_P, c_int64,
                                                  INT32_P, c_int64, c_int, c_int64, POINTER(c_int64), c_int64,
                                                  POINTER(c_void_p)]),
    "topos_hip_program_gradient": (c_int, [c_void_p, c_int64, POINTER(c_int64)]),
    "topos_hip_program_info": (c_int, [c_void_p, POINTER(ctypes.c_uint64), POINTER(c_int64), POINTER(c_int64)]),
    "topos_hip_program_bind": (c_int, [c_void_p, c_int, c_int32, c_void_p]),
    "topos_hip_program_bind_selection": (c_int, [c_void_p, c_int32, INT32_P, c_int64, c_float]),
    "topos_hip_program_run": (c_int, [c_void_p, c_void_p]),
    "topos_hip_program_replay": (c_int, [c_void_p, c_void_p]),
    "topos_hip_program_run_profiled": (c_int, [c_void_p, c_void_p, FLOAT_P]),
    "topos_hip_program_launch": (c_int, [c_void_p, c_int64, POINTER(c_char_p), POINTER(ctypes.c_double),
                                         POINTER(ctypes.c_double)]),
    "topos_hip_program_output": (c_int, [c_void_p, c_int64, POINTER(c_void_p)]),
    "topos_hip_program_read": (c_int, [c_void_p, c_int64, FLOAT_P, c_int64]),
    "topos_hip_last_refusal": (c_char_p, []),
    "topos_hip_program_describe": (c_char_p, [c_void_p]),
    "topos_hip_program_destroy": (None, [c_void_p]),
    "topos_hip_sgd_step_f32": (c_int, [c_void_p, c_void_p, c_int64, c_float, c_void_p]),
    "topos_hip_adamw_step_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_float, c_float, c_float,
                                         c_float, c_float, c_float, c_float, c_float, c_float, c_int, c_void_p]),
    "topos_hip_adamw_step_multi_f32": (c_int, [POINTER(AdamwTensor), c_int64, c_float, c_float, c_float, c_float,
                                               c_float, c_float, c_float, c_float, c_float, c_void_p]),
}

for _name, (_restype, _argtypes) in PROTOTYPES.items():
    _function = getattr(lib, _name)
    _function.restype = _restype
    _function.argtypes = _argtypes

# The structures above follow include/topos_hip.h at this version.
ABI_VERSION = 2
if lib.topos_hip_abi_version() != ABI_VERSION:
    raise ImportError(f"{LIBRARY_PATH} has ABI version {lib.topos_hip_abi_version()}, this binding "
                      f"{ABI_VERSION}; rebuild with `python poorgrad_amd/build.py`")


class HipError(RuntimeError):
    """A non-OK status from the library, carrying the code."""

    def __init__(self, code: int, what: str):
        reason = lib.topos_hip_status_reason().decode()
        text = lib.topos_hip_status_string(code).decode()
        super().__init__(f"{what}: {text}" + (f" ({reason})" if reason else ""))
        self.code = code


def checked(code: int, what: str) -> None:
    if code != OK:
        raise HipError(code, what)


def status() -> int:
    return lib.topos_hip_status()


def status_reason() -> str:
    return lib.topos_hip_status_reason().decode()
