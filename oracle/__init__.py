"""ctypes binding of the CPU oracle (oracle/oracle.c); oracle/interpreter.py plays
recorded tapes over it.

TEST INFRASTRUCTURE ONLY: the parity tests, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` use it as the checker. Product code
never imports it.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_double, c_float, c_int, c_int64, c_size_t, c_uint64
from pathlib import Path

import numpy as np

_PATH = Path(__file__).resolve().parent / "liboracle.so"
if not _PATH.exists():
    raise ImportError(f"{_PATH} is not built; run `python poorgrad_amd/build.py`")
lib = ctypes.CDLL(str(_PATH))

_F = POINTER(c_float)
_D = POINTER(c_double)
_U64 = POINTER(c_uint64)

_PROTOTYPES = {
    "oracle_splitmix64": (c_uint64, [_U64]),
    "oracle_unit": (c_double, [_U64]),
    "oracle_standard_normal": (c_double, [_U64]),
    "oracle_uniform_f32": (None, [_U64, c_double, c_size_t, _F]),
    "oracle_normal_f32": (None, [_U64, c_double, c_size_t, _F]),
    "oracle_uniform_f64": (None, [_U64, c_double, c_size_t, _D]),
    "oracle_normal_f64": (None, [_U64, c_double, c_size_t, _D]),
    "oracle_gemm_f32": (None, [_F, c_int64, c_int64, _F, c_int64, c_int64, c_int64, c_int64, c_int64, _F]),
    "oracle_gemm_rows_f32": (None, [_F, c_int64, c_int64, _F, c_int64, c_int64, c_int64, c_int64, c_int64,
                                    c_int64, c_int64, _F]),
    "oracle_unary_f32": (c_float, [c_int, c_float]),
    "oracle_binary_f32": (c_float, [c_int, c_float, c_float]),
    "oracle_map_f32": (None, [c_int, _F, c_size_t, _F]),
    "oracle_zip_f32": (None, [c_int, _F, _F, c_size_t, _F]),
    "oracle_sum_f32": (c_float, [_F, c_size_t]),
    "oracle_sum_along_f32": (None, [_F, c_int64, c_int64, c_int64, _F]),
    "oracle_max_along_f32": (None, [_F, c_int64, c_int64, c_int64, _F]),
    "oracle_log_softmax_rows_f32": (None, [_F, c_int64, c_int64, _F]),
    "oracle_softmax_rows_f32": (None, [_F, c_int64, c_int64, _F]),
    "oracle_log_sum_exp_rows_f32": (None, [_F, c_int64, c_int64, _F]),
    "oracle_layer_norm_rows_f32": (None, [_F, c_int64, c_int64, _F, _F, c_float, _F]),
    "oracle_bf16_from_f32": (ctypes.c_uint16, [c_float]),
    "oracle_bf16_round": (None, [_F, c_size_t, POINTER(ctypes.c_uint16)]),
    "oracle_bf16_widen": (None, [POINTER(ctypes.c_uint16), c_size_t, _F]),
}
for _name, (_res, _args) in _PROTOTYPES.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

NEG, EXP, LN, SQRT, TANH = range(5)
ADD, SUB, MUL, DIV, POWF, MAX, STEP = range(7)


def _f(array: np.ndarray):
    assert array.dtype == np.float32 and array.flags.c_contiguous
    return array.ctypes.data_as(_F)


class Generator:
    """The seeded splitmix64 stream of src/neural/init.rs:50-102; successive
    draws continue one state, as an initializer closure does."""

    def __init__(self, seed: int):
        self._state = c_uint64(seed)

    def uniform(self, count: int, scale: float) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        lib.oracle_uniform_f32(ctypes.byref(self._state), scale, count, _f(out))
        return out

    def normal(self, count: int, deviation: float) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        lib.oracle_normal_f32(ctypes.byref(self._state), deviation, count, _f(out))
        return out

    def uniform64(self, count: int, scale: float) -> np.ndarray:
        out = np.empty(count, dtype=np.float64)
        lib.oracle_uniform_f64(ctypes.byref(self._state), scale, count, out.ctypes.data_as(_D))
        return out

    def normal64(self, count: int, deviation: float) -> np.ndarray:
        out = np.empty(count, dtype=np.float64)
        lib.oracle_normal_f64(ctypes.byref(self._state), deviation, count, out.ctypes.data_as(_D))
        return out

    def next_u64(self) -> int:
        return lib.oracle_splitmix64(ctypes.byref(self._state))


# Host threads a large product's rows are spread over (1: single-threaded, as
# the reference interpreter runs). Every output row is computed by the same
# sequential loop whichever thread runs it, so the bits do not depend on this.
THREADS = 1


def _gemm_threaded(a, a_strides, b, b_strides, m, k, n, out) -> None:
    import concurrent.futures

    chunk = (m + THREADS - 1) // THREADS
    chunk = (chunk + 3) // 4 * 4
    ranges = [(r, min(r + chunk, m)) for r in range(0, m, chunk)]

    def run(span):
        lib.oracle_gemm_rows_f32(_f(a), a_strides[0], a_strides[1], _f(b), b_strides[0], b_strides[1], m, n, k,
                                 span[0], span[1], _f(out))

    with concurrent.futures.ThreadPoolExecutor(max_workers=THREADS) as pool:
        list(pool.map(run, ranges))


def gemm(a: np.ndarray, a_strides, b: np.ndarray, b_strides, m: int, k: int, n: int,
         rows: tuple[int, int] | None = None) -> np.ndarray:
    """gemm::multiply over flat buffers read through (row, column) strides;
    `rows` restricts the product to a row range (zeros elsewhere)."""
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    b = np.ascontiguousarray(b, dtype=np.float32).ravel()
    out = np.zeros(m * n, dtype=np.float32)
    if rows is None and THREADS > 1 and m >= 8 * THREADS and m * n * k >= (1 << 27):
        _gemm_threaded(a, a_strides, b, b_strides, m, k, n, out)
    elif rows is None:
        lib.oracle_gemm_f32(_f(a), a_strides[0], a_strides[1], _f(b), b_strides[0], b_strides[1], m, n, k, _f(out))
    else:
        lib.oracle_gemm_rows_f32(_f(a), a_strides[0], a_strides[1], _f(b), b_strides[0], b_strides[1], m, n, k,
                                 rows[0], rows[1], _f(out))
    return out.reshape(m, n)


def map_(op: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib.oracle_map_f32(op, _f(x), x.size, _f(y))
    return y


def zip_(op: int, x: np.ndarray, y: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(np.broadcast_to(y, x.shape), dtype=np.float32)
    out = np.empty_like(x)
    lib.oracle_zip_f32(op, _f(x), _f(y), x.size, _f(out))
    return out


def sum_(x: np.ndarray) -> np.float32:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.float32(lib.oracle_sum_f32(_f(x), x.size))


def sum_along(x: np.ndarray, axis: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    outer = int(np.prod(x.shape[:axis], dtype=np.int64))
    inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
    out = np.empty(x.shape[:axis] + x.shape[axis + 1:], dtype=np.float32)
    lib.oracle_sum_along_f32(_f(x), outer, x.shape[axis], inner, _f(out))
    return out


def max_along(x: np.ndarray, axis: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    outer = int(np.prod(x.shape[:axis], dtype=np.int64))
    inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
    out = np.empty(x.shape[:axis] + x.shape[axis + 1:], dtype=np.float32)
    lib.oracle_max_along_f32(_f(x), outer, x.shape[axis], inner, _f(out))
    return out


def _rows(fn, x: np.ndarray, full: bool) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape if full else x.shape[:1], dtype=np.float32)
    fn(_f(x), x.shape[0], x.shape[1], _f(out))
    return out


def log_softmax_rows(x: np.ndarray) -> np.ndarray:
    return _rows(lib.oracle_log_softmax_rows_f32, x, True)


def softmax_rows(x: np.ndarray) -> np.ndarray:
    return _rows(lib.oracle_softmax_rows_f32, x, True)


def log_sum_exp_rows(x: np.ndarray) -> np.ndarray:
    return _rows(lib.oracle_log_sum_exp_rows_f32, x, False)


def layer_norm_rows(x: np.ndarray, scale: np.ndarray, shift: np.ndarray, epsilon: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    shift = np.ascontiguousarray(shift, dtype=np.float32)
    out = np.empty_like(x)
    lib.oracle_layer_norm_rows_f32(_f(x), x.shape[0], x.shape[1], _f(scale), _f(shift), epsilon, _f(out))
    return out


# ---- the bf16 payload (src/payload/bf16.rs) ----

def bf16_round(x: np.ndarray) -> np.ndarray:
    """Bf16::from_f32 elementwise: uint16 bit patterns."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib.oracle_bf16_round(_f(x), x.size, out.ctypes.data_as(POINTER(ctypes.c_uint16)))
    return out


def bf16_widen(h: np.ndarray) -> np.ndarray:
    """Bf16::to_f32 elementwise."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib.oracle_bf16_widen(h.ctypes.data_as(POINTER(ctypes.c_uint16)), h.size, _f(out))
    return out


def gemm_bf16(a: np.ndarray, a_strides, b: np.ndarray, b_strides, m: int, k: int, n: int) -> np.ndarray:
    """Bf16::gemm (src/payload/bf16.rs:235-262): widen both operands, the f32
    gemm::multiply, one rounding per output."""
    return bf16_round(gemm(bf16_widen(a), a_strides, bf16_widen(b), b_strides, m, k, n))
