"""Pins the oracle's fused-row helpers and its f32::max tie (CPU only).

* oracle_layer_norm_rows_f32, oracle_log_softmax_rows_f32,
  oracle_softmax_rows_f32 and oracle_log_sum_exp_rows_f32 are each compared
  bit for bit with the interpreter (oracle/interpreter.py) evaluating the
  recorded facade: LayerNorm::express (src/neural/layer_norm.rs:100-132) with
  the epsilon leaf 1e-5, LogSoftmax (src/function/log_softmax.rs:51-60),
  softmax = log_softmax.exp (src/graph/composite.rs:43-45) and LogSumExp
  (src/function/log_sum_exp.rs:53-61) along axis 1. The interpreter is built
  only from the individually pinned primitives (ordered folds, glibc maps,
  IEEE +,-,*,/), so equality pins each fused helper to the composition.
  Planted mistakes (a misplaced epsilon, a reordered variance, a reciprocal
  for the division, a reversed sum, a shift by the row's first term, a
  divided softmax) are shown to fail the same comparison.
* max_f32's signed-zero tie (src/payload/elementary.rs:137-139: f32::max,
  which rustc lowers to llvm.maxnum.f32) against LLVM's maxnum built here by
  clang on runtime operands (tests/native/maxnum_probe.c).
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

import oracle
from poorgrad_amd import topos as t
from tests.program_util import run_oracle

NATIVE = Path(__file__).resolve().parent / "native"
WIDTHS = [(6, 768), (3, 4096), (2, 50257)]


def _rows(rows: int, columns: int, seed: int) -> np.ndarray:
    g = oracle.Generator(seed)
    x = g.normal(rows * columns, 1.0).reshape(rows, columns)
    # A spread of scales, so exponentials and the variance cover a wide range.
    return (x * np.float32(1 + 3 * (seed % 4))).astype(np.float32)


def _bits(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _facade_layer_norm(x, scale, shift, epsilon):
    tape = t.Tape()
    xv = tape.input(x.shape)
    sv, bv = tape.parameter(scale.shape), tape.parameter(shift.shape)
    ev = tape.leaf(t.Constant((), float(np.float32(epsilon))))
    out = t.layer_norm(xv, sv, bv, ev)
    return run_oracle(tape, [out], [scale, shift], {0: x})[out.id]


def _facade_rows(x, which):
    tape = t.Tape()
    xv = tape.input(x.shape)
    out = {"log_softmax": lambda v: v.log_softmax(1), "softmax": lambda v: v.softmax(1),
           "logsumexp": lambda v: v.logsumexp(1)}[which](xv)
    return run_oracle(tape, [out], [], {0: x})[out.id]


@pytest.mark.parametrize("rows, columns", WIDTHS)
def test_layer_norm_helper_is_the_recorded_facade(rows, columns):
    x = _rows(rows, columns, 11)
    g = oracle.Generator(12)
    scale, shift = g.normal(columns, 1.0), g.normal(columns, 1.0)
    want = _facade_layer_norm(x, scale, shift, 1e-5)
    assert np.array_equal(_bits(oracle.layer_norm_rows(x, scale, shift, 1e-5)), _bits(want))


@pytest.mark.parametrize("rows, columns", WIDTHS)
@pytest.mark.parametrize("which", ["log_softmax", "softmax", "logsumexp"])
def test_row_helpers_are_the_recorded_facades(rows, columns, which):
    x = _rows(rows, columns, 13 + columns % 7)
    helper = {"log_softmax": oracle.log_softmax_rows, "softmax": oracle.softmax_rows,
              "logsumexp": oracle.log_sum_exp_rows}[which]
    want = _facade_rows(x, which)
    assert np.array_equal(_bits(helper(x)), _bits(want))


# ---- planted mistakes: each restated in numpy/oracle primitives, each must
# ---- differ from the recorded facade, so the comparison above would catch it.

def _mean(x):
    return oracle.sum_along(x, 1) / np.float32(x.shape[1])


def _layer_norm_eps_outside(x, scale, shift, epsilon):
    mean = _mean(x)[:, None]
    centred = x - mean
    variance = _mean(centred * centred)[:, None]
    deviation = oracle.map_(oracle.SQRT, np.ascontiguousarray(variance)) + np.float32(epsilon)
    return (centred / deviation) * scale + shift


def _layer_norm_moment_variance(x, scale, shift, epsilon):
    mean = _mean(x)[:, None]
    variance = (_mean(x * x)[:, None] - mean * mean).astype(np.float32)
    deviation = oracle.map_(oracle.SQRT, np.ascontiguousarray(variance + np.float32(epsilon)))
    return ((x - mean) / deviation) * scale + shift


def _layer_norm_reciprocal(x, scale, shift, epsilon):
    mean = _mean(x)[:, None]
    centred = x - mean
    variance = _mean(centred * centred)[:, None]
    deviation = oracle.map_(oracle.SQRT, np.ascontiguousarray(variance + np.float32(epsilon)))
    return (centred * (np.float32(1) / deviation)) * scale + shift


@pytest.mark.parametrize("mutant", [_layer_norm_eps_outside, _layer_norm_moment_variance, _layer_norm_reciprocal])
@pytest.mark.parametrize("rows, columns", WIDTHS[:2])
def test_planted_layer_norm_mistakes_fail(mutant, rows, columns):
    x = _rows(rows, columns, 11)
    g = oracle.Generator(12)
    scale, shift = g.normal(columns, 1.0), g.normal(columns, 1.0)
    want = _facade_layer_norm(x, scale, shift, 1e-5)
    with np.errstate(all="ignore"):
        got = mutant(x, scale, shift, 1e-5).astype(np.float32)
    assert not np.array_equal(_bits(got), _bits(want))


def _log_softmax_reversed_sum(x):
    peak = oracle.max_along(x, 1)[:, None]
    shifted = x - peak
    flipped = np.ascontiguousarray(oracle.map_(oracle.EXP, shifted)[:, ::-1])
    return shifted - oracle.map_(oracle.LN, oracle.sum_along(flipped, 1))[:, None]


def _log_sum_exp_first_shift(x):
    # Shifted by the row's first term instead of its maximum.
    peak = np.ascontiguousarray(x[:, 0])
    total = oracle.sum_along(oracle.map_(oracle.EXP, x - peak[:, None]), 1)
    return peak + oracle.map_(oracle.LN, total)


def _softmax_divided(x):
    e = oracle.map_(oracle.EXP, x - oracle.max_along(x, 1)[:, None])
    return e / oracle.sum_along(e, 1)[:, None]


@pytest.mark.parametrize("mutant, which", [(_log_softmax_reversed_sum, "log_softmax"),
                                           (_log_sum_exp_first_shift, "logsumexp"),
                                           (_softmax_divided, "softmax")])
@pytest.mark.parametrize("rows, columns", WIDTHS[:2])
def test_planted_row_mistakes_fail(mutant, which, rows, columns):
    x = _rows(rows, columns, 13 + columns % 7)
    with np.errstate(all="ignore"):
        got = mutant(x).astype(np.float32)
    assert not np.array_equal(_bits(got), _bits(_facade_rows(x, which)))


# ---- the f32::max tie against LLVM's maxnum ----

@pytest.fixture(scope="module")
def maxnum():
    path = NATIVE / "libmaxnum_probe.so"
    if not path.exists():
        pytest.skip("tests/native/libmaxnum_probe.so is not built (poorgrad_amd/build.py builds it)")
    lib = ctypes.CDLL(str(path))
    lib.probe_maxnum.restype = ctypes.c_float
    lib.probe_maxnum.argtypes = [ctypes.c_float, ctypes.c_float]
    return lib.probe_maxnum


def _f32bits(x: float) -> int:
    return int(np.float32(x).view(np.uint32))


CASES = [(-0.0, 0.0), (0.0, -0.0), (-0.0, -0.0), (0.0, 0.0), (float("nan"), -0.0), (-0.0, float("nan")),
         (1.0, -1.0), (-1.0, 1.0), (float("inf"), float("nan")), (float("nan"), float("nan")),
         (-float("inf"), -0.0), (1e-45, -1e-45)]


@pytest.mark.parametrize("a, b", CASES)
def test_max_tie_is_llvm_maxnum(maxnum, a, b):
    got = np.float32(oracle.lib.oracle_binary_f32(oracle.MAX, a, b))
    want = np.float32(maxnum(a, b))
    if np.isnan(want):
        assert np.isnan(got)
    else:
        assert _f32bits(got) == _f32bits(want)


def test_relu_of_negative_zero_is_llvm_maxnum(maxnum):
    # relu = maximum(zero_like) (src/function/relu.rs): max(-0, +0).
    x = np.array([-0.0, 0.0, -1.0, 2.0], dtype=np.float32)
    got = oracle.zip_(oracle.MAX, x, np.zeros_like(x))
    want = np.array([maxnum(float(v), 0.0) for v in x], dtype=np.float32)
    assert np.array_equal(_bits(got), _bits(want))
    assert _f32bits(got[0]) == 0x80000000  # the first operand wins the tie


def test_reversed_tie_would_fail(maxnum):
    # A max that keeps the second operand on a tie (glibc fmaxf's choice)
    # disagrees with maxnum on (-0, +0): the comparison above catches it.
    def second_on_tie(a, b):
        return b if a == b else max(a, b)
    assert _f32bits(second_on_tie(-0.0, 0.0)) != _f32bits(maxnum(-0.0, 0.0))
