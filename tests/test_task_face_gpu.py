"""The offered task face on a real device: host buffers in, product out,
exactly as a `Backend::Hip` arm of `Task::offer` would be called."""
import numpy as np
import pytest

import oracle
from poorgrad_amd import tasks
from tests.conftest import banner
from tests.gpu_util import assert_bitwise

pytestmark = pytest.mark.gpu


def test_gemm_task_exact_and_fast(hip):
    banner("task face gemm")
    m, k, n = 200, 300, 400
    g = oracle.Generator(7)
    a = g.normal(m * k, 1.0)
    b = g.normal(k * n, 1.0)
    expected = oracle.gemm(a, (k, 1), b, (n, 1), m, k, n)
    exact = tasks.gemm_f32(a, (k, 1), b, (n, 1), m, k, n, hip.EXACT)
    assert exact is not None
    assert_bitwise(exact, expected, "task exact")
    fast = tasks.gemm_f32(a, (k, 1), b, (n, 1), m, k, n, hip.FAST)
    bound = 1e-5 * (np.abs(a.reshape(m, k).astype(np.float64)) @ np.abs(b.reshape(k, n).astype(np.float64)))
    assert (np.abs(fast - expected) <= bound).all()
    # A transposed right operand (G . B^T): strides [1, k] over a [n, k] buffer.
    bt = np.ascontiguousarray(b.reshape(k, n).T)
    assert_bitwise(tasks.gemm_f32(a, (k, 1), bt, (1, k), m, k, n, hip.EXACT), expected, "task b^T")


def test_map_task(hip):
    banner("task face map")
    x = oracle.Generator(9).normal(1 << 18, 4.0)
    for op, ref in ((0, oracle.EXP), (1, oracle.LN), (2, oracle.SQRT), (3, oracle.TANH)):
        got = tasks.map_f32(op, x)
        assert got is not None
        assert_bitwise(got, oracle.map_(ref, x), f"map {op}")
