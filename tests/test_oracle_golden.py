"""Pins the CPU oracle to the reference's own golden vectors and closed forms
(oracle/ restates src/payload and src/neural; these checks make a dropped term,
a wrong seed or a transposed operand fail)."""
import math
from fractions import Fraction
import struct

import numpy as np
import pytest

import oracle


def f64_bits(x: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def f32_of_f64_bits(bits: int) -> int:
    return struct.unpack("<I", struct.pack("<f", np.float32(struct.unpack("<d", struct.pack("<Q", bits))[0])))[0]


# src/neural/tests/init_tests.rs:81-134: seeded streams pinned forever.
GOLDEN_UNIFORM_7 = [0xbfcc341e1ba6cdf8, 0xbfeeecf0ca02f0e8, 0x3fe9a610202eac4a, 0x3fc53aeb70673e28]
GOLDEN_NORMAL_7_DEV2 = [0x3fffa194ec47d228, 0xc00dd3fde5949e97, 0x3f800ea29c8645d7, 0xbff0efc91ba890b4]
GOLDEN_XAVIER_7_2x2 = [0xbfd14566a85c9c0a, 0xbff2f01dbe7ab6a2, 0x3fef69c081567c5c, 0x3fca0063d7a5b7aa]
GOLDEN_KAIMING_7_2x2 = [0x3fefa194ec47d228, 0xbffdd3fde5949e97, 0x3f700ea29c8645d7, 0xbfe0efc91ba890b4]


@pytest.mark.parametrize("golden, draw", [
    (GOLDEN_UNIFORM_7, lambda g: g.uniform64(4, 1.0)),
    (GOLDEN_NORMAL_7_DEV2, lambda g: g.normal64(4, 2.0)),
    (GOLDEN_XAVIER_7_2x2, lambda g: g.uniform64(4, math.sqrt(6.0 / 4.0))),   # xavier: sqrt(6/(2+2))
    (GOLDEN_KAIMING_7_2x2, lambda g: g.normal64(4, math.sqrt(2.0 / 2.0))),   # kaiming: sqrt(2/fan_in)
])
def test_seeded_streams_match_reference_goldens(golden, draw):
    doubles = draw(oracle.Generator(7))
    assert [f64_bits(float(d)) for d in doubles] == golden


def test_f32_stream_is_the_f64_stream_rounded_once():
    singles = oracle.Generator(7).normal(4, 2.0)
    assert [int(s.view(np.uint32)) for s in singles] == [f32_of_f64_bits(b) for b in GOLDEN_NORMAL_7_DEV2]


def test_splitmix64_known_answer():
    # splitmix64 from state 0: the published first outputs of the generator.
    g = oracle.Generator(0)
    assert [g.next_u64() for _ in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def logical_reference(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """src/payload/tests/gemm_tests.rs:10-30: ascending inner index, seeded
    from the first term, pure-Python loops in f32."""
    rows, inner = a.shape
    columns = b.shape[1]
    out = np.empty((rows, columns), dtype=np.float32)
    for i in range(rows):
        for j in range(columns):
            total = np.float32(a[i, 0]) * np.float32(b[0, j])
            for s in range(1, inner):
                total = np.float32(total + np.float32(a[i, s]) * np.float32(b[s, j]))
            out[i, j] = total
    return out


def varied(rows, columns, seed):
    # src/payload/tests/gemm_tests.rs:50-56
    index = np.arange(rows * columns, dtype=np.int64)
    return (((index * 7 + seed * 13) % 23 - 11) / 4.0).astype(np.float32).reshape(rows, columns)


@pytest.mark.parametrize("m, k, n", [(1, 1, 1), (2, 3, 4), (5, 8, 13), (16, 16, 16), (7, 1, 9), (3, 17, 2)])
def test_gemm_matches_logical_order(m, k, n):
    rng = np.random.default_rng(m * 100 + k * 10 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    expected = logical_reference(a, b)
    got = oracle.gemm(a, (k, 1), b, (n, 1), m, k, n)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
    # Transposed views of the same logical operands: strides [1, m] and [1, k].
    at = np.ascontiguousarray(a.T)
    bt = np.ascontiguousarray(b.T)
    got_t = oracle.gemm(at, (1, m), bt, (1, k), m, k, n)
    assert np.array_equal(got_t.view(np.uint32), expected.view(np.uint32))


def test_gemm_varied_values_exact():
    a, b = varied(5, 7, 1), varied(7, 3, 2)
    assert np.array_equal(oracle.gemm(a, (7, 1), b, (3, 1), 5, 7, 3), logical_reference(a, b))


def test_gemm_negative_zero_terms_keep_their_sign():
    # src/payload/tests/gemm_tests.rs:130-139
    a = np.array([[-0.0, 0.0]], dtype=np.float32)
    b = np.array([[0.0], [-0.0]], dtype=np.float32)
    out = oracle.gemm(a, (2, 1), b, (1, 1), 1, 2, 1)
    assert out.view(np.uint32)[0, 0] == np.float32(-0.0).view(np.uint32)


def test_gemm_is_not_fused_multiply_add():
    # (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 needs 25 bits: the separately rounded
    # product is 1 + 2^-11 (tie to even), so adding -(1 + 2^-11) gives 0; a
    # fused multiply-add would keep 2^-24.
    a = np.array([[1.0 + 2.0**-12, 1.0]], dtype=np.float32)
    b = np.array([[1.0 + 2.0**-12], [-(1.0 + 2.0**-11)]], dtype=np.float32)
    out = oracle.gemm(a, (2, 1), b, (1, 1), 1, 2, 1)[0, 0]
    assert out == np.float32(0.0)
    exact = Fraction(1 + 2**-12) ** 2 - Fraction(1 + 2**-11)
    assert exact == Fraction(2) ** -24


def test_plan_exact_gemm_32x32_closed_form():
    # src/engine/tests/plan_tests.rs:542-571: a = (v % 37) * 0.21 - 3.7, b = (v % 29) * 0.17 - 2.3.
    v = np.arange(32 * 32)
    a = ((v % 37) * np.float32(0.21) - np.float32(3.7)).astype(np.float32)
    a = np.array([np.float32(np.float32(x % 37) * np.float32(0.21)) - np.float32(3.7) for x in v], dtype=np.float32)
    b = np.array([np.float32(np.float32(x % 29) * np.float32(0.17)) - np.float32(2.3) for x in v], dtype=np.float32)
    a, b = a.reshape(32, 32), b.reshape(32, 32)
    assert np.array_equal(oracle.gemm(a, (32, 1), b, (32, 1), 32, 32, 32), logical_reference(a, b))


def test_reductions_closed_forms():
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4) - 5.5
    # sum_along over every axis equals the ordered fold.
    for axis in range(3):
        moved = np.moveaxis(x, axis, -1)
        expected = np.empty(moved.shape[:-1], dtype=np.float32)
        for idx in np.ndindex(expected.shape):
            total = moved[idx][0]
            for value in moved[idx][1:]:
                total = np.float32(total + value)
            expected[idx] = total
        assert np.array_equal(oracle.sum_along(x, axis), expected)
        assert np.array_equal(oracle.max_along(x, axis), moved.max(axis=-1))
    assert oracle.sum_(np.array([1e8, 1.0, -1e8], dtype=np.float32)) == np.float32(0.0)  # ordered, not exact


def test_max_nan_loses_and_zero_tie_keeps_first():
    assert oracle.lib.oracle_binary_f32(oracle.MAX, float("nan"), 2.0) == 2.0
    assert oracle.lib.oracle_binary_f32(oracle.MAX, 2.0, float("nan")) == 2.0
    tie = np.float32(oracle.lib.oracle_binary_f32(oracle.MAX, -0.0, 0.0))
    assert tie.view(np.uint32) == np.float32(-0.0).view(np.uint32)
    assert oracle.lib.oracle_binary_f32(oracle.STEP, 1.0, 1.0) == 1.0  # ties answer one
    assert oracle.lib.oracle_binary_f32(oracle.STEP, float("nan"), 0.0) == 0.0


def test_log_softmax_special_cases():
    # Uniform logits: every log-probability is -ln(3) (src/neural/tests/loss_tests.rs:6-18).
    out = oracle.log_softmax_rows(np.zeros((2, 3), dtype=np.float32))
    assert np.allclose(out, -math.log(3.0), atol=1e-7)
    # Extreme logits: the winner's log-probability is exactly zero (loss_tests.rs:100-132).
    out = oracle.log_softmax_rows(np.array([[1000.0, 0.0, -1000.0]], dtype=np.float32))
    assert out[0, 0] == 0.0 and out[0, 2] == -2000.0
    # softmax sums to one within rounding; LSE of a constant row is c + ln(n).
    p = oracle.softmax_rows(np.array([[1.0, 2.0, 3.0, 4.0]], dtype=np.float32))
    assert abs(float(p.sum()) - 1.0) < 1e-6
    assert abs(oracle.log_sum_exp_rows(np.full((1, 4), 2.0, dtype=np.float32))[0] - (2.0 + math.log(4.0))) < 1e-6


def test_layer_norm_closed_form():
    x = np.array([[1.0, 2.0, 3.0, 4.0]], dtype=np.float32)
    out = oracle.layer_norm_rows(x, np.ones(4, np.float32), np.zeros(4, np.float32), 0.0)
    # mean 2.5, biased variance 1.25
    expected = (x - 2.5) / np.sqrt(np.float32(1.25))
    assert np.allclose(out, expected, atol=1e-6)
    shifted = oracle.layer_norm_rows(x, np.full(4, 2.0, np.float32), np.full(4, 1.0, np.float32), 0.0)
    assert np.allclose(shifted, 2.0 * expected + 1.0, atol=1e-6)


def test_bf16_rounding_golden_cases():
    """Bf16::from_f32 against the reference's own cases
    (src/payload/tests/bf16_tests.rs:6-52): ties to even, the carry into the
    extremes, signed zeros, NaN kept a NaN, and every bit pattern
    round-tripping through f32."""
    f = np.float32

    def h(x):
        return int(oracle.lib.oracle_bf16_from_f32(f(x)))

    assert h(1.003_906_25) == h(1.0) == 0x3F80            # 1 + 2^-8 ties to the even 1.0
    assert h(1.011_718_75) == h(1.015_625) == 0x3F82      # 1 + 3 * 2^-8 ties to the even neighbour
    assert h(1.006) == h(1.007_812_5) == 0x3F81           # off a tie: the nearest
    assert h(np.finfo(np.float32).max) == 0x7F80          # carries into infinity
    assert h(-np.finfo(np.float32).max) == 0xFF80
    assert h(-0.0) == 0x8000 and h(0.0) == 0x0000
    assert np.isnan(oracle.bf16_widen(np.array([h(np.nan)], np.uint16))[0])
    every = np.arange(1 << 16, dtype=np.uint16)
    back = oracle.bf16_round(oracle.bf16_widen(every))
    nan = np.isnan(oracle.bf16_widen(every))
    assert np.array_equal(back[~nan], every[~nan])
    assert np.isnan(oracle.bf16_widen(back[nan])).all()


def test_bf16_matmul_accumulates_in_f32_and_rounds_once():
    """src/payload/tests/bf16_tests.rs:117-127: [256, 1, 1] . [1, 1, 1] is 258
    (per-op bf16 accumulation would answer 256)."""
    left = oracle.bf16_round(np.array([[256.0, 1.0, 1.0]], np.float32))
    right = oracle.bf16_round(np.array([[1.0], [1.0], [1.0]], np.float32))
    product = oracle.gemm_bf16(left, (3, 1), right, (1, 1), 1, 3, 1)
    assert oracle.bf16_widen(product)[0, 0] == 258.0
