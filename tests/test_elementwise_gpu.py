"""Maps and generated chains on the GPU against the host libm and the
oracle's op-by-op composition (every intermediate rounded to f32, as the
interpreter materialises it): bit-identical."""
import ctypes
import os
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from poorgrad_amd import device
from tests.conftest import banner
from tests.gpu_util import assert_bitwise, to_device

pytestmark = pytest.mark.gpu

_CHECK = Path(__file__).resolve().parent / "native" / "libfaithful_check.so"


@pytest.fixture(scope="module")
def host_libm():
    lib = ctypes.CDLL(str(_CHECK))
    lib.host_libm_range.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64,
                                    ctypes.POINTER(ctypes.c_uint32), ctypes.c_int]
    return lib


@pytest.mark.parametrize("operation, name", [(0, "exp"), (1, "ln"), (2, "sqrt"), (3, "tanh")])
def test_map_every_f32_input_matches_host_libm(hip, host_libm, operation, name):
    """All 2^32 inputs, in chunks: the device map against the host glibc."""
    banner(f"exhaustive map {name}")
    checker_function = {0: 0, 1: 1, 2: 3, 3: 2}[operation]  # faithful_check numbering
    chunk = 1 << 26
    threads = max(1, min(16, os.cpu_count() or 1))
    expected = np.empty(chunk, dtype=np.uint32)
    for start in range(0, 1 << 32, chunk):
        inputs = torch.arange(start, start + chunk, dtype=torch.int64, device="cuda").to(torch.int32)
        x = inputs.view(torch.float32)
        y = device.map_(operation, x)
        got = y.view(torch.int32).cpu().numpy().view(np.uint32).copy()
        got_f = got.view(np.float32)
        got[np.isnan(got_f)] = 0x7FC00000
        host_libm.host_libm_range(checker_function, start, chunk,
                                  expected.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), threads)
        if not np.array_equal(got, expected):
            bad = np.flatnonzero(got != expected)[:5]
            raise AssertionError(f"{name}: {len(np.flatnonzero(got != expected))} differ in chunk 0x{start:08x}; "
                                 f"inputs {[hex(start + int(i)) for i in bad]}")


POW_FAMILIES = ["random bits", "positive bases", "negative bases", "bases near one", "overflow edges", "dyadic"]


@pytest.mark.parametrize("family", range(len(POW_FAMILIES)), ids=POW_FAMILIES)
def test_chain_powf_matches_host_libm_on_dense_samples(hip, host_libm, family):
    """powf in a generated chain against the box host's glibc powf on 2^24
    seeded pairs per input family (the families of the CPU check of the
    restated source), NaN as a class."""
    from poorgrad_amd import _native as n

    banner(f"chain powf {POW_FAMILIES[family]}")
    count = 1 << 24
    host_libm.pow_pairs.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_float),
                                    ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint32)]
    x = np.empty(count, np.float32)
    y = np.empty(count, np.float32)
    expected = np.empty(count, np.uint32)
    host_libm.pow_pairs(family, 11, count, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                        y.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                        expected.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    chain = device.Chain((count,), [((1,), 0), ((1,), 0)], [(n.CHAIN_POWF, -1, -2)], [0])
    got = chain(to_device(x), to_device(y))[0].cpu().numpy().view(np.uint32).copy()
    got[np.isnan(got.view(np.float32))] = 0x7FC00000
    if not np.array_equal(got, expected):
        bad = np.flatnonzero(got != expected)
        raise AssertionError(f"{len(bad)} pairs differ, e.g. powf({x[bad[0]]!r}, {y[bad[0]]!r}): "
                             f"0x{got[bad[0]]:08x} vs host 0x{expected[bad[0]]:08x}")


def compose(steps, inputs, outputs, shape):
    """The oracle's op-by-op evaluation of a chain over materialised views."""
    from poorgrad_amd import _native as n

    unary = {n.CHAIN_NEG: oracle.NEG, n.CHAIN_EXP: oracle.EXP, n.CHAIN_LN: oracle.LN,
             n.CHAIN_SQRT: oracle.SQRT, n.CHAIN_TANH: oracle.TANH}
    binary = {n.CHAIN_ADD: oracle.ADD, n.CHAIN_SUB: oracle.SUB, n.CHAIN_MUL: oracle.MUL,
              n.CHAIN_DIV: oracle.DIV, n.CHAIN_MAX: oracle.MAX, n.CHAIN_STEP: oracle.STEP,
              n.CHAIN_POWF: oracle.POWF}
    values = []

    def ref(r):
        return inputs[-r - 1] if r < 0 else values[r]

    for op, left, right in steps:
        if op in unary:
            values.append(oracle.map_(unary[op], ref(left)))
        else:
            values.append(oracle.zip_(binary[op], ref(left), ref(right)))
    return [ref(o) for o in outputs]


def materialise(buffer, shape, strides, offset):
    return np.lib.stride_tricks.as_strided(buffer[offset:], shape=shape,
                                           strides=[4 * s for s in strides]).copy()


def run_chain(shape, views, steps, outputs):
    """views: list of (buffer, strides, offset)."""
    chain = device.Chain(shape, [(st, off) for _, st, off in views], steps, outputs)
    got = chain(*[to_device(buf) for buf, _, _ in views])
    torch.cuda.synchronize()
    want = compose(steps, [materialise(buf, shape, st, off) for buf, st, off in views], outputs, shape)
    for g, w in zip(got, want):
        assert_bitwise(g, w, f"chain {shape}")
    return chain


@pytest.mark.parametrize("shape", [(64, 128), (7, 13), (3, 5, 8), (1,), (1024, 4096), (2, 3, 4, 20)])
def test_silu_bias_chain(hip, shape):
    """x / (exp(-x) + 1) + b, b broadcast along axis 0 (examples/llama/model.rs:258,
    src/neural/linear.rs:94-105)."""
    from poorgrad_amd import _native as n

    banner(f"silu+bias chain {shape}")
    g = oracle.Generator(11)
    volume = int(np.prod(shape))
    x = g.normal(volume, 1.0)
    b = g.normal(shape[-1], 1.0)
    one = np.array([1.0], np.float32)
    contiguous = [int(np.prod(shape[d + 1:])) for d in range(len(shape))]
    along0 = [0] * (len(shape) - 1) + [1]
    run_chain(shape, [(x, contiguous, 0), (b, along0, 0), (one, [0] * len(shape), 0)],
              [(n.CHAIN_NEG, -1, 0), (n.CHAIN_EXP, 0, 0), (n.CHAIN_ADD, 1, -3), (n.CHAIN_DIV, -1, 2),
               (n.CHAIN_ADD, 3, -2)], [4])


@pytest.mark.parametrize("shape", [(256, 768), (5, 7), (8192, 3072)])
def test_gelu_chain(hip, shape):
    """0.5 x (1 + tanh(0.7978846 (x + 0.044715 x^3))) with scalar leaves
    broadcast_like (examples/gpt2/model.rs:85-98), node for node."""
    from poorgrad_amd import _native as n

    banner(f"gelu chain {shape}")
    x = oracle.Generator(5).normal(int(np.prod(shape)), 2.0)
    consts = [np.array([v], np.float32) for v in (0.5, 1.0, 0.7978846, 0.044715)]
    contiguous = [shape[1], 1]
    views = [(x, contiguous, 0)] + [(c, [0, 0], 0) for c in consts]
    X, HALF, ONE, ROOT, COEF = -1, -2, -3, -4, -5
    steps = [(n.CHAIN_MUL, X, X), (n.CHAIN_MUL, 0, X), (n.CHAIN_MUL, 1, COEF),   # cubic
             (n.CHAIN_ADD, X, 2), (n.CHAIN_MUL, 3, ROOT), (n.CHAIN_TANH, 4, 0),  # inner
             (n.CHAIN_ADD, 5, ONE), (n.CHAIN_MUL, X, 6), (n.CHAIN_MUL, 7, HALF)]
    run_chain(shape, views, steps, [8, 5])  # the output and the tanh (kept for backward)


def test_chain_views_transposed_offset_and_column_broadcast(hip):
    """A transposed operand, a narrowed window with an offset, and a per-row
    statistic broadcast along axis 1 (stride [1, 0])."""
    from poorgrad_amd import _native as n

    banner("chain strided views")
    rows, cols = 37, 44
    g = oracle.Generator(3)
    t = g.normal(rows * cols, 1.0)           # stored [cols, rows]: read transposed
    wide = g.normal(rows * (cols + 9), 1.0)  # narrowed: columns 5..5+cols of [rows, cols+9]
    stat = g.normal(rows, 1.0) + 3.0         # per-row: broadcast along axis 1
    run_chain((rows, cols), [(t, [1, rows], 0), (wide, [cols + 9, 1], 5), (stat, [1, 0], 0)],
              [(n.CHAIN_SUB, -1, -2), (n.CHAIN_DIV, 0, -3), (n.CHAIN_MAX, 1, -1), (n.CHAIN_STEP, -2, -1),
               (n.CHAIN_SQRT, -3, 0), (n.CHAIN_LN, -3, 0), (n.CHAIN_MUL, 3, 4), (n.CHAIN_ADD, 6, 5)],
              [2, 7])


def test_chain_signed_zeros_and_specials(hip):
    from poorgrad_amd import _native as n

    banner("chain specials")
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4e38, -1.0, 1.0, 2.0, 0.5],
                 dtype=np.float32)
    y = np.array([-0.0, 0.0, np.inf, np.inf, 1.0, -1e-45, 1e-45, 3.4e38, -0.0, np.nan, 2.0, -0.5],
                 dtype=np.float32)
    steps = [(op, -1, -2) for op in (n.CHAIN_ADD, n.CHAIN_SUB, n.CHAIN_MUL, n.CHAIN_DIV, n.CHAIN_MAX,
                                     n.CHAIN_STEP)]
    steps += [(op, -1, 0) for op in (n.CHAIN_NEG, n.CHAIN_EXP, n.CHAIN_LN, n.CHAIN_SQRT, n.CHAIN_TANH)]
    run_chain((12,), [(x, [1], 0), (y, [1], 0)], steps, list(range(len(steps))))
