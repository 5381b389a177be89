"""The composed formulas' dedicated device forms against the oracle
interpreter, over shapes beyond the reference's bench:

* WindowProduct (src/engine/pattern/window.rs:58-150,
  src/payload/tensor.rs:1475-1544): conv2d's im2col chain is never
  materialised; the forward product and the kernel gradient gather the patch
  matrix from the source (strides 1-3, padding 0-2, square and oblong
  kernels, a permuted source view);
* ReduceWindow (src/engine/pattern/reduce_window.rs): max_pool's lanes read
  the source through window views (one launch, the recorded lane order);
* BatchNormTraining (src/engine/pattern/batch_norm.rs): the statistics, the
  normalisation and the affine map as one column program.

Exact: every readable value bitwise. Fast: the window products and every
fold stay exact, so only the input gradient (a matrix-core product) is
held to the envelope."""
import numpy as np
import pytest

from poorgrad_amd import topos as t
from tests.conftest import banner
from tests.gpu_util import assert_bitwise
from tests.program_util import run_device, run_oracle

pytestmark = pytest.mark.gpu

# (batch, channels, height, width, filters, kernel_h, kernel_w, stride, padding, permuted source)
CONVS = [
    (2, 3, 9, 11, 4, 3, 3, 2, 0, False),
    (3, 2, 8, 8, 5, 3, 2, 1, 2, False),
    (2, 4, 7, 10, 3, 1, 1, 1, 0, True),
    (1, 3, 12, 12, 6, 5, 5, 3, 1, True),
    (4, 16, 14, 14, 32, 3, 3, 1, 1, False),
]


def _conv_step(batch, channels, height, width, filters, kh, kw, stride, padding, permuted):
    tape = t.Tape()
    if permuted:  # the source is a transposed view of the input
        x = tape.input((batch, channels, width, height))
        source = x.permute([0, 1, 3, 2])
    else:
        x = tape.input((batch, channels, height, width))
        source = x
    w = tape.parameter((filters, channels, kh, kw))
    b = tape.parameter((filters,))
    y = t.conv2d(source, w, b, stride, padding)
    r = tape.input(y.shape)
    loss = (y * r).sum()
    gx, gw, gb = tape.differentiate(loss, [x, w, b])
    rng = np.random.default_rng(batch * 100 + channels * 10 + kh)
    params = [rng.standard_normal(w.shape).astype(np.float32), rng.standard_normal(b.shape).astype(np.float32)]
    dense = {x.node.slot: rng.standard_normal(x.shape).astype(np.float32),
             r.node.slot: rng.standard_normal(r.shape).astype(np.float32)}
    return tape, [y, loss, gx, gw, gb], params, dense


@pytest.mark.parametrize("case", CONVS, ids=lambda c: "x".join(map(str, c[:9])) + ("p" if c[9] else ""))
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_window_product_conv_step(hip, case, posture):
    banner(f"window product conv {case} {posture}")
    tape, roots, params, dense = _conv_step(*case)
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    want = run_oracle(tape, roots, params, dense)
    got, program = run_device(tape, roots, params, dense, numerics=numerics)
    assert "gemm window patches " in program.describe and "gemm window patches^T" in program.describe
    assert "pad [" not in program.describe
    y, loss, gx, gw, gb = roots
    for r in (y, gw, gb):
        assert_bitwise(got[r.id], want[r.id], f"{posture} node {r.id} {r.shape}")
    if numerics == hip.EXACT:
        assert_bitwise(got[loss.id], want[loss.id], "loss")
        assert_bitwise(got[gx.id], want[gx.id], "input gradient")
    else:
        e = want[gx.id].astype(np.float64)
        assert np.abs(got[gx.id].astype(np.float64) - e).max() <= 1e-3 * max(np.abs(e).max(), 1e-3)


@pytest.mark.parametrize("size, stride", [(2, 2), (3, 2), (3, 1), (2, 3)])
def test_reduce_window_reads_the_source(hip, size, stride):
    """max_pool with overlapping (stride < size) and gapped (stride > size)
    windows, ties and signed zeros included, with its gradient: bitwise, and
    no lane copy."""
    banner(f"reduce window size {size} stride {stride}")
    tape = t.Tape()
    x = tape.input((3, 4, 11, 13))
    pooled = t.max_pool(x, size, stride)
    r = tape.input(pooled.shape)
    loss = (pooled * r).sum()
    (gx,) = tape.differentiate(loss, [x])
    rng = np.random.default_rng(size * 10 + stride)
    values = rng.integers(-3, 4, x.shape).astype(np.float32)  # many ties
    values[0, 0, :2, :] = -0.0
    dense = {x.node.slot: values, r.node.slot: rng.standard_normal(r.shape).astype(np.float32)}
    want = run_oracle(tape, [pooled, gx], [], dense)
    got, program = run_device(tape, [pooled, gx], [], dense)
    assert "copy [" not in program.describe
    for v in (pooled, gx):
        assert_bitwise(got[v.id], want[v.id], f"node {v.id} {v.shape}")


@pytest.mark.parametrize("rows, features", [(256, 512), (64, 100), (7, 33), (1024, 48)])
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_batch_norm_is_one_column_program(hip, rows, features, posture):
    """BatchNorm's statistics and output (src/neural/batch_norm.rs:149-176)
    in one launch, and its training gradients, bitwise in both postures
    (no product is involved)."""
    banner(f"batch norm column program {rows}x{features} {posture}")
    tape = t.Tape()
    x = tape.input((rows, features))
    scale, shift = tape.parameter((features,)), tape.parameter((features,))
    epsilon = tape.leaf(t.Constant((), 1e-5))
    out, mean, variance = t.batch_norm(x, scale, shift, epsilon)
    r = tape.input(out.shape)
    loss = (out * r).sum()
    gx, gs, gb = tape.differentiate(loss, [x, scale, shift])
    rng = np.random.default_rng(rows + features)
    params = [rng.standard_normal(features).astype(np.float32), rng.standard_normal(features).astype(np.float32)]
    dense = {x.node.slot: (3 * rng.standard_normal((rows, features)) + 1).astype(np.float32),
             r.node.slot: rng.standard_normal((rows, features)).astype(np.float32)}
    roots = [out, mean, variance, gx, gs, gb]
    numerics = hip.EXACT if posture == "exact" else hip.FAST
    want = run_oracle(tape, roots, params, dense)
    got, program = run_device(tape, roots, params, dense, numerics=numerics)
    assert program.describe.count("columns [") >= 1
    for v in roots:
        assert_bitwise(got[v.id], want[v.id], f"{posture} node {v.id} {v.shape}")
