"""The topos interpreter, restated over a recorded tape (poorgrad_amd.topos):
``Network::run`` (src/engine/run.rs:417-526) evaluating every wanted node in
recording order with ``Function::forward`` (src/function/function.rs:432-478).

TEST INFRASTRUCTURE ONLY: parity tests compare the device program with this
evaluation. Views are numpy views (a view changes no values,
src/payload/layout.rs); every arithmetic operation goes through the C oracle
(oracle.c), or through numpy's IEEE single-precision +, -, *, / which round
each element once exactly like the interpreter's f32 operators.
"""
from __future__ import annotations

import numpy as np

import oracle
from poorgrad_amd import topos as t


class Sel:
    """A Selection payload (src/payload/storage.rs:45-50)."""

    def __init__(self, indices, vocab: int, one: float = 1.0):
        self.indices = np.asarray(indices, dtype=np.int64)
        self.vocab = int(vocab)
        self.one = np.float32(one)

    def dense(self) -> np.ndarray:
        # Tensor::get on a selection (tensor.rs:220-240): one at the index, +0 elsewhere.
        out = np.zeros((len(self.indices), self.vocab), dtype=np.float32)
        out[np.arange(len(self.indices)), self.indices] = self.one
        return out


def _dense(x) -> np.ndarray:
    return x.dense() if isinstance(x, Sel) else np.ascontiguousarray(x, dtype=np.float32)


def _expand(x: np.ndarray, axis: int, shape) -> np.ndarray:
    return np.broadcast_to(np.expand_dims(x, axis), shape)


def _matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Tensor::matmul (tensor.rs:921-1027): one gemm::multiply per batch slice."""
    a, b = _dense(a), _dense(b)
    m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
    batch = a.shape[:-2]
    out = np.empty(batch + (m, n), dtype=np.float32)
    for index in np.ndindex(*batch):
        out[index] = oracle.gemm(a[index], (k, 1), b[index], (n, 1), m, k, n)
    return out


def _log_softmax(x: np.ndarray, axis: int) -> np.ndarray:
    """LogSoftmax::forward (src/function/log_softmax.rs:51-60), term by term."""
    x = _dense(x)
    peak = _expand(oracle.max_along(x, axis), axis, x.shape)
    shifted = x - peak
    normalizer = oracle.map_(oracle.LN, oracle.sum_along(oracle.map_(oracle.EXP, shifted), axis))
    return shifted - _expand(normalizer, axis, x.shape)


def _log_sum_exp(x: np.ndarray, axis: int) -> np.ndarray:
    """LogSumExp::forward (src/function/log_sum_exp.rs:53-61)."""
    x = _dense(x)
    peak = oracle.max_along(x, axis)
    shifted = x - _expand(peak, axis, x.shape)
    return peak + oracle.map_(oracle.LN, oracle.sum_along(oracle.map_(oracle.EXP, shifted), axis))


def _scatter(g: np.ndarray, selection: Sel, rows: int) -> np.ndarray:
    """Tensor::scatter (tensor.rs:1582-1618): zero-seeded, in source order."""
    g = _dense(g)
    acc = np.zeros((rows,) + g.shape[1:], dtype=np.float32)
    for source, target in enumerate(selection.indices):
        acc[target] = acc[target] + g[source]
    return acc


def _unfold(x: np.ndarray, axis: int, size: int, step: int, dilation: int) -> np.ndarray:
    """Tensor::unfold, the strided window view of Layout::unfold
    (src/payload/layout.rs:299-331): (count, size) at `axis`, window starts
    `step` apart, window elements `dilation` apart."""
    x = _dense(x)
    count = (x.shape[axis] - dilation * (size - 1) - 1) // step + 1
    shape = x.shape[:axis] + (count, size) + x.shape[axis + 1:]
    # An extent-1 axis never advances, so its stride is 0 (layout.rs:311-329):
    # a single window takes any step.
    along = x.strides[axis]
    strides = x.strides[:axis] + (0 if count == 1 else along * step, 0 if size == 1 else along * dilation) \
        + x.strides[axis + 1:]
    return np.lib.stride_tricks.as_strided(x, shape, strides, writeable=False)


def _fold(x: np.ndarray, axis: int, size: int, step: int, dilation: int, extent: int) -> np.ndarray:
    """Tensor::fold (src/payload/tensor.rs:1392-1462): each position sums, from
    +0 and in ascending window-element order k, the terms of the windows w
    with w * step + k * dilation == position."""
    x = _dense(x)
    count = x.shape[axis]
    out = np.zeros(x.shape[:axis] + (extent,) + x.shape[axis + 2:], dtype=np.float32)
    positions = np.arange(extent)
    lead = (slice(None),) * axis
    for k in range(size):
        rest = positions - k * dilation
        valid = (rest >= 0) & (rest % step == 0) & (rest // step < count)
        target, window = positions[valid], rest[valid] // step
        out[lead + (target,)] = out[lead + (target,)] + x[lead + (window, k)]
    return out


def forward(node: t.Node, operands: list, parameters: list, inputs: list):
    """Function::forward of one node."""
    op = node.op
    if op == t.LEAF:
        p = node.payload
        if isinstance(p, t.Constant):
            return np.full(p.shape, np.float32(p.value), dtype=np.float32)
        if isinstance(p, t.Dense):
            return p.array
        return Sel(p.indices, p.vocab, p.one)
    if op == t.PARAMETER:
        return parameters[node.slot]
    if op == t.INPUT:
        return inputs[node.slot]
    a = operands[0] if operands else None
    b = operands[1] if len(operands) > 1 else None
    if op in (t.ADD, t.SUB, t.MUL, t.DIV):
        x, y = _dense(a), _dense(b)
        return {t.ADD: np.add, t.SUB: np.subtract, t.MUL: np.multiply, t.DIV: np.divide}[op](x, y)
    if op == t.NEG:
        return -_dense(a)
    unary = {t.TANH: oracle.TANH, t.EXP: oracle.EXP, t.LN: oracle.LN, t.SQRT: oracle.SQRT}
    if op in unary:
        return oracle.map_(unary[op], _dense(a))
    binary = {t.POWF: oracle.POWF, t.MAXIMUM: oracle.MAX, t.STEP: oracle.STEP}
    if op in binary:
        return oracle.zip_(binary[op], _dense(a), _dense(b))
    if op == t.RELU:
        x = _dense(a)
        return oracle.zip_(oracle.MAX, x, np.zeros_like(x))  # maximum(zero_like)
    if op == t.MATMUL:
        return _matmul(a, b)
    if op == t.TRANSPOSE:
        x = _dense(a)
        return x.T if x.ndim == 2 else x
    if op == t.SUM:
        return np.array(oracle.sum_(_dense(a)), dtype=np.float32)
    if op == t.SUM_ALONG:
        return oracle.sum_along(_dense(a), node.params[0])
    if op == t.BROADCAST:
        return np.broadcast_to(_dense(a).ravel()[0], node.shape)
    if op == t.BROADCAST_ALONG:
        return _expand(_dense(a), node.params[0], node.shape)
    if op == t.RESHAPE:
        return _dense(a).reshape(node.shape)
    if op == t.PERMUTE:
        return np.transpose(_dense(a), node.params)
    if op == t.NARROW:
        axis, start, length = node.params
        x = _dense(a)
        index = [slice(None)] * x.ndim
        index[axis] = slice(start, start + length)
        return x[tuple(index)]
    if op == t.PAD:
        axis, start, full = node.params
        x = _dense(a)
        out = np.zeros(node.shape, dtype=np.float32)  # zero_like of an element: +0
        index = [slice(None)] * x.ndim
        index[axis] = slice(start, start + x.shape[axis])
        out[tuple(index)] = x
        return out
    if op == t.UNFOLD:
        return _unfold(a, *node.params[:4])
    if op == t.FOLD:
        return _fold(a, *node.params[:5])
    if op == t.GATHER:
        return _dense(a)[b.indices]
    if op == t.SCATTER:
        return _scatter(a, b, node.params[0])
    if op == t.LOG_SOFTMAX:
        return _log_softmax(a, node.params[0])
    if op == t.LOG_SUM_EXP:
        return _log_sum_exp(a, node.params[0])
    raise NotImplementedError(t.NAMES[op])


def run(tape: t.Tape, readable, parameters: list, inputs: list) -> dict:
    """Evaluates the ancestors of `readable` (Values or node indices) in
    recording order and returns {node index: value}."""
    targets = [r.id if isinstance(r, t.Value) else int(r) for r in readable]
    wanted = [False] * len(tape.nodes)
    for i in targets:
        wanted[i] = True
    for i in range(len(tape.nodes) - 1, -1, -1):
        if wanted[i]:
            for link in tape.nodes[i].operands:
                wanted[link] = True
    # A value is dropped after its last wanted consumer (the releases of a
    # forward-only plan, src/engine/plan.rs:612-621), so full-width graphs fit
    # in host memory; numpy views keep their bases alive as long as needed.
    keep = set(targets)
    last_use = [-1] * len(tape.nodes)
    for i, node in enumerate(tape.nodes):
        if wanted[i]:
            for link in node.operands:
                last_use[link] = i
    values: list = [None] * len(tape.nodes)
    for i, node in enumerate(tape.nodes):
        if wanted[i]:
            values[i] = forward(node, [values[link] for link in node.operands], parameters, inputs)
            for link in node.operands:
                if last_use[link] == i and link not in keep:
                    values[link] = None
    out = {}
    for i in targets:
        v = values[i]
        out[i] = v.dense() if isinstance(v, Sel) else np.array(v, dtype=np.float32)
    return out
