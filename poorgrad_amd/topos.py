"""The recording surface of topos, restated in Python: a Tape of nodes, Value
proxies with the reference's operation set, the composites built on it, and
``Tape.differentiate`` — the reverse scan that records gradients as ordinary
nodes. A recorded graph lowers to the device-program table of
``include/topos_hip.h`` (the columns a compiled ``Plan`` exposes).

This is the host side above the C ABI. topos records with Rust
(``src/graph``), which this image cannot compile; recording here follows the
same rules node for node so that the programs the library executes are the
plans topos would hand it:

* the op set and each rule's recorded backward are those of
  ``src/function/*.rs`` (``function.rs:26-59``), evaluated in the order the
  rules write them;
* ``differentiate`` follows ``src/graph/tape.rs:335-411``: a ones seed, ancestor
  marking through present cotangents, and zero-seeded accumulation
  ``zero_like() + contribution`` in reverse scan order;
* composites follow ``src/graph/composite.rs`` (softmax, mean_along, concat)
  and the neural facades ``src/neural/{linear,layer_norm,loss}.rs``.

No arithmetic happens here: payloads are recorded, never computed.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from typing import Iterable, Sequence

import numpy as np

# Function variants (include/topos_hip.h TOPOS_HIP_OP_*).
LEAF, PARAMETER, INPUT, ADD, SUB, MUL, DIV, NEG, TANH, EXP, LN, MATMUL, TRANSPOSE, SUM, SUM_ALONG = range(15)
BROADCAST, BROADCAST_ALONG, RESHAPE, PERMUTE, NARROW, PAD, UNFOLD, FOLD, GATHER, SCATTER = range(15, 25)
LOG_SOFTMAX, LOG_SUM_EXP, SQRT, POWF, MAXIMUM, RELU, STEP = range(25, 32)

NAMES = ["Leaf", "Parameter", "Input", "Add", "Sub", "Mul", "Div", "Neg", "Tanh", "Exp", "Ln", "MatMul",
         "Transpose", "Sum", "SumAlong", "Broadcast", "BroadcastAlong", "Reshape", "Permute", "Narrow", "Pad",
         "Unfold", "Fold", "Gather", "Scatter", "LogSoftmax", "LogSumExp", "Sqrt", "Powf", "Maximum", "Relu",
         "Step"]

MAX_RANK = 6


# ---- payloads (src/payload/storage.rs:36-51) ----

@dataclass(frozen=True)
class Constant:
    """Storage::Constant: one value over a shape (Tensor::filled / counted)."""
    shape: tuple
    value: float


@dataclass(frozen=True, eq=False)
class Dense:
    """Storage::Dense, row-major."""
    array: np.ndarray

    @property
    def shape(self) -> tuple:
        return tuple(self.array.shape)


@dataclass(frozen=True, eq=False)
class Selection:
    """Storage::Selection (Tensor::selection, src/payload/tensor.rs:312-342):
    row r is `one` at column indices[r] and +0 elsewhere."""
    indices: np.ndarray
    vocab: int
    one: float = 1.0

    @property
    def shape(self) -> tuple:
        return (len(self.indices), self.vocab)


def counted(shape, count: int) -> Constant:
    """Data::counted (src/payload/tensor.rs:705-707): `count` as f32 everywhere."""
    return Constant(tuple(shape), float(np.float32(count)))


@dataclass
class Node:
    op: int
    operands: tuple
    shape: tuple
    params: tuple = ()
    slot: int = -1
    payload: object = None  # leaves
    selection: bool = False  # selection inputs
    one: float = 1.0


def _without(shape: tuple, axis: int) -> tuple:
    return shape[:axis] + shape[axis + 1:]


class Tape:
    """The recording tape (src/graph/tape.rs): nodes in recording order."""

    def __init__(self):
        self.nodes: list[Node] = []
        self.parameter_shapes: list[tuple] = []
        self.input_shapes: list[tuple] = []
        self.parameter_nodes: list[int] = []

    # -- sources --
    def _record(self, op: int, operands: Sequence[int], shape, **kw) -> "Value":
        shape = tuple(int(s) for s in shape)
        assert len(shape) <= MAX_RANK, f"rank {len(shape)} exceeds the device's {MAX_RANK} axes"
        assert all(s > 0 for s in shape), "tensors must hold at least one element"
        self.nodes.append(Node(op, tuple(operands), shape, **kw))
        return Value(self, len(self.nodes) - 1)

    def parameter(self, shape) -> "Value":
        slot = len(self.parameter_shapes)
        self.parameter_shapes.append(tuple(shape))
        value = self._record(PARAMETER, (), shape, slot=slot)
        self.parameter_nodes.append(value.id)
        return value

    def input(self, shape) -> "Value":
        slot = len(self.input_shapes)
        self.input_shapes.append(tuple(shape))
        return self._record(INPUT, (), shape, slot=slot)

    def selection_input(self, rows: int, vocab: int, one: float = 1.0) -> "Value":
        slot = len(self.input_shapes)
        self.input_shapes.append((rows, vocab))
        return self._record(INPUT, (), (rows, vocab), slot=slot, selection=True, one=float(np.float32(one)))

    def leaf(self, payload) -> "Value":
        if isinstance(payload, Dense):
            payload = Dense(np.ascontiguousarray(payload.array, dtype=np.float32))
        return self._record(LEAF, (), payload.shape, payload=payload)

    def value(self, index: int) -> "Value":
        return Value(self, index)

    # -- the recorded reverse scan (src/graph/tape.rs:335-411) --
    def differentiate(self, loss: "Value", wrt: Iterable["Value"]) -> list["Value"]:
        assert loss.shape == (), "differentiate requires a scalar loss; reduce it with `sum` first"
        output = loss.id
        cotangents: list = [None] * (output + 1)
        cotangents[output] = loss.literal(counted(loss.shape, 1))
        ancestors = [False] * (output + 1)
        ancestors[output] = True
        for index in range(output, -1, -1):
            if not ancestors[index]:
                continue
            node = self.nodes[index]
            if not node.operands:
                continue  # sources: gradients stop here and are read out below
            operands = [Value(self, link) for link in node.operands]
            gradient = cotangents[index]
            recorded = _backward(node, operands, Value(self, index), gradient)
            assert len(recorded) == len(node.operands)
            for link, contribution in zip(node.operands, recorded):
                if contribution is None:
                    continue
                ancestors[link] = True
                existing = cotangents[link]
                seeded = existing if existing is not None else Value(self, link).zero_like()
                cotangents[link] = seeded + contribution
        out = []
        for target in wrt:
            gradient = cotangents[target.id] if target.id <= output else None
            out.append(gradient if gradient is not None else target.literal(counted(target.shape, 0)))
        return out

    # -- lowering to the device program --
    def program(self, roots: Sequence["Value"], observe: Sequence["Value"] = ()) -> "ProgramTable":
        """The node table of the plan that reads `roots` (and `observe`):
        every recorded node in order, the readable ones flagged
        (Request::roots / observe, src/engine/request.rs)."""
        return ProgramTable(self, [v.id for v in roots] + [v.id for v in observe])


class Value:
    """A proxy to one recorded node (src/graph/value.rs); operators record."""

    __slots__ = ("tape", "id")
    __array_priority__ = 1000

    def __init__(self, tape: Tape, index: int):
        self.tape, self.id = tape, index

    @property
    def node(self) -> Node:
        return self.tape.nodes[self.id]

    @property
    def shape(self) -> tuple:
        return self.node.shape

    def literal(self, payload) -> "Value":
        return self.tape.leaf(payload)

    def _apply(self, op, operands, shape, params=()) -> "Value":
        return self.tape._record(op, [o.id for o in operands], shape, params=tuple(int(p) for p in params))

    def _coerce(self, other) -> "Value":
        # Value op Data: the payload records as a literal (value.rs:539-575).
        return other if isinstance(other, Value) else self.literal(other)

    def _binary(self, op, other) -> "Value":
        other = self._coerce(other)
        assert other.shape == self.shape, f"tensors have different shapes: {self.shape} vs {other.shape}"
        return self._apply(op, [self, other], self.shape)

    # elementwise
    def __add__(self, other): return self._binary(ADD, other)
    def __sub__(self, other): return self._binary(SUB, other)
    def __mul__(self, other): return self._binary(MUL, other)
    def __truediv__(self, other): return self._binary(DIV, other)
    def __neg__(self): return self._apply(NEG, [self], self.shape)
    def tanh(self): return self._apply(TANH, [self], self.shape)
    def exp(self): return self._apply(EXP, [self], self.shape)
    def ln(self): return self._apply(LN, [self], self.shape)
    def sqrt(self): return self._apply(SQRT, [self], self.shape)
    def powf(self, exponent): return self._binary(POWF, exponent)
    def maximum(self, other): return self._binary(MAXIMUM, other)
    def relu(self): return self._apply(RELU, [self], self.shape)
    def step(self, threshold): return self._binary(STEP, threshold)

    # constants of this shape (Differentiable::zero_like / one_like on a trace)
    def zero_like(self) -> "Value": return self.literal(counted(self.shape, 0))
    def one_like(self) -> "Value": return self.literal(counted(self.shape, 1))

    # tensorial
    def matmul(self, rhs: "Value") -> "Value":
        a, b = self.shape, rhs.shape
        assert len(a) >= 2 and len(a) == len(b) and a[:-2] == b[:-2] and a[-1] == b[-2], f"matmul {a} x {b}"
        return self._apply(MATMUL, [self, rhs], a[:-1] + (b[-1],))

    def transpose(self) -> "Value":
        s = self.shape
        assert len(s) <= 2, "transpose supports rank 2 at most"
        return self._apply(TRANSPOSE, [self], s[::-1] if len(s) == 2 else s)

    def sum(self) -> "Value":
        return self._apply(SUM, [self], ())

    def sum_along(self, axis: int) -> "Value":
        return self._apply(SUM_ALONG, [self], _without(self.shape, axis), [axis])

    def broadcast_like(self, reference: "Value") -> "Value":
        assert math.prod(self.shape) == 1, "broadcast requires a single-element tensor"
        return self._apply(BROADCAST, [self, reference], reference.shape)

    def broadcast_along(self, axis: int, reference: "Value") -> "Value":
        assert self.shape == _without(reference.shape, axis), "broadcast_along needs the remaining shape"
        return self._apply(BROADCAST_ALONG, [self, reference], reference.shape, [axis])

    def reshape(self, shape) -> "Value":
        shape = tuple(shape)
        assert math.prod(shape) == math.prod(self.shape), "reshape changes the number of elements"
        return self._apply(RESHAPE, [self], shape)

    def permute(self, order) -> "Value":
        order = tuple(order)
        assert sorted(order) == list(range(len(self.shape))), "permute order must cover every axis"
        return self._apply(PERMUTE, [self], tuple(self.shape[a] for a in order), order)

    def unsqueeze(self, axis: int) -> "Value":
        s = list(self.shape)
        s.insert(axis, 1)
        return self.reshape(s)

    def squeeze(self, axis: int) -> "Value":
        s = list(self.shape)
        assert s[axis] == 1, "squeeze requires an extent-1 axis"
        del s[axis]
        return self.reshape(s)

    def narrow(self, axis: int, start: int, length: int) -> "Value":
        s = list(self.shape)
        assert 0 < length and start + length <= s[axis], "narrow window exceeds the axis"
        s[axis] = length
        return self._apply(NARROW, [self], s, [axis, start, length])

    def pad(self, axis: int, start: int, full_extent: int) -> "Value":
        s = list(self.shape)
        assert start + s[axis] <= full_extent, "pad window exceeds the full extent"
        s[axis] = full_extent
        return self._apply(PAD, [self], s, [axis, start, full_extent])

    def unfold(self, axis: int, size: int, step: int, dilation: int) -> "Value":
        """Unfold::infer_shape (src/function/unfold.rs:40-70): `axis` becomes
        the (count, size) pair of sliding windows."""
        s = list(self.shape)
        assert axis < len(s) and size > 0 and step > 0 and dilation > 0, "unfold parameters"
        span = dilation * (size - 1) + 1
        assert span <= s[axis], f"unfold window span {span} exceeds axis {axis} extent {s[axis]}"
        s[axis] = (s[axis] - span) // step + 1
        s.insert(axis + 1, size)
        return self._apply(UNFOLD, [self], s, [axis, size, step, dilation])

    def fold(self, axis: int, size: int, step: int, dilation: int, extent: int) -> "Value":
        """Fold::infer_shape (src/function/fold.rs:42-82): the (count, size)
        pair at `axis` folds back onto an axis of `extent`."""
        s = list(self.shape)
        assert axis + 1 < len(s) and size > 0 and step > 0 and dilation > 0, "fold parameters"
        span = dilation * (size - 1) + 1
        assert span <= extent, f"fold window span {span} exceeds the target extent {extent}"
        assert s[axis] == (extent - span) // step + 1 and s[axis + 1] == size, "fold window pair"
        s[axis] = extent
        del s[axis + 1]
        return self._apply(FOLD, [self], s, [axis, size, step, dilation, extent])

    def gather(self, selection: "Value") -> "Value":
        rows, vocab = selection.shape
        assert vocab == self.shape[0], "gather selection vocabulary must match the table rows"
        return self._apply(GATHER, [self, selection], (rows,) + self.shape[1:])

    def scatter(self, selection: "Value", rows: int) -> "Value":
        assert selection.shape == (self.shape[0], rows), "scatter selection shape"
        return self._apply(SCATTER, [self, selection], (rows,) + self.shape[1:], [rows])

    def log_softmax(self, axis: int) -> "Value":
        return self._apply(LOG_SOFTMAX, [self], self.shape, [axis])

    def logsumexp(self, axis: int) -> "Value":
        return self._apply(LOG_SUM_EXP, [self], _without(self.shape, axis), [axis])

    # composites (src/graph/composite.rs)
    def softmax(self, axis: int) -> "Value":
        return self.log_softmax(axis).exp()

    def mean_along(self, axis: int) -> "Value":
        extent = self.shape[axis]
        return self.sum_along(axis) / counted(_without(self.shape, axis), extent)

    def abs(self) -> "Value":
        return self.maximum(-self)


def concat(values: Sequence[Value], axis: int) -> Value:
    """concat = the sum of each value padded into place (composite.rs:142-183)."""
    if len(values) == 1:
        return values[0]
    combined = sum(v.shape[axis] for v in values)
    offset, total = 0, None
    for v in values:
        padded = v.pad(axis, offset, combined)
        offset += v.shape[axis]
        total = padded if total is None else total + padded
    return total


def _swapped(value: Value) -> Value:
    """The trailing-axes swap of src/function/matmul.rs:89-97."""
    rank = len(value.shape)
    if rank <= 2:
        return value.transpose()
    order = list(range(rank))
    order[-2], order[-1] = order[-1], order[-2]
    return value.permute(order)


def _inverse(order) -> list:
    inverse = [0] * len(order)
    for position, axis in enumerate(order):
        inverse[axis] = position
    return inverse


def _backward(node: Node, operands: list, output: Value, g: Value) -> list:
    """Each variant's recorded derivative rule (src/function/*.rs, `backward`),
    written in the rule's own evaluation order."""
    op = node.op
    if op == ADD:
        return [g, g]
    if op == SUB:
        return [g, -g]
    if op == MUL:
        left, right = operands
        return [g * right, g * left]
    if op == DIV:
        _, right = operands
        first = g / right
        return [first, -(g * output / right)]
    if op == NEG:
        return [-g]
    if op == TANH:
        derivative = output.one_like() - output * output
        return [g * derivative]
    if op == EXP:
        return [g * output]
    if op == LN:
        return [g / operands[0]]
    if op == SQRT:
        return [g / (output + output)]
    if op == POWF:
        base, exponent = operands
        lowered = exponent - exponent.one_like()
        base_cotangent = g * exponent * base.powf(lowered)
        exponent_cotangent = g * output * base.ln()
        return [base_cotangent, exponent_cotangent]
    if op == MAXIMUM:
        left, right = operands
        winners = left.step(right)
        left_cotangent = g * winners
        right_cotangent = g * (winners.one_like() - winners)
        return [left_cotangent, right_cotangent]
    if op == RELU:
        operand = operands[0]
        return [g * operand.step(operand.zero_like())]
    if op == STEP:
        return [None, None]
    if op == MATMUL:
        left, right = operands
        first = g.matmul(_swapped(right))
        return [first, _swapped(left).matmul(g)]
    if op == TRANSPOSE:
        return [g.transpose()]
    if op == SUM:
        return [g.broadcast_like(operands[0])]
    if op == SUM_ALONG:
        return [g.broadcast_along(node.params[0], operands[0])]
    if op == BROADCAST:
        return [g.sum().broadcast_like(operands[0]), None]
    if op == BROADCAST_ALONG:
        return [g.sum_along(node.params[0]), None]
    if op == RESHAPE:
        return [g.reshape(operands[0].shape)]
    if op == PERMUTE:
        return [g.permute(_inverse(node.params))]
    if op == NARROW:
        axis, start, _ = node.params
        return [g.pad(axis, start, operands[0].shape[axis])]
    if op == PAD:
        axis, start, _ = node.params
        return [g.narrow(axis, start, operands[0].shape[axis])]
    if op == UNFOLD:
        axis, size, step, dilation = node.params[:4]
        return [g.fold(axis, size, step, dilation, operands[0].shape[axis])]
    if op == FOLD:
        axis, size, step, dilation, _ = node.params[:5]
        return [g.unfold(axis, size, step, dilation)]
    if op == GATHER:
        table, selection = operands
        return [g.scatter(selection, table.shape[0]), None]
    if op == SCATTER:
        return [g.gather(operands[1]), None]
    if op == LOG_SOFTMAX:
        axis = node.params[0]
        total = g.sum_along(axis).broadcast_along(axis, g)
        return [g - output.exp() * total]
    if op == LOG_SUM_EXP:
        axis = node.params[0]
        operand = operands[0]
        probabilities = (operand - output.broadcast_along(axis, operand)).exp()
        return [g.broadcast_along(axis, operand) * probabilities]
    raise NotImplementedError(f"no recorded derivative for {NAMES[op]}")


# ---- neural facades (src/neural) ----

def linear(x: Value, weights: Value, bias: Value) -> Value:
    """Linear::express (src/neural/linear.rs:94-105): x.W + b repeated along axis 0."""
    product = x.matmul(weights)
    return product + bias.broadcast_along(0, product)


def layer_norm(x: Value, scale: Value, shift: Value, epsilon: Value) -> Value:
    """LayerNorm::express (src/neural/layer_norm.rs:100-132); `epsilon` is a
    single-value leaf."""
    mean = x.mean_along(1)
    centered = x - mean.broadcast_along(1, x)
    variance = (centered * centered).mean_along(1)
    deviation = (variance + epsilon.broadcast_like(variance)).sqrt()
    normalized = centered / deviation.broadcast_along(1, x)
    return normalized * scale.broadcast_along(0, x) + shift.broadcast_along(0, x)


def rms_norm(x: Value, scale: Value, epsilon: Value) -> Value:
    """RmsNorm::express (src/neural/rms_norm.rs:89-114): x / sqrt(mean_j(x^2)
    + epsilon) * scale; `epsilon` is a single-value leaf."""
    power = (x * x).mean_along(1)
    root = (power + epsilon.broadcast_like(power)).sqrt()
    return x / root.broadcast_along(1, x) * scale.broadcast_along(0, x)


def cross_entropy(logits: Value, targets: Value) -> Value:
    """cross_entropy (src/neural/loss.rs:44-63)."""
    assert len(logits.shape) == 2 and targets.shape == logits.shape
    normalizers = (targets.sum_along(1) * logits.logsumexp(1)).sum()
    alignment = (targets * logits).sum()
    return (normalizers - alignment) / targets.sum()


def conv2d(x: Value, weights: Value, bias: Value, stride: int, padding: int) -> Value:
    """conv2d (src/neural/convolution.rs:24-118): pad, two single-axis
    unfolds, the im2col reshape of the permuted windows, one rank-2 product
    with the permuted kernel, the bias along the rows, and the NCHW view."""
    batch, channels, height, width = x.shape
    filters, kernel_channels, kernel_height, kernel_width = weights.shape
    assert kernel_channels == channels and bias.shape == (filters,) and stride > 0, "conv2d shapes"
    padded = x
    if padding > 0:
        padded = padded.pad(2, padding, height + 2 * padding)
        padded = padded.pad(3, padding, width + 2 * padding)
    windows = padded.unfold(2, kernel_height, stride, 1).unfold(4, kernel_width, stride, 1)
    out_height, out_width = windows.shape[2], windows.shape[4]
    patches = windows.permute([0, 2, 4, 1, 3, 5]).reshape(
        [batch * out_height * out_width, channels * kernel_height * kernel_width])
    kernel = weights.permute([1, 2, 3, 0]).reshape([channels * kernel_height * kernel_width, filters])
    product = patches.matmul(kernel)
    shifted = product + bias.broadcast_along(0, product)
    return shifted.reshape([batch, out_height, out_width, filters]).permute([0, 3, 1, 2])


def window_lanes(x: Value, size: int, stride: int) -> Value:
    """window_lanes (src/neural/pooling.rs:10-28): [b, c, oh, ow, size*size]."""
    assert len(x.shape) == 4 and size > 0 and stride > 0, "pooling input must be rank 4"
    windows = x.unfold(2, size, stride, 1).unfold(4, size, stride, 1)
    axes = windows.shape
    return windows.permute([0, 1, 2, 4, 3, 5]).reshape([axes[0], axes[1], axes[2], axes[4], size * size])


def max_pool(x: Value, size: int, stride: int) -> Value:
    """max_pool (src/neural/pooling.rs:30-41): a left-biased fold of `maximum`
    over the window lanes, then the lane axis squeezed."""
    lanes = window_lanes(x, size, stride)
    largest = lanes.narrow(4, 0, 1)
    for lane in range(1, size * size):
        largest = largest.maximum(lanes.narrow(4, lane, 1))
    return largest.squeeze(4)


def batch_norm(x: Value, scale: Value, shift: Value, epsilon: Value):
    """BatchNorm::express (src/neural/batch_norm.rs:104-121, normalize at
    :149-176): statistics of the batch itself, the biased variance; returns
    (output, mean, variance). `epsilon` is a single-value leaf."""
    assert len(x.shape) == 2 and scale.shape == (x.shape[1],), "batch-norm input must be rank 2"
    mean = x.mean_along(0)
    centered = x - mean.broadcast_along(0, x)
    variance = (centered * centered).mean_along(0)
    deviation = (variance + epsilon.broadcast_like(variance)).sqrt()
    normalized = centered / deviation.broadcast_along(0, centered)
    output = normalized * scale.broadcast_along(0, centered) + shift.broadcast_along(0, centered)
    return output, mean, variance


# ---- the program table ----

class ProgramTable:
    """The lowered plan: the node table, leaf payloads and the readable set
    (include/topos_hip.h topos_hip_node / topos_hip_leaf)."""

    def __init__(self, tape: Tape, readable: Sequence[int]):
        from . import _native as n

        self.tape = tape
        self.readable = list(dict.fromkeys(readable))
        nodes = tape.nodes
        self.count = len(nodes)
        table = (n.Node * self.count)()
        leaves, data, indices = [], [], []
        data_len = 0
        index_len = 0
        for i, x in enumerate(nodes):
            r = table[i]
            r.op = x.op
            r.rank = len(x.shape)
            for d, s in enumerate(x.shape):
                r.shape[d] = s
            r.operands[0] = x.operands[0] if len(x.operands) > 0 else -1
            r.operands[1] = x.operands[1] if len(x.operands) > 1 else -1
            for d, p in enumerate(x.params):
                r.params[d] = p
            r.slot = x.slot
            r.flags = 0
            if x.op == INPUT and x.selection:
                r.flags |= n.NODE_SELECTION
                r.params[0] = int(np.float32(x.one).view(np.uint32))
            if x.op == LEAF:
                payload = x.payload
                leaf = n.Leaf()
                if isinstance(payload, Constant):
                    leaf.kind, leaf.value = n.LEAF_CONSTANT, payload.value
                elif isinstance(payload, Dense):
                    flat = payload.array.ravel()
                    leaf.kind, leaf.offset, leaf.count = n.LEAF_DENSE, data_len, flat.size
                    data.append(flat)
                    data_len += flat.size
                elif isinstance(payload, Selection):
                    idx = np.ascontiguousarray(payload.indices, dtype=np.int32)
                    leaf.kind, leaf.value, leaf.offset, leaf.count = n.LEAF_SELECTION, payload.one, index_len, idx.size
                    indices.append(idx)
                    index_len += idx.size
                else:
                    raise TypeError(f"unknown leaf payload {payload!r}")
                r.slot = len(leaves)
                leaves.append(leaf)
        for i in self.readable:
            table[i].flags |= n.NODE_READABLE
        self.nodes = table
        self.leaves = (n.Leaf * max(1, len(leaves)))(*leaves)
        self.n_leaves = len(leaves)
        self.leaf_data = np.concatenate(data).astype(np.float32) if data else np.zeros(1, np.float32)
        self.leaf_data_len = data_len
        self.leaf_indices = np.concatenate(indices).astype(np.int32) if indices else np.zeros(1, np.int32)
        self.leaf_indices_len = index_len

    def create_backward(self, numerics: int, target: int, wrt: Sequence[int]):
        """topos_hip_program_create_backward: this forward table plus the
        library's own reverse scan from `target`; returns the native handle."""
        from . import _native as n

        handle = ctypes.c_void_p()
        wanted = (ctypes.c_int64 * max(1, len(wrt)))(*wrt)
        code = n.lib.topos_hip_program_create_backward(
            self.nodes, self.count, self.leaves, self.n_leaves,
            self.leaf_data.ctypes.data_as(n.FLOAT_P), self.leaf_data_len,
            self.leaf_indices.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), self.leaf_indices_len,
            numerics, int(target), wanted, len(wrt), ctypes.byref(handle))
        if code != n.OK:
            raise n.HipError(code, "program create backward: " + n.lib.topos_hip_last_refusal().decode())
        return handle

    def create(self, numerics: int):
        """topos_hip_program_create; returns the native handle."""
        from . import _native as n

        handle = ctypes.c_void_p()
        code = n.lib.topos_hip_program_create(
            self.nodes, self.count, self.leaves, self.n_leaves,
            self.leaf_data.ctypes.data_as(n.FLOAT_P), self.leaf_data_len,
            self.leaf_indices.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), self.leaf_indices_len,
            numerics, ctypes.byref(handle))
        if code != n.OK:
            raise n.HipError(code, "program create: " + n.lib.topos_hip_last_refusal().decode())
        return handle
