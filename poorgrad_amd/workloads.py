"""The benchmark configurations recorded as train steps on the topos surface
(poorgrad_amd.topos), plus their synthetic data.

* ``mlp``: the MNIST-shaped step of BASELINE configs[0] — 784 -> 128 -> 10,
  ReLU, softmax cross-entropy, Kaiming-uniform weights, zero biases.
* ``gpt2``: the GPT-2-small step of configs[3] — pre-LayerNorm blocks, causal
  softmax attention batched as rank-3 products over (batch x heads), GELU MLP
  of 4x width, tied embeddings, cross-entropy over the vocabulary — with any
  dimensions (the parity tests record the same graph at a small size).
* ``llama``: the Llama-style decoder of configs[4] — RMSNorm, rotary position
  embeddings rotated by narrow/neg/concat, causal attention batched over
  (batch x heads), SwiGLU MLP, bias-free projections, an untied head
  (examples/llama/model.rs:80-330) — forward and backward, no optimizer.
* ``cnn``: the convolutional examples (examples/mnist/main.rs:59-99,
  examples/cifar10/main.rs) — conv2d -> ReLU -> max_pool stages over the
  window views, flatten, an affine head, cross-entropy.
* ``batch_norm_mlp``: examples/makemore/mlp_batchnorm.rs — embedding gather,
  a bias-free hidden product, BatchNorm by the batch's own statistics, tanh,
  an affine head, cross-entropy.

All use the recorded-gradients route (src/graph/tape.rs:335-411;
examples/makemore/mlp_compiled.rs:142-204): one forward program reads the
loss and every parameter's gradient. The recipes follow the reference's
facades and examples (src/neural/{linear,layer_norm,loss}.rs,
examples/gpt2/model.rs:60-199); targets and token ids are Tensor::selection
payloads.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .topos import (Constant, Dense, Selection, Tape, Value, batch_norm, concat, conv2d, cross_entropy, layer_norm,
                    linear, max_pool, rms_norm)

# ---- synthetic data: src/neural/init.rs:45-102, vectorized ----

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def _splitmix(seed: int, count: int, skip: int = 0) -> np.ndarray:
    """Outputs skip+1 .. skip+count of splitmix64 from `seed` (init.rs:50-56)."""
    with np.errstate(over="ignore"):
        steps = np.arange(skip + 1, skip + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + steps * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def unit(seed: int, count: int, skip: int = 0) -> np.ndarray:
    """unit() draws in [0, 1) (init.rs:58-60), as f64."""
    return (_splitmix(seed, count, skip) >> np.uint64(11)).astype(np.float64) / float(1 << 53)


def uniform(seed: int, scale: float, shape) -> np.ndarray:
    """init::uniform (init.rs:88-91): (unit * 2 - 1) * scale, rounded to f32."""
    count = int(np.prod(shape))
    return ((unit(seed, count) * 2.0 - 1.0) * scale).astype(np.float32).reshape(shape)


def normal(seed: int, deviation: float, shape) -> np.ndarray:
    """init::normal (init.rs:93-102): Box-Muller on consecutive draw pairs.
    (numpy's f64 log/cos may differ from the C library's in the last bit, so
    this is the reference's generator up to that rounding: synthetic data.)"""
    count = int(np.prod(shape))
    u = unit(seed, 2 * count)
    radius = np.sqrt(-2.0 * np.log(1.0 - u[0::2]))
    angle = 2.0 * math.pi * u[1::2]
    return (radius * np.cos(angle) * deviation).astype(np.float32).reshape(shape)


def labels(seed: int, count: int, classes: int) -> np.ndarray:
    """Uniform class indices: splitmix64 outputs modulo the class count."""
    return (_splitmix(seed, count) % np.uint64(classes)).astype(np.int32)


@dataclass
class Workload:
    """A recorded train step: parameters (slot order), their initial values,
    feeds, and the loss and gradients the program reads."""
    tape: Tape
    parameters: list
    initial: list
    loss: Value
    gradients: list
    dense_inputs: dict = field(default_factory=dict)      # slot -> array
    selection_inputs: dict = field(default_factory=dict)  # slot -> (indices, one)
    config: dict = field(default_factory=dict)

    @property
    def roots(self) -> list:
        return [self.loss] + list(self.gradients)

    def parameter_count(self) -> int:
        return int(sum(a.size for a in self.initial))


def mlp(batch: int = 64, sizes=(784, 128, 10), weight_seeds=(7, 8), input_seed: int = 11,
        label_seed: int = 13, record_gradients: bool = True) -> Workload:
    """Linear -> ReLU -> Linear, cross_entropy over
    one-hot targets; inputs U[0,1), Kaiming-uniform weights
    U(-sqrt(6/fan_in), +sqrt(6/fan_in)), zero biases."""
    tape = Tape()
    params, initial = [], []
    for (fan_in, fan_out), seed in zip(zip(sizes[:-1], sizes[1:]), weight_seeds):
        w = tape.parameter((fan_in, fan_out))
        b = tape.parameter((fan_out,))
        params += [w, b]
        initial += [uniform(seed, math.sqrt(6.0 / fan_in), (fan_in, fan_out)), np.zeros(fan_out, np.float32)]
    x = tape.input((batch, sizes[0]))
    targets = tape.selection_input(batch, sizes[-1])
    h = x
    for layer in range(len(sizes) - 1):
        h = linear(h, params[2 * layer], params[2 * layer + 1])
        if layer < len(sizes) - 2:
            h = h.relu()
    loss = cross_entropy(h, targets)
    # Without recorded gradients the tape is the forward graph alone: the
    # engine-backward route appends the reverse scan on the device.
    gradients = tape.differentiate(loss, params) if record_gradients else []
    feeds = unit(input_seed, batch * sizes[0]).astype(np.float32).reshape(batch, sizes[0])
    return Workload(tape, params, initial, loss, gradients, dense_inputs={x.node.slot: feeds},
                    selection_inputs={targets.node.slot: (labels(label_seed, batch, sizes[-1]), 1.0)},
                    config={"model": "mlp", "sizes": list(sizes), "batch": batch})


def cnn(batch: int = 64, channels: int = 1, side: int = 28, filters=(8, 16), classes: int = 10,
        weight_seed: int = 11, input_seed: int = 17, label_seed: int = 19,
        record_gradients: bool = True) -> Workload:
    """The MNIST example's model (examples/mnist/main.rs:59-99; with
    channels=3, side=32, filters=(16, 32, 64) the CIFAR-10 one): per stage
    conv2d (3x3, stride 1, padding 1, Kaiming-normal kernels
    sqrt(2 / (c * 9)), zero biases), ReLU, 2x2 max_pool; then the flattened
    features through an affine head (Kaiming-normal), cross-entropy over
    one-hot targets. Images are U[0, 1) draws (synthetic data)."""
    tape = Tape()
    params, initial = [], []
    stages = []
    c = channels
    for s, f in enumerate(filters):
        w = tape.parameter((f, c, 3, 3))
        b = tape.parameter((f,))
        params += [w, b]
        initial += [normal(weight_seed + s, math.sqrt(2.0 / (c * 9)), (f, c, 3, 3)), np.zeros(f, np.float32)]
        stages.append((w, b))
        c = f
    reduced = side >> len(filters)
    flat = c * reduced * reduced
    head_w = tape.parameter((flat, classes))
    head_b = tape.parameter((classes,))
    params += [head_w, head_b]
    initial += [normal(weight_seed + len(filters), math.sqrt(2.0 / flat), (flat, classes)),
                normal(weight_seed + len(filters) + 1, math.sqrt(2.0 / classes), (classes,))]
    images = tape.input((batch, channels, side, side))
    targets = tape.selection_input(batch, classes)
    h = images
    for w, b in stages:
        h = max_pool(conv2d(h, w, b, 1, 1).relu(), 2, 2)
    logits = linear(h.reshape([batch, flat]), head_w, head_b)
    loss = cross_entropy(logits, targets)
    gradients = tape.differentiate(loss, params) if record_gradients else []
    pixels = unit(input_seed, batch * channels * side * side).astype(np.float32).reshape(batch, channels, side, side)
    return Workload(tape, params, initial, loss, gradients, dense_inputs={images.node.slot: pixels},
                    selection_inputs={targets.node.slot: (labels(label_seed, batch, classes), 1.0)},
                    config={"model": "cnn", "batch": batch, "channels": channels, "side": side,
                            "filters": list(filters)})


def batch_norm_mlp(batch: int = 64, vocab: int = 27, context: int = 3, embed: int = 10, hidden: int = 100,
                   weight_seed: int = 7, token_seed: int = 13, record_gradients: bool = True) -> Workload:
    """examples/makemore/mlp_batchnorm.rs:55-126: embeddings gathered by the
    context's token ids and flattened, a bias-free hidden product, BatchNorm
    (scale one, shift zero, epsilon 1e-5; normalized by the batch's own
    statistics), tanh, an affine output, cross-entropy over the next token.
    Embeddings N(0, 1), Xavier-uniform weights; token ids are uniform draws
    (synthetic data)."""
    tape = Tape()
    table = tape.parameter((vocab, embed))
    hidden_w = tape.parameter((context * embed, hidden))
    scale = tape.parameter((hidden,))
    shift = tape.parameter((hidden,))
    out_w = tape.parameter((hidden, vocab))
    out_b = tape.parameter((vocab,))
    epsilon = tape.leaf(Constant((), 1e-5))
    params = [table, hidden_w, scale, shift, out_w, out_b]
    xavier = lambda seed, fan_in, fan_out, shape: uniform(seed, math.sqrt(6.0 / (fan_in + fan_out)), shape)
    initial = [normal(weight_seed + 1, 1.0, (vocab, embed)),
               xavier(weight_seed, context * embed, hidden, (context * embed, hidden)),
               np.ones(hidden, np.float32), np.zeros(hidden, np.float32),
               xavier(weight_seed + 2, hidden, vocab, (hidden, vocab)),
               xavier(weight_seed + 3, hidden, vocab, (vocab,))]
    contexts = tape.selection_input(batch * context, vocab)
    targets = tape.selection_input(batch, vocab)
    preactivation = table.gather(contexts).reshape([batch, context * embed]).matmul(hidden_w)
    normalized, _, _ = batch_norm(preactivation, scale, shift, epsilon)
    product = normalized.tanh().matmul(out_w)
    loss = cross_entropy(product + out_b.broadcast_along(0, product), targets)
    gradients = tape.differentiate(loss, params) if record_gradients else []
    return Workload(tape, params, initial, loss, gradients,
                    selection_inputs={contexts.node.slot: (labels(token_seed, batch * context, vocab), 1.0),
                                      targets.node.slot: (labels(token_seed + 1, batch, vocab), 1.0)},
                    config={"model": "batch_norm_mlp", "batch": batch, "vocab": vocab, "context": context,
                            "embed": embed, "hidden": hidden})


def _gelu(x: Value, half: Value, one: Value, root: Value, coefficient: Value) -> Value:
    """examples/gpt2/model.rs:85-98: 0.5 x (1 + tanh(0.7978846 (x + 0.044715 x^3)))."""
    cubic = x * x * x * coefficient.broadcast_like(x)
    inner = ((x + cubic) * root.broadcast_like(x)).tanh()
    return x * (inner + one.broadcast_like(inner)) * half.broadcast_like(x)


def _weights(init: str):
    """The weight draw: init::normal(seed, 0.02) (the configs' N(0, 0.02)), or
    init::uniform(seed, 0.02 * sqrt(3)) of the same deviation, whose draws use
    integer and correctly rounded f64 arithmetic only, so every machine draws
    the same bits (the full-shape parity fixtures use it)."""
    if init == "normal":
        return lambda seed, shape: normal(seed, 0.02, shape)
    if init == "uniform":
        return lambda seed, shape: uniform(seed, 0.02 * math.sqrt(3.0), shape)
    raise ValueError(f"unknown weight init {init!r}")


def gpt2(batch: int = 8, context: int = 1024, vocab: int = 50257, width: int = 768, heads: int = 12,
         layers: int = 12, positions: int = 1024, weight_seed: int = 7, token_seed: int = 13,
         init: str = "normal", record_gradients: bool = True) -> Workload:
    """BASELINE configs[3] (or the same graph at other dimensions): GPT-2 with
    pre-LayerNorm blocks, causal attention, GELU MLP, tied embeddings."""
    assert width % heads == 0 and context <= positions
    head = width // heads
    rows = batch * context
    tape = Tape()
    params, initial = [], []
    seed = [weight_seed]

    draw = _weights(init)

    def weight(shape):
        p = tape.parameter(shape)
        params.append(p)
        initial.append(draw(seed[0], shape))
        seed[0] += 1
        return p

    def filled(shape, value):
        p = tape.parameter(shape)
        params.append(p)
        initial.append(np.full(shape, value, np.float32))
        return p

    wte = weight((vocab, width))
    wpe = weight((positions, width))
    blocks = []
    for _ in range(layers):
        blocks.append({
            "ln1": (filled((width,), 1.0), filled((width,), 0.0)),
            "attn": (weight((width, 3 * width)), filled((3 * width,), 0.0)),
            "proj": (weight((width, width)), filled((width,), 0.0)),
            "ln2": (filled((width,), 1.0), filled((width,), 0.0)),
            "fc": (weight((width, 4 * width)), filled((4 * width,), 0.0)),
            "out": (weight((4 * width, width)), filled((width,), 0.0)),
        })
    ln_f = (filled((width,), 1.0), filled((width,), 0.0))

    # Leaves shared by every block (examples/gpt2/model.rs:363-388).
    causal = np.where(np.arange(context)[None, :] <= np.arange(context)[:, None], 0.0, -np.inf).astype(np.float32)
    mask = tape.leaf(Dense(causal))
    scale = tape.leaf(Constant((), float(np.float32(1.0 / math.sqrt(head)))))
    epsilon = tape.leaf(Constant((), float(np.float32(1e-5))))
    half, one = tape.leaf(Constant((), 0.5)), tape.leaf(Constant((), 1.0))
    root = tape.leaf(Constant((), float(np.float32(0.7978846))))
    coefficient = tape.leaf(Constant((), float(np.float32(0.044715))))

    tokens = tape.selection_input(rows, vocab)
    targets = tape.selection_input(rows, vocab)
    where = tape.leaf(Selection(np.tile(np.arange(context, dtype=np.int32), batch), positions))

    def split_heads(fused: Value, part: int) -> Value:
        x = fused.narrow(1, part * width, width).reshape((batch, context, heads, head))
        return x.permute((0, 2, 1, 3)).reshape((batch * heads, context, head))

    x = wte.gather(tokens) + wpe.gather(where)
    for b in blocks:
        h = layer_norm(x, *b["ln1"], epsilon)
        fused = linear(h, *b["attn"])
        q, k, v = split_heads(fused, 0), split_heads(fused, 1), split_heads(fused, 2)
        scores = q.matmul(k.permute((0, 2, 1)))
        weights = (scores * scale.broadcast_like(scores) + mask.broadcast_along(0, scores)).softmax(2)
        attended = weights.matmul(v).reshape((batch, heads, context, head)).permute((0, 2, 1, 3))
        x = x + linear(attended.reshape((rows, width)), *b["proj"])
        h = layer_norm(x, *b["ln2"], epsilon)
        x = x + linear(_gelu(linear(h, *b["fc"]), half, one, root, coefficient), *b["out"])
    logits = layer_norm(x, *ln_f, epsilon).matmul(wte.transpose())
    loss = cross_entropy(logits, targets)
    # Without recorded gradients the tape is the forward graph alone: the
    # engine-backward route appends the reverse scan on the device.
    gradients = tape.differentiate(loss, params) if record_gradients else []

    stream = labels(token_seed, rows + batch, vocab).reshape(batch, context + 1)
    token_ids = stream[:, :-1].reshape(-1)
    next_ids = stream[:, 1:].reshape(-1)  # next-token targets
    return Workload(tape, params, initial, loss, gradients,
                    selection_inputs={tokens.node.slot: (token_ids, 1.0), targets.node.slot: (next_ids, 1.0)},
                    config={"model": "gpt2", "batch": batch, "context": context, "vocab": vocab, "width": width,
                            "heads": heads, "layers": layers})


def rope_tables(context: int, head: int, base: float = 10000.0):
    """examples/llama/model.rs:88-117: column j and j + head/2 share the
    frequency base^(-2 (j mod head/2) / head); angles in f64, tables rounded to
    f32."""
    half = head // 2
    position = np.arange(context, dtype=np.float64)[:, None]
    column = np.arange(head)[None, :] % half
    angle = position * np.power(base, -2.0 * column / head)
    return np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)


def llama(batch: int = 2, context: int = 2048, vocab: int = 32000, width: int = 2048, heads: int = 16,
          hidden: int = 5632, layers: int = 8, epsilon: float = 1e-6, weight_seed: int = 7,
          token_seed: int = 13, host_weights: bool = True, init: str = "normal",
          record_gradients: bool = True) -> Workload:
    """BASELINE configs[4] (or the same graph at other dimensions): a Llama-style
    decoder, forward and backward (the loss and every parameter's gradient).
    Blocks follow examples/llama/model.rs: pre-norm RMSNorm (:280-300), q/k/v/o
    projections without bias, rotary embeddings on q and k (:119-131), causal
    softmax attention with scale 1/sqrt(head) (:177-198), SwiGLU
    x / (exp(-x) + 1) * up (:252-258); final RMSNorm and an untied head.
    host_weights=False leaves `initial` as the parameter shapes (a caller that
    draws the weights on the device; 542M host draws take minutes)."""
    assert width % heads == 0 and (width // heads) % 2 == 0
    head = width // heads
    half = head // 2
    rows = batch * context
    tape = Tape()
    params, initial = [], []
    seed = [weight_seed]

    draw = _weights(init)

    def weight(shape):
        p = tape.parameter(shape)
        params.append(p)
        initial.append(draw(seed[0], shape) if host_weights else shape)
        seed[0] += 1
        return p

    def ones(shape):
        p = tape.parameter(shape)
        params.append(p)
        initial.append(np.ones(shape, np.float32) if host_weights else shape)
        return p

    embed = weight((vocab, width))
    blocks = []
    for _ in range(layers):
        blocks.append({
            "norm1": ones((width,)),
            "q": weight((width, width)), "k": weight((width, width)), "v": weight((width, width)),
            "o": weight((width, width)),
            "norm2": ones((width,)),
            "gate": weight((width, hidden)), "up": weight((width, hidden)), "down": weight((hidden, width)),
        })
    final_norm = ones((width,))
    lm_head = weight((width, vocab))

    # Leaves shared by every block.
    cos, sin = rope_tables(context, head)
    cos_leaf, sin_leaf = tape.leaf(Dense(cos)), tape.leaf(Dense(sin))
    causal = np.where(np.arange(context)[None, :] <= np.arange(context)[:, None], 0.0, -np.inf).astype(np.float32)
    mask = tape.leaf(Dense(causal))
    scale = tape.leaf(Constant((), float(np.float32(1.0 / math.sqrt(head)))))
    eps = tape.leaf(Constant((), float(np.float32(epsilon))))
    one = tape.leaf(Constant((), 1.0))

    tokens = tape.selection_input(rows, vocab)
    targets = tape.selection_input(rows, vocab)

    def split_heads(x: Value) -> Value:
        return x.reshape((batch, context, heads, head)).permute((0, 2, 1, 3)).reshape((batch * heads, context, head))

    def rotate(x: Value) -> Value:
        # value * cos + rotate_half(value) * sin over [batch x heads, context, head]
        flipped = concat([-x.narrow(2, half, half), x.narrow(2, 0, half)], 2)
        return x * cos_leaf.broadcast_along(0, x) + flipped * sin_leaf.broadcast_along(0, x)

    x = embed.gather(tokens)
    for b in blocks:
        h = rms_norm(x, b["norm1"], eps)
        q = rotate(split_heads(h.matmul(b["q"])))
        k = rotate(split_heads(h.matmul(b["k"])))
        v = split_heads(h.matmul(b["v"]))
        scores = q.matmul(k.permute((0, 2, 1)))
        weights = (scores * scale.broadcast_like(scores) + mask.broadcast_along(0, scores)).softmax(2)
        attended = weights.matmul(v).reshape((batch, heads, context, head)).permute((0, 2, 1, 3))
        x = x + attended.reshape((rows, width)).matmul(b["o"])
        h = rms_norm(x, b["norm2"], eps)
        gated = h.matmul(b["gate"])
        activated = gated / ((-gated).exp() + one.broadcast_like(gated))
        x = x + (activated * h.matmul(b["up"])).matmul(b["down"])
    logits = rms_norm(x, final_norm, eps).matmul(lm_head)
    loss = cross_entropy(logits, targets)
    # Without recorded gradients the tape is the forward graph alone: the
    # engine-backward route appends the reverse scan on the device.
    gradients = tape.differentiate(loss, params) if record_gradients else []

    stream = labels(token_seed, rows + batch, vocab).reshape(batch, context + 1)
    token_ids = stream[:, :-1].reshape(-1)
    next_ids = stream[:, 1:].reshape(-1)
    return Workload(tape, params, initial, loss, gradients,
                    selection_inputs={tokens.node.slot: (token_ids, 1.0), targets.node.slot: (next_ids, 1.0)},
                    config={"model": "llama", "batch": batch, "context": context, "vocab": vocab, "width": width,
                            "heads": heads, "hidden": hidden, "layers": layers})


def llama_product_flops(w: Workload) -> float:
    """2·m·n·k over the forward products, times three (forward, and the two
    backward products of each)."""
    c = w.config
    rows, width, hidden, vocab = c["batch"] * c["context"], c["width"], c["hidden"], c["vocab"]
    head = width // c["heads"]
    per_layer = 2 * rows * width * width * 4 + 2 * rows * width * hidden * 3
    attention = 2 * 2 * c["batch"] * c["heads"] * c["context"] ** 2 * head
    return 3.0 * (c["layers"] * (per_layer + attention) + 2 * rows * width * vocab)
