"""Writes the full-shape parity fixtures: the oracle interpreter (oracle/,
the restated topos interpreter) on the widest slices of BASELINE configs[3]
and configs[4] that one CPU process evaluates in minutes:

* gpt2_full_width.json: GPT-2 at batch 1, context 1024, width 768, 12 heads,
  vocabulary 50257, 2 layers (the config's every row, column and product shape
  per sequence, at 2 of its 12 layers);
* llama_full_width.json: the Llama-style decoder at batch 1, context 2048,
  width 2048, 16 heads, SwiGLU 5632, vocabulary 32000, 1 layer;
* gpt2_batch8.json: GPT-2 at the headline batch, 8 x 1024 tokens (products
  with M = 8192, the 96-way batched attention, the tied-embedding gradient
  (768, 50257, 8192) with its split along k), full width and vocabulary, 2
  layers;
* llama_batch2.json: the Llama-style decoder at its config batch, 2 x 2048
  tokens (M = 4096, 32-way attention), full width, 1 layer.

The oracle's products spread their rows over the host's cores (at most 8);
each row is still one sequential loop, so the bits are the single-threaded
oracle's.

Weights use the uniform draw of the same deviation (integer and correctly
rounded f64 arithmetic only), so the GPU box re-derives the same parameters
bit for bit. Each fixture holds the loss bits and, per gradient, the SHA-256
of its f32 bits, its largest magnitude and 64 sampled elements (seeded flat
indices, their bits), plus SHA-256 digests of the inputs so a test can tell an
input mismatch from a result mismatch.

Run in the build container (no GPU): python tests/golden/make_full_shape_fixtures.py [gpt2|llama]
"""
from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HERE = Path(__file__).resolve().parent
SAMPLES = 64


def configs():
    from poorgrad_amd import workloads

    return {
        "gpt2": (HERE / "gpt2_full_width.json",
                 lambda: workloads.gpt2(batch=1, context=1024, vocab=50257, width=768, heads=12, layers=2,
                                        positions=1024, init="uniform")),
        "llama": (HERE / "llama_full_width.json",
                  lambda: workloads.llama(batch=1, context=2048, vocab=32000, width=2048, heads=16, hidden=5632,
                                          layers=1, init="uniform")),
        "gpt2_batch8": (HERE / "gpt2_batch8.json",
                        lambda: workloads.gpt2(batch=8, context=1024, vocab=50257, width=768, heads=12, layers=2,
                                               positions=1024, init="uniform")),
        "llama_batch2": (HERE / "llama_batch2.json",
                         lambda: workloads.llama(batch=2, context=2048, vocab=32000, width=2048, heads=16,
                                                 hidden=5632, layers=1, init="uniform")),
    }


def digest(array) -> str:
    return hashlib.sha256(np.ascontiguousarray(array, dtype=np.float32).tobytes()).hexdigest()


def input_digests(w) -> dict:
    """Digests of everything the run reads: parameters, dense leaves (masks,
    rotary tables), selection indices."""
    from poorgrad_amd import topos as t

    h = hashlib.sha256()
    for a in w.initial:
        h.update(np.ascontiguousarray(a, dtype=np.float32).tobytes())
    leaves = hashlib.sha256()
    for node in w.tape.nodes:
        if node.op == t.LEAF and isinstance(node.payload, t.Dense):
            leaves.update(np.ascontiguousarray(node.payload.array, dtype=np.float32).tobytes())
    selections = hashlib.sha256()
    for slot in sorted(w.selection_inputs):
        selections.update(np.ascontiguousarray(w.selection_inputs[slot][0], dtype=np.int64).tobytes())
    return {"parameters": h.hexdigest(), "dense_leaves": leaves.hexdigest(), "selections": selections.hexdigest()}


def sample_indices(size: int, gradient: int) -> np.ndarray:
    return np.unique(np.random.default_rng(1000 + gradient).integers(0, size, SAMPLES))


def summarize(w, values: dict) -> dict:
    loss = np.asarray(values[w.loss.id], dtype=np.float32).reshape(())
    gradients = []
    for i, g in enumerate(w.gradients):
        v = np.ascontiguousarray(values[g.id], dtype=np.float32)
        flat = v.ravel()
        picks = sample_indices(flat.size, i)
        gradients.append({"shape": list(v.shape), "sha256": digest(v), "max_abs": float(np.abs(flat).max()),
                          "sample_indices": picks.tolist(),
                          "sample_bits": flat[picks].view(np.uint32).tolist()})
    return {"loss_bits": int(loss.view(np.uint32)), "loss": float(loss), "gradients": gradients}


def make(name: str) -> None:
    import os

    import oracle
    from tests.program_util import run_oracle

    oracle.THREADS = max(1, min(8, os.cpu_count() or 1))

    path, build = configs()[name]
    start = time.time()
    w = build()
    print(f"[{name}] recorded {len(w.tape.nodes)} nodes, {w.parameter_count()} parameters "
          f"in {time.time() - start:.0f} s", flush=True)
    start = time.time()
    values = run_oracle(w.tape, w.roots, w.initial, {}, w.selection_inputs)
    print(f"[{name}] oracle ran in {time.time() - start:.0f} s", flush=True)
    record = {"config": w.config, "init": "uniform", "inputs": input_digests(w), **summarize(w, values)}
    path.write_text(json.dumps(record, indent=1) + "\n")
    print(f"[{name}] wrote {path} (loss {record['loss']})", flush=True)


if __name__ == "__main__":
    for name in sys.argv[1:] or list(configs()):
        make(name)
