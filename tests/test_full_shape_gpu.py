"""Parity at the configs' full widths and batches: the device program of the
GPT-2 train step (configs[3]: context 1024, width 768, 12 heads, vocabulary
50257, at 2 of its 12 layers, at batch 1 and at the headline batch 8) and of
the Llama-style decoder (configs[4]: context 2048, width 2048, 16 heads,
SwiGLU 5632, vocabulary 32000, at 1 of its 8 layers, at batch 1 and at its
batch 2) against fixtures the oracle interpreter wrote
(tests/golden/make_full_shape_fixtures.py). These sizes reach the paths the
small-size tests cannot: 50257-wide streamed row programs, the gathered
ordered sum over 411M terms, split-k vocabulary products, the headline's
M = 8192 products, 96-way batched attention and the tied-embedding gradient
(768, 50257, 8192), and 1024- and 2048-wide attention row programs.

Exact posture: the loss bits and every gradient's SHA-256 over its f32 bits
equal the oracle's (bit-identical, the plan = interpreter contract of
src/engine/tests/plan_tests.rs:9-22). Fast posture: the loss within 1e-4
relative and the sampled gradient elements within 1e-3 of each gradient's
largest magnitude, the rule of the small-size fast tests."""
import hashlib
import json

import numpy as np
import pytest

from tests.conftest import banner
from tests.golden.make_full_shape_fixtures import configs, input_digests

pytestmark = pytest.mark.gpu

CASES = configs()


def _run(w, numerics):
    import torch

    from poorgrad_amd.program import DeviceProgram

    program = DeviceProgram(w.tape, w.roots, numerics=numerics)
    held = []
    for slot, array in enumerate(w.initial):
        t = torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).cuda()
        held.append(t)
        program.bind_parameter(slot, t)
    for slot, (indices, one) in w.selection_inputs.items():
        program.bind_selection(slot, indices, one)
    program.run()
    torch.cuda.synchronize()
    return program


@pytest.mark.parametrize("model", ["gpt2", "llama", "gpt2_batch8", "llama_batch2"])
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_full_width_train_step_matches_oracle_fixture(hip, model, posture):
    path, build = CASES[model]
    fixture = json.loads(path.read_text())
    banner(f"full width {model} {posture}: recording")
    w = build()
    assert input_digests(w) == fixture["inputs"], "this host derives other inputs than the fixture's"
    banner(f"full width {model} {posture}: device program")
    program = _run(w, hip.EXACT if posture == "exact" else hip.FAST)
    loss = np.asarray(program.read(w.loss), dtype=np.float32).reshape(())
    if posture == "exact":
        assert int(loss.view(np.uint32)) == fixture["loss_bits"], (float(loss), fixture["loss"])
    else:
        assert abs(float(loss) - fixture["loss"]) <= 1e-4 * max(abs(fixture["loss"]), 1.0)
    for i, (g, want) in enumerate(zip(w.gradients, fixture["gradients"])):
        value = np.ascontiguousarray(program.read(g), dtype=np.float32)
        assert list(value.shape) == want["shape"]
        flat = value.ravel()
        picks = np.asarray(want["sample_indices"], dtype=np.int64)
        expected = np.asarray(want["sample_bits"], dtype=np.uint32).view(np.float32)
        if posture == "exact":
            got_bits = flat[picks].view(np.uint32)
            assert np.array_equal(got_bits, expected.view(np.uint32)), f"gradient {i} {want['shape']}: samples"
            assert hashlib.sha256(value.tobytes()).hexdigest() == want["sha256"], f"gradient {i} {want['shape']}"
        else:
            scale = max(want["max_abs"], 1e-3)
            error = np.abs(flat[picks].astype(np.float64) - expected.astype(np.float64)).max()
            assert error <= 1e-3 * scale, f"gradient {i} {want['shape']}: {error} against scale {scale}"
