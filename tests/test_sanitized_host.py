"""The library's host code (planner, code generation, backward scan, task
face, status and poison paths) under AddressSanitizer and
UndefinedBehaviorSanitizer: a sanitized build of libtopos_hip.so
(poorgrad_amd/build.py build_sanitized, host code only) planning the
benchmark programs (window programs included), planning from four threads at
once, and the refusal paths under the fake runtime, in a fresh interpreter
with the sanitizer runtime preloaded. Any report fails the test."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent

SCENARIO = r'''
import ctypes
import numpy as np
from poorgrad_amd import _native as n
assert n.lib.topos_hip_fake_runtime(1 << 30) == n.OK
from poorgrad_amd import topos as t, workloads
from poorgrad_amd.program import DeviceProgram

for numerics in (n.EXACT, n.FAST):
    for make in (lambda g: workloads.mlp(record_gradients=g),
                 lambda g: workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=4, layers=2, positions=24,
                                          record_gradients=g),
                 lambda g: workloads.llama(batch=2, context=16, vocab=37, width=32, heads=4, hidden=48, layers=1,
                                           record_gradients=g)):
        w = make(True)
        a = DeviceProgram(w.tape, w.roots, numerics=numerics)
        f = make(False)
        b = DeviceProgram.engine_backward(f.tape, f.loss, f.parameters, numerics=numerics)
        assert a.describe == b.describe
        print("planned", a.info["launches"])

tape = t.Tape()
x = tape.input((16, 24))
y = tape.input((16, 24))
z = x.powf(y)
print("powf", DeviceProgram(tape, [(z + x).exp(), z.log_softmax(1)]).info["launches"])

# Window programs: the convolutional and BatchNorm steps, both routes.
for numerics in (n.EXACT, n.FAST):
    for make in (lambda g: workloads.cnn(batch=2, side=8, filters=(2, 3), record_gradients=g),
                 lambda g: workloads.batch_norm_mlp(batch=4, record_gradients=g)):
        w = make(True)
        a = DeviceProgram(w.tape, w.roots, numerics=numerics)
        f = make(False)
        b = DeviceProgram.engine_backward(f.tape, f.loss, f.parameters, numerics=numerics)
        assert a.describe == b.describe
        print("planned", a.info["launches"])

# Planning from four threads at once (the generated-kernel cache and the
# compile queue are shared): every plan equals the serial one.
import threading
def make_program(i):
    w = workloads.gpt2(batch=2, context=8, vocab=19 + i, width=16, heads=2, layers=1, positions=8)
    return DeviceProgram(w.tape, w.roots, numerics=n.FAST if i % 2 else n.EXACT).describe
expected = [make_program(i) for i in range(4)]
results = [None] * 4
def worker(i):
    results[i] = make_program(i)
threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
for th in threads: th.start()
for th in threads: th.join()
assert results == expected
print("threads", len(results))

# Refusals: a window pair that disagrees with its extent, malformed tables, a
# non-scalar backward target.
tape = t.Tape()
x = tape.input((6,))
tape._record(t.UNFOLD, [x.id], (3, 3), params=(0, 3, 3, 1))
try:
    tape.program([t.Value(tape, 1)]).create(n.EXACT)
    raise AssertionError("a wrong unfold shape was accepted")
except n.HipError as e:
    assert e.code == n.INVALID_ARGUMENT
tape = t.Tape()
x = tape.input((4, 3))
tape.nodes.append(t.Node(t.ADD, (0, 7), (4, 3)))
try:
    tape.program([t.Value(tape, 1)]).create(n.EXACT)
except n.HipError as e:
    assert e.code == n.INVALID_ARGUMENT
tape = t.Tape()
p = tape.parameter((4, 3))
try:
    DeviceProgram.engine_backward(tape, (p * p).sum_along(1), [p])
except n.HipError as e:
    assert e.code == n.INVALID_ARGUMENT

# The task face: declines, span overflow, then the injected runtime failure
# that poisons the library.
buf = (ctypes.c_float * 16)()
out = (ctypes.c_float * 4)()
assert n.lib.topos_hip_gemm_f32(buf, 16, 1 << 63, 1 << 63, buf, 16, 2, 1, 2, 2, 2, n.EXACT, out) == n.INVALID_ARGUMENT
big = np.ones(512 * 512, np.float32)
res = np.empty(512 * 512, np.float32)
fp = ctypes.POINTER(ctypes.c_float)
codes = [n.lib.topos_hip_gemm_f32(big.ctypes.data_as(fp), big.size, 512, 1, big.ctypes.data_as(fp), big.size, 512, 1,
                                  512, 512, 512, n.FAST, res.ctypes.data_as(fp)) for _ in range(3)]
print("task", codes)
print("done")
'''


def test_host_code_is_clean_under_asan_and_ubsan():
    import importlib.util

    spec = importlib.util.spec_from_file_location("_topos_builder", ROOT / "poorgrad_amd" / "build.py")
    builder = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(builder)
    library = builder.SANITIZED / "libtopos_hip.so"
    sources = [builder.CSRC / s for s in builder.SOURCES] + [builder.CSRC / "backend.hpp", builder.CSRC / "codegen.hpp"]
    if not library.exists() or library.stat().st_mtime < max(s.stat().st_mtime for s in sources):
        library = builder.build_sanitized()
    env = dict(os.environ, LD_PRELOAD=str(builder.sanitizer_runtime()), TOPOS_HIP_LIBRARY=str(library),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", PYTHONMALLOC="malloc",
               PYTHONPATH=str(ROOT))
    result = subprocess.run([sys.executable, "-c", SCENARIO], capture_output=True, text=True, cwd=ROOT, env=env,
                            timeout=900)
    report = result.stderr[-6000:]
    assert "AddressSanitizer" not in result.stderr and "runtime error:" not in result.stderr, report
    assert result.returncode == 0, report
    assert result.stdout.strip().endswith("done"), result.stdout + report
    # The injected runtime failure happened (the fake runtime counts calls) or
    # every call was served; either way the codes are statuses, not crashes.
    assert "task" in result.stdout
