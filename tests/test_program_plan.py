"""Planning device programs without a GPU: the fake runtime
(topos_hip_fake_runtime, the Api::fake pattern of
src/backend/cuda/kernels/context.rs:101-162) plans and compiles every
generated kernel for gfx950 but runs nothing. Each scenario runs in a fresh
interpreter (the runtime choice is process-wide)."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent

PREAMBLE = r'''
import numpy as np
from poorgrad_amd import _native as n
assert n.lib.topos_hip_fake_runtime(1 << 30) == n.OK
from poorgrad_amd import topos as t, workloads
from poorgrad_amd.program import DeviceProgram
'''


def run(code: str) -> str:
    result = subprocess.run([sys.executable, "-c", PREAMBLE + code], capture_output=True, text=True, cwd=ROOT,
                            timeout=600)
    assert result.returncode == 0, result.stderr[-3000:]
    return result.stdout


def test_an_elementwise_tree_is_one_generated_kernel():
    out = run(r'''
tape = t.Tape()
x = tape.input((64, 32))
b = tape.parameter((32,))
y = ((-x).exp() + x.one_like())
z = x / y + b.broadcast_along(0, x)
p = DeviceProgram(tape, [z])
print(p.info["launches"])
print(p.describe)
''')
    lines = out.splitlines()
    assert lines[0] == "1", out
    assert "chain Add [64,32]" in out


def test_a_reduction_absorbs_its_elementwise_operand():
    out = run(r'''
tape = t.Tape()
x = tape.input((16, 48))
s = (x * x + x).sum_along(0)
p = DeviceProgram(tape, [s])
print(p.info["launches"])
print(p.describe)
''')
    assert out.splitlines()[0] == "1", out
    assert "fold sum axis 0 [16,48] 1 inputs, 2 steps" in out


def test_a_row_group_is_one_launch():
    # LayerNorm's forward (mean, centring, variance, deviation, scale and
    # shift; src/neural/layer_norm.rs:100-132) and a softmax over its result:
    # every reduction runs along the last axis, so the whole group is one
    # row program writing only what is read outside it.
    out = run(r'''
tape = t.Tape()
x = tape.input((64, 40))
g = tape.parameter((40,))
b = tape.parameter((40,))
eps = tape.leaf(t.Constant((), 1e-5))
h = t.layer_norm(x, g, b, eps)
w = h.softmax(1)
p = DeviceProgram(tape, [w])
print(p.info["launches"])
print(p.describe)
''')
    assert out.splitlines()[0] == "1", out
    assert "rows [64,40]" in out and "4 folds, 1+0 outputs" in out


def test_views_launch_nothing():
    out = run(r'''
tape = t.Tape()
a = tape.parameter((8, 6))
v = a.transpose().narrow(0, 1, 4).reshape((4, 1, 8)).permute((2, 0, 1))   # a unit-axis reshape: a view
s = v.sum_along(0)
p = DeviceProgram(tape, [s])
print(p.info["launches"])
w = a.transpose().narrow(0, 1, 4).reshape((2, 2, 8)).sum_along(0)         # splitting a strided axis: a view
q = DeviceProgram(tape, [w])
print(q.info["launches"])
u = a.transpose().reshape((48,)).reshape((6, 8)).sum_along(0)              # merging strided axes: copied first
r = DeviceProgram(tape, [u])
print(r.info["launches"])
''')
    assert out.splitlines()[:3] == ["1", "1", "2"], out


def test_mlp_step_plans_with_side_branches_and_an_arena():
    out = run(r'''
w = workloads.mlp()
for numerics in (n.EXACT, n.FAST):
    p = DeviceProgram(w.tape, w.roots, numerics=numerics)
    info = p.info
    print(info["arena_bytes"] > 0, info["launches"], p.describe.count("[side]"))
''')
    for line in out.splitlines():
        ok, launches, side = line.split()
        assert ok == "True" and int(launches) > 10 and int(side) > 0, out


def test_window_views_launch_nothing_and_fold_is_one_kernel():
    """Unfold is a strided view (Layout::unfold, src/payload/layout.rs:299-331):
    a chain reads the overlapping windows directly. Fold
    (src/payload/tensor.rs:1392-1462) is one kernel."""
    out = run(r'''
tape = t.Tape()
x = tape.input((4, 3, 10, 12))
windows = x.unfold(2, 3, 2, 1).unfold(4, 3, 2, 1)
y = (windows * windows).exp()
folded = y.fold(4, 3, 2, 1, 12).fold(2, 3, 2, 1, 10)
p = DeviceProgram(tape, [y, folded])
d = p.describe
print(p.info["launches"], d.count("fold ["), d.count("chain"))
''')
    launches, folds, chains = map(int, out.split())
    assert launches == 3 and folds == 2 and chains == 1, out


def test_wrong_window_shapes_are_invalid_arguments():
    out = run(r'''
tape = t.Tape()
x = tape.input((6,))
tape._record(t.UNFOLD, [x.id], (3, 3), params=(0, 3, 3, 1))   # two windows, not three
table = tape.program([t.Value(tape, 1)])
try:
    table.create(n.EXACT)
except n.HipError as e:
    print(e.code, "unfolded shape" in n.lib.topos_hip_last_refusal().decode())
tape = t.Tape()
x = tape.input((3, 3))
tape._record(t.FOLD, [x.id], (9,), params=(0, 3, 2, 1, 9))    # extent 9 makes four windows
table = tape.program([t.Value(tape, 1)])
try:
    table.create(n.EXACT)
except n.HipError as e:
    print(e.code, "fold window pair" in n.lib.topos_hip_last_refusal().decode())
''')
    assert out.split() == ["5", "True", "5", "True"], out  # TOPOS_HIP_INVALID_ARGUMENT


def test_the_convolutional_and_batch_norm_graphs_plan():
    out = run(r'''
for make in (lambda: workloads.cnn(batch=4), lambda: workloads.batch_norm_mlp(batch=8)):
    w = make()
    for numerics in (n.EXACT, n.FAST):
        p = DeviceProgram(w.tape, w.roots, numerics=numerics)
        print(p.info["launches"], p.describe.count("fold ["))
''')
    rows = [list(map(int, line.split())) for line in out.strip().splitlines()]
    assert len(rows) == 4 and rows[0][1] >= 6 and rows[2][1] == 0, out


def test_malformed_tables_are_invalid_arguments():
    out = run(r'''
tape = t.Tape()
x = tape.input((4, 4))
y = x + x
table = tape.program([y])
table.nodes[1].operands[0] = 5   # a forward reference
try:
    table.create(n.EXACT)
except n.HipError as e:
    print(e.code)
tape = t.Tape()
s = tape.leaf(t.Selection(np.array([0, 9], np.int32), 4))   # index out of vocabulary
table = tape.program([s])
try:
    table.create(n.EXACT)
except n.HipError as e:
    print(e.code)
''')
    assert out.split() == ["5", "5"], out  # TOPOS_HIP_INVALID_ARGUMENT


def test_the_gpt2_graph_plans():
    out = run(r'''
w = workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=4, layers=2, positions=24)
p = DeviceProgram(w.tape, w.roots, numerics=n.FAST)
d = p.describe
print(p.info["launches"], d.count("gemm mfma"), d.count("[side]"), d.count(": rows ["))
''')
    launches, gemms, side, rows = map(int, out.split())
    assert launches > 100 and gemms > 20 and side > 10 and rows >= 10, out


def test_the_llama_graph_plans():
    out = run(r'''
w = workloads.llama(batch=2, context=16, vocab=37, width=32, heads=4, hidden=48, layers=2)
p = DeviceProgram(w.tape, w.roots, numerics=n.FAST)
d = p.describe
print(p.info["launches"], d.count("gemm mfma"), d.count(": rows ["))
''')
    launches, gemms, rows = map(int, out.split())
    assert launches > 60 and gemms >= 2 * 3 * 8 and rows >= 5, out


def test_consecutive_chains_join():
    # a = x*x + y has two consumers, so it is materialised; the chains that
    # follow over the same shape join its launch (one kernel, several
    # outputs), except one that reads it transposed, which must wait for the
    # whole of it.
    out = run(r'''
tape = t.Tape()
x = tape.input((48, 48))
y = tape.input((48, 48))
a = x * x + y
b = a * x
c = (b + a).exp()
d = a.transpose() * y
p = DeviceProgram(tape, [c, b, d])
print(p.info["launches"])
print(p.describe)
''')
    lines = out.splitlines()
    assert lines[0] == "2", out
    assert "chain Add+Mul+Exp [48,48]" in out and ", 3 outputs" in out, out


def test_engine_backward_plans_the_recorded_gradients_program():
    """The engine-backward route (the library's own reverse scan,
    Run::backward of src/engine/run.rs:229-318, over a forward-only table)
    records the same nodes, in the same order, as Tape::differentiate's
    recorded route (src/graph/tape.rs:335-411): the two programs plan to the
    same launches, descriptions and arena."""
    out = run(r'''
cases = [
    lambda g: workloads.mlp(record_gradients=g),
    lambda g: workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=4, layers=2, positions=24,
                             record_gradients=g),
    lambda g: workloads.llama(batch=2, context=16, vocab=37, width=32, heads=4, hidden=48, layers=2,
                              record_gradients=g),
    lambda g: workloads.cnn(batch=4, record_gradients=g),
    lambda g: workloads.batch_norm_mlp(batch=8, record_gradients=g),
]
for make in cases:
    for numerics in (n.EXACT, n.FAST):
        recorded = make(True)
        forward = make(False)
        a = DeviceProgram(recorded.tape, recorded.roots, numerics=numerics)
        b = DeviceProgram.engine_backward(forward.tape, forward.loss, forward.parameters, numerics=numerics)
        assert a.describe == b.describe, (a.describe[:2000], b.describe[:2000])
        assert a.info == b.info, (a.info, b.info)
        print(a.info["launches"])
''')
    assert len(out.split()) == 10, out


def test_engine_backward_refuses_a_non_scalar_target():
    out = run(r'''
tape = t.Tape()
x = tape.parameter((4, 3))
y = (x * x).sum_along(1)
try:
    DeviceProgram.engine_backward(tape, y, [x])
except n.HipError as e:
    print(e.code, "scalar" in str(e))
''')
    assert out.split() == ["5", "True"], out


def test_powf_of_tensors_plans_into_a_chain_and_a_row_program():
    """Powf of recorded tensors is a chain step (and a row-program step), its
    generated code compiled for gfx950 through hipRTC with the restated powf."""
    out = run(r'''
tape = t.Tape()
x = tape.input((16, 24))
y = tape.input((16, 24))
z = x.powf(y)
p = DeviceProgram(tape, [(z + x).exp(), z.log_softmax(1)])
d = p.describe
print("Powf" in d, p.info["launches"])
''')
    ok, launches = out.split()
    assert ok == "True" and int(launches) >= 1, out


def test_composed_formulas_plan_their_dedicated_forms():
    """The reference pattern bench's three composed formulas
    (benches/pattern.rs; src/backend/formula.rs:30-37): conv2d's im2col chain
    becomes one window product with no pad or copy launch (WindowProduct);
    max_pool's lanes are read through window views, one launch
    (ReduceWindow); BatchNorm's statistics, normalisation and affine map are
    one column program (BatchNormTraining). The coverage cells say so."""
    out = run(r'''
import ctypes
for numerics in (n.EXACT, n.FAST):
    tape = t.Tape()
    x = tape.input((64, 16, 14, 14)); w = tape.parameter((32, 16, 3, 3)); b = tape.parameter((32,))
    conv = DeviceProgram(tape, [t.conv2d(x, w, b, 1, 1)], numerics=numerics).describe
    tape = t.Tape()
    pool = DeviceProgram(tape, [t.max_pool(tape.input((64, 32, 28, 28)), 2, 2)], numerics=numerics)
    tape = t.Tape()
    x = tape.input((256, 512)); s = tape.parameter((512,)); h = tape.parameter((512,))
    o, mean, var = t.batch_norm(x, s, h, tape.leaf(t.Constant((), 1e-5)))
    norm = DeviceProgram(tape, [o, mean, var], numerics=numerics)
    print("gemm window patches" in conv, "pad [" not in conv, "copy [64,14,14" not in conv,
          pool.info["launches"], norm.info["launches"], "columns [256,512]" in norm.describe)
fidelity, precisions = ctypes.c_int(), ctypes.c_uint()
for formula in (n.lib.topos_hip_coverage(2, ctypes.byref(fidelity), ctypes.byref(precisions)),
                n.lib.topos_hip_coverage(3, ctypes.byref(fidelity), ctypes.byref(precisions)),
                n.lib.topos_hip_coverage(4, ctypes.byref(fidelity), ctypes.byref(precisions))):
    print(formula, fidelity.value, precisions.value)
''')
    lines = out.splitlines()
    assert lines[0] == lines[1] == "True True True 1 1 True", out
    assert lines[2:] == ["1 0 1"] * 3, out


def test_max_pool_lanes_in_a_training_step_read_the_source():
    """In a training step the pooled lanes also feed maximum's gradient rules:
    every lane is still a view of the window source, so no copy is planned."""
    out = run(r'''
w = workloads.cnn(batch=8)
d = DeviceProgram(w.tape, w.roots).describe
print("copy [8,8,14,14,2,2]" in d, "copy [8,16,7,7,2,2]" in d, d.count("gemm window"))
''')
    assert out.split() == ["False", "False", "4"], out


def test_a_transposed_view_is_copied_in_tiles():
    # The key gradient of attention, (q^T dS)^T read through the head
    # permutation: a copy whose innermost axis steps 4 KB through its input
    # while another axis is contiguous, moved in 64 x 64 tiles through LDS
    # (the tile kernel compiles for gfx950 with the rest).
    out = run(r'''
w = workloads.gpt2(batch=2, context=64, vocab=61, width=128, heads=2, layers=1, positions=64)
p = DeviceProgram(w.tape, w.roots, numerics=n.FAST)
print(p.describe)
''')
    assert "copy (tiles) [2,64,2,64]" in out, out
    assert "copy [2,64,2,64]" not in out, out


def test_trailing_branches_fed_by_the_main_stream_run_on_it():
    """Side branches that cannot start before the main stream's last launch
    ends and read no side output run on the main stream (the GPT-2 step's
    embedding scatters); the tied embedding's final accumulation, which reads
    the head's side-stream weight gradient, stays on the side stream."""
    out = run(r'''
w = workloads.gpt2(batch=2, context=16, vocab=37, width=32, heads=4, layers=2, positions=24)
p = DeviceProgram(w.tape, w.roots, numerics=n.FAST)
for line in p.describe.splitlines()[1:]:
    print(line)
''')
    lines = out.splitlines()
    scatters = [line for line in lines if ": scatter " in line]
    assert len(scatters) == 2 and not any("[side]" in line for line in scatters), out
    assert "[side]" in lines[-1] and "chain Add [37,32]" in lines[-1], out
