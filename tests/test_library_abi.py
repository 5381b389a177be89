"""The C ABI library loads, exports every symbol include/topos_hip.h declares,
and answers its manifest and device-free declines without a GPU."""
import ctypes
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "topos_hip.h").read_text()
    return sorted(set(re.findall(r"\b(topos_hip_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    from poorgrad_amd import _native as n

    symbols = declared_symbols()
    assert len(symbols) >= 15
    for name in symbols:
        assert hasattr(n.lib, name), f"{name} is declared but not exported"
        assert name in n.PROTOTYPES, f"{name} has no ctypes prototype"


def test_manifest_answers_without_a_device():
    from poorgrad_amd import _native as n
    import ctypes

    assert n.lib.topos_hip_abi_version() == 2
    assert n.lib.topos_hip_compiled() == 1
    fidelity, precisions = ctypes.c_int(-1), ctypes.c_uint(0)
    assert n.lib.topos_hip_coverage(n.FORMULA_GEMM, ctypes.byref(fidelity), ctypes.byref(precisions)) == 1
    assert (fidelity.value, precisions.value) == (n.ENVELOPE, n.PRECISION_F32)
    assert n.lib.topos_hip_coverage(n.FORMULA_MAP, ctypes.byref(fidelity), ctypes.byref(precisions)) == 1
    assert (fidelity.value, precisions.value) == (n.BIT_IDENTICAL, n.PRECISION_F32)
    for formula in (n.FORMULA_WINDOW_PRODUCT, n.FORMULA_REDUCE_WINDOW, n.FORMULA_BATCH_NORM_TRAINING):
        assert n.lib.topos_hip_coverage(formula, ctypes.byref(fidelity), ctypes.byref(precisions)) == 1
        assert (fidelity.value, precisions.value) == (n.BIT_IDENTICAL, n.PRECISION_F32)
    assert n.lib.topos_hip_coverage(n.FORMULA_BATCH_NORM_INFERENCE, None, None) == 0


def test_coverage_matches_the_integration_table():
    """The Rust manifest written out for topos (the coverage table of the
    binding's documentation) and the library's own answers agree cell by cell,
    as formula_tests.rs checks the chains against the matrix for every member."""
    from poorgrad_amd import _native as n

    text = (ROOT / "INTEGRATION.md").read_text()
    table = text[text.index("| Formula | Coverage | Fidelity | Precisions |"):]
    rows = []
    for line in table.splitlines()[2:]:
        if not line.startswith("|"):
            break
        rows.append([cell.strip() for cell in line.strip("|").split("|")])
    codes = {"Gemm": n.FORMULA_GEMM, "Map": n.FORMULA_MAP, "WindowProduct": n.FORMULA_WINDOW_PRODUCT,
             "ReduceWindow": n.FORMULA_REDUCE_WINDOW, "BatchNormTraining": n.FORMULA_BATCH_NORM_TRAINING,
             "BatchNormInference": n.FORMULA_BATCH_NORM_INFERENCE}
    assert sorted(r[0] for r in rows) == sorted(codes), "the table names every Formula variant once"
    for formula, coverage, fidelity, precisions in rows:
        f, p = ctypes.c_int(-1), ctypes.c_uint(0)
        served = n.lib.topos_hip_coverage(codes[formula], ctypes.byref(f), ctypes.byref(p))
        assert served == (coverage == "Serves"), formula
        if served:
            assert f.value == {"BitIdentical": n.BIT_IDENTICAL, "Envelope": n.ENVELOPE}[fidelity], formula
            want = sum({"F32": n.PRECISION_F32, "F64": n.PRECISION_F64}[x.strip()] for x in precisions.split(","))
            assert p.value == want, formula
    assert n.lib.topos_hip_dispatch() == n.DISPATCH_OFFERED
    assert "const DISPATCH: Dispatch = Dispatch::Offered;" in text


def test_task_face_declines_need_no_device():
    from poorgrad_amd import tasks

    # GEMV shapes, sub-threshold sizes: declined before any device work.
    assert tasks.gemm_f32(np.ones(8), (8, 1), np.ones(8), (1, 1), 1, 8, 1) is None
    assert tasks.gemm_f32(np.ones(64), (8, 1), np.ones(64), (8, 1), 8, 8, 8) is None
    assert tasks.map_f32(0, np.ones(100, np.float32)) is None
    # A slice that does not span its matrix is a contract violation
    # (src/payload/gemm.rs:57-89 panics; the ABI answers INVALID_ARGUMENT).
    with pytest.raises(ValueError):
        tasks.gemm_f32(np.ones(3), (2, 1), np.ones(4), (2, 1), 2, 2, 2)


def test_task_face_span_overflow_is_a_contract_violation():
    import ctypes

    from poorgrad_amd import _native as n

    # Strides whose span 1 + (m-1)*rs + (k-1)*cs wraps size_t must not pass the
    # length check (the reference's span arithmetic panics on overflow).
    buf = (ctypes.c_float * 16)()
    out = (ctypes.c_float * 4)()
    huge = 1 << 63
    for a_rs, a_cs in ((huge, huge), (1, (1 << 64) - 1), ((1 << 64) - 1, 2)):
        code = n.lib.topos_hip_gemm_f32(buf, 16, a_rs, a_cs, buf, 16, 2, 1, 2, 2, 2, n.EXACT, out)
        assert code == n.INVALID_ARGUMENT, (a_rs, a_cs, code)


def _run_isolated(code: str) -> str:
    # Setup and poison are process-wide and sticky: each scenario runs in a
    # fresh interpreter.
    result = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=ROOT,
                            timeout=300)
    assert result.returncode == 0, result.stderr
    return result.stdout


def test_status_without_device_is_no_device_not_failure():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a device is visible here")
    out = _run_isolated("from poorgrad_amd import _native as n; print(n.status())")
    from poorgrad_amd import _native as n

    assert int(out.strip()) == n.NO_DEVICE


def test_runtime_failure_poisons_and_every_later_offer_declines():
    # The fake runtime (Api::fake, src/backend/cuda/kernels/context.rs:101-162)
    # fails its third device call: the first task fails and poisons, the
    # status reports the poison with its reason, and later tasks decline.
    code = r'''
import numpy as np
from poorgrad_amd import _native as n, tasks
assert n.lib.topos_hip_fake_runtime(2) == n.OK
assert n.status() == n.OK
a = np.ones(256 * 256, np.float32)
import ctypes
product = np.empty(256 * 256, np.float32)
f = lambda x: x.ctypes.data_as(n.FLOAT_P)
first = n.lib.topos_hip_gemm_f32(f(a), a.size, 256, 1, f(a), a.size, 256, 1, 256, 256, 256, n.FAST, f(product))
print(first, n.status(), n.status_reason())
second = tasks.gemm_f32(a, (256, 1), a, (256, 1), 256, 256, 256)
print(second is None)
assert n.lib.topos_hip_fake_runtime(0) == n.INVALID_ARGUMENT  # too late: already set up
'''
    lines = _run_isolated(code).strip().splitlines()
    from poorgrad_amd import _native as n

    first, status, reason = lines[0].split(" ", 2)
    assert int(first) == n.RUNTIME_ERROR
    assert int(status) == n.POISONED
    assert "fake runtime failure" in reason
    assert lines[1] == "True"


def test_fake_runtime_serves_until_its_failing_call():
    code = r'''
import numpy as np
from poorgrad_amd import _native as n, tasks
assert n.lib.topos_hip_fake_runtime(1000) == n.OK
a = np.ones(256 * 256, np.float32)
print(tasks.gemm_f32(a, (256, 1), a, (256, 1), 256, 256, 256, n.EXACT) is not None, n.status())
'''
    from poorgrad_amd import _native as n

    served, status = _run_isolated(code).split()
    assert served == "True" and int(status) == n.OK


def test_chain_source_is_generated_and_compiles_for_gfx950():
    # In the fake runtime the chain is generated and compiled by hipRTC for
    # gfx950 (no device needed), just not loaded.
    code = r'''
from poorgrad_amd import _native as n
from poorgrad_amd.device import Chain
import torch
assert n.lib.topos_hip_fake_runtime(1000) == n.OK
# y = x / (exp(-x) + 1) + b, b broadcast along axis 0
chain = Chain((8, 16), [((16, 1), 0), ((0, 1), 0), ((0, 0), 0)],
              [(n.CHAIN_NEG, -1, 0), (n.CHAIN_EXP, 0, 0), (n.CHAIN_ADD, 1, -3),
               (n.CHAIN_DIV, -1, 2), (n.CHAIN_ADD, 3, -2)], [4])
print(len(chain.source))
print("topos_faithful::exp_f32" in chain.source)
'''
    size, has_exp = _run_isolated(code).split()
    assert int(size) > 1000 and has_exp == "True"
