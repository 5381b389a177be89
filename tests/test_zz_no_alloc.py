"""The no-allocation product (topos_hip_gemm_f32_device_noalloc) against the
allocating device-face product (topos_hip_gemm_f32_device), both called
through the C ABI on the same operands. Both launch the same kernels with the
same split along k whenever the partials fit the fixed array; only the home
of the split partials differs (a fixed device array instead of the library's
workspace), so the results must then agree bit for bit, and each must meet
the oracle's bar (gemm::multiply, src/payload/gemm.rs:140-211): bitwise under
Exact, within |c - exact| <= 1e-5 * sum_k |a_ik b_kj| under Fast.

Two calls in a row share the fixed array, the second with a smaller product,
so the second runs over the first's leftover partials. A product whose split
would need more than the array splits into fewer ranges: within the envelope.
In a fresh process the no-allocation entry runs first, under HIP graph
capture too, and the library's workspace is shown never to be created."""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:  # the child process runs this file as a script
    sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

pytestmark = pytest.mark.gpu

# (m, k, n, seed). Under Fast both split k: 16 partials of 512 x 512 (16 MiB)
# then 8 of 256 x 384, each within the 64 MiB array.
CASES = [(512, 4096, 512, 21), (256, 2048, 384, 22)]


def _product(entry, a, a_strides, b, b_strides, m, k, n, numerics, out=None):
    import torch

    from poorgrad_amd import _native as nat

    if out is None:
        out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    code = getattr(nat.lib, entry)(a.data_ptr(), a_strides[0], a_strides[1], b.data_ptr(), b_strides[0],
                                   b_strides[1], m, k, n, numerics, out.data_ptr(), n,
                                   torch.cuda.current_stream().cuda_stream)
    nat.checked(code, entry)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _operands(m, k, n, seed, transposed):
    from tests.gpu_util import to_device

    g = oracle.Generator(seed)
    a = g.normal(m * k, 1.0).reshape(m, k)
    b = g.normal(k * n, 1.0).reshape(k, n)
    if transposed:  # A^T . G: the left operand stored [k, m], strides [1, m]
        return a, b, to_device(np.ascontiguousarray(a.T)), (1, m), to_device(b), (n, 1)
    return a, b, to_device(a), (k, 1), to_device(b), (n, 1)


def _within_envelope(got, a, b, rows=None):
    rows = slice(None) if rows is None else rows
    exact = oracle.gemm(np.ascontiguousarray(a[rows]), (a.shape[1], 1), b, (b.shape[1], 1), a[rows].shape[0],
                        a.shape[1], b.shape[1])
    bound = 1e-5 * (np.abs(a[rows].astype(np.float64)) @ np.abs(b.astype(np.float64)))
    return bool((np.abs(got[rows].astype(np.float64) - exact) <= bound).all())


@pytest.mark.parametrize("transposed", [False, True], ids=["a_b", "at_b"])
@pytest.mark.parametrize("posture", ["exact", "fast"])
def test_noalloc_product_equals_allocating_product(hip, posture, transposed):
    from tests.conftest import banner
    from tests.gpu_util import assert_bitwise

    numerics = hip.EXACT if posture == "exact" else hip.FAST
    prepared = [(case, _operands(*case, transposed)) for case in CASES]
    allocating = []
    for (m, k, n, seed), (_, _, da, ast, db, bst) in prepared:
        banner(f"noalloc: allocating product {posture} {m}x{k}x{n} transposed={transposed}")
        allocating.append(_product("topos_hip_gemm_f32_device", da, ast, db, bst, m, k, n, numerics))
    # The no-allocation calls back to back: the second, smaller product runs
    # over the first's partials left in the shared array.
    fixed = []
    for (m, k, n, seed), (_, _, da, ast, db, bst) in prepared:
        banner(f"noalloc: no-allocation product {posture} {m}x{k}x{n} transposed={transposed}")
        fixed.append(_product("topos_hip_gemm_f32_device_noalloc", da, ast, db, bst, m, k, n, numerics))
    for ((m, k, n, seed), (a, b, *_)), want, got in zip(prepared, allocating, fixed):
        assert_bitwise(got, want, f"noalloc vs allocating {posture} {m}x{k}x{n}")
        if numerics == hip.EXACT:
            exact = oracle.gemm(a.ravel(), (k, 1), b.ravel(), (n, 1), m, k, n)
            assert_bitwise(got, exact, f"noalloc vs oracle {m}x{k}x{n}")
        else:
            assert _within_envelope(got, a, b), f"envelope {m}x{k}x{n}"


def test_noalloc_splits_within_its_array(hip):
    """2048 x 2048 over k = 8192 splits six ways under Fast on the allocating
    entry (96 MiB of partials); the no-allocation entry takes the four ranges
    its 64 MiB array holds. Both within the envelope (rows sampled against the
    oracle); Exact needs no scratch and stays bitwise equal."""
    import torch

    from tests.conftest import banner
    from tests.gpu_util import assert_bitwise, to_device

    m, k, n = 2048, 8192, 2048
    banner(f"noalloc: capped split {m}x{k}x{n}")
    g = oracle.Generator(31)
    a = g.normal(m * k, 1.0).reshape(m, k)
    b = g.normal(k * n, 1.0).reshape(k, n)
    da, db = to_device(a), to_device(b)
    got = _product("topos_hip_gemm_f32_device_noalloc", da, (k, 1), db, (n, 1), m, k, n, hip.FAST)
    assert hip.lib.topos_hip_last_refusal() == b""
    rows = np.r_[0:8, 1021:1029, m - 8:m]
    assert _within_envelope(got, a, b, rows), "capped split outside the envelope"
    again = _product("topos_hip_gemm_f32_device_noalloc", da, (k, 1), db, (n, 1), m, k, n, hip.FAST)
    assert_bitwise(again, got, "capped split repeats")
    banner(f"noalloc: exact at {m}x{k}x{n}")
    want = _product("topos_hip_gemm_f32_device", da, (k, 1), db, (n, 1), m, k, n, hip.EXACT)
    exact = _product("topos_hip_gemm_f32_device_noalloc", da, (k, 1), db, (n, 1), m, k, n, hip.EXACT)
    assert_bitwise(exact, want, "noalloc exact, large")
    del da, db
    torch.cuda.empty_cache()


def test_noalloc_allocates_nothing_in_a_fresh_process_and_under_capture(hip):
    """A child process calls the no-allocation entry before anything else:
    the library's workspace stays uncreated (topos_hip_workspace_bytes() is
    0) through a split Fast product, its replay inside a captured HIP graph
    (global capture mode, where an allocation would fail the capture) and a
    second smaller product; only the allocating entry then creates it."""
    from tests.conftest import banner

    banner("noalloc: fresh child process, graph capture")
    done = subprocess.run([sys.executable, "-u", str(Path(__file__).resolve()), "child"], cwd=str(ROOT),
                          capture_output=True, text=True, timeout=300)
    print(done.stdout[-4000:], flush=True)
    assert done.returncode == 0, done.stderr[-4000:]
    assert "child: ok" in done.stdout


def _child() -> None:
    import torch

    from poorgrad_amd import _native as nat
    from tests.gpu_util import assert_bitwise, to_device

    assert nat.status() == nat.OK, nat.status_reason()
    assert nat.lib.topos_hip_workspace_bytes() == 0
    results = []
    for (m, k, n, seed) in CASES:
        print(f"child: noalloc {m}x{k}x{n}", flush=True)
        a, b, da, ast, db, bst = _operands(m, k, n, seed, False)
        eager = _product("topos_hip_gemm_f32_device_noalloc", da, ast, db, bst, m, k, n, nat.FAST)
        assert nat.lib.topos_hip_workspace_bytes() == 0, "the no-allocation entry created the workspace"
        assert _within_envelope(eager, a, b), "envelope"
        results.append((m, k, n, da, ast, db, bst, eager))
    # Capture the first product, then replay it with eager work between the
    # replays: every replay gives the eager bits.
    m, k, n, da, ast, db, bst, eager = results[0]
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    graph = torch.cuda.CUDAGraph()
    print("child: capture", flush=True)
    with torch.cuda.graph(graph):
        stream = torch.cuda.current_stream().cuda_stream
        code = nat.lib.topos_hip_gemm_f32_device_noalloc(da.data_ptr(), ast[0], ast[1], db.data_ptr(), bst[0],
                                                         bst[1], m, k, n, nat.FAST, out.data_ptr(), n, stream)
        assert code == nat.OK, nat.lib.topos_hip_last_refusal()
    for replay in range(3):
        print(f"child: replay {replay}", flush=True)
        out.fill_(float("nan"))
        # Eager work between replays: the second product through the same array.
        m2, k2, n2, da2, ast2, db2, bst2, eager2 = results[1]
        again = _product("topos_hip_gemm_f32_device_noalloc", da2, ast2, db2, bst2, m2, k2, n2, nat.FAST)
        assert_bitwise(again, eager2, "eager product between replays")
        graph.replay()
        torch.cuda.synchronize()
        assert_bitwise(out.cpu().numpy(), eager, f"replay {replay}")
    assert nat.lib.topos_hip_workspace_bytes() == 0, "capture or replay created the workspace"
    # The allocating entry does create it: the diagnostic sees allocations.
    _product("topos_hip_gemm_f32_device", da, ast, db, bst, m, k, n, nat.FAST)
    assert nat.lib.topos_hip_workspace_bytes() > 0
    del graph
    print("child: ok", flush=True)


if __name__ == "__main__" and sys.argv[1:] == ["child"]:
    _child()
