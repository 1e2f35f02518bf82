"""The reference's conformance suite (packages/tensor-backend/src/conformance.ts
runConformance) on HipBackend: ops.json, ops-numerics.json and
ops-quantized.json in f32, f16 and bf16, natively and with the optional ops
hidden (the compose fallbacks), plus the scope / dispose checks."""
import numpy as np
import pytest

from conformance import run_all
from fixtures import load_cases
from laya_hip import compose as C

pytestmark = pytest.mark.gpu

CASES = load_cases("ops.json") + load_cases("ops-numerics.json") + load_cases("ops-quantized.json")


@pytest.fixture(scope="module")
def backend():
    from laya_hip.backend import HipBackend
    b = HipBackend(0)
    yield b
    b.destroy()


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_all_cases(backend, dtype):
    print(f"conformance {dtype}", flush=True)
    ran, failures = run_all(backend, CASES, dtype)
    assert ran > 100
    assert not failures, f"{len(failures)} failing of {ran}:\n" + "\n".join(failures)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_all_cases_composed(backend, dtype):
    """withoutOptionalOps (conformance.ts:131-143): numerics, quantized and
    fused optional ops through the compose.ts compositions on the same
    device; cumsum has no composition and stays native, as in the
    reference's own composed run (backend-mlx/test/conformance.test.ts:33-35)."""
    hidden = tuple(o for o in C.NUMERICS_OPS if o != "cumsum") + C.QUANTIZED_OPS + ("geglu", "meanPool")
    b = C.without_optional_ops(backend, hidden)
    ran, failures = run_all(b, CASES, dtype)
    assert not failures, f"{len(failures)} failing of {ran}:\n" + "\n".join(failures)


def test_scope_disposes_intermediates_and_keeps_results(backend):
    """conformance.ts:311-318 and backend-cpu/test/backend.test.ts:32-54."""
    from laya_hip.host import host
    b = backend
    x = b.fromHost(host("f32", [2], [1, 2]))
    before = b.pool_stats()["live_blocks"]
    y = b.scope(lambda: b.add(b.exp(x), x))
    assert b.pool_stats()["live_blocks"] == before + 1  # the exp intermediate is gone
    got = b.read(y).data
    np.testing.assert_allclose(got, [np.e + 1, np.exp(2) + 2], rtol=1e-5, atol=1e-5)
    b.dispose(y)
    b.dispose(x)
    b.dispose(x)  # idempotent
    with pytest.raises(RuntimeError, match="after dispose"):
        b.exp(x)
    with pytest.raises(RuntimeError, match="boom"):
        b.scope(lambda: (b.exp(b.fromHost(host("f32", [1], [1]))), (_ for _ in ()).throw(RuntimeError("boom"))))


def test_from_host_copies_at_call_time(backend):
    from laya_hip.host import host
    data = np.array([1, 2], np.float32)
    h = host("f32", [2], data)
    t = backend.fromHost(h)
    h.data[0] = 9
    assert list(backend.read(t).data) == [1, 2]
    backend.dispose(t)
