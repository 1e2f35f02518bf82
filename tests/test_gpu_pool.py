"""Masked mean pooling on the GPU (Backend.meanPool, index.ts:242-243;
compose.ts:96-105): the two-pass kernel for 16-bit activations (column
chunks of 512, row slices, four row groups added in a fixed order) against
numpy's f64 mean of the same stored values.  The shapes leave a partial last
column chunk (D = 1032), uneven row slices (L = 517) and a sequence with no
visible token (its mean is 0, as compose.ts divides by max(count, 1)).
Sums are f32, so the bound is relative: 1e-5 of the largest |mean|.  Two
runs give the same bits (no atomics)."""
import numpy as np
import pytest

from gpu_util import read32, rounded, to_host
from laya_hip.host import HostTensor

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("B,L,D", [(3, 517, 1032), (16, 2048, 1024), (1, 7, 8)])
def test_meanpool_16bit(b, dtype, B, L, D):
    rng = np.random.default_rng(B * 1000 + L)
    x = rounded(rng.standard_normal((B, L, D)) * 2 + 0.25, dtype)
    lens = rng.integers(1, L + 1, B)
    lens[0] = 0 if B > 1 else lens[0]
    mask = (np.arange(L)[None, :] < lens[:, None]).astype(np.uint8)
    X = b.fromHost(to_host(x, dtype))
    Mk = b.fromHost(HostTensor("bool", (B, L), mask))
    got = read32(b, b.meanPool(X, Mk))
    again = read32(b, b.meanPool(X, Mk))
    np.testing.assert_array_equal(got, again)
    cnt = mask.sum(1).astype(np.float64)
    want = (x.astype(np.float64) * mask[:, :, None]).sum(1) / np.maximum(cnt, 1.0)[:, None]
    assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))
    if B > 1:
        assert np.all(got[0] == 0.0)  # no visible token
    for t in (X, Mk):
        b.dispose(t)
