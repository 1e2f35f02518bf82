"""Row ops of the decision head on the GPU (laya/src/model.ts:218-224):
`sort` and `softmax` over rows of marker scores (up to 255 markers), which
take the block-per-row kernel for contiguous rows of 16..1024 values.

- sort: bit for bit against numpy's stable sort of the values as stored in
  the output dtype -- ascending, NaN last, equal values (-0 and +0 among
  them) in their original order, which is what the library's stable
  insertion sort gives for other shapes;
- softmax: against numpy in f64, 1e-6 absolute on probabilities, with
  masked logits (-1e4) as the head writes them.
"""
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


def _row_values(rng, rows, n):
    x = rng.standard_normal((rows, n)).astype(np.float32)
    x[:, ::7] = np.round(x[:, ::7])  # duplicates
    x[0, :4] = [0.0, -0.0, 0.0, -0.0]  # signed zeros keep their order
    x[1, 3] = np.nan
    x[1, n // 2] = np.nan
    x[2, :] = 1.5  # all equal
    return x


@pytest.mark.parametrize("n", [15, 16, 255, 1000, 1024])
def test_sort_rows_f32(b, n):
    rng = np.random.default_rng(n)
    x = _row_values(rng, 7, n)
    X = b.fromHost(HostTensor("f32", x.shape, x))
    got = np.asarray(b.read(b.sort(X, -1)).data, np.float32).reshape(x.shape)
    want = np.sort(x, axis=-1, kind="stable")
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    b.dispose(X)


@pytest.mark.parametrize("n", [16, 255])
def test_sort_rows_i32_and_f16(b, n):
    rng = np.random.default_rng(100 + n)
    xi = rng.integers(-50, 50, (5, n)).astype(np.int32)
    Xi = b.fromHost(HostTensor("i32", xi.shape, xi))
    got = np.asarray(b.read(b.sort(Xi, -1)).data, np.int32).reshape(xi.shape)
    np.testing.assert_array_equal(got, np.sort(xi, axis=-1, kind="stable"))
    xh = rounded(_row_values(rng, 5, n), "f16")
    Xh = b.fromHost(to_host(xh, "f16"))
    goth = read32(b, b.sort(Xh, -1)).reshape(xh.shape)
    np.testing.assert_array_equal(goth.view(np.uint32), np.sort(xh, axis=-1, kind="stable").view(np.uint32))
    for t in (Xi, Xh):
        b.dispose(t)


@pytest.mark.parametrize("n", [16, 255, 1024])
def test_softmax_rows(b, n):
    rng = np.random.default_rng(200 + n)
    x = (rng.standard_normal((9, n)) * 3).astype(np.float32)
    x[:, n - n // 3:] = -1e4  # masked marker slots
    X = b.fromHost(HostTensor("f32", x.shape, x))
    got = np.asarray(b.read(b.softmax(X, -1)).data, np.float32).reshape(x.shape)
    z = x.astype(np.float64)
    e = np.exp(z - z.max(-1, keepdims=True))
    want = e / e.sum(-1, keepdims=True)
    assert np.max(np.abs(got - want)) <= 1e-6
    b.dispose(X)


@pytest.mark.parametrize("n", [63, 64, 255, 1000])
@pytest.mark.parametrize("op", ["sum", "mean", "max", "min"])
def test_reduce_rows(b, op, n):
    """Float reductions over contiguous rows (`sum(plogp, -1)` in the head):
    rows of 64 or more values take one block per row.  Sum and mean within
    1e-5 of f64 (relative to the row's sum of |x|); max and min exact, a NaN
    in the row winning as in numpy."""
    rng = np.random.default_rng(300 + n)
    x = rng.standard_normal((6, n)).astype(np.float32)
    x[3, n // 3] = np.nan
    X = b.fromHost(HostTensor("f32", x.shape, x))
    got = np.asarray(b.read(getattr(b, op)(X, -1)).data, np.float32)
    want = getattr(np, op)(x.astype(np.float64), axis=-1)
    if op in ("sum", "mean"):
        scale = np.abs(x.astype(np.float64)).sum(-1) / (n if op == "mean" else 1)
        ok = np.isnan(want) == np.isnan(got)
        assert ok.all()
        fin = ~np.isnan(want)
        assert np.all(np.abs(got[fin] - want[fin]) <= 1e-5 * scale[fin])
    else:
        np.testing.assert_array_equal(got, want.astype(np.float32))
    b.dispose(X)
