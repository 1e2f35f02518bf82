"""Empty and degenerate shapes through the Backend ops on the GPU.

A HIP launch with an empty grid is an error, so the library returns before
launching anything when an op's output is empty.  These cases check that
every such early return still leaves a well-formed result, with the values
the mathematics fixes (the reference's fixtures hold no empty shapes):
- shape-preserving ops on a tensor with a 0 dimension give an empty result
  of the same shape;
- linear and matmul with no rows give an empty result. With K = 0 they give
  the bias, or zeros, since an empty dot product is 0;
- a sum over an empty axis is 0;
- meanPool over a sequence of length 0 is 0, as compose.ts:96-105 divides by
  max(count, 1);
- max over an empty axis has no value. It is refused with an error before
  any launch;
- attention over no keys is NaN, like a fully masked query row.
"""
import numpy as np
import pytest

from laya_hip import ffi as F
from laya_hip.host import HostTensor

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _t(b, dtype, shape, fill=None):
    np_dt = {"f32": np.float32, "f16": np.float16, "i32": np.int32, "bool": np.uint8}[dtype]
    a = np.zeros(shape, np_dt) if fill is None else np.asarray(fill, np_dt).reshape(shape)
    return b.fromHost(HostTensor(dtype, shape, a))


def _read(b, t):
    h = b.read(t)
    return np.asarray(h.data).reshape(h.shape)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_shape_preserving_ops_on_empty(b, dtype):
    x = _t(b, dtype, (0, 8))
    y = _t(b, dtype, (3, 0))
    outs = [b.add(x, x), b.scale(x, 2.0), b.exp(x), b.softmax(y, -1), b.sort(y, -1), b.cumsum(x, 0),
            b.softmax(x, -1), b.sort(x, -1)]
    for o, shape in zip(outs, [(0, 8), (0, 8), (0, 8), (3, 0), (3, 0), (0, 8), (0, 8), (0, 8)]):
        got = _read(b, o)
        assert got.shape == shape and got.size == 0
        b.dispose(o)
    w = _t(b, dtype, (8,), np.ones(8))
    ln = b.layerNorm(x, w, None, 1e-5)
    assert _read(b, ln).shape == (0, 8)
    for t in (x, y, w, ln):
        b.dispose(t)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_linear_without_rows(b, dtype):
    rng = np.random.default_rng(1)
    x = _t(b, dtype, (2, 0, 64))
    w = _t(b, dtype, (32, 64), rng.standard_normal((32, 64)) * 0.1)
    bias = _t(b, dtype, (32,), rng.standard_normal(32))
    y = b.linear(x, w, bias)
    got = _read(b, y)
    assert got.shape == (2, 0, 32)
    z = b.matmul(_t(b, dtype, (0, 64)), b.transpose(w, [1, 0]))
    assert _read(b, z).shape == (0, 32)
    for t in (x, w, bias, y, z):
        b.dispose(t)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_linear_with_empty_inner_dimension(b, dtype):
    """K = 0: each output is the bias exactly (no rounding is involved)."""
    rng = np.random.default_rng(2)
    bias_v = rng.standard_normal(8).astype(np.float16).astype(np.float32)
    x = _t(b, dtype, (4, 0))
    w = _t(b, dtype, (8, 0))
    bias = _t(b, dtype, (8,), bias_v)
    got = _read(b, b.linear(x, w, bias)).astype(np.float32)
    np.testing.assert_array_equal(got, np.broadcast_to(bias_v, (4, 8)))
    got0 = _read(b, b.linear(x, w, None)).astype(np.float32)
    np.testing.assert_array_equal(got0, np.zeros((4, 8), np.float32))
    m = _read(b, b.matmul(_t(b, dtype, (3, 0)), _t(b, dtype, (0, 5)))).astype(np.float32)
    np.testing.assert_array_equal(m, np.zeros((3, 5), np.float32))


def test_reductions_over_an_empty_axis(b):
    x = _t(b, "f32", (3, 0))
    np.testing.assert_array_equal(_read(b, b.sum(x, 1)), np.zeros(3, np.float32))
    xi = _t(b, "i32", (0, 4))
    np.testing.assert_array_equal(_read(b, b.sum(xi, 0)), np.zeros(4, np.int32))
    with pytest.raises(F.HipError, match="empty axis"):
        b.max(x, 1)
    for t in (x, xi):
        b.dispose(t)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_meanpool_of_empty_sequences(b, dtype):
    x = _t(b, dtype, (2, 0, 64))
    mask = _t(b, "bool", (2, 0))
    got = _read(b, b.meanPool(x, mask))
    np.testing.assert_array_equal(got, np.zeros((2, 64), np.float32))
    assert _read(b, b.meanPool(_t(b, dtype, (0, 5, 64)), _t(b, "bool", (0, 5)))).shape == (0, 64)
    for t in (x, mask):
        b.dispose(t)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("masked", [False, True])
def test_sdpa_without_keys(b, dtype, masked):
    """Attention over Lk = 0 keys: a softmax over an empty set, 0 / 0, is NaN
    in every output, as for a query row whose keys are all masked (the
    oracle's cr_sdpa and both kernels give those rows NaN).  A masked call
    builds no mask summary and launches nothing invalid.  The query and
    value shapes are those of the encoder's MFMA path (D = 64)."""
    q = _t(b, dtype, (2, 3, 40, 64), np.ones(2 * 3 * 40 * 64))
    k = _t(b, dtype, (2, 3, 0, 64))
    v = _t(b, dtype, (2, 3, 0, 64))
    m = _t(b, "bool", (2, 1, 40, 0)) if masked else None
    o = b.sdpa(q, k, v, m, 0.125)
    got = _read(b, o).astype(np.float32)
    assert got.shape == (2, 3, 40, 64) and np.all(np.isnan(got))
    for t in (q, k, v, m, o):
        if t is not None:
            b.dispose(t)
