"""Native quantizedEmbedding (hb_qgather; Backend.quantizedEmbedding,
index.ts:250-256) bit for bit against numpy.  A looked-up value is the
code times its group's f16 scale, plus the f16 zero when affine:
- f16 output: the exact value rounded once to f16 (the product of an f16
  code and an f16 scale, or their fused multiply-add with the zero);
- f32 output: the exact value rounded once to f32.

Shapes with K % 8 == 0 and group % 8 == 0 take the 8-values-per-thread
kernel, including a partial last group (K = 1000, group 64).  The others
(groups of 4 and 12; K = 20 with groups of 10, q8 only) take the
one-value-per-thread kernel.  Both must give the same bits."""
import numpy as np
import pytest

from laya_hip.host import HostQuantized, HostTensor, quant_groups

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _table(rng, V, K, bits, group, mode):
    lo, hi = {(8, "symmetric"): (-128, 127), (8, "affine"): (0, 255), (4, "symmetric"): (-8, 7),
              (4, "affine"): (0, 15)}[(bits, mode)]
    codes = rng.integers(lo, hi + 1, (V, K)).astype(np.int32)
    G = quant_groups(K, group)
    scales = (rng.uniform(0.002, 0.05, (V, G)) * rng.choice([-1, 1], (V, G))).astype(np.float16)
    zeros = rng.uniform(-1, 1, (V, G)).astype(np.float16) if mode == "affine" else None
    if bits == 8:
        packed = (codes & 255).astype(np.uint8)
    else:
        nib = (codes & 15).astype(np.uint8)
        packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return codes, scales, zeros, packed


# (K, group) x (bits, mode) cases the format allows (in * bits % 32 == 0;
# K = 20 takes q8 only, its q4 refusal is a CPU test)
CASES = [(K, g, bits, mode) for K, g in [(1024, 64), (1000, 64), (16, 4), (24, 12), (20, 10)]
         for bits, mode in [(8, "symmetric"), (8, "affine"), (4, "symmetric"), (4, "affine")] if (K * bits) % 32 == 0]


@pytest.mark.parametrize("out_dtype", ["f16", "f32"])
@pytest.mark.parametrize("K,group,bits,mode", CASES)
def test_quantized_embedding_bits(b, out_dtype, bits, mode, K, group):
    rng = np.random.default_rng(K * 10 + bits + (mode == "affine"))
    V = 300
    codes, scales, zeros, packed = _table(rng, V, K, bits, group, mode)
    h = HostQuantized((V, K), bits, group, mode, packed, HostTensor("f32", scales.shape, scales.astype(np.float32)),
                      None if zeros is None else HostTensor("f32", zeros.shape, zeros.astype(np.float32)))
    q = b.fromHostQuantized(h, out_dtype)
    assert q is not None
    ids = rng.integers(0, V, (2, 129)).astype(np.int32)
    ids[0, :3] = [0, V - 1, 7]
    I = b.fromHost(HostTensor("i32", ids.shape, ids))
    got = np.asarray(b.read(b.quantizedEmbedding(q.w, q.scales, q.biases, q, I)).data)
    g = np.arange(K) // group
    c = codes[ids].astype(np.float64)
    s = scales[ids][..., g].astype(np.float64)
    exact = c * s  # a zero code times a negative scale is -0
    if zeros is not None:
        exact = exact + zeros[ids][..., g].astype(np.float64)
    want = exact.astype(np.float16 if out_dtype == "f16" else np.float32)
    assert got.shape == want.shape
    np.testing.assert_array_equal(got.view(np.uint16 if out_dtype == "f16" else np.uint32),
                                  want.view(np.uint16 if out_dtype == "f16" else np.uint32))
    b.dispose(I)
