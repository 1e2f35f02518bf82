"""The package's quantizer (laya_hip.quant, restating laya/src/quant.ts
quantizeMatrix) produces the same bytes as the CPU oracle's C restatement,
which tests/test_oracle.py pins to the reference's quant tests."""
import numpy as np
import pytest

from laya_hip.quant import quantize_matrix
from oracle import cpu_ref as cr


def _cases():
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((96, 192)) * 0.02).astype(np.float32)
    w[0] = 0                                # all-zero row
    w[1, :64] = 0.01                        # constant group
    w[2, 5] = 0.5                           # outlier
    w[3, :32] = np.float32(np.float16(1 / 127)) * 2.5  # exact half-way values
    yield w, 96, 192
    yield (rng.standard_normal((64, 768)) * 0.02).astype(np.float32), 64, 768


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [64, 32, 16])
@pytest.mark.parametrize("refine", [False, True])
def test_quantizer_matches_oracle_bytes(bits, group, refine):
    for w, r, c in _cases():
        q, s, b = quantize_matrix(w, r, c, bits, group, refine=refine)
        oq, os_, ob = cr.quantize_matrix(w, r, c, bits, group, refine=refine)
        np.testing.assert_array_equal(q, oq)
        np.testing.assert_array_equal(s.view(np.uint16), os_)
        if bits == 4:
            np.testing.assert_array_equal(b.view(np.uint16), ob)
        else:
            assert b is None


def test_quantizer_rejects_bad_shapes():
    with pytest.raises(ValueError, match="must divide"):
        quantize_matrix(np.zeros(20, np.float32), 2, 10, 8, 64)
    with pytest.raises(ValueError, match="even"):
        quantize_matrix(np.zeros(18, np.float32), 2, 9, 4, 9)
