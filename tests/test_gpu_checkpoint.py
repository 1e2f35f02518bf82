"""Checkpoints loaded from disk onto HipBackend: the tiny golden checkpoint
read by laya_hip.checkpoint (float, and quantized q8 / q4 with the weights
dequantized on load or kept packed on the device) through the unchanged
encoder loader, against the golden activations (packages/laya/test/
quant.test.ts:207-222, 337-360 do the same through load())."""
import os

import numpy as np
import pytest

from fixtures import arr, tiny
from gpu_util import read32
from laya_hip import checkpoint as C
from laya_hip.modernbert import loadModernBert, parseModernBertConfig
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu

TINY = os.path.join(os.path.dirname(__file__), "golden", "tiny", "model.safetensors")


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _encode(b, weights, dtype):
    cfgj, _, act = tiny()
    # a consuming getter hands each tensor out once: the prefix is given, as
    # laya passes it (packages/laya/src/model.ts:332)
    enc = loadModernBert(b, parseModernBertConfig(cfgj), weights.get, dtype=dtype, prefix="encoder.")
    ids = arr(act["inputs"]["input_ids"])
    mask = arr(act["inputs"]["attention_mask"])
    out = read32(b, enc.forward(ids, mask, ids.shape[0], ids.shape[1]))
    enc.dispose()
    return out, arr(act["stages"]["encoder.final_norm"]), mask


def test_float_checkpoint_from_disk(b):
    out, want, _ = _encode(b, C.read_weights(TINY), "f32")
    assert np.max(np.abs(out - want)) <= 1e-4


def _oracle_weights(data):
    """Oracle weights from a quantized file: fl16(q*s + z) of the stored codes
    by the oracle's own dequantizer, plain tensors as stored (f32)."""
    f = C.read_safetensors(data)
    W = {}
    for n in f.names():
        if n.endswith((".scales", ".biases")) or not n.startswith("encoder."):
            continue
        dt, shape = f.info(n)
        if f.has(n + ".scales"):
            s = np.asarray(f.array(n + ".scales"), np.float32)
            z = np.asarray(f.array(n + ".biases"), np.float32) if f.has(n + ".biases") else None
            codes = np.asarray(f.array(n))
            if dt == "I8":
                q = codes.astype(np.int32)
            else:
                q = np.empty((shape[0], 2 * shape[1]), np.int32)
                q[:, 0::2], q[:, 1::2] = codes & 15, codes >> 4
            W[n[8:]] = cr.dequant_exact_f16(q, s, z, q.shape[1] // s.shape[1]).view(np.float16).astype(np.float32)
        else:
            W[n[8:]] = np.asarray(f.array(n), np.float32)
    return W


@pytest.mark.parametrize("bits,sanity", [(8, 5e-2), (4, 5e-1)])
def test_quantized_checkpoint_host_and_device_paths(b, bits, sanity):
    """Both loading paths against the f32 oracle on the same dequantized
    weights (the f16 parity bar, 5e-2), and loosely against the float
    golden stages (the quantization error itself)."""
    data, _ = C.quantize_safetensors(TINY, bits)
    host_out, want, mask = _encode(b, C.read_weights(data, dtype="f16"), "f16")
    dev_out, _, _ = _encode(b, C.read_weights(data, quantized="device"), "f16")
    cfgj, _, act = tiny()
    ids = arr(act["inputs"]["input_ids"])
    ref = cr.encoder_forward(cr.EncoderConfig.from_json(cfgj), _oracle_weights(data), ids, mask)
    valid = mask != 0
    e_host = float(np.max(np.abs(host_out[valid] - ref[valid])))
    e_dev = float(np.max(np.abs(dev_out[valid] - ref[valid])))
    e_float = float(np.max(np.abs(host_out[valid] - want[valid])))
    print(f"tiny q{bits}: vs oracle on the dequantized weights host {e_host:.3e} device {e_dev:.3e}; "
          f"vs the float golden stages {e_float:.3e}")
    assert e_host <= 5e-2 and e_dev <= 5e-2
    assert e_float <= sanity
