"""Checkpoint I/O (laya_hip.checkpoint) on the CPU: the safetensors reader and
writer, the quantized-format metadata, and the converter and dequantizing
loader on the tiny golden checkpoint.  The cases follow the reference's
packages/laya/test/quant.test.ts:109-247."""
import os

import numpy as np
import pytest

from fixtures import read_safetensors as fixture_read
from laya_hip import checkpoint as C
from laya_hip.host import HostQuantized, HostTensor
from oracle import cpu_ref as cr

TINY = os.path.join(os.path.dirname(__file__), "golden", "tiny", "model.safetensors")


def test_reader_matches_the_fixture_reader():
    f = C.read_safetensors(TINY)
    want = fixture_read(TINY)
    assert sorted(f.names()) == sorted(want)
    for n in f.names():
        np.testing.assert_array_equal(np.asarray(f.array(n), np.float32), np.asarray(want[n], np.float32))


def test_writer_round_trip_and_alignment():
    t = {"a": C.RawTensor("F16", (2, 3), np.arange(6, dtype=np.float16).reshape(2, 3)),
         "b": C.RawTensor("I8", (5,), np.array([-1, 0, 1, 2, 3], np.int8)),
         "c": C.RawTensor("BF16", (1,), np.array([0x3F80], np.uint16))}
    data = C.write_safetensors(t, {"k": "v"})
    hlen = int.from_bytes(data[:8], "little")
    assert (8 + hlen) % 8 == 0
    f = C.read_safetensors(data)
    assert f.metadata == {"k": "v"}
    for n, r in t.items():
        assert f.info(n) == (r.dtype, r.shape)
        np.testing.assert_array_equal(f.array(n), r.data)
    with pytest.raises(ValueError):
        C.read_safetensors(data[:12])


def test_quant_metadata():
    """quant.test.ts:109-119."""
    assert C.quant_metadata({}) is None
    assert C.quant_metadata(None) is None
    m = C.quant_metadata({"laya_quant": "q4", "group_size": "64", "version": "1", "laya_quant_source_dtype": "F16"})
    assert (m.scheme, m.bits, m.group_size, m.version, m.source_dtype) == ("q4", 4, 64, "1", "F16")
    assert C.quant_metadata({"laya_quant": "q8", "group_size": "row", "version": "1"}).group_size is None
    with pytest.raises(ValueError, match="unknown quantization scheme"):
        C.quant_metadata({"laya_quant": "q3", "version": "1"})
    with pytest.raises(ValueError, match='format version "2" is not supported'):
        C.quant_metadata({"laya_quant": "q8", "version": "2"})
    with pytest.raises(ValueError, match="invalid group_size"):
        C.quant_metadata({"laya_quant": "q8", "version": "1", "group_size": "0"})


def test_should_quantize():
    """quant.test.ts:121-136."""
    sq = C.should_quantize
    assert sq("encoder.layers.0.attn.Wqkv.weight", "F16", (3072, 1024), 4)
    assert sq("encoder.embeddings.tok_embeddings.weight", "F16", (50368, 1024), 4)
    assert not sq("encoder.embeddings.tok_embeddings.weight", "F16", (50368, 1024), 4, embeddings=False)
    assert sq("head.layers.1.linear2.weight", "F16", (1024, 4096), 4)
    assert not sq("encoder.layers.1.attn_norm.weight", "F16", (1024,), 4)
    assert not sq("head.layers.0.norm1.weight", "F16", (1024,), 4)
    assert not sq("head.layers.0.linear1.bias", "F16", (4096,), 4)
    assert not sq("type_emb.weight", "F16", (3, 1024), 4)
    assert not sq("scorer.layers.3.weight", "F16", (1, 1024), 4)
    assert not sq("act_head.layers.0.weight", "F16", (256, 1028), 4)  # 1028 is not a multiple of 64
    assert sq("act_head.layers.0.weight", "F16", (256, 1028), 8, group_size="row")
    assert not sq("encoder.layers.0.mlp.Wi.weight", "F16", (5248, 1024), 4, exclude=(r"mlp",))
    assert not sq("x.weight", "I32", (128, 128), 4)


@pytest.mark.parametrize("bits", [8, 4])
def test_quantize_tiny_checkpoint(bits):
    """quant.test.ts:168-205: exact metadata, companions, untouched small
    tensors, weights back within the per-group bound, consuming getter."""
    data, report = C.quantize_safetensors(TINY, bits, metadata={"laya_quant_source": "tiny"})
    f = C.read_safetensors(data)
    assert f.metadata == {"laya_quant_source": "tiny", "laya_quant": f"q{bits}", "group_size": "64",
                          "version": C.QUANT_FORMAT_VERSION, "laya_quant_source_dtype": "F32"}
    src = C.read_safetensors(TINY)
    assert len(report["quantized"]) + len(report["kept"]) == len(src.names())
    assert report["bytes_in"] == sum(src.bytes(n).size for n in src.names())
    assert report["bytes_out"] == len(data)
    assert "encoder.layers.0.attn.Wqkv.weight" in report["quantized"]
    assert "encoder.embeddings.tok_embeddings.weight" in report["quantized"]
    for name in report["quantized"]:
        rows, cols = src.info(name)[1]
        assert f.info(name) == ("I8" if bits == 8 else "U8", (rows, cols) if bits == 8 else (rows, cols // 2))
        assert f.info(name + ".scales") == ("F16", (rows, cols // 64))
        assert f.has(name + ".biases") == (bits == 4)
    for name in report["kept"]:
        assert bytes(f.bytes(name)) == bytes(src.bytes(name)), name
        assert not f.has(name + ".scales")
    assert {"temperature", "type_emb.weight", "encoder.final_norm.weight"} <= set(report["kept"])
    ws = C.read_weights(data, dtype="f32")
    name = "encoder.layers.1.mlp.Wi.weight"
    got = ws.get(name)
    assert got.dtype == "f32" and tuple(got.shape) == src.info(name)[1]
    want = np.asarray(src.array(name), np.float32)
    s = np.asarray(f.array(name + ".scales"), np.float32)
    cols = got.shape[1]
    bound = (1.0 if bits == 8 else 1.5) * np.repeat(s, 64, axis=1) + 1e-6
    assert np.all(np.abs(got.data - want) <= bound)
    assert ws.get(name) is None  # consumed
    assert name not in ws.remaining()
    assert not any(n.endswith((".scales", ".biases")) for n in ws.remaining())


def test_mixed_precision_q8_patterns():
    """quant.test.ts:224-235."""
    data, report = C.quantize_safetensors(TINY, 4, q8=(r"attn\.",))
    f = C.read_safetensors(data)
    assert f.info("encoder.layers.0.attn.Wqkv.weight")[0] == "I8"
    assert not f.has("encoder.layers.0.attn.Wqkv.weight.biases")
    assert f.info("encoder.layers.0.mlp.Wi.weight")[0] == "U8"
    assert sorted(report["promoted"]) == sorted(n for n in report["quantized"] if "attn." in n)
    t = C.read_weights(data).get("encoder.layers.0.attn.Wqkv.weight")
    assert t.dtype == "f16" and t.data.dtype == np.float16


def test_plain_untouched_and_corrupt_files_fail():
    """quant.test.ts:237-247."""
    plain = C.read_weights(TINY, dtype="f16")
    assert plain.get("encoder.layers.0.attn.Wqkv.weight").dtype == "f32"  # dtype applies to dequantized tensors
    data, _ = C.quantize_safetensors(TINY, 4)
    f = C.read_safetensors(data)
    tensors = {n: f.raw(n) for n in f.names()}
    del tensors["encoder.layers.0.attn.Wqkv.weight.biases"]
    with pytest.raises(ValueError, match=r"q4 needs \.biases"):
        C.read_weights(C.write_safetensors(tensors, f.metadata))
    with pytest.raises(ValueError, match='format version "9"'):
        C.read_weights(C.write_safetensors({}, {"laya_quant": "q4", "version": "9"}))
    with pytest.raises(ValueError, match="already quantized"):
        C.quantize_safetensors(data, 8)


@pytest.mark.parametrize("bits", [8, 4])
def test_device_getter_hands_out_packed_matrices(bits):
    """quant.test.ts:315-335: quantized="device" gives HostQuantized views of
    the stored codes; the host-dequantized weights equal the oracle's
    fl16(q*s + z) of those codes bit for bit."""
    data, report = C.quantize_safetensors(TINY, bits)
    dev = C.read_weights(data, quantized="device")
    hostw = C.read_weights(data, dtype="f16")
    for name in report["quantized"]:
        h = dev.get(name)
        assert isinstance(h, HostQuantized) and h.bits == bits
        assert h.mode == ("symmetric" if bits == 8 else "affine")
        ref = hostw.get(name)
        assert isinstance(ref, HostTensor) and ref.dtype == "f16"
        G = h.shape[1] // h.groupSize
        codes = np.asarray(h.data, np.uint8).reshape(h.shape[0], -1)
        if bits == 8:
            q = codes.view(np.int8).astype(np.int32)
        else:
            q = np.empty(h.shape, np.int32)
            q[:, 0::2], q[:, 1::2] = codes & 15, codes >> 4
        s = np.asarray(h.scales.data, np.float32).reshape(h.shape[0], G)
        z = None if h.biases is None else np.asarray(h.biases.data, np.float32).reshape(h.shape[0], G)
        want = cr.dequant_exact_f16(q, s, z, h.groupSize)  # the oracle: fl16(q*s + z), rounded once
        np.testing.assert_array_equal(np.asarray(ref.data).view(np.uint16).reshape(h.shape), want)
    plain = dev.get("encoder.final_norm.weight")
    assert isinstance(plain, HostTensor) and plain.dtype == "f32"


@pytest.mark.parametrize("patch,msg", [
    ({"head_layers": None}, "must specify encoder and head_layers"),
    ({"encoder": None}, "must specify encoder and head_layers"),
    ({"head_max_len": 4}, "4 < head_max_len < max_len"),
    ({"head_max_len": 128}, "4 < head_max_len < max_len"),
    ({"max_len": 257}, "4 < head_max_len < max_len"),
])
def test_load_checkpoint_validates_the_config_before_reading_weights(tmp_path, patch, msg):
    """load.ts:53 runs validateConfig (agent.ts:96-105) before any weight is
    read: an invalid rl_agent_config.json fails with the reference's message
    even when model.safetensors is unreadable, and no backend call is made
    (the backend argument is None)."""
    import json
    import shutil
    from laya_hip.model import loadCheckpoint, validateConfig
    from laya_hip.modernbert import parseModernBertConfig

    src = os.path.dirname(TINY)
    d = tmp_path / "ckpt"
    shutil.copytree(src, d)
    cfg = json.load(open(d / "rl_agent_config.json"))
    enc = parseModernBertConfig(json.load(open(d / "encoder" / "config.json")))
    validateConfig(cfg, enc)  # the fixture's own config is valid
    for k, v in patch.items():
        if v is None:
            del cfg[k]
        else:
            cfg[k] = v
    json.dump(cfg, open(d / "rl_agent_config.json", "w"))
    (d / "model.safetensors").write_bytes(b"not a safetensors file")
    with pytest.raises(ValueError, match=msg):
        loadCheckpoint(None, str(d))
