"""CPU tests of the host-side logic: view strides, masks, the quantized
layout helpers and the config parser (no GPU)."""
import numpy as np
import pytest

from fixtures import arr, case, tiny
from laya_hip.backend import HipBackend, _broadcast_shape, _contig
from laya_hip.host import HostQuantized, HostTensor, pack_quantized, unpack_quantized, validate_quantized
from laya_hip.modernbert import attentionMasks, parseModernBertConfig
from oracle import cpu_ref as cr


def _view_ok(shape, strides, new_shape):
    """Checks _nocopy_strides against numpy on a strided view of arange."""
    base = np.arange(10000)
    itemsize = base.itemsize
    v = np.lib.stride_tricks.as_strided(base, shape, [s * itemsize for s in strides])
    st = HipBackend._nocopy_strides(shape, strides, new_shape)
    want = v.reshape(new_shape)  # numpy copies when it must
    if st is None:
        return None
    got = np.lib.stride_tricks.as_strided(base, new_shape, [s * itemsize for s in st])
    np.testing.assert_array_equal(got, want)
    return st


def test_nocopy_reshape_strides():
    # contiguous -> anything
    assert _view_ok((2, 3, 4), _contig((2, 3, 4)), (6, 4)) == (4, 1)
    assert _view_ok((2, 3, 4), _contig((2, 3, 4)), (2, 1, 12)) is not None
    # the encoder's split parts: [1, B, nh, L, hd] slices of a transposed qkv
    B, L, nh, hd = 2, 5, 3, 4
    qkv_strides = _contig((B, L, 3, nh, hd))
    perm = (2, 0, 3, 1, 4)
    shape = tuple((B, L, 3, nh, hd)[p] for p in perm)
    strides = tuple(qkv_strides[p] for p in perm)
    part_shape = (1,) + shape[1:]
    st = _view_ok(part_shape, strides, (B, nh, L, hd))
    assert st is not None
    # a transposed view cannot flatten its swapped axes
    assert _view_ok((4, 3), (1, 4), (12,)) is None
    # sdpa's [B,H,L,D] view of a [B,L,H,D] buffer transposes back for free
    B, H, L, D = 2, 3, 5, 4
    ostr = (L * H * D, D, H * D, 1)
    t_shape, t_str = (B, L, H, D), (ostr[0], ostr[2], ostr[1], ostr[3])
    assert _view_ok(t_shape, t_str, (B, L, H * D)) == (L * H * D, H * D, 1)


def test_broadcast_shape():
    assert _broadcast_shape((2, 3, 4), (3, 1)) == (2, 3, 4)
    assert _broadcast_shape((2, 1, 4), (2, 3, 4), (1, 3, 1)) == (2, 3, 4)
    with pytest.raises(ValueError):
        _broadcast_shape((2, 3), (4,))


def test_attention_masks_match_oracle_and_fixture():
    full = arr(case("sdpa/full_attention")["inputs"][3])
    sliding = arr(case("sdpa/sliding_attention")["inputs"][3])
    B, L = full.shape[0], full.shape[3]
    f, s = attentionMasks(full.reshape(B, L), B, L, 16)
    np.testing.assert_array_equal(f.data, full)
    np.testing.assert_array_equal(s.data, sliding)
    rng = np.random.default_rng(0)
    valid = np.zeros((3, 70), np.uint8)
    for b, n in enumerate([70, 33, 1]):
        valid[b, :n] = 1
    f2, s2 = attentionMasks(valid, 3, 70, 128)
    of, os_ = cr.attention_masks(valid, 3, 70, 128)
    np.testing.assert_array_equal(f2.data, of)
    np.testing.assert_array_equal(s2.data, os_)


def test_pack_unpack_roundtrip_and_layout():
    rng = np.random.default_rng(1)
    for bits, mode, lo, hi in [(8, "symmetric", -128, 127), (8, "affine", 0, 255), (4, "symmetric", -8, 7),
                               (4, "affine", 0, 15)]:
        q = rng.integers(lo, hi + 1, (6, 64))
        data = pack_quantized(q, bits)
        h = HostQuantized((6, 64), bits, 32, mode, data, HostTensor("f32", (6, 2), np.ones((6, 2), np.float32)),
                          HostTensor("f32", (6, 2), np.zeros((6, 2), np.float32)) if mode == "affine" else None)
        validate_quantized(h)
        np.testing.assert_array_equal(unpack_quantized(h).reshape(6, 64), q)
    # even column in the low nibble (index.ts:101-105)
    assert list(pack_quantized([1, 2, 15, 0], 4)) == [0x21, 0x0F]


def test_validate_quantized_errors():
    s = HostTensor("f32", (4, 1), np.ones((4, 1), np.float32))
    with pytest.raises(ValueError, match="multiple of 32"):
        validate_quantized(HostQuantized((4, 6), 4, 64, "affine", np.zeros(12, np.uint8), s, s))
    with pytest.raises(ValueError, match="missing biases"):
        validate_quantized(HostQuantized((4, 64), 8, 64, "affine", np.zeros(256, np.uint8), s, None))
    with pytest.raises(ValueError, match="takes no biases"):
        validate_quantized(HostQuantized((4, 64), 8, 64, "symmetric", np.zeros(256, np.uint8), s, s))
    with pytest.raises(ValueError, match="data has"):
        validate_quantized(HostQuantized((4, 64), 8, 64, "symmetric", np.zeros(10, np.uint8), s, None))


def test_parse_config_matches_fixture():
    cfgj, _, act = tiny()
    c = parseModernBertConfig(cfgj)
    assert list(c.layerTypes) == act["layer_types"]
    assert c.headDim == 32 and c.normEps == 1e-5 and not c.normBias
    assert c.ropeBase == {"full_attention": 160000.0, "sliding_attention": 10000.0}
    r = parseModernBertConfig({**cfgj, "global_rope_theta": 1, "rope_parameters": {
        "full_attention": {"rope_theta": 5, "rope_type": "default"}, "sliding_attention": {"rope_theta": 7}}})
    assert r.ropeBase == {"full_attention": 5.0, "sliding_attention": 7.0}
    with pytest.raises(ValueError, match="Unsupported encoder"):
        parseModernBertConfig({**cfgj, "model_type": "bert"})
    with pytest.raises(ValueError, match="activation"):
        parseModernBertConfig({**cfgj, "hidden_activation": "silu"})
    with pytest.raises(ValueError, match="head dimension"):
        parseModernBertConfig({**cfgj, "num_attention_heads": 3})
    with pytest.raises(ValueError, match="layer_types"):
        parseModernBertConfig({**cfgj, "layer_types": ["full_attention"]})
    with pytest.raises(ValueError, match="RoPE"):
        parseModernBertConfig({**cfgj, "rope_parameters": {"full_attention": {"rope_type": "yarn"}}})


def test_block_size_classes_match_the_library_rule():
    """HipBackend keeps disposed blocks by the library pool's size class
    (runtime.hip, size_class): 256-byte steps up to 64 KiB, then steps of a
    sixteenth of the next power of two."""
    sc = HipBackend._size_class
    assert [sc(n) for n in (0, 1, 255, 256, 257, 65536)] == [256, 256, 256, 256, 512, 65536]
    assert sc(65537) == 65536 + 8192  # next power 131072, step 8192
    assert sc(100_000) == 106496  # 13 * 8192
    assert sc(1 << 20) == 1 << 20
    assert sc((1 << 20) + 1) == (1 << 20) + (1 << 17)  # next power 2 MiB, step 128 KiB
    for n in (1, 300, 4096, 70_000, 3_000_000, 123_456_789):
        c = sc(n)
        assert c >= n and sc(c) == c  # a class is its own class
