"""A recorded encoder forward (HipBackend.capture, hb_capture_* /
hb_graph_*): replays give the eager forward's bits.  Each replay is followed
by eager work on the same backend (an eager encode, which reuses blocks of
the pool) and a read that synchronizes; every replay is checked.  The shapes
take both GEMM kernels: the small-M one, and at M = 4096 rows the large-M one
with panel-order operands from the LayerNorm, attention and GeGLU kernels.  New token
ids, and then a new padding pattern in the attention masks, written in place
into the recorded inputs (HipBackend.write) give the eager result for those
inputs: every replay re-summarises the masks it reads.  Destroying the graph returns its blocks: the pool's live block count
comes back to where it was before the recording."""
import numpy as np
import pytest

from laya_hip import ffi as F
from laya_hip.host import HostTensor
from laya_hip.modernbert import attentionMasks, loadModernBert, parseModernBertConfig

pytestmark = pytest.mark.gpu

CFG = {"vocab_size": 1000, "hidden_size": 256, "intermediate_size": 384, "num_hidden_layers": 4,
       "num_attention_heads": 4, "local_attention": 64}


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _weights(rng):
    H, I, V = CFG["hidden_size"], CFG["intermediate_size"], CFG["vocab_size"]
    n = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float16)  # noqa: E731
    W = {"embeddings.tok_embeddings.weight": n(V, H), "embeddings.norm.weight": np.ones(H, np.float16),
         "final_norm.weight": np.ones(H, np.float16)}
    for i in range(CFG["num_hidden_layers"]):
        p = f"layers.{i}."
        if i:
            W[p + "attn_norm.weight"] = np.ones(H, np.float16)
        W[p + "attn.Wqkv.weight"] = n(3 * H, H)
        W[p + "attn.Wo.weight"] = n(H, H)
        W[p + "mlp_norm.weight"] = np.ones(H, np.float16)
        W[p + "mlp.Wi.weight"] = n(2 * I, H)
        W[p + "mlp.Wo.weight"] = n(H, I)
    return W


def _bits(b, t):
    return np.asarray(b.read(t).data).view(np.uint16).copy()


@pytest.mark.parametrize("B,T", [(1, 128), (2, 96), (8, 512)])  # M = 4096: the large-M GEMM, panel operands
def test_recorded_encoder_replays(b, B, T):
    rng = np.random.default_rng(B * 100 + T)
    W = _weights(rng)
    enc = loadModernBert(b, parseModernBertConfig(CFG),
                         lambda nm: HostTensor("f16", W[nm[8:]].shape, W[nm[8:]])
                         if nm.startswith("encoder.") and nm[8:] in W else None, dtype="f16")
    ids = rng.integers(0, CFG["vocab_size"], (B, T)).astype(np.int32)
    valid = np.ones((B, T), np.uint8)
    valid[-1, T - 17:] = 0  # a padded tail in the last sequence
    inp = enc.uploadInputs(ids, valid, B, T)

    def eager():
        y = enc.encode(inp)
        out = _bits(b, y)
        b.dispose(y)
        return out

    want = eager()
    blocks0 = b.pool_stats()["live_blocks"]
    g = b.capture(lambda: enc.encode(inp))
    for _ in range(3):
        got = _bits(b, g.run())
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(eager(), want)  # eager work between replays
    # new ids, written in place into the recorded input
    ids2 = rng.integers(0, CFG["vocab_size"], (B, T)).astype(np.int32)
    b.write(inp["ids"], HostTensor("i32", (B, T), ids2))
    got2 = _bits(b, g.run())
    want2 = eager()
    np.testing.assert_array_equal(got2, want2)
    assert not np.array_equal(want2, want)
    # a new padding pattern, written in place into the recorded masks: the
    # replay summarises the new masks (tiles that were hidden are now seen
    # and the other way round), as does the eager forward after the write
    valid3 = np.ones((B, T), np.uint8)
    valid3[0, T // 2 + 3:] = 0
    if B > 1:
        valid3[-1, :] = 1
    full3, sliding3 = attentionMasks(valid3, B, T, CFG["local_attention"])
    b.write(inp["masks"]["full_attention"], full3)
    b.write(inp["masks"]["sliding_attention"], sliding3)
    b.write(inp["mask"], HostTensor("bool", (B, T), valid3))
    got3 = _bits(b, g.run())
    want3 = eager()
    np.testing.assert_array_equal(got3, want3)
    fresh = enc.uploadInputs(ids2, valid3, B, T)
    y = enc.encode(fresh)
    np.testing.assert_array_equal(_bits(b, y), want3)
    b.dispose(y)
    enc.disposeInputs(fresh)
    assert not np.array_equal(want3, want2)
    np.testing.assert_array_equal(_bits(b, g.run()), want3)  # replays again after eager work
    out = g.out
    g.destroy()
    b.dispose(out)  # the recorded output belongs to the caller
    assert b.pool_stats()["live_blocks"] == blocks0
    enc.disposeInputs(inp)
    enc.dispose()


def test_recorded_quantized_linear_replays(b):
    """A quantized linear at M = 4096 rows (its weight dequantized once per
    call into a 16-bit copy from the pool, then the large-M GEMM), recorded
    and replayed: every replay gives the eager bits, also after x is
    rewritten in place; the copy's block stays with the graph and returns to
    the pool when the graph is destroyed."""
    from laya_hip import compose as C
    from laya_hip.host import HostQuantized, pack_quantized
    from oracle import cpu_ref as cr
    rng = np.random.default_rng(9)
    N, K, M = 768, 768, 4096
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    q, s, z = cr.quantize_matrix(w, N, K, 4, 64, refine=False)
    h = HostQuantized((N, K), 4, 64, "affine", pack_quantized(q, 4), HostTensor("f16", s.shape, s.view(np.float16)),
                      HostTensor("f16", z.shape, z.view(np.float16)))
    Q = C.upload_quantized(b, h, "f16")
    X = b.fromHost(HostTensor("f16", (M, K), rng.standard_normal((M, K)).astype(np.float16)))

    def eager():
        y = C.quantized_linear(b, X, Q)
        out = _bits(b, y)
        b.dispose(y)
        return out

    want = eager()
    blocks0 = b.pool_stats()["live_blocks"]
    g = b.capture(lambda: C.quantized_linear(b, X, Q))
    for _ in range(3):
        np.testing.assert_array_equal(_bits(b, g.run()), want)
        np.testing.assert_array_equal(eager(), want)  # eager work between replays
    b.write(X, HostTensor("f16", (M, K), rng.standard_normal((M, K)).astype(np.float16)))
    got2 = _bits(b, g.run())
    want2 = eager()
    np.testing.assert_array_equal(got2, want2)
    assert not np.array_equal(want2, want)
    out = g.out
    g.destroy()
    b.dispose(out)
    assert b.pool_stats()["live_blocks"] == blocks0
    C.dispose_quantized(b, Q)
    b.dispose(X)


def test_recording_refuses_synchronizing_calls(b):
    """A read inside a recording is refused with a clear error (the host-side
    check runs before the stream is touched); the recording is dropped and
    the backend keeps working eagerly."""
    x = b.fromHost(HostTensor("f32", (4, 64), np.ones((4, 64), np.float32)))

    def bad():
        y = b.scale(x, 2.0)
        b.read(y)
        return y

    with pytest.raises(F.HipError, match="recording a graph"):
        b.capture(bad, warmup=False)
    assert b._capture_held is None
    y = b.scale(x, 3.0)
    np.testing.assert_array_equal(np.asarray(b.read(y).data).reshape(4, 64), np.full((4, 64), 3.0, np.float32))
    for t in (x, y):
        b.dispose(t)


def test_summary_recorded_without_warmup_is_rebuilt_eagerly(b):
    """Mask summaries first enqueued inside a recording (capture with
    warmup=False, and a recording that raises part-way) are written only by a
    replay: an eager forward on the same masks afterwards rebuilds them and
    gives the bits of a forward on a fresh upload of the same inputs."""
    B, T = 2, 256
    rng = np.random.default_rng(77)
    W = _weights(rng)
    enc = loadModernBert(b, parseModernBertConfig(CFG),
                         lambda nm: HostTensor("f16", W[nm[8:]].shape, W[nm[8:]])
                         if nm.startswith("encoder.") and nm[8:] in W else None, dtype="f16")
    ids = rng.integers(0, CFG["vocab_size"], (B, T)).astype(np.int32)
    valid = np.ones((B, T), np.uint8)
    valid[0, 150:] = 0
    valid[1, 40:] = 0

    def run(inp):
        y = enc.encode(inp)
        out = _bits(b, y)
        b.dispose(y)
        return out

    ref_inp = enc.uploadInputs(ids, valid, B, T)
    want = run(ref_inp)  # also sets up the RoPE tables outside any recording
    enc.disposeInputs(ref_inp)

    inp = enc.uploadInputs(ids, valid, B, T)
    g = b.capture(lambda: enc.encode(inp), warmup=False)
    np.testing.assert_array_equal(run(inp), want)  # eager, before any replay
    np.testing.assert_array_equal(_bits(b, g.run()), want)
    out = g.out
    g.destroy()
    b.dispose(out)
    enc.disposeInputs(inp)

    inp2 = enc.uploadInputs(ids, valid, B, T)

    def aborts():
        enc.encode(inp2)
        raise KeyError("abort the recording")

    with pytest.raises(KeyError):
        b.capture(aborts, warmup=False)
    np.testing.assert_array_equal(run(inp2), want)
    enc.disposeInputs(inp2)
    enc.dispose()
