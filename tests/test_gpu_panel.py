"""Panel-order activations (laya_hip.h, HB_X_PANEL / HB_Y_PANEL): the layout,
and bit identity of every panel-order path with its row-major twin.

The encoder writes a LayerNorm output and the fused GeGLU output in panel
order when a large-M linear layer consumes them (M >= 4096), so the GEMM
reads one 1 KB block per load.  Only the addressing changes: the LayerNorm,
the GEMM and its epilogues must give the same bits as with row-major
operands, for f16 and bf16, plain, GeGLU, residual and quantized weights,
with ragged M (padding rows in the last block, partial 256-row tiles).
The values themselves are checked against the oracle by the linear and
encoder tests; the batch-independence test of the encoder compares a B = 32
forward (panel order) with B = 1 (row-major) bit for bit."""
import numpy as np
import pytest

from gpu_util import read32, rounded, to_host
from laya_hip import ffi as F
from laya_hip.backend import _PanelRows
from laya_hip.host import HostQuantized, HostTensor, pack_quantized
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _bits(b, t) -> np.ndarray:
    return np.asarray(b.read(t).data).view(np.uint16)


def _panel_ref(a: np.ndarray) -> np.ndarray:
    """The documented layout: block (i, j) of 32 x 16 at (i * K/16 + j) * 512,
    chunk 32*h + r = row 32i + r, columns 16j + 8h .. +7; padding rows 0."""
    M, K = a.shape
    Mp = (M + 31) // 32 * 32
    p = np.zeros((Mp, K), a.dtype)
    p[:M] = a
    return p.reshape(Mp // 32, 32, K // 16, 2, 8).transpose(0, 2, 3, 1, 4).reshape(-1)


@pytest.mark.parametrize("M,K", [(100, 48), (4100, 768), (32, 16)])
def test_pack_unpack_layout(b, M, K):
    rng = np.random.default_rng(M)
    a = rng.standard_normal((M, K)).astype(np.float16)
    X = b.fromHost(HostTensor("f16", (M, K), a))
    Mp = (M + 31) // 32 * 32
    P = b._new((Mp * K,), "f16")
    b._call("pack", "hb_panel_pack", b.ctx, b._ptr(X), K, P._st.ptr, M, K)
    np.testing.assert_array_equal(_bits(b, P), _panel_ref(a).view(np.uint16))
    Y = b._new((M, K), "f16")
    b._call("unpack", "hb_panel_unpack", b.ctx, P._st.ptr, Y._st.ptr, K, M, K)
    np.testing.assert_array_equal(_bits(b, Y), a.view(np.uint16))
    for t in (X, P, Y):
        b.dispose(t)


def test_panel_entry_points_reject_unsupported_calls(b):
    X = b.fromHost(HostTensor("f16", (64, 40), np.zeros((64, 40), np.float16)))
    P = b._new((64 * 48,), "f16")
    with pytest.raises(RuntimeError, match="K % 16"):
        b._call("pack", "hb_panel_pack", b.ctx, b._ptr(X), 40, P._st.ptr, 64, 40)
    W = b.fromHost(HostTensor("f16", (64, 40), np.zeros((64, 40), np.float16)))
    Y = b._new((64, 64), "f16")
    # panel-order operands only on the large-M kernel (checked before any launch)
    with pytest.raises(RuntimeError, match="panel-order operands need"):
        b._call("linear", "hb_linear", b.ctx, F.HB_F16, b._ptr(X), 40, b._ptr(W), 0, 0, 0, Y._st.ptr, 64, 64, 64,
                40, F.HB_X_PANEL)
    for t in (X, P, W, Y):
        b.dispose(t)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("pdt", [None, "same", "f32"])
@pytest.mark.parametrize("D", [768, 256, 1024, 2048])
def test_layernorm_panel_bits(b, dtype, pdt, D):
    """Panel-order LayerNorm = row-major LayerNorm bit for bit, for row widths
    of every register-group count the kernel is built for (D / 256 = 1, 3, 4,
    8) and a last 8-row block that is only half full (M = 4100)."""
    M = 4100
    rng = np.random.default_rng(3)
    x = rounded(rng.standard_normal((M, D)) * 2 + 0.5, dtype)
    X = b.fromHost(to_host(x, dtype))
    Wt = Bt = None
    if pdt is not None:
        wd = dtype if pdt == "same" else "f32"
        Wt = b.fromHost(to_host(rounded(1 + 0.1 * rng.standard_normal(D), wd), wd))
        Bt = b.fromHost(to_host(rounded(0.1 * rng.standard_normal(D), wd), wd))
    ref = _bits(b, b._ready(b.layerNorm(X, Wt, Bt, 1e-5)))
    h = b.layerNorm(X, Wt, Bt, 1e-5)
    pan = b._as_panel(h)
    assert isinstance(pan, _PanelRows)
    raw = np.empty(((M + 31) // 32 * 32) * D, np.uint16)
    b._call("read", "hb_download", b.ctx, raw.ctypes.data, pan.st.ptr, raw.nbytes)
    want = _panel_ref(ref.reshape(M, D))
    np.testing.assert_array_equal(raw, want)  # padding rows are zeros
    np.testing.assert_array_equal(_bits(b, h), ref)  # row-major again on read (the LayerNorm re-run)


def _chain(b, X, g, Wqkv, Wi, Wo, R, dtype, materialize):
    """LN -> Wqkv; LN -> Wi + GeGLU -> Wo + residual, as in one encoder layer."""
    def ln():
        h = b.layerNorm(X, g, None, 1e-5)
        return b._ready(h) if materialize else h
    h1 = ln()
    qkv = b.linear(h1, Wqkv)
    if not materialize:
        assert isinstance(h1._lazy, _PanelRows)
    m = b.geglu(b.linear(ln(), Wi))
    if materialize:
        m = b._ready(m)
    out = b.add(R, b.linear(m, Wo))
    if not materialize:
        assert isinstance(m._lazy, _PanelRows)
    return _bits(b, qkv), _bits(b, out), _bits(b, m)  # m: a panel-order GeGLU output is unpacked on read


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("M", [4160, 8192])
def test_panel_gemm_chain_bits(b, dtype, M):
    H, I = 768, 1152
    rng = np.random.default_rng(M + (dtype == "bf16"))
    up = lambda a: b.fromHost(to_host(rounded(a, dtype), dtype))  # noqa: E731
    X = up(rng.standard_normal((M, H)))
    g = up(1 + 0.1 * rng.standard_normal(H))
    Wqkv, Wi, Wo = up(rng.normal(0, 0.02, (3 * H, H))), up(rng.normal(0, 0.02, (2 * I, H))), \
        up(rng.normal(0, 0.02, (H, I)))
    R = up(rng.standard_normal((M, H)))
    print(f"panel chain {dtype} M={M}", flush=True)
    fused = _chain(b, X, g, Wqkv, Wi, Wo, R, dtype, materialize=False)
    plain = _chain(b, X, g, Wqkv, Wi, Wo, R, dtype, materialize=True)
    unpacks = b.stats["panel_unpacks"]
    np.testing.assert_array_equal(fused[0], plain[0])
    np.testing.assert_array_equal(fused[1], plain[1])
    np.testing.assert_array_equal(fused[2], plain[2])
    assert unpacks > 0
    # and the values: rows of the chain against the oracle (f16 / bf16 rounding at every op)
    rows = np.sort(rng.choice(M, 64, replace=False))
    x32 = read32(b, X)[rows]
    w32 = lambda t: read32(b, t)  # noqa: E731
    h = rounded(cr.layer_norm(x32, w32(g), None, 1e-5), dtype)
    qkv = rounded(cr.linear(h, w32(Wqkv)), dtype)
    got = fused[0].reshape(M, 3 * H)[rows]
    got = got.view(np.float16).astype(np.float32) if dtype == "f16" else \
        (got.astype(np.uint32) << 16).view(np.float32)
    assert np.max(np.abs(got - qkv)) / np.max(np.abs(qkv)) <= (2e-3 if dtype == "f16" else 8e-3)
    for t in (X, g, Wqkv, Wi, Wo, R):
        b.dispose(t)


@pytest.mark.parametrize("bits", [8, 4])
def test_panel_quantized_bits(b, bits):
    from laya_hip import compose as C
    M, H, N = 4160, 768, 2304
    rng = np.random.default_rng(bits)
    w = rounded(rng.normal(0, 0.02, (N, H)), "f16")
    q, s, z = cr.quantize_matrix(w, N, H, bits, 64, refine=bits == 4)
    h = HostQuantized((N, H), bits, 64, "symmetric" if bits == 8 else "affine", pack_quantized(q, bits),
                      HostTensor("f16", s.shape, s.view(np.float16)),
                      HostTensor("f16", z.shape, z.view(np.float16)) if z is not None else None)
    Q = C.upload_quantized(b, h, "f16")
    X = b.fromHost(to_host(rounded(rng.standard_normal((M, H)), "f16"), "f16"))
    hp = b.layerNorm(X, None, None, 1e-5)
    y_pan = C.quantized_linear(b, hp, Q)
    assert isinstance(hp._lazy, _PanelRows)
    y_row = C.quantized_linear(b, b._ready(b.layerNorm(X, None, None, 1e-5)), Q)
    np.testing.assert_array_equal(_bits(b, y_pan), _bits(b, y_row))
    C.dispose_quantized(b, Q)
    b.dispose(X)


@pytest.mark.parametrize("window", [None, 128])
def test_panel_attention_output_into_wo(b, window):
    """The encoder's attention block (modernbert/src/index.ts:348-353): the
    sdpa output stays pending through transpose + reshape, attn Wo reads it
    in panel order (hb_sdpa_panel), bit for bit as with the row-major output,
    with a padding mask (global) and a sliding-window mask."""
    from laya_hip.modernbert import attentionMasks
    B, L, nh, hd = 8, 512, 12, 64
    H = nh * hd
    rng = np.random.default_rng(11)
    lens = rng.integers(64, L + 1, B)
    valid = (np.arange(L)[None, :] < lens[:, None]).astype(np.uint8)
    full, sliding = attentionMasks(valid, B, L, 128)
    mask = b.fromHost(full if window is None else sliding)
    qkv = b.fromHost(to_host(rounded(rng.standard_normal((B, L, 3 * H)), "f16"), "f16"))
    Wo = b.fromHost(to_host(rounded(rng.normal(0, 0.02, (H, H)), "f16"), "f16"))
    R = b.fromHost(to_host(rounded(rng.standard_normal((B, L, H)), "f16"), "f16"))

    def block(materialize):
        t = b.transpose(b.reshape(qkv, [B, L, 3, nh, hd]), [2, 0, 3, 1, 4])
        q, k, v = [b.reshape(x, [B, nh, L, hd]) for x in b.split(t, 3, 0)]
        att = b.sdpa(b.rope(q, 1e4), b.rope(k, 1e4), v, mask, hd ** -0.5)
        if materialize:
            b._ready(att)
        merged = b.reshape(b.transpose(att, [0, 2, 1, 3]), [B, L, H])
        y = b.add(R, b.linear(merged, Wo))
        if not materialize:
            assert isinstance(merged._lazy, _PanelRows)
        return _bits(b, y), _bits(b, att)

    pan, pan_att = block(False)
    row, row_att = block(True)
    np.testing.assert_array_equal(pan, row)
    np.testing.assert_array_equal(pan_att, row_att)  # the pending output read on its own, row-major


def test_encoder_forwards_release_every_block(b):
    """Pending layerNorm / sdpa / geglu tensors, their shared views and panel
    copies are all freed: repeated forwards of a 3-layer encoder at M = 4096
    (every panel path taken) leave the pool's live block count unchanged, and
    so does a forward whose intermediate is read half-way."""
    from laya_hip.modernbert import loadModernBert, parseModernBertConfig
    H, I, NH, V, B, T = 768, 1152, 12, 1000, 8, 512
    cfgj = {"vocab_size": V, "hidden_size": H, "intermediate_size": I, "num_hidden_layers": 3,
            "num_attention_heads": NH, "local_attention": 128}
    rng = np.random.default_rng(12)
    n = lambda *s: (rng.standard_normal(s, dtype=np.float32) * 0.02).astype(np.float16)  # noqa: E731
    W = {"embeddings.tok_embeddings.weight": n(V, H), "embeddings.norm.weight": np.ones(H, np.float16),
         "final_norm.weight": np.ones(H, np.float16)}
    for i in range(3):
        p = f"layers.{i}."
        if i:
            W[p + "attn_norm.weight"] = np.ones(H, np.float16)
        W.update({p + "attn.Wqkv.weight": n(3 * H, H), p + "attn.Wo.weight": n(H, H),
                  p + "mlp_norm.weight": np.ones(H, np.float16), p + "mlp.Wi.weight": n(2 * I, H),
                  p + "mlp.Wo.weight": n(H, I)})
    enc = loadModernBert(b, parseModernBertConfig(cfgj),
                         lambda nm: HostTensor("f16", W[nm[8:]].shape, W[nm[8:]]) if nm[8:] in W else None,
                         dtype="f16")
    lens = rng.integers(64, T + 1, B)
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    valid = (np.arange(T)[None, :] < lens[:, None]).astype(np.uint8)
    inp = enc.uploadInputs(ids, valid, B, T)
    first = _bits(b, enc.encode(inp))  # the mask summaries are built (and cached) here
    before = b.pool_stats()["live_blocks"]
    for _ in range(2):
        b.dispose(enc.encode(inp))
        assert b.pool_stats()["live_blocks"] == before
    x = b.scope(lambda: enc.embeddings(inp["ids"]))
    h = enc.layer(0, x, inp["masks"]["full_attention"])
    mid = _bits(b, h)  # an intermediate read in the middle of the pending chain
    assert np.isfinite(mid.view(np.float16).astype(np.float32)).all()
    for t in (x, h):
        b.dispose(t)
    assert b.pool_stats()["live_blocks"] == before
    np.testing.assert_array_equal(_bits(b, enc.encode(inp)), first)  # and the result is unchanged
    enc.disposeInputs(inp)
    enc.dispose()
