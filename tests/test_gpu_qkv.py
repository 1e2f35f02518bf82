"""The attention block's q / k / v projection fused with its layout glue and
RoPE (hb_linear_qkv), on the GPU.

- Through the C ABI: the head-major [3, B, H, L, 64] output equals, bit for
  bit, what the separate ops store -- hb_linear's row-major product, viewed
  as modernbert/src/index.ts:348-350 views it, then hb_rope on q and k --
  for f16 and bf16, with x row-major and in panel order, on the config-3
  shape and on a ragged one (L not a multiple of the 256-row tile, so tiles
  span sequences); and the product is within the GEMM tolerance of the CPU
  oracle.  Calls it cannot take (a bias, M below the large-M kernel's range,
  M not a multiple of L, f32) are refused.
- Through the Backend contract (HipBackend(fuse_qkv=True)): an attention
  block called as ModernBert.layer calls it takes the fused launch, and its
  sdpa output equals bit for bit the one computed from separately roped
  operands; a full-depth encoder forward with the fused projection equals
  the default one bit for bit.
"""
import numpy as np
import pytest

from gpu_util import max_rel, read32, rounded, to_host
from laya_hip import ffi as F
from laya_hip.modernbert import attentionMasks
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0, fuse_qkv=True)
    yield be
    be.destroy()


def _bits(b, ptr, n):
    out = np.empty(n, np.uint16)
    b.n.call("read", "hb_download", b.ctx, out.ctypes.data, ptr, out.nbytes)
    return out


def _separate(b, Y, B, L, H, base, dtype):
    """[3, B, H, L, 64] bits from the separate ops: the row-major product
    viewed per head, then hb_rope on q and k."""
    qkv = b.transpose(b.reshape(Y, [B, L, 3, H, 64]), [2, 0, 3, 1, 4])
    parts = [b.reshape(t, [B, H, L, 64]) for t in b.split(qkv, 3, 0)]
    outs = []
    for i, t in enumerate(parts):
        r = b.rope(t, base) if i < 2 else t
        h = b.read(r)
        outs.append(np.asarray(h.data).view(np.uint16).reshape(B, H, L, 64))
        if r is not t:
            b.dispose(r)
    for t in parts + [qkv]:
        b.dispose(t)
    return np.stack(outs)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("B,L,H,K,panel", [(32, 512, 12, 768, False),  # config 3's Wqkv
                                           (32, 130, 4, 128, False),   # ragged: tiles span sequences
                                           (16, 320, 12, 768, True)])  # x in panel order
def test_linear_qkv_equals_separate_ops(b, dtype, B, L, H, K, panel):
    print(f"hb_linear_qkv B={B} L={L} H={H} K={K} panel={panel} {dtype}", flush=True)
    rng = np.random.default_rng(B * L + H + K)
    M, N = B * L, 3 * H * 64
    base = 160000.0
    x = rounded(rng.standard_normal((M, K)), dtype)
    w = rounded(rng.normal(0, 0.02, (N, K)), dtype)
    X, W = b.fromHost(to_host(x, dtype)), b.fromHost(to_host(w, dtype))
    dt = F.HB_F16 if dtype == "f16" else F.HB_BF16
    # the separate ops: row-major product (realized by reading it), views, rope
    Y = b.linear(X, W)
    y = read32(b, Y)
    want = _separate(b, Y, B, L, H, base, dtype)
    # the fused entry point, x row-major or packed in panel order
    out = b._malloc(M * N * 2)
    xp, flags, packed = b._ptr(X), 0, None
    if panel:
        packed = b._malloc((M + 31) // 32 * 32 * K * 2)
        b.n.call("pack", "hb_panel_pack", b.ctx, xp, K, packed.ptr, M, K)
        xp, flags = packed.ptr, flags | F.HB_X_PANEL
    b.n.call("linear", "hb_linear_qkv", b.ctx, dt, xp, K, b._ptr(W), 0, out.ptr, M, K, L, H, base, flags)
    got = _bits(b, out.ptr, 3 * M * H * 64).reshape(3, B, H, L, 64)
    np.testing.assert_array_equal(got, want)
    # the product itself against the oracle (rows are independent: a sample)
    rows = np.sort(rng.choice(M, 256, replace=False))
    ref = cr.linear(x[rows], w)
    assert max_rel(y[rows], ref) <= (2e-3 if dtype == "f16" else 8e-3)
    for t in (X, W, Y):
        b.dispose(t)
    out.release()
    if packed is not None:
        packed.release()


def test_linear_qkv_rejects_what_it_cannot_take(b):
    x = b._malloc(4096 * 64 * 2)
    with pytest.raises(F.HipError, match="multiple of L"):
        b.n.call("linear", "hb_linear_qkv", b.ctx, F.HB_F16, x.ptr, 64, x.ptr, 0, x.ptr, 4096, 64, 1000, 1, 1e4, 0)
    with pytest.raises(F.HipError, match="M >= 4096"):
        b.n.call("linear", "hb_linear_qkv", b.ctx, F.HB_F16, x.ptr, 64, x.ptr, 0, x.ptr, 2048, 64, 512, 1, 1e4, 0)
    with pytest.raises(F.HipError, match="f16 or bf16"):
        b.n.call("linear", "hb_linear_qkv", b.ctx, F.HB_F32, x.ptr, 64, x.ptr, 0, x.ptr, 4096, 64, 512, 1, 1e4, 0)
    with pytest.raises(F.HipError, match="no bias"):
        b.n.call("linear", "hb_linear_qkv", b.ctx, F.HB_F16, x.ptr, 64, x.ptr, x.ptr, x.ptr, 4096, 64, 512, 1, 1e4,
                 F.HB_EPI_BIAS)
    x.release()


@pytest.mark.parametrize("kind", ["full_attention", "sliding_attention"])
def test_attention_block_takes_the_fused_projection(b, kind):
    """linear -> reshape -> transpose -> split -> rope -> sdpa, as
    modernbert/src/index.ts:348-352 calls them, launches hb_linear_qkv and
    gives the sdpa output of separately roped operands, bit for bit."""
    print(f"fused attention block {kind}", flush=True)
    rng = np.random.default_rng(7)
    B, L, H, K = 16, 512, 12, 768
    base = 160000.0 if kind == "full_attention" else 10000.0
    lens = rng.integers(64, L + 1, B)
    valid = (np.arange(L)[None, :] < lens[:, None]).astype(np.uint8)
    full, sliding = attentionMasks(valid, B, L, 128)
    mask = b.fromHost(full if kind == "full_attention" else sliding)
    x = rounded(rng.standard_normal((B, L, K)), "f16")
    w = rounded(rng.normal(0, 0.02, (3 * H * 64, K)), "f16")
    X, W = b.fromHost(to_host(x, "f16")), b.fromHost(to_host(w, "f16"))

    def views(Y):
        qkv = b.transpose(b.reshape(Y, [B, L, 3, H, 64]), [2, 0, 3, 1, 4])
        return [b.reshape(t, [B, H, L, 64]) for t in b.split(qkv, 3, 0)]

    before = b.stats["linear_fused_qkv"]
    q, k, v = views(b.linear(X, W))
    got = read32(b, b.sdpa(b.rope(q, base), b.rope(k, base), v, mask, 0.125))
    assert b.stats["linear_fused_qkv"] == before + 1
    # the same block from separately launched, separately roped operands
    q2, k2, v2 = views(b.linear(X, W))
    qr, kr = b.rope(q2, base), b.rope(k2, base)
    b.read(qr), b.read(kr)  # launches the product row-major and hb_rope on q and k
    want = read32(b, b.sdpa(qr, kr, v2, mask, 0.125))
    assert b.stats["linear_fused_qkv"] == before + 1
    np.testing.assert_array_equal(got, want)
    assert np.isfinite(got).all()


def test_encoder_with_the_fused_projection_equals_the_default(b):
    """A 4-layer ModernBERT-base-shape forward (B = 16, T = 512, ragged
    lengths) with the fused q / k / v projection gives the default forward's
    bits (RoPE inside sdpa)."""
    from laya_hip.backend import HipBackend
    from laya_hip.host import HostTensor
    from laya_hip.modernbert import loadModernBert, parseModernBertConfig
    print("encoder fused vs default", flush=True)
    cfgj = {"vocab_size": 1000, "hidden_size": 768, "intermediate_size": 1152, "num_hidden_layers": 4,
            "num_attention_heads": 12, "local_attention": 128}
    rng = np.random.default_rng(11)
    W = {"embeddings.tok_embeddings.weight": rng.normal(0, 0.02, (1000, 768)),
         "embeddings.norm.weight": np.ones(768), "final_norm.weight": np.ones(768)}
    for i in range(4):
        p = f"layers.{i}."
        if i:
            W[p + "attn_norm.weight"] = np.ones(768)
        W[p + "attn.Wqkv.weight"] = rng.normal(0, 0.02, (2304, 768))
        W[p + "attn.Wo.weight"] = rng.normal(0, 0.02, (768, 768))
        W[p + "mlp_norm.weight"] = np.ones(768)
        W[p + "mlp.Wi.weight"] = rng.normal(0, 0.02, (2304, 768))
        W[p + "mlp.Wo.weight"] = rng.normal(0, 0.02, (768, 1152))
    W = {k: np.asarray(v, np.float16) for k, v in W.items()}
    B, T = 16, 512
    ids = rng.integers(0, 1000, (B, T)).astype(np.int32)
    valid = (np.arange(T)[None, :] < rng.integers(64, T + 1, B)[:, None]).astype(np.uint8)
    cfg = parseModernBertConfig(cfgj)

    def run(be):
        enc = loadModernBert(be, cfg, lambda n: HostTensor("f16", W[n[8:]].shape, W[n[8:]])
                             if n.startswith("encoder.") and n[8:] in W else None, dtype="f16")
        out = np.asarray(be.read(enc.forward(ids, valid, B, T)).data).view(np.uint16).copy()
        enc.dispose()
        return out

    before = b.stats["linear_fused_qkv"]
    fused = run(b)
    assert b.stats["linear_fused_qkv"] == before + 4
    plain_be = HipBackend(0)
    try:
        plain = run(plain_be)
        assert plain_be.stats["linear_fused_qkv"] == 0 and plain_be.stats["sdpa_fused_rope"] == 4
    finally:
        plain_be.destroy()
    np.testing.assert_array_equal(fused, plain)
