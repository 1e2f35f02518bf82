"""Bandwidth-kernel and attention parity on the GPU at the BASELINE config-3
shapes (B=32, T=512, H=768, 12 heads of 64): LayerNorm, RoPE, GeGLU and SDPA
(global and sliding-window masks, padded batches) against the CPU oracle.
SDPA is checked on a subset of (batch, head) pairs, which are independent."""
import numpy as np
import pytest

from gpu_util import max_rel, read32, rounded, to_host
from laya_hip.host import HostTensor
from laya_hip.modernbert import attentionMasks
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_layernorm_config3(b, dtype):
    rng = np.random.default_rng(1)
    x = rounded(rng.standard_normal((16384, 768)) * 2 + 0.5, dtype)
    w = rounded(rng.uniform(0.5, 1.5, 768), dtype)
    X, Wt = b.fromHost(to_host(x, dtype)), b.fromHost(to_host(w, dtype))
    got = read32(b, b.layerNorm(X, Wt, None, 1e-5))
    ref = cr.layer_norm(x, w, None, 1e-5)
    assert max_rel(got, ref) <= (2e-3 if dtype == "f16" else 8e-3)
    # generic-width path (D not a multiple of 256)
    x2 = rounded(rng.standard_normal((100, 96)), dtype)
    got2 = read32(b, b.layerNorm(b.fromHost(to_host(x2, dtype)), None, None, 1e-5))
    assert max_rel(got2, cr.layer_norm(x2, None, None, 1e-5)) <= (2e-3 if dtype == "f16" else 8e-3)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rope_and_geglu_config3(b, dtype):
    rng = np.random.default_rng(2)
    x = rounded(rng.standard_normal((32, 12, 512, 64)), dtype)
    X = b.fromHost(to_host(x, dtype))
    for base in (10000.0, 160000.0):
        got = read32(b, b.rope(X, base))
        assert max_rel(got, cr.rope(x, base)) <= (2e-3 if dtype == "f16" else 8e-3)
    m = rounded(rng.standard_normal((16384, 2304)), dtype)
    got = read32(b, b.geglu(b.fromHost(to_host(m, dtype))))
    assert max_rel(got, cr.geglu(m)) <= (2e-3 if dtype == "f16" else 8e-3)


def _qkv_views(b, qkv_dev, B, L, nh, hd):
    qkv = b.transpose(b.reshape(qkv_dev, [B, L, 3, nh, hd]), [2, 0, 3, 1, 4])
    return [b.reshape(t, [B, nh, L, hd]) for t in b.split(qkv, 3, 0)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("kind", ["full_attention", "sliding_attention"])
def test_sdpa_encoder_layout_config3(b, kind, dtype):
    """sdpa(rope(q), rope(k), v) on strided q/k/v views of a [B, L, 3*H]
    projection, as ModernBert.layer calls it (modernbert/src/index.ts:348-352)."""
    print(f"sdpa {kind} {dtype}", flush=True)
    rng = np.random.default_rng(3)
    B, L, nh, hd = 32, 512, 12, 64
    lens = rng.integers(64, 513, B)
    lens[0] = 512
    valid = (np.arange(L)[None, :] < lens[:, None]).astype(np.uint8)
    full, sliding = attentionMasks(valid, B, L, 128)
    mask_h = full if kind == "full_attention" else sliding
    base = 160000.0 if kind == "full_attention" else 10000.0
    qkv = rounded(rng.standard_normal((B, L, 3 * nh * hd)), dtype)
    dev = b.fromHost(to_host(qkv, dtype))
    mask = b.fromHost(mask_h)
    q, k, v = _qkv_views(b, dev, B, L, nh, hd)
    att = b.sdpa(b.rope(q, base), b.rope(k, base), v, mask, hd ** -0.5)
    got = read32(b, att)  # [B, nh, L, hd]; the launch happens here, on first use
    assert b.stats["sdpa_fused_rope"] > 0
    t = qkv.reshape(B, L, 3, nh, hd).transpose(2, 0, 3, 1, 4)
    tol = 5e-3 if dtype == "f16" else 2e-2
    for bb, hh in [(0, 0), (1, 5), (7, 11), (31, 3), (int(np.argmin(lens)), 7)]:
        qs, ks, vs = (np.ascontiguousarray(t[i][bb:bb + 1, hh:hh + 1]) for i in range(3))
        rq = rounded(cr.rope(qs, base), dtype)
        rk = rounded(cr.rope(ks, base), dtype)
        ref = cr.sdpa(rq, rk, vs, mask_h.data[bb:bb + 1], hd ** -0.5)
        err = max_rel(got[bb:bb + 1, hh:hh + 1], ref)
        assert err <= tol, f"(b={bb}, h={hh}, len={lens[bb]}): max-rel {err:.2e}"


@pytest.mark.parametrize("kind", ["full_attention", "sliding_attention"])
def test_sdpa_at_the_maximum_sequence_length(b, kind):
    """One sequence of ModernBERT's max_position_embeddings (8192) tokens with
    a padded tail, through the encoder's call (rope(q), rope(k), strided views
    of one projection).  Query rows are independent, so the oracle runs on a
    sample of them: both ends of a 128-query tile, the middle of the
    sequence, the last valid query and padded queries (which attend to every
    valid key under the sliding mask)."""
    print(f"sdpa L=8192 {kind}", flush=True)
    rng = np.random.default_rng(6)
    B, L, nh, hd, n_valid = 1, 8192, 12, 64, 7192
    valid = (np.arange(L)[None, :] < n_valid).astype(np.uint8)
    full, sliding = attentionMasks(valid, B, L, 128)
    mask_h = full if kind == "full_attention" else sliding
    base = 160000.0 if kind == "full_attention" else 10000.0
    qkv = rounded(rng.standard_normal((B, L, 3 * nh * hd)), "f16")
    dev = b.fromHost(to_host(qkv, "f16"))
    mask = b.fromHost(mask_h)
    q, k, v = _qkv_views(b, dev, B, L, nh, hd)
    got = read32(b, b.sdpa(b.rope(q, base), b.rope(k, base), v, mask, hd ** -0.5))
    sel = np.array([0, 1, 127, 128, 4095, 4096, 7000, n_valid - 1, n_valid, L - 1])
    t = qkv.reshape(B, L, 3, nh, hd).transpose(2, 0, 3, 1, 4)
    for hh in (0, 11):
        qs, ks, vs = (np.ascontiguousarray(t[i][:, hh:hh + 1]) for i in range(3))
        rq = rounded(cr.rope(qs, base), "f16")[:, :, sel]
        rk = rounded(cr.rope(ks, base), "f16")
        m = mask_h.data if kind == "full_attention" else mask_h.data[:, :, sel]
        ref = cr.sdpa(rq, rk, vs, m, hd ** -0.5)
        err = max_rel(got[:, hh:hh + 1, sel], ref)
        assert err <= 5e-3, f"(h={hh}): max-rel {err:.2e}"
    for x in (dev, mask):
        b.dispose(x)


def test_sdpa_fused_rope_is_bit_identical_to_separate_rope(b):
    rng = np.random.default_rng(4)
    B, L, nh, hd = 2, 300, 12, 64
    qkv = rounded(rng.standard_normal((B, L, 3 * nh * hd)), "f16")
    valid = np.ones((B, L), np.uint8)
    valid[1, 200:] = 0
    full, sliding = attentionMasks(valid, B, L, 128)
    dev = b.fromHost(to_host(qkv, "f16"))
    mask = b.fromHost(sliding)
    q, k, v = _qkv_views(b, dev, B, L, nh, hd)
    fused = b.read(b.sdpa(b.rope(q, 10000.0), b.rope(k, 10000.0), v, mask, 0.125)).data
    rq = b.fromHost(b.read(b.rope(q, 10000.0)))  # materialised rotation, re-uploaded
    rk = b.fromHost(b.read(b.rope(k, 10000.0)))
    plain = b.read(b.sdpa(rq, rk, v, mask, 0.125)).data
    np.testing.assert_array_equal(fused.view(np.uint16), plain.view(np.uint16))


def test_sdpa_generic_path_matches_oracle(b):
    """f32 and head dims other than 64 take the generic kernel."""
    rng = np.random.default_rng(5)
    for (B, H, L, D) in [(2, 3, 40, 16), (1, 2, 100, 32), (2, 2, 70, 128)]:
        q, k, v = (rng.standard_normal((B, H, L, D)).astype(np.float32) for _ in range(3))
        valid = np.ones((B, L), np.uint8)
        valid[-1, L // 2:] = 0
        _, sliding = attentionMasks(valid, B, L, 16)
        dev = [b.fromHost(to_host(a, "f32")) for a in (q, k, v)]
        got = read32(b, b.sdpa(b.rope(dev[0], 10000.0), dev[1], dev[2], b.fromHost(sliding), 0.25))
        ref = cr.sdpa(cr.rope(q, 10000.0), k, v, sliding.data, 0.25)
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_sdpa_negative_key_and_value_row_strides(b):
    """hb_sdpa through the C ABI with K and V given as row-reversed views (the
    base pointer at their last row, row stride -64 elements), otherwise
    meeting every condition of the MFMA kernel: the call takes the generic
    kernel, which addresses negative strides, and matches the oracle on the
    reversed keys and values.  Also a masked call."""
    from laya_hip import ffi as F
    rng = np.random.default_rng(12)
    B, H, L, D = 2, 3, 192, 64
    valid = np.ones((B, L), np.uint8)
    valid[1, 130:] = 0
    full, sliding = attentionMasks(valid, B, L, 128)
    x = [rounded(rng.standard_normal((B, H, L, D)), "f16") for _ in range(3)]
    q, k, v = (b.fromHost(to_host(a, "f16")) for a in x)
    out = b._malloc(B * H * L * D * 2)
    for mh in (None, sliding):
        m = None if mh is None else b.fromHost(mh)
        print(f"sdpa negative strides mask={mh is not None}", flush=True)
        st = F.i64s((H * L * D, L * D, D, 1))
        rev = F.i64s((H * L * D, L * D, -D, 1))
        last = (L - 1) * D * 2  # bytes to the last row of a (b, h) block
        mp, ms = (0, None) if m is None else (b._ptr(m), F.i64s((L * L, 0, L, 1)))
        b.n.call("sdpa", "hb_sdpa", b.ctx, F.HB_F16, b._ptr(q), st, b._ptr(k) + last, rev, b._ptr(v) + last, rev,
                 mp, ms, 0, out.ptr, st, B, H, L, L, D, 0.125, 0.0, 0.0)
        got = np.empty(B * H * L * D, np.uint16)
        b.n.call("read", "hb_download", b.ctx, got.ctypes.data, out.ptr, got.nbytes)
        got = got.view(np.float16).astype(np.float32).reshape(B, H, L, D)
        ref = cr.sdpa(x[0], x[1][:, :, ::-1].copy(), x[2][:, :, ::-1].copy(),
                      None if mh is None else mh.data, 0.125)
        assert max_rel(got, ref) <= 5e-3
        if m is not None:
            b.dispose(m)
    for t in (q, k, v):
        b.dispose(t)
    out.release()
