"""hb_sdpa_noalloc, the attention entry point that allocates nothing, through
the C ABI: two calls in a row (the second smaller, another mask kind and
dtype) give hb_sdpa's outputs bit for bit and leave the context's pool as it
was (no block taken, none cached); an unmasked call matches too; a shape
whose mask summary would not fit the 2 MiB scratch is refused with an error
before anything is launched (its operands are real, full-size tensors)."""
import numpy as np
import pytest

from laya_hip import ffi as F
from laya_hip.host import HostTensor, f32_to_bf16_bits
from laya_hip.modernbert import attentionMasks

pytestmark = pytest.mark.gpu

D = 64


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _host(a, dtype):
    a = np.asarray(a, np.float32)
    if dtype == "f32":
        return HostTensor("f32", a.shape, a)
    if dtype == "f16":
        return HostTensor("f16", a.shape, a.astype(np.float16))
    return HostTensor("bf16", a.shape, f32_to_bf16_bits(a).reshape(a.shape))


def _case(b, rng, B, H, L, mask_kind, dtype, D=D):
    """q, k, v [B, H, L, D], a mask (None, "full" [B,1,1,L] or "sliding"
    [B,1,L,L] from attentionMasks with window 128) and two output blocks."""
    lens = rng.integers(L // 2, L + 1, B)
    valid = (np.arange(L)[None, :] < lens[:, None]).astype(np.uint8)
    full, sliding = attentionMasks(valid, B, L, 128)
    ts = [b.fromHost(_host(rng.standard_normal((B, H, L, D)), dtype)) for _ in range(3)]
    m = None if mask_kind is None else b.fromHost(full if mask_kind == "full" else sliding)
    ms = None if m is None else ((L, 0, 0, 1) if mask_kind == "full" else (L * L, 0, L, 1))
    outs = [b._malloc(B * H * L * D * (4 if dtype == "f32" else 2)) for _ in range(2)]
    return ts, m, ms, outs


def _call_pair(b, B, H, L, mask_kind, dtype, seed, D=D):
    rng = np.random.default_rng(seed)
    (q, k, v), m, ms, (o1, o2) = _case(b, rng, B, H, L, mask_kind, dtype, D)
    dt = {"f16": F.HB_F16, "bf16": F.HB_BF16, "f32": F.HB_F32}[dtype]
    st = F.i64s((H * L * D, L * D, D, 1))
    mp = b._ptr(m) if m is not None else 0
    msa = F.i64s(ms) if ms is not None else None
    scale = D ** -0.5
    args = (b.ctx, dt, b._ptr(q), st, b._ptr(k), st, b._ptr(v), st, mp, msa)
    b.n.call("sdpa", "hb_sdpa", *args, 0, o1.ptr, st, B, H, L, L, D, scale, 0.0, 0.0)
    b.flush()
    before = b.pool_stats()
    print(f"hb_sdpa_noalloc B={B} H={H} L={L} D={D} mask={mask_kind} {dtype}", flush=True)
    b.n.call("sdpa", "hb_sdpa_noalloc", *args, o2.ptr, st, B, H, L, L, D, scale)
    after = b.pool_stats()
    assert after == before, f"the pool changed: {before} -> {after}"
    n = B * H * L * D
    bits = np.uint32 if dtype == "f32" else np.uint16
    got = np.empty(n, bits)
    want = np.empty(n, bits)
    b.n.call("read", "hb_download", b.ctx, want.ctypes.data, o1.ptr, want.nbytes)
    b.n.call("read", "hb_download", b.ctx, got.ctypes.data, o2.ptr, got.nbytes)
    np.testing.assert_array_equal(got, want)
    vals = {"f32": lambda w: w.view(np.float32), "f16": lambda w: w.view(np.float16),
            "bf16": lambda w: (w.astype(np.uint32) << 16).view(np.float32)}[dtype](want)
    assert np.isfinite(vals).all()
    for t in (q, k, v, m):
        if t is not None:
            b.dispose(t)
    for o in (o1, o2):
        o.release()


def test_noalloc_sdpa_two_calls_match_hb_sdpa(b):
    _call_pair(b, 4, 12, 512, "sliding", "f16", 1)  # the config-3 attention shape, 4 of its 32 sequences
    _call_pair(b, 2, 4, 200, "full", "bf16", 2)     # smaller, ragged tiles, the other mask kind and dtype


def test_noalloc_sdpa_without_mask(b):
    _call_pair(b, 1, 3, 130, None, "f16", 3)


@pytest.mark.parametrize("dtype,Dh", [("f32", 64), ("f16", 128)])
def test_noalloc_sdpa_masked_generic_path(b, dtype, Dh):
    """Masked calls that take the generic kernel (f32, or a head dim other
    than 64) read no mask summary: they are served, build nothing in the
    scratch, leave the pool as it was and give hb_sdpa's bits."""
    _call_pair(b, 2, 2, 160, "sliding", dtype, 5, D=Dh)
    _call_pair(b, 1, 2, 96, "full", dtype, 6, D=Dh)


def test_noalloc_sdpa_refuses_a_summary_larger_than_its_scratch(b):
    B, H, L = 64, 1, 8192  # summary 64 * 64 * 128 * 8 = 4 MiB > 2 MiB
    rng = np.random.default_rng(4)
    big = [b.fromHost(HostTensor("f16", (B, H, L, D), np.zeros((B, H, L, D), np.float16))) for _ in range(3)]
    m = b.fromHost(HostTensor("bool", (B, 1, 1, L), (rng.random((B, 1, 1, L)) < 0.9).astype(np.uint8)))
    o = b._malloc(B * H * L * D * 2)
    st = F.i64s((H * L * D, L * D, D, 1))
    with pytest.raises(F.HipError, match="scratch"):
        b.n.call("sdpa", "hb_sdpa_noalloc", b.ctx, F.HB_F16, b._ptr(big[0]), st, b._ptr(big[1]), st,
                 b._ptr(big[2]), st, b._ptr(m), F.i64s((L, 0, 0, 1)), o.ptr, st, B, H, L, L, D, 0.125)
    b.flush()
    for t in (*big, m):
        b.dispose(t)
    o.release()
