"""The large-M GEMM with several tiles per block, on the GPU, through the C ABI.

When a block streams several output tiles (more tiles than CUs, and K stages
that are a multiple of 6 or at least 12), an interior tile's output leaves
during the next tile's first stages instead of in one burst, and a residual
tile is copied in from a later stage; edge tiles (ragged M or N) and outputs
in the other layout still leave in one burst.  A tile whose K stages are not
a multiple of 6 ends with a tail that hands the next tile's registers over
(every remainder 1..5 is covered).  Each case checks:
- bit for bit, 128-row windows of the output (first, middle, last rows)
  against hb_linear on those 128 rows alone, which takes the small-M
  kernels: every MFMA kernel gives a row the same bits;
- the windows against the CPU oracle (max-rel 2e-3 fp16 / 8e-3 bf16);
- a GeGLU output written in panel order equals, after hb_panel_unpack, the
  row-major one bit for bit.
"""
import numpy as np
import pytest

from gpu_util import max_rel, rounded, to_host
from laya_hip import ffi as F
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _bits(b, ptr, n):
    out = np.empty(n, np.uint16)
    b.n.call("read", "hb_download", b.ctx, out.ctypes.data, ptr, out.nbytes)
    return out


def _linear(b, dt, xp, M, K, wp, N, bp=0, rp=0, geglu=False, flags=0):
    """y = hb_linear(x [M, K] row-major, ...) into a new buffer; N output
    columns (N / 2 with GeGLU)."""
    No = N // 2 if geglu else N
    y = b._malloc(((M + 31) // 32 * 32) * No * 2)
    flags |= (F.HB_EPI_BIAS if bp else 0) | (F.HB_EPI_RESID if rp else 0) | (F.HB_EPI_GEGLU if geglu else 0)
    b.n.call("linear", "hb_linear", b.ctx, dt, xp, K, wp, bp, rp, No if rp else 0, y.ptr, No, M, No, K, flags)
    return y


def _to_f32(bits, dtype):
    if dtype == "f16":
        return bits.view(np.float16).astype(np.float32)
    from laya_hip.host import bf16_bits_to_f32
    return bf16_bits_to_f32(bits)


CASES = [
    # M, N (2N with GeGLU), K, geglu, bias, residual
    (12900, 2304, 768, False, False, False),  # Wqkv-like, the last row panel partial (a burst edge tile)
    (16384, 2300, 768, False, False, False),  # the last column tile partial
    (32768, 768, 768, False, True, True),     # two tiles per block with bias and residual
    (32768, 768, 1152, False, False, True),   # mlp Wo shape, K = 1152, residual
    (16384, 2304, 768, True, False, False),   # GeGLU, row-major output
    (16384, 2304, 1024, False, False, False),  # 16 K stages (a tail of 4), the large config's Wqkv
    (32768, 1024, 1024, False, True, True),    # the large config's attn Wo: partial last column tile
    (32768, 1024, 2624, False, False, True),   # the large config's mlp Wo: 41 stages (a tail of 5)
    (16384, 2304, 832, True, False, False),    # GeGLU, 13 stages (a tail of 1)
    (16384, 2304, 896, False, True, False),    # 14 stages (a tail of 2)
    (8192, 2304, 960, False, False, True),     # 15 stages (a tail of 3), residual
    (16384, 2304, 1000, False, True, False),   # K % 64 != 0 (a zeroed K tail) over 16 stages, streamed
    (32768, 1024, 1000, False, False, True),   # 128-column tiles with a K tail and a residual
    (16384, 2304, 1000, True, False, False),   # GeGLU with a K tail, streamed
]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("M,N,K,geglu,bias,resid", CASES)
def test_streamed_tiles_equal_single_tile_rows(b, dtype, M, N, K, geglu, bias, resid):
    print(f"streamed GEMM M={M} N={N} K={K} geglu={geglu} bias={bias} resid={resid} {dtype}", flush=True)
    rng = np.random.default_rng(M + N + K + int(geglu))
    dt = F.HB_F16 if dtype == "f16" else F.HB_BF16
    No = N // 2 if geglu else N
    x = rounded(rng.standard_normal((M, K)), dtype)
    w = rounded(rng.normal(0, 0.03, (N, K)), dtype)
    bv = rounded(rng.standard_normal(N), dtype) if bias else None
    r = rounded(rng.standard_normal((M, No)), dtype) if resid else None
    X, Wt = b.fromHost(to_host(x, dtype)), b.fromHost(to_host(w, dtype))
    Bt = b.fromHost(to_host(bv, dtype)) if bias else None
    R = b.fromHost(to_host(r, dtype)) if resid else None
    xp, wp = b._ptr(X), b._ptr(Wt)
    bp = b._ptr(Bt) if bias else 0
    rp = b._ptr(R) if resid else 0
    y = _linear(b, dt, xp, M, K, wp, N, bp, rp, geglu)
    full = _bits(b, y.ptr, M * No).reshape(M, No)
    for s in (0, (M // 2) // 32 * 32, M - 128):
        ys = _linear(b, dt, xp + s * K * 2, 128, K, wp, N, bp, rp + s * No * 2 if resid else 0, geglu)
        win = _bits(b, ys.ptr, 128 * No).reshape(128, No)
        ys.release()
        np.testing.assert_array_equal(full[s:s + 128], win, err_msg=f"rows {s}..{s + 127}")
        lin = rounded(cr.linear(x[s:s + 128], w, bv), dtype)
        ref = rounded(cr.geglu(lin), dtype) if geglu else lin
        ref = ref + r[s:s + 128] if resid else ref
        err = max_rel(_to_f32(win, dtype), ref)
        assert err <= (2e-3 if dtype == "f16" else 8e-3), f"rows {s}..: max-rel {err:.2e}"
    assert np.isfinite(_to_f32(full, dtype)).all()
    y.release()
    for t in (X, Wt, Bt, R):
        if t is not None:
            b.dispose(t)


@pytest.mark.parametrize("K", [768, 1024])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_streamed_panel_output_equals_row_major(b, dtype, bias, K):
    """The GeGLU linear with its output in panel order (streamed, as the
    encoder's Wi runs: an interior tile's GELU products are formed while the
    next tile computes) equals the row-major output (every GELU in the
    epilogue) bit for bit, with x row-major and in panel order, with and
    without a bias, at 12 K stages and at 16 (a tail of 4 per tile)."""
    print(f"streamed GeGLU panel output {dtype} bias={bias} K={K}", flush=True)
    M, N = 16384, 2304
    rng = np.random.default_rng(5)
    dt = F.HB_F16 if dtype == "f16" else F.HB_BF16
    x = rounded(rng.standard_normal((M, K)), dtype)
    w = rounded(rng.normal(0, 0.03, (N, K)), dtype)
    X, Wt = b.fromHost(to_host(x, dtype)), b.fromHost(to_host(w, dtype))
    Bt = b.fromHost(to_host(rounded(rng.standard_normal(N), dtype), dtype)) if bias else None
    xp, wp = b._ptr(X), b._ptr(Wt)
    bp = b._ptr(Bt) if bias else 0
    rowmajor = _linear(b, dt, xp, M, K, wp, N, bp, geglu=True)
    want = _bits(b, rowmajor.ptr, M * (N // 2))
    packed = b._malloc(M * K * 2)
    b.n.call("pack", "hb_panel_pack", b.ctx, xp, K, packed.ptr, M, K)
    for src, flags in ((xp, 0), (packed.ptr, F.HB_X_PANEL)):
        yp = _linear(b, dt, src, M, K, wp, N, bp, geglu=True, flags=flags | F.HB_Y_PANEL)
        out = b._malloc(M * (N // 2) * 2)
        b.n.call("unpack", "hb_panel_unpack", b.ctx, yp.ptr, out.ptr, N // 2, M, N // 2)
        np.testing.assert_array_equal(_bits(b, out.ptr, M * (N // 2)), want)
        yp.release()
        out.release()
    packed.release()
    rowmajor.release()
    for t in (X, Wt, Bt):
        if t is not None:
            b.dispose(t)
