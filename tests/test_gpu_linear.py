"""Linear-layer parity on the GPU (BASELINE configs 1 and 2).

GEMM outputs of the MFMA kernels against the CPU oracle's f64-accumulated
linear on the same rounded inputs: max-rel (max|y - r| / max|r|) <= 2e-3 for
fp16 and 8e-3 for bf16; quantized weights <= 1e-2 against the oracle's
dequantize-then-linear.  At M = 8192 / 16384 the oracle runs on a random
subset of rows (rows are independent).  The one-hot test reads single
dequantized weights back bit for bit: fl16(q*s + z), the value host
dequantization uploads (backend-webgpu/test/quantized.test.ts:107-160)."""
import numpy as np
import pytest

from gpu_util import max_rel, read32, rounded, to_host
from laya_hip.host import HostQuantized, HostTensor, QuantizedLinearOptions, pack_quantized
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu

SHAPES = {"Wqkv": (2304, 768), "Wo": (768, 768), "Wi": (2304, 768), "WoMlp": (768, 1152)}
MS = [128, 512, 2048, 8192, 16384]


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _rows(M, rng, n=384):
    return np.arange(M) if M <= n else np.sort(rng.choice(M, n, replace=False))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("M", MS)
def test_linear_config1(b, name, M, dtype):
    N, K = SHAPES[name]
    print(f"linear {name} M={M} {dtype}", flush=True)
    rng = np.random.default_rng(M + N + K)
    x = rounded(rng.standard_normal((M, K)), dtype)
    w = rounded(rng.normal(0, 0.02, (N, K)), dtype)
    X, Wt = b.fromHost(to_host(x, dtype)), b.fromHost(to_host(w, dtype))
    geglu = name == "Wi"
    if geglu:
        y = b.geglu(b.linear(X, Wt))
    else:
        y = b.linear(X, Wt)
    got = read32(b, y)
    rows = _rows(M, rng)
    lin = cr.linear(x[rows], w)
    ref = cr.geglu(rounded(lin, dtype)) if geglu else lin
    err = max_rel(got[rows], ref)
    tol = 2e-3 if dtype == "f16" else 8e-3
    assert err <= tol, f"{name} M={M} {dtype}: max-rel {err:.2e}"
    for t in (X, Wt, y):
        b.dispose(t)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_linear_bias_resid_ragged(b, dtype):
    """Bias and residual epilogues, and ragged M / N / K (tails of every tile)."""
    rng = np.random.default_rng(7)
    for (M, N, K) in [(130, 200, 256), (37, 48, 72), (1, 3072, 1024), (333, 100, 256), (50, 96, 128), (4100, 770, 776)]:
        x = rounded(rng.standard_normal((M, K)), dtype)
        w = rounded(rng.normal(0, 0.05, (N, K)), dtype)
        bias = rounded(rng.standard_normal(N), dtype)
        r = rounded(rng.standard_normal((M, N)), dtype)
        X, Wt, Bt, R = (b.fromHost(to_host(a, dtype)) for a in (x, w, bias, r))
        y = b.add(R, b.linear(X, Wt, Bt))
        got = read32(b, y)
        lin = rounded(cr.linear(x, w, bias), dtype)
        ref = r + lin
        err = max_rel(got, ref)
        assert err <= (2e-3 if dtype == "f16" else 8e-3), f"M={M} N={N} K={K}: {err:.2e}"
        for t in (X, Wt, Bt, R, y):
            b.dispose(t)
    assert b.stats["linear_fused_resid"] > 0


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_linear_geglu_bias_ragged(b, dtype):
    """GeGLU epilogue with a bias (value and gate halves of the bias) and
    ragged output widths, on both the small-M and the large-M kernels."""
    rng = np.random.default_rng(9)
    for (M, N2, K) in [(300, 770, 136), (4100, 770, 776), (4096, 2304, 768)]:
        x = rounded(rng.standard_normal((M, K)), dtype)
        w = rounded(rng.normal(0, 0.05, (N2, K)), dtype)
        bias = rounded(rng.standard_normal(N2), dtype)
        X, Wt, Bt = (b.fromHost(to_host(a, dtype)) for a in (x, w, bias))
        y = b.geglu(b.linear(X, Wt, Bt))
        got = read32(b, y)
        rows = _rows(M, rng)
        ref = cr.geglu(rounded(cr.linear(x[rows], w, bias), dtype))
        err = max_rel(got[rows], ref)
        assert err <= (2e-3 if dtype == "f16" else 8e-3), f"M={M} N={N2} K={K}: {err:.2e}"
        for t in (X, Wt, Bt, y):
            b.dispose(t)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_fused_geglu_is_bit_identical_to_separate_geglu(b, dtype):
    """linear -> geglu fused into the GEMM epilogue gives the same bits as a
    materialised linear followed by the standalone GeGLU kernel."""
    rng = np.random.default_rng(10)
    for M in (300, 4096):
        x = rounded(rng.standard_normal((M, 768)), dtype)
        w = rounded(rng.normal(0, 0.05, (2304, 768)), dtype)
        X, Wt = b.fromHost(to_host(x, dtype)), b.fromHost(to_host(w, dtype))
        fused = b.read(b.geglu(b.linear(X, Wt))).data
        sep = b.read(b.geglu(b._ready(b.linear(X, Wt)))).data
        assert b.stats["linear_fused_geglu"] > 0
        np.testing.assert_array_equal(fused, sep)
        b.dispose(X)
        b.dispose(Wt)


def test_linear_f32_path(b):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((70, 45)).astype(np.float32)
    w = rng.standard_normal((33, 45)).astype(np.float32)
    X, Wt = b.fromHost(to_host(x, "f32")), b.fromHost(to_host(w, "f32"))
    got = read32(b, b.linear(X, Wt))
    np.testing.assert_allclose(got, cr.linear(x, w), rtol=1e-5, atol=1e-5)


def _quantized(rng, N, K, bits, g=64):
    w = rounded(rng.normal(0, 0.02, (N, K)), "f16")
    q, s, z = cr.quantize_matrix(w, N, K, bits, g, refine=bits == 4)
    mode = "symmetric" if bits == 8 else "affine"
    h = HostQuantized((N, K), bits, g, mode, pack_quantized(q, bits), HostTensor("f16", s.shape, s.view(np.float16)),
                      HostTensor("f16", z.shape, z.view(np.float16)) if z is not None else None)
    sf = s.view(np.float16).astype(np.float32)
    zf = z.view(np.float16).astype(np.float32) if z is not None else None
    return h, q, sf, zf


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("M", [512, 2048, 8192])
def test_qlinear_config2(b, name, M, bits):
    from laya_hip import compose as C
    N, K = SHAPES[name]
    print(f"qlinear {name} M={M} q{bits}", flush=True)
    rng = np.random.default_rng(M + N + bits)
    h, q, sf, zf = _quantized(rng, N, K, bits)
    x = rounded(rng.standard_normal((M, K)), "f16")
    X = b.fromHost(to_host(x, "f16"))
    Q = C.upload_quantized(b, h, "f16")
    assert Q.native
    geglu = name == "Wi"
    y = C.quantized_linear(b, X, Q)
    if geglu:
        y = b.geglu(y)
    got = read32(b, y)
    rows = _rows(M, rng)
    lin = cr.quantized_linear(x[rows], q, sf, zf, 64, dtype="f16")
    ref = cr.geglu(rounded(lin, "f16")) if geglu else lin
    err = max_rel(got[rows], ref)
    assert err <= 1e-2, f"{name} M={M} q{bits}: max-rel {err:.2e}"
    C.dispose_quantized(b, Q)
    b.dispose(X)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("M", [512, 2048, 4160])
def test_qlinear_bf16(b, M, bits):
    """Quantized weights with bf16 activations: the dequantized weight is
    rounded once to bf16 (quant.ts:189-243, dequantRows then the compute
    dtype) on every path -- M = 512 and M = 2048 (128 x 64 tiles, the loader
    dequantizing each stage) and M = 4160 (dequantized once, then the
    large-M kernel with a partial row tile) -- against the oracle's
    dequantize-then-linear in bf16, max-rel <= 1e-2."""
    from laya_hip import compose as C
    N, K = SHAPES["Wqkv"]
    rng = np.random.default_rng(7 * M + bits)
    h, q, sf, zf = _quantized(rng, N, K, bits)
    x = rounded(rng.standard_normal((M, K)), "bf16")
    X = b.fromHost(to_host(x, "bf16"))
    Q = C.upload_quantized(b, h, "bf16")
    assert Q.native
    got = read32(b, C.quantized_linear(b, X, Q))
    rows = _rows(M, rng)
    ref = cr.quantized_linear(x[rows], q, sf, zf, 64, dtype="bf16")
    err = max_rel(got[rows], ref)
    assert err <= 1e-2, f"bf16 M={M} q{bits}: max-rel {err:.2e}"
    C.dispose_quantized(b, Q)
    b.dispose(X)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_quantized_small_m_slab_bits_equal_large_m(b, dtype):
    """Quantized weights on the small-M slab kernel (the slab's codes, scales
    and zeros fetched to LDS and dequantized once into the f16 slab): against
    the oracle's dequantize-then-linear (max-rel <= 1e-2), and bit for bit
    against the same rows inside a 4096-row input, which the large-M kernel
    computes with the same dequantization and k16 order.  Shapes: attn Wo and
    mlp Wo (K = 1152) with residuals, Wi + GeGLU, a ragged output width with
    K = 576; q8 symmetric and q4 affine; groups of 64 and 32."""
    from laya_hip import compose as C
    rng = np.random.default_rng(41)
    cases = [(128, 768, 768, False, 8, 64, True), (512, 768, 1152, False, 4, 64, True),
             (77, 2304, 768, True, 4, 32, False), (200, 784, 576, False, 8, 32, False)]
    for (M, N2, K, geglu, bits, g, resid) in cases:
        print(f"quantized slab M={M} N={N2} K={K} geglu={geglu} q{bits} g{g} resid={resid} {dtype}", flush=True)
        h, q, sf, zf = _quantized(rng, N2, K, bits, g)
        Q = C.upload_quantized(b, h, dtype)
        assert Q.native
        N = N2 // 2 if geglu else N2
        x = rounded(rng.standard_normal((M, K)), dtype)
        r = rounded(rng.standard_normal((M, N)), dtype)

        def run(xs, rs):
            X, R = b.fromHost(to_host(xs, dtype)), b.fromHost(to_host(rs, dtype))
            y = C.quantized_linear(b, X, Q)
            y = b.geglu(y) if geglu else y
            y = b.add(R, y) if resid else y
            out = np.asarray(b.read(y).data)
            got = read32(b, y)
            for t in (X, R, y):
                b.dispose(t)
            return out, got

        out, got = run(x, r)
        lin = cr.quantized_linear(x, q, sf, zf, g, dtype=dtype)
        ref = cr.geglu(rounded(lin, dtype)) if geglu else lin
        ref = r + rounded(ref, dtype) if resid else ref
        err = max_rel(got, ref)
        assert err <= 1e-2, f"M={M} N={N2} K={K} q{bits}: max-rel {err:.2e}"
        xb = np.concatenate([x, rounded(rng.standard_normal((4096 - M, K)), dtype)])
        rb = np.concatenate([r, rounded(rng.standard_normal((4096 - M, N)), dtype)])
        big, _ = run(xb, rb)
        np.testing.assert_array_equal(out, big[:M])
        C.dispose_quantized(b, Q)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_quantized_mid_m_bits_equal_large_m(b, dtype):
    """Between M = 1024 and 4096 a quantized linear on 128 x 64 tiles
    dequantizes each W stage in its loader (Wqkv at M = 2048, attn Wo and
    mlp Wo); Wqkv at M = 3072 runs 128 x 128 tiles on the weight dequantized
    once into a 16-bit copy.  Every path gives a row the same bits: the rows
    of an M-row call equal the same rows inside a 4096-row call, which the
    large-M kernel computes on the weight dequantized once.  Each call is
    also checked against the oracle's dequantize-then-linear (max-rel <=
    1e-2).  q8 symmetric and q4 affine, residuals, a ragged M."""
    from laya_hip import compose as C
    rng = np.random.default_rng(43)
    cases = [(2048, 2304, 768, 8, False), (3072, 2304, 768, 4, False), (2048, 768, 768, 4, True),
             (1024, 768, 1152, 8, False), (2000, 768, 768, 8, True)]
    for (M, N, K, bits, resid) in cases:
        print(f"quantized mid-M M={M} N={N} K={K} q{bits} resid={resid} {dtype}", flush=True)
        h, q, sf, zf = _quantized(rng, N, K, bits)
        Q = C.upload_quantized(b, h, dtype)
        assert Q.native
        x = rounded(rng.standard_normal((4096, K)), dtype)
        r = rounded(rng.standard_normal((4096, N)), dtype)

        def run(xs, rs):
            X, R = b.fromHost(to_host(xs, dtype)), b.fromHost(to_host(rs, dtype))
            y = C.quantized_linear(b, X, Q)
            y = b.add(R, y) if resid else y
            out = np.asarray(b.read(y).data)
            got = read32(b, y)
            for t in (X, R, y):
                b.dispose(t)
            return out, got

        (small, got), (big, _) = run(x[:M], r[:M]), run(x, r)
        np.testing.assert_array_equal(small, big[:M])
        rows = _rows(M, rng)
        lin = cr.quantized_linear(x[rows], q, sf, zf, 64, dtype=dtype)
        ref = r[rows] + rounded(lin, dtype) if resid else lin
        err = max_rel(got[rows], ref)
        assert err <= 1e-2, f"M={M} N={N} K={K} q{bits}: max-rel {err:.2e}"
        C.dispose_quantized(b, Q)


@pytest.mark.parametrize("bits,mode", [(8, "symmetric"), (4, "affine"), (8, "affine"), (4, "symmetric")])
def test_qlinear_one_hot_reads_exact_weights(b, bits, mode):
    """x = identity rows: y[k, n] = dequant(W)[n, k] must equal fl16(q*s + z)
    exactly (subnormal scales included)."""
    from laya_hip import compose as C
    rng = np.random.default_rng(bits)
    N, K, g = 64, 128, 32
    lo, hi = {(8, "symmetric"): (-127, 127), (8, "affine"): (0, 255), (4, "symmetric"): (-8, 7),
              (4, "affine"): (0, 15)}[(bits, mode)]
    q = rng.integers(lo, hi + 1, (N, K))
    s16 = rng.uniform(1e-6, 0.05, (N, K // g)).astype(np.float16)
    s16[0, 0] = np.float16(3e-7)  # subnormal
    z16 = rng.uniform(-0.1, 0.1, (N, K // g)).astype(np.float16)
    h = HostQuantized((N, K), bits, g, mode, pack_quantized(q, bits), HostTensor("f16", s16.shape, s16),
                      HostTensor("f16", z16.shape, z16) if mode == "affine" else None)
    Q = C.upload_quantized(b, h, "f16")
    assert Q.native
    X = b.fromHost(to_host(np.eye(K, dtype=np.float32), "f16"))
    got = b.read(C.quantized_linear(b, X, Q)).data.astype(np.float16).view(np.uint16)
    want = cr.dequant_exact_f16(q, s16.astype(np.float32), z16.astype(np.float32) if mode == "affine" else None, g)
    np.testing.assert_array_equal(got, want.T)
    E = C.quantized_embedding(b, Q, b.fromHost(HostTensor("i32", (N,), np.arange(N, dtype=np.int32))))
    np.testing.assert_array_equal(b.read(E).data.view(np.uint16), want)


def test_small_output_linear_epilogues(b):
    """Small outputs with a long K (M * N <= 16384, K >= 256) run one wave per
    output (gemm_dot) with the SIMT kernel's epilogue: f32 GeGLU with bias
    (K = 300, not a multiple of 8), bias plus a fused residual, and an f32
    linear on q4 weights, all against the oracle."""
    from laya_hip import compose as C
    rng = np.random.default_rng(21)
    M, N, K = 3, 20, 300
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((2 * N, K)) * 0.1).astype(np.float32)
    bias = rng.standard_normal(2 * N).astype(np.float32)
    r = rng.standard_normal((M, N)).astype(np.float32)
    X, Wt, Bt, R = (b.fromHost(to_host(a, "f32")) for a in (x, w, bias, r))
    got = read32(b, b.add(R, b.geglu(b.linear(X, Wt, Bt))))
    want = cr.geglu(cr.linear(x, w, bias)) + r
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    n_fused = b.stats["linear_fused_resid"]
    R2 = b.fromHost(to_host(rng.standard_normal((M, 2 * N)).astype(np.float32), "f32"))
    got = read32(b, b.add(R2, b.linear(X, Wt, Bt)))  # the residual in the epilogue
    assert b.stats["linear_fused_resid"] == n_fused + 1
    np.testing.assert_allclose(got, cr.linear(x, w, bias) + read32(b, R2), rtol=1e-5, atol=1e-5)
    b.dispose(R2)
    M, N, K = 4, 64, 512
    h, q, sf, zf = _quantized(rng, N, K, 4)
    Q = C.upload_quantized(b, h, "f32")
    x = rng.standard_normal((M, K)).astype(np.float32)
    Xq = b.fromHost(to_host(x, "f32"))
    got = read32(b, C.quantized_linear(b, Xq, Q))
    want = cr.quantized_linear(x, q, sf, zf, 64, dtype="f32")
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    C.dispose_quantized(b, Q)
    for t in (X, Wt, Bt, R, Xq):
        b.dispose(t)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_small_m_slab_edges_and_bits_equal_large_m(b, dtype):
    """The weight-stationary small-M kernel (16-bit weights, K % 64 == 0) on
    its edges: rows not a multiple of 32, output widths that end inside a
    32-column block, a bias that is an offset view (not 8-byte aligned),
    GeGLU, residuals, K from 64 to 1152.  Against the oracle (max-rel 2e-3 /
    8e-3), and bit for bit against the large-M kernel: the same X rows placed
    in a 4096-row input give the same output rows.  (Output rows of a length
    that is not a multiple of 8 take the f32 SIMT kernels instead, whose
    summation order depends on the shape.)"""
    rng = np.random.default_rng(21)
    cases = [(77, 784, 192, True, "offset", False), (300, 2304, 768, True, "aligned", False),
             (1, 768, 1152, False, "aligned", True), (129, 200, 1024, False, None, True),
             (33, 96, 64, False, "offset", True), (500, 2304, 768, False, None, False)]
    for (M, N2, K, geglu, bmode, resid) in cases:
        x = rounded(rng.standard_normal((M, K)), dtype)
        w = rounded(rng.normal(0, 0.05, (N2, K)), dtype)
        N = N2 // 2 if geglu else N2
        bias = rounded(rng.standard_normal(N2 + 1), dtype)
        r = rounded(rng.standard_normal((M, N)), dtype)
        X, Wt, Bfull, R = (b.fromHost(to_host(a, dtype)) for a in (x, w, bias, r))
        Bt = None if bmode is None else (b.slice(Bfull, [1], [N2 + 1]) if bmode == "offset" else b.slice(Bfull, [0], [N2]))
        bv = None if bmode is None else (bias[1:] if bmode == "offset" else bias[:N2])
        y = b.linear(X, Wt, Bt)
        y = b.geglu(y) if geglu else y
        y = b.add(R, y) if resid else y
        got = read32(b, y)
        lin = rounded(cr.linear(x, w, bv), dtype)
        ref = rounded(cr.geglu(lin), dtype) if geglu else lin
        ref = r + ref if resid else ref
        err = max_rel(got, ref)
        assert err <= (2e-3 if dtype == "f16" else 8e-3), f"M={M} N={N2} K={K} geglu={geglu}: {err:.2e}"
        # the same rows through the large-M kernel
        xb = np.concatenate([x, rounded(rng.standard_normal((4096 - M, K)), dtype)])
        rb = np.concatenate([r, rounded(rng.standard_normal((4096 - M, N)), dtype)])
        XB, RB = b.fromHost(to_host(xb, dtype)), b.fromHost(to_host(rb, dtype))
        yb = b.linear(XB, Wt, Bt)
        yb = b.geglu(yb) if geglu else yb
        yb = b.add(RB, yb) if resid else yb
        big = np.asarray(b.read(yb).data)
        np.testing.assert_array_equal(np.asarray(b.read(y).data), big[:M])
        for t in (X, Wt, Bfull, R, y, XB, RB, yb) + ((Bt,) if Bt is not None else ()):
            b.dispose(t)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_small_m_slab_takes_panel_operands(b, dtype):
    """The small-M slab kernel reads x in panel order (HB_X_PANEL) and writes
    a GeGLU output in panel order (HB_Y_PANEL), through the C ABI: bit for bit
    the row-major results, for row counts that are not multiples of 32 (the
    panel's padding rows) and a K longer than the registers (1152).  Calls
    that take the 128 x 128 kernel, and small-M quantized calls, refuse
    panel operands."""
    from laya_hip import ffi as F
    rng = np.random.default_rng(31)
    dt = F.HB_F16 if dtype == "f16" else F.HB_BF16

    def bits(ptr, n):
        out = np.empty(n, np.uint16)
        b.n.call("read", "hb_download", b.ctx, out.ctypes.data, ptr, out.nbytes)
        return out

    for (M, N2, K, geglu, with_bias) in [(1, 768, 768, False, False), (33, 2304, 768, True, True),
                                         (100, 768, 1152, False, True), (128, 2304, 768, False, False),
                                         (128, 2304, 768, True, False)]:
        print(f"slab panel M={M} N={N2} K={K} geglu={geglu} {dtype}", flush=True)
        No = N2 // 2 if geglu else N2
        x = rounded(rng.standard_normal((M, K)), dtype)
        w = rounded(rng.normal(0, 0.05, (N2, K)), dtype)
        bias = rounded(rng.standard_normal(N2), dtype)
        X, Wt, Bt = (b.fromHost(to_host(a, dtype)) for a in (x, w, bias))
        xp, wp, bp = b._ptr(X), b._ptr(Wt), (b._ptr(Bt) if with_bias else 0)
        flags = (F.HB_EPI_GEGLU if geglu else 0) | (F.HB_EPI_BIAS if with_bias else 0)
        Mp = (M + 31) // 32 * 32
        ref = b._malloc(M * No * 2)
        b.n.call("linear", "hb_linear", b.ctx, dt, xp, K, wp, bp, 0, 0, ref.ptr, No, M, No, K, flags)
        want = bits(ref.ptr, M * No)
        packed = b._malloc(Mp * K * 2)
        b.n.call("pack", "hb_panel_pack", b.ctx, xp, K, packed.ptr, M, K)
        y = b._malloc(M * No * 2)
        b.n.call("linear", "hb_linear", b.ctx, dt, packed.ptr, K, wp, bp, 0, 0, y.ptr, No, M, No, K,
                 flags | F.HB_X_PANEL)
        np.testing.assert_array_equal(bits(y.ptr, M * No), want)
        yp = b._malloc(Mp * No * 2)
        b.n.call("linear", "hb_linear", b.ctx, dt, packed.ptr, K, wp, bp, 0, 0, yp.ptr, No, M, No, K,
                 flags | F.HB_X_PANEL | F.HB_Y_PANEL)
        b.n.call("unpack", "hb_panel_unpack", b.ctx, yp.ptr, y.ptr, No, M, No)
        np.testing.assert_array_equal(bits(y.ptr, M * No), want)
        for m in (ref, packed, y, yp):
            m.release()
        for t in (X, Wt, Bt):
            b.dispose(t)
    # 2048 rows of a 2304-wide product take the 128 x 128 kernel: refused
    x = b._malloc(2048 * 768 * 2)
    w = b._malloc(2304 * 768 * 2)
    y = b._malloc(2048 * 2304 * 2)  # sized for the call, which is refused before any launch
    with pytest.raises(F.HipError, match="panel-order operands"):
        b.n.call("linear", "hb_linear", b.ctx, dt, x.ptr, 768, w.ptr, 0, 0, 0, y.ptr, 2304, 2048, 2304, 768,
                 F.HB_X_PANEL)
    with pytest.raises(F.HipError, match="panel-order operands"):  # quantized weights below 4096 rows
        b.n.call("quantizedLinear", "hb_qlinear", b.ctx, dt, x.ptr, 768, w.ptr, w.ptr, 0, 0, 0, 0, x.ptr, 768,
                 128, 768, 768, 8, 64, 0, F.HB_X_PANEL)
    for m in (x, w, y):
        m.release()
