"""Call-site helpers for the contract's optional ops, restated from
packages/tensor-backend/src/compose.ts: each uses the backend's native
kernel when it has one and a composition of required ops otherwise, so a
caller runs on every backend.  `without_optional_ops` mirrors
conformance.ts:131-143 (hide native optional ops to test the compositions).
"""
from __future__ import annotations

import math

import numpy as np

from .host import HostQuantized, HostTensor, QuantizedTensor, to_f32, unpack_quantized, validate_quantized

NUMERICS_OPS = ("equal", "notEqual", "less", "lessEqual", "greater", "greaterEqual", "logicalAnd", "logicalOr",
                "logicalNot", "sqrt", "rsqrt", "pow", "neg", "abs", "tanh", "sigmoid", "erf", "argmax", "argmin",
                "mean", "min", "cumsum")
QUANTIZED_OPS = ("fromHostQuantized", "quantizedLinear", "quantizedEmbedding")
FLOATS = ("f32", "f16", "bf16", "f64")


def has_native(b, op: str) -> bool:
    return callable(getattr(b, op, None))


class without_optional_ops:
    """A view of `b` without the given optional ops (compose.ts fallbacks run)."""

    def __init__(self, b, ops=NUMERICS_OPS):
        object.__setattr__(self, "_b", b)
        object.__setattr__(self, "_hidden", set(ops))

    def __getattr__(self, name):
        if name in self._hidden:
            raise AttributeError(name)
        return getattr(self._b, name)


def _as_float(b, x):
    return x if x.dtype in FLOATS else b.cast(x, "f32")


def _bit(b, x):
    return b.cast(b.cast(x, "bool"), "f32")


def zeros_like(b, x, dtype=None):
    return b.scope(lambda: b.cast(b.scale(_bit(b, x), 0), dtype or x.dtype))


def ones_like(b, x, dtype=None):
    return b.scope(lambda: b.cast(b.cast(b.exp(b.scale(_bit(b, x), 0)), "bool"), dtype or x.dtype))


# ---------------------------------------------------------------- fused (compose.ts:86-105)

def geglu(b, x):
    """gelu(value) * gate, [value, gate] = split(x, 2, -1)."""
    if has_native(b, "geglu"):
        return b.geglu(x)

    def f():
        value, gate = b.split(x, 2, len(x.shape) - 1)
        return b.mul(b.gelu(value), gate)
    return b.scope(f)


def mean_pool(b, x, mask):
    """Masked mean over axis 1 in f32: x [B, L, D], mask [B, L] -> [B, D]."""
    if has_native(b, "meanPool"):
        return b.meanPool(x, mask)

    def f():
        B, L = x.shape[0], x.shape[1]
        m = b.cast(b.reshape(mask, [B, L, 1]), "f32")
        total = b.sum(b.mul(b.cast(x, "f32"), m), 1)
        n = b.sum(m, 1)
        return b.div(total, b.maximum(n, ones_like(b, n)))
    return b.scope(f)


# ---------------------------------------------------------------- numerics (compose.ts:109-304)

def logicalNot(b, x):
    if has_native(b, "logicalNot"):
        return b.logicalNot(x)
    return b.scope(lambda: b.cast(b.sub(ones_like(b, _bit(b, x)), _bit(b, x)), "bool"))


def logicalAnd(b, x, y):
    if has_native(b, "logicalAnd"):
        return b.logicalAnd(x, y)
    return b.scope(lambda: b.cast(b.mul(_bit(b, x), _bit(b, y)), "bool"))


def logicalOr(b, x, y):
    if has_native(b, "logicalOr"):
        return b.logicalOr(x, y)
    return b.scope(lambda: b.cast(b.maximum(_bit(b, x), _bit(b, y)), "bool"))


def _diff(b, x, y):
    def wide(t):
        if t.dtype == "bool":
            return b.cast(t, "i32")
        return t if (t.dtype == "i32" or t.dtype in FLOATS) else b.cast(t, "f32")
    return b.sub(wide(x), wide(y))


def greater(b, x, y):
    if has_native(b, "greater"):
        return b.greater(x, y)
    return b.scope(lambda: b.cast(b.relu(_diff(b, x, y)), "bool"))


def less(b, x, y):
    if has_native(b, "less"):
        return b.less(x, y)
    return greater(b, y, x)


def notEqual(b, x, y):
    if has_native(b, "notEqual"):
        return b.notEqual(x, y)
    return b.scope(lambda: b.cast(_diff(b, x, y), "bool"))


def equal(b, x, y):
    if has_native(b, "equal"):
        return b.equal(x, y)
    return b.scope(lambda: logicalNot(b, notEqual(b, x, y)))


def lessEqual(b, x, y):
    if has_native(b, "lessEqual"):
        return b.lessEqual(x, y)
    return b.scope(lambda: logicalNot(b, greater(b, x, y)))


def greaterEqual(b, x, y):
    if has_native(b, "greaterEqual"):
        return b.greaterEqual(x, y)
    return b.scope(lambda: logicalNot(b, less(b, x, y)))


def neg(b, x):
    if has_native(b, "neg"):
        return b.neg(x)
    if x.dtype in FLOATS:
        return b.scale(x, -1)
    if x.dtype == "bool":
        return b.scope(lambda: b.sub(zeros_like(b, x, "i32"), b.cast(x, "i32")))
    return b.scope(lambda: b.sub(zeros_like(b, x, x.dtype), x))


def abs(b, x):  # noqa: A001 - contract name
    if has_native(b, "abs"):
        return b.abs(x)
    return b.scope(lambda: b.maximum(x, neg(b, x)))


def sqrt(b, x):
    if has_native(b, "sqrt"):
        return b.sqrt(x)
    return b.scope(lambda: b.exp(b.scale(b.log(_as_float(b, x)), 0.5)))


def rsqrt(b, x):
    if has_native(b, "rsqrt"):
        return b.rsqrt(x)
    return b.scope(lambda: b.exp(b.scale(b.log(_as_float(b, x)), -0.5)))


def pow(b, x, y):  # noqa: A001 - contract name
    if has_native(b, "pow"):
        return b.pow(x, y)
    return b.scope(lambda: b.exp(b.mul(_as_float(b, y), b.log(_as_float(b, x)))))


def sigmoid(b, x):
    if has_native(b, "sigmoid"):
        return b.sigmoid(x)

    def f():
        fx = _as_float(b, x)
        one = ones_like(b, fx)
        return b.div(one, b.add(one, b.exp(neg(b, fx))))
    return b.scope(f)


def tanh(b, x):
    if has_native(b, "tanh"):
        return b.tanh(x)

    def f():
        fx = _as_float(b, x)
        return b.sub(b.scale(sigmoid(b, b.scale(fx, 2)), 2), ones_like(b, fx))
    return b.scope(f)


def erf(b, x):
    """compose.ts:231-255: series below 1, Laplace continued fraction above."""
    if has_native(b, "erf"):
        return b.erf(x)

    def f():
        fx = _as_float(b, x)
        one = ones_like(b, fx)
        c = lambda v: b.scale(one, v)  # noqa: E731
        x2 = b.mul(fx, fx)
        term = fx
        s = fx
        for n in range(1, 11):
            term = b.mul(term, b.scale(x2, -1 / n))
            s = b.add(s, b.scale(term, 1 / (2 * n + 1)))
        series = b.scale(s, 1.1283791670955126)
        z = abs(b, fx)
        t = b.add(b.scale(x2, 2), one)
        fr = zeros_like(b, fx)
        for n in range(28, 0, -1):
            fr = b.div(c((2 * n - 1) * (2 * n)), b.sub(b.add(t, c(4 * n)), fr))
        erfc = b.div(b.mul(b.exp(neg(b, x2)), b.scale(z, 1.1283791670955126)), b.sub(t, fr))
        tail = b.sub(one, erfc)
        signed = b.where(less(b, fx, zeros_like(b, fx)), neg(b, tail), tail)
        return b.where(less(b, z, one), series, signed)
    return b.scope(f)


def mean(b, x, axis, keepDims=False):
    if has_native(b, "mean"):
        return b.mean(x, axis, keepDims)
    n = x.shape[axis]
    return b.scope(lambda: b.scale(b.sum(_as_float(b, x), axis, keepDims), 1 / n))


def min(b, x, axis, keepDims=False):  # noqa: A001 - contract name
    if has_native(b, "min"):
        return b.min(x, axis, keepDims)
    if x.dtype == "bool":
        return b.scope(lambda: logicalNot(b, b.max(logicalNot(b, x), axis, keepDims)))
    return b.scope(lambda: neg(b, b.max(neg(b, x), axis, keepDims)))


def cumsum(b, x, axis):
    if has_native(b, "cumsum"):
        return b.cumsum(x, axis)
    raise RuntimeError(f"cumsum: the {b.name} backend has no native cumsum and there is no default composition")


def _arg_reduce(b, x, axis, keepDims, which):
    if not has_native(b, "cumsum"):
        raise RuntimeError(f"{which}: the {b.name} backend has neither a native {which} nor a native cumsum")
    n = x.shape[axis]

    def f():
        best = b.max(x, axis, True) if which == "argmax" else min(b, x, axis, True)
        ones = ones_like(b, x, "i32")
        iota = b.sub(cumsum(b, ones, axis), ones)
        cand = b.where(equal(b, x, best), iota, b.cast(b.scale(ones_like(b, x, "f32"), n), "i32"))
        return b.cast(min(b, cand, axis, keepDims), "i32")
    return b.scope(f)


def argmax(b, x, axis, keepDims=False):
    if has_native(b, "argmax"):
        return b.argmax(x, axis, keepDims)
    return _arg_reduce(b, x, axis, keepDims, "argmax")


def argmin(b, x, axis, keepDims=False):
    if has_native(b, "argmin"):
        return b.argmin(x, axis, keepDims)
    return _arg_reduce(b, x, axis, keepDims, "argmin")


# ---------------------------------------------------------------- quantized (compose.ts:306-438)

def has_native_quantized(b) -> bool:
    return all(has_native(b, op) for op in QUANTIZED_OPS)


def is_quantized(x) -> bool:
    return isinstance(x, QuantizedTensor)


def _upload_float(b, h: HostTensor, dtype: str):
    src = h if (h.dtype == "f32" or b.supports(h.dtype)) else HostTensor("f32", h.shape, to_f32(h))
    t = b.fromHost(src)
    if t.dtype == dtype:
        return t
    c = b.cast(t, dtype)
    b.dispose(t)
    return c


def upload_quantized(b, h: HostQuantized, dtype: str) -> QuantizedTensor:
    """compose.ts:342-365: native layout when the backend accepts it, else
    the compose layout (q values as floats, dequantized per call)."""
    validate_quantized(h)
    if dtype not in FLOATS:
        raise TypeError(f"uploadQuantized: dtype must be float, got {dtype}")
    if has_native_quantized(b):
        q = b.fromHostQuantized(h, dtype)
        if q is not None:
            return q
    N, K = h.shape
    q = unpack_quantized(h)
    done = []
    try:
        done.append(_upload_float(b, HostTensor("f32", (N, K), q.astype(np.float32).reshape(N, K)), dtype))
        done.append(_upload_float(b, h.scales, dtype))
        if h.mode == "affine":
            done.append(_upload_float(b, h.biases, dtype))
    except BaseException:
        for t in done:
            b.dispose(t)
        raise
    return QuantizedTensor((N, K), h.bits, h.groupSize, h.mode, dtype, False, done[0], done[1],
                           done[2] if len(done) > 2 else None)


def dispose_quantized(b, q: QuantizedTensor) -> None:
    b.dispose(q.w)
    b.dispose(q.scales)
    if q.biases is not None:
        b.dispose(q.biases)


def _dequant_rows(b, w, scales, biases, group: int, dtype: str):
    """compose.ts:379-398: f32 dequantization, rounded once to `dtype`."""
    def f():
        R, K = w.shape
        G = math.ceil(K / group)
        full = K // group
        fl = lambda t: b.cast(t, "f32")  # noqa: E731

        def part(w0, w1, g0, g1):
            n = g1 - g0
            gs = (w1 - w0) // n
            wq = b.reshape(fl(b.slice(w, [0, w0], [R, w1])), [R, n, gs])
            s = b.reshape(fl(b.slice(scales, [0, g0], [R, g1])), [R, n, 1])
            v = b.mul(wq, s)
            if biases is not None:
                v = b.add(v, b.reshape(fl(b.slice(biases, [0, g0], [R, g1])), [R, n, 1]))
            return b.reshape(v, [R, w1 - w0])
        pieces = []
        if full:
            pieces.append(part(0, full * group, 0, full))
        if G > full:
            pieces.append(part(full * group, K, full, G))
        v = pieces[0] if len(pieces) == 1 else b.concat(pieces, 1)
        return v if v.dtype == dtype else b.cast(v, dtype)
    return b.scope(f)


def dequantize(b, q: QuantizedTensor):
    if q.native:
        raise RuntimeError(f"dequantize: {b.name} keeps this matrix in its native layout")
    return _dequant_rows(b, q.w, q.scales, q.biases, q.groupSize, q.dtype)


def quantized_linear(b, x, q: QuantizedTensor, bias=None):
    """compose.ts:407-414: y = x . dequant(q)^T (+ bias) in x's dtype."""
    if x.shape[-1] != q.shape[1]:
        raise ValueError(f"quantizedLinear: x [{x.shape}] vs w [{q.shape}]")
    if q.native:
        if not has_native(b, "quantizedLinear"):
            raise RuntimeError(f"quantizedLinear: the {b.name} backend has no native quantizedLinear")
        return b.quantizedLinear(x, q.w, q.scales, q.biases, q, bias)
    dt = x.dtype if x.dtype in FLOATS else "f32"
    return b.scope(lambda: b.linear(x, _dequant_rows(b, q.w, q.scales, q.biases, q.groupSize, dt), bias))


def quantized_embedding(b, q: QuantizedTensor, ids):
    """compose.ts:417-428."""
    if q.native:
        if not has_native(b, "quantizedEmbedding"):
            raise RuntimeError(f"quantizedEmbedding: the {b.name} backend has no native quantizedEmbedding")
        return b.quantizedEmbedding(q.w, q.scales, q.biases, q, ids)

    def f():
        n = ids.size
        flat = b.reshape(ids, [n])
        rows = _dequant_rows(b, b.embedding(q.w, flat), b.embedding(q.scales, flat),
                             b.embedding(q.biases, flat) if q.biases is not None else None, q.groupSize, q.dtype)
        return b.reshape(rows, list(ids.shape) + [q.shape[1]])
    return b.scope(f)


def linear_any(b, x, w, bias=None):
    """compose.ts:431-433: `linear` for a weight that may be quantized."""
    return quantized_linear(b, x, w, bias) if is_quantized(w) else b.linear(x, w, bias)


def embedding_any(b, table, ids):
    return quantized_embedding(b, table, ids) if is_quantized(table) else b.embedding(table, ids)
