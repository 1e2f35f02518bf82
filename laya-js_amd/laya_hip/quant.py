"""laya-js quantized checkpoint format v1: the matrix quantizer.

Restates `quantizeMatrix` (packages/laya/src/quant.ts:96-187; format in
docs/QUANTIZATION.md "Format"): each row is split into groups of `group`
consecutive values with their own f16 parameters -- q8: symmetric,
q in [-127, 127], scale = max|w| / 127; q4: affine, q in [0, 15], bias = min,
scale = (max - min) / 15 -- optionally refined by alternating "assign q by
rounding" and a least-squares refit (`REFINE_STEPS` rounds), keeping the
parameters with the smallest squared error.  Scale and bias are rounded to
f16 before q is chosen.  JS semantics are kept where they decide values:
Math.round rounds halves toward +inf, the per-group sums run sequentially in
f64, and f16 rounding is round-to-nearest-even from f64.

Vectorised over all groups of the matrix (one pass per position within a
group), so quantizing a ModernBERT-base checkpoint takes seconds.
"""
from __future__ import annotations

import numpy as np

REFINE_STEPS = 8
DEFAULT_GROUP_SIZE = 64


def _f16(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore", invalid="ignore"):
        return x.astype(np.float16).astype(np.float64)


def _js_round(x: np.ndarray) -> np.ndarray:
    f = np.floor(x)
    return np.where(x - f >= 0.5, f + 1.0, f)


def _assign(w, s, b, qmin, qmax):
    """q = clamp(round((w - b) / s)) per group; returns (q, squared error)."""
    ok = (s > 0) & np.isfinite(s)
    s_ok = np.where(ok, s, 1.0)[:, None]
    with np.errstate(invalid="ignore", divide="ignore"):
        v = np.where(ok[:, None], _js_round((w - b[:, None]) / s_ok), 0.0)
    v = np.clip(v, qmin, qmax)
    rec = v * np.where(ok, s, 0.0)[:, None] + b[:, None]
    d = w - rec
    err = np.zeros(w.shape[0])
    for k in range(w.shape[1]):  # sequential, as the reference sums
        err += d[:, k] * d[:, k]
    return v.astype(np.int32), err


def _seq_sum(a: np.ndarray) -> np.ndarray:
    acc = np.zeros(a.shape[0])
    for k in range(a.shape[1]):
        acc += a[:, k]
    return acc


def quantize_matrix(values, rows: int, cols: int, bits: int, group: int | None = None, refine: bool = True):
    """-> (q int32 [rows, cols], scales f16 [rows, G], biases f16 [rows, G] | None)."""
    group = cols if group is None else group
    v = np.asarray(values, np.float32).reshape(rows, cols)
    if bits not in (8, 4):
        raise ValueError(f"quantizeMatrix: bits must be 8 or 4, got {bits}")
    if not (isinstance(group, int) and group > 0 and cols % group == 0):
        raise ValueError(f"quantizeMatrix: group size {group} must divide {cols}")
    if bits == 4 and (cols % 2 or group % 2):
        raise ValueError("quantizeMatrix: q4 needs an even column count and group size")
    G = cols // group
    w = v.astype(np.float64).reshape(rows * G, group)
    steps = REFINE_STEPS if refine else 0
    n = float(group)
    if bits == 8:
        qmin, qmax = -127, 127
        s = _f16(np.abs(w).max(axis=1) / 127)
        b = np.zeros_like(s)
    else:
        qmin, qmax = 0, 15
        lo, hi = w.min(axis=1), w.max(axis=1)
        b = _f16(lo)
        s = _f16((hi - b) / 15)
    best_q, best_err = _assign(w, s, b, qmin, qmax)
    best_s, best_b = s.copy(), b.copy()
    active = np.ones(w.shape[0], bool)
    for _ in range(steps):
        q = best_q.astype(np.float64)
        if bits == 8:
            num = _seq_sum(q * w)
            den = _seq_sum(q * q)
            live = active & (den != 0)
            with np.errstate(invalid="ignore", divide="ignore"):
                s_new = _f16(np.where(live, num / np.where(den != 0, den, 1.0), 0.0))
            b_new = np.zeros_like(s_new)
        else:
            sq, sw, sqq, sqw = _seq_sum(q), _seq_sum(w), _seq_sum(q * q), _seq_sum(q * w)
            den = n * sqq - sq * sq
            live = active & (den != 0)
            with np.errstate(invalid="ignore", divide="ignore"):
                s_new = _f16(np.where(live, (n * sqw - sq * sw) / np.where(den != 0, den, 1.0), 0.0))
                b_new = _f16((sw - s_new * sq) / n)
        q_new, err_new = _assign(w, s_new, b_new, qmin, qmax)
        better = live & (err_new < best_err)
        best_q = np.where(better[:, None], q_new, best_q)
        best_err = np.where(better, err_new, best_err)
        best_s = np.where(better, s_new, best_s)
        best_b = np.where(better, b_new, best_b)
        active = better
        if not active.any():
            break
    q = best_q.reshape(rows, cols)
    scales = best_s.reshape(rows, G).astype(np.float16)
    biases = best_b.reshape(rows, G).astype(np.float16) if bits == 4 else None
    return q, scales, biases
