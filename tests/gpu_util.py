"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import numpy as np

from laya_hip.host import HostTensor, f32_to_bf16_bits, bf16_bits_to_f32

NP16 = {"f16": np.float16}


def to_host(a: np.ndarray, dtype: str) -> HostTensor:
    a = np.asarray(a, np.float32)
    if dtype == "f16":
        return HostTensor("f16", a.shape, a.astype(np.float16))
    if dtype == "bf16":
        return HostTensor("bf16", a.shape, f32_to_bf16_bits(a).reshape(a.shape))
    return HostTensor("f32", a.shape, a)


def rounded(a: np.ndarray, dtype: str) -> np.ndarray:
    """Values as stored in `dtype`, as f32."""
    a = np.asarray(a, np.float32)
    if dtype == "f16":
        return a.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(a)).reshape(a.shape)
    return a


def read32(b, t) -> np.ndarray:
    h = b.read(t)
    if h.dtype == "bf16":
        return bf16_bits_to_f32(h.data).reshape(h.shape)
    return np.asarray(h.data, np.float32)


def max_rel(got, ref) -> float:
    """max |y - r| / max |r| (the GEMM parity metric: elementwise relative
    error is ill-posed near zero)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))
