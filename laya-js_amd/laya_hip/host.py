"""Host-side types of the tensor-backend contract, restated for Python.

HostTensor / HostQuantized / QuantizedTensor and the quantized pack, unpack
and validate helpers follow packages/tensor-backend/src/index.ts:39-137 and
src/host.ts:1-185.  Host data are numpy arrays: f32 -> float32, f16 ->
float16, bf16 -> uint16 raw bits, i32 -> int32, bool -> uint8 (0/1), u8,
i8, u16, i16, u32, f64 -> float64, i64/u64 -> int64/uint64.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional

import numpy as np

NP_DTYPE = {
    "f32": np.float32, "f16": np.float16, "bf16": np.uint16, "i32": np.int32, "bool": np.uint8, "u8": np.uint8,
    "i8": np.int8, "u16": np.uint16, "i16": np.int16, "u32": np.uint32, "f64": np.float64, "i64": np.int64,
    "u64": np.uint64,
}
FLOATS = ("f32", "f16", "bf16", "f64")


@dataclass(frozen=True)
class HostTensor:
    dtype: str
    shape: tuple
    data: np.ndarray


def host(dtype: str, shape, data=None) -> HostTensor:
    """host.ts:45-58: a HostTensor of `shape`, zero-filled or from `data`."""
    shape = tuple(int(d) for d in shape)
    n = int(np.prod(shape)) if shape else 1
    if data is None:
        arr = np.zeros(n, NP_DTYPE[dtype])
    else:
        src = np.asarray(data)
        if src.size != n:
            raise ValueError(f"host(): {src.size} values for shape [{','.join(map(str, shape))}]")
        if dtype == "bf16" and src.dtype != np.uint16:
            arr = f32_to_bf16_bits(src.astype(np.float32).ravel())
        elif dtype == "bool":
            arr = (src.ravel() != 0).astype(np.uint8)
        else:
            arr = src.astype(NP_DTYPE[dtype]).ravel()
    return HostTensor(dtype, shape, arr.reshape(shape))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """host.ts:63-69: round-to-nearest-even f32 -> bf16 bits (NaN -> 0x7fc0)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, 0x7FC0, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_f32(t: HostTensor) -> np.ndarray:
    """host.ts:77-92: any HostTensor -> float32 values."""
    if t.dtype == "bf16":
        return bf16_bits_to_f32(t.data)
    return np.asarray(t.data).astype(np.float32)


def to_f64(t: HostTensor) -> np.ndarray:
    if t.dtype == "bf16":
        return bf16_bits_to_f32(t.data).astype(np.float64)
    return np.asarray(t.data).astype(np.float64)


# ---------------------------------------------------------------- quantized

@dataclass(frozen=True)
class QuantizedLinearOptions:
    bits: int
    groupSize: int
    mode: str  # "symmetric" | "affine"


@dataclass(frozen=True)
class HostQuantized:
    """index.ts:98-115: W [out, in], row-major packed `in*bits/8` bytes per row
    (4-bit: even column in the low nibble); scales (and affine biases) float
    [out, ceil(in/groupSize)]."""
    shape: tuple
    bits: int
    groupSize: int
    mode: str
    data: np.ndarray  # uint8
    scales: HostTensor
    biases: Optional[HostTensor]


@dataclass(frozen=True)
class QuantizedTensor:
    """index.ts:122-137.  native=True: w / scales / biases are in the
    backend's own layout; False: compose layout (q values as floats)."""
    shape: tuple
    bits: int
    groupSize: int
    mode: str
    dtype: str
    native: bool
    w: Any
    scales: Any
    biases: Any


def quant_groups(in_features: int, group_size: int) -> int:
    return -(-in_features // group_size)


def validate_quantized(h: HostQuantized) -> None:
    """host.ts:136-154."""
    N, K = h.shape
    where = f"quantized [{N}, {K}] q{h.bits}/{h.mode}/g{h.groupSize}"
    if h.bits not in (4, 8):
        raise ValueError(f"{where}: bits must be 4 or 8")
    if h.mode not in ("symmetric", "affine"):
        raise ValueError(f'{where}: mode must be "symmetric" or "affine"')
    if not (isinstance(N, int) and N > 0 and isinstance(K, int) and K > 0):
        raise ValueError(f"{where}: bad shape")
    if not (isinstance(h.groupSize, int) and h.groupSize > 0):
        raise ValueError(f"{where}: bad group size")
    if (K * h.bits) % 32:
        raise ValueError(f"{where}: in · bits must be a multiple of 32")
    if h.data.size != N * K * h.bits // 8:
        raise ValueError(f"{where}: data has {h.data.size} bytes, want {N * K * h.bits // 8}")
    G = quant_groups(K, h.groupSize)

    def check(t, name):
        if t is None:
            raise ValueError(f"{where}: missing {name}")
        if t.dtype not in ("f32", "f16", "bf16"):
            raise TypeError(f"{where}: {name} must be float")
        if len(t.shape) != 2 or t.shape[0] != N or t.shape[1] != G:
            raise ValueError(f"{where}: {name} has shape [{','.join(map(str, t.shape))}], want [{N}, {G}]")

    check(h.scales, "scales")
    if h.mode == "affine":
        check(h.biases, "biases")
    elif h.biases is not None:
        raise ValueError(f"{where}: symmetric quantization takes no biases")


def unpack_quantized(h: HostQuantized) -> np.ndarray:
    """host.ts:157-172: int32 q values [out * in] (signed for symmetric)."""
    d = np.asarray(h.data, np.uint8).ravel()
    signed = h.mode == "symmetric"
    if h.bits == 8:
        return d.view(np.int8).astype(np.int32) if signed else d.astype(np.int32)
    lo = (d & 15).astype(np.int32)
    hi = (d >> 4).astype(np.int32)
    if signed:
        lo = (lo ^ 8) - 8
        hi = (hi ^ 8) - 8
    q = np.empty(d.size * 2, np.int32)
    q[0::2] = lo
    q[1::2] = hi
    return q


def pack_quantized(q, bits: int) -> np.ndarray:
    """host.ts:175-185."""
    q = np.asarray(q, np.int64).ravel()
    if bits == 8:
        return (q & 255).astype(np.uint8)
    if q.size % 2:
        raise ValueError("packQuantized: 4-bit needs an even value count")
    return ((q[0::2] & 15) | ((q[1::2] & 15) << 4)).astype(np.uint8)
