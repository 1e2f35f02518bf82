"""Checkpoint I/O: safetensors files and laya-js quantized checkpoints
(format version 1), host side.

Restates the reference's loaders:
- `read_weights` / `consuming_weights` / `dequantizing_weights` /
  `sanitize_name` (packages/laya/src/weights.ts:15-161);
- `quant_metadata`, `group_quantized`, `dequantize_matrix`,
  `should_quantize` / `bits_of` / `group_of` and `quantize_safetensors`
  (packages/laya/src/quant.ts:65-77, 189-243, 246-360, 363-403).

The file format is safetensors: an 8-byte little-endian header length, a
JSON header (`name -> {dtype, shape, data_offsets}` plus `__metadata__`),
then the tensor bytes.  A quantized checkpoint stores each quantized matrix
`W` as I8 [rows, cols] (q8) or U8 [rows, cols/2] (q4, even column in the low
nibble) with `W.scales` (and for q4 `W.biases`) F16 [rows, cols/g]; its
`__metadata__` carries `laya_quant`, `group_size`, `version` and
`laya_quant_source_dtype`.  Files are memory-mapped, so a checkpoint is
never read into host memory twice.
"""
from __future__ import annotations

import json
import re
import struct
from dataclasses import dataclass
from typing import Callable, Optional

import numpy as np

from .host import HostQuantized, HostTensor
from .quant import DEFAULT_GROUP_SIZE, quantize_matrix

QUANT_FORMAT_VERSION = "1"

# safetensors dtype -> numpy storage type (BF16 kept as raw 16-bit patterns)
SAFE_NP = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16, "I64": np.int64,
           "I32": np.int32, "I16": np.int16, "I8": np.int8, "U64": np.uint64, "U32": np.uint32, "U16": np.uint16,
           "U8": np.uint8, "BOOL": np.uint8}
# safetensors dtype -> contract dtype (weights.ts:13)
DTYPES = {"F16": "f16", "BF16": "bf16", "F32": "f32", "I32": "i32", "BOOL": "bool", "U8": "bool"}


@dataclass(frozen=True)
class RawTensor:
    """A tensor as read from the file: safetensors dtype + data view."""
    dtype: str
    shape: tuple
    data: np.ndarray


class SafetensorsFile:
    """A parsed safetensors file over a byte buffer or a memory-mapped path."""

    def __init__(self, source):
        if isinstance(source, (bytes, bytearray, memoryview)):
            buf = np.frombuffer(source, np.uint8)
        else:
            buf = np.memmap(source, np.uint8, mode="r")
        if buf.size < 8:
            raise ValueError("safetensors: file shorter than its header length")
        (n,) = struct.unpack("<Q", bytes(buf[:8]))
        if 8 + n > buf.size:
            raise ValueError("safetensors: header runs past the end of the file")
        header = json.loads(bytes(buf[8:8 + n]).decode("utf-8"))
        self.metadata = {str(k): str(v) for k, v in (header.pop("__metadata__", None) or {}).items()}
        self._buf = buf
        self._base = 8 + n
        self._info = {}
        for name, e in header.items():
            dt, shape, (b0, b1) = e["dtype"], tuple(int(d) for d in e["shape"]), e["data_offsets"]
            if dt not in SAFE_NP:
                raise TypeError(f"safetensors: unsupported dtype {dt} for {name}")
            want = int(np.prod(shape)) * np.dtype(SAFE_NP[dt]).itemsize if shape else np.dtype(SAFE_NP[dt]).itemsize
            if b1 - b0 != want or self._base + b1 > buf.size:
                raise ValueError(f"safetensors: {name}: data_offsets [{b0}, {b1}) do not hold {dt} {list(shape)}")
            self._info[name] = (dt, shape, b0, b1)

    def names(self) -> list:
        return list(self._info)

    def has(self, name: str) -> bool:
        return name in self._info

    def info(self, name: str) -> tuple:
        dt, shape, _, _ = self._info[name]
        return dt, shape

    def bytes(self, name: str) -> np.ndarray:
        _, _, b0, b1 = self._info[name]
        return self._buf[self._base + b0:self._base + b1]

    def array(self, name: str) -> np.ndarray:
        dt, shape, _, _ = self._info[name]
        return self.bytes(name).view(SAFE_NP[dt]).reshape(shape)

    def raw(self, name: str) -> RawTensor:
        dt, shape = self.info(name)
        return RawTensor(dt, shape, self.array(name))


def read_safetensors(source) -> SafetensorsFile:
    return SafetensorsFile(source)


def write_safetensors(tensors: dict, metadata: Optional[dict] = None) -> bytes:
    """Serialises {name: RawTensor | (dtype, shape, array)} with the
    tensors' bytes in insertion order and 8-byte-aligned data."""
    header, chunks, off = {}, [], 0
    for name, t in tensors.items():
        dt, shape, data = (t.dtype, t.shape, t.data) if isinstance(t, RawTensor) else t
        b = np.ascontiguousarray(data).view(np.uint8).reshape(-1).tobytes()
        header[name] = {"dtype": dt, "shape": [int(d) for d in shape], "data_offsets": [off, off + len(b)]}
        chunks.append(b)
        off += len(b)
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    h = json.dumps(header, separators=(",", ":")).encode("utf-8")
    h += b" " * ((8 - len(h) % 8) % 8)
    return struct.pack("<Q", len(h)) + h + b"".join(chunks)


# ---------------------------------------------------------------- quantized format

@dataclass(frozen=True)
class QuantMetadata:
    scheme: str
    bits: int
    group_size: Optional[int]  # None = one group per row
    version: str
    source_dtype: Optional[str]


def quant_metadata(metadata: Optional[dict]) -> Optional[QuantMetadata]:
    """quant.ts:65-77: the scheme of a quantized checkpoint, None for a float
    one; unknown schemes, versions and group sizes raise."""
    scheme = (metadata or {}).get("laya_quant")
    if scheme is None:
        return None
    if scheme not in ("q8", "q4"):
        raise ValueError(f'laya: unknown quantization scheme laya_quant={json.dumps(scheme)} (expected "q8" or "q4")')
    version = metadata.get("version", "")
    if version != QUANT_FORMAT_VERSION:
        raise ValueError(f"laya: quantized checkpoint format version {json.dumps(version)} is not supported "
                         f"(this laya reads version {QUANT_FORMAT_VERSION})")
    g = metadata.get("group_size")
    group = None
    if g is not None and g != "row":
        try:
            group = int(g)
            ok = str(group) == g.strip() and group > 0
        except ValueError:
            ok = False
        if not ok:
            raise ValueError(f"laya: invalid group_size {json.dumps(g)} in quantized checkpoint")
    return QuantMetadata(scheme, 8 if scheme == "q8" else 4, group, version, metadata.get("laya_quant_source_dtype"))


@dataclass
class QuantizedMatrix:
    bits: int
    rows: int
    cols: int
    data: np.ndarray  # q8: int8 [rows*cols]; q4: uint8 [rows*cols/2]
    scales: np.ndarray  # float16 [rows, G]
    biases: Optional[np.ndarray]  # q4: float16 [rows, G]
    group_size: int


def group_quantized(tensors: dict) -> tuple:
    """quant.ts:375-403: splits a quantized file's tensors into quantized
    matrices (with their .scales / .biases folded in) and plain tensors."""
    quantized, plain, companion = {}, {}, set()
    for name, t in tensors.items():
        scales = tensors.get(name + ".scales")
        if scales is None:
            continue
        where = f"laya: quantized tensor {name}"
        if scales.dtype != "F16" or len(scales.shape) != 2:
            raise ValueError(f"{where}: .scales must be F16 [rows, groups]")
        rows, G = scales.shape
        biases = None
        if t.dtype == "I8":
            bits, cols = 8, t.shape[1] if len(t.shape) > 1 else -1
        elif t.dtype == "U8":
            bits, cols = 4, 2 * t.shape[1] if len(t.shape) > 1 else -1
            bt = tensors.get(name + ".biases")
            if bt is None or bt.dtype != "F16" or tuple(bt.shape) != (rows, G):
                raise ValueError(f"{where}: q4 needs .biases F16 [{rows}, {G}]")
            biases = np.asarray(bt.data).reshape(rows, G)
            companion.add(name + ".biases")
        else:
            raise ValueError(f"{where}: dtype {t.dtype} is not a quantized dtype (I8 or U8)")
        if len(t.shape) != 2 or t.shape[0] != rows or cols % G:
            raise ValueError(f"{where}: shape [{','.join(map(str, t.shape))}] does not match .scales "
                             f"[{rows},{G}]")
        companion.add(name + ".scales")
        quantized[name] = QuantizedMatrix(bits, rows, cols, np.asarray(t.data).reshape(-1),
                                          np.asarray(scales.data).reshape(rows, G), biases, cols // G)
    for name, t in tensors.items():
        if name not in quantized and name not in companion:
            plain[name] = t
    return quantized, plain


def _codes(m: QuantizedMatrix) -> np.ndarray:
    if m.bits == 8:
        return m.data.view(np.int8).reshape(m.rows, m.cols)
    b = m.data.view(np.uint8).reshape(m.rows, m.cols // 2)
    q = np.empty((m.rows, m.cols), np.uint8)
    q[:, 0::2] = b & 15
    q[:, 1::2] = b >> 4
    return q


def dequantize_matrix(m: QuantizedMatrix, dtype: str = "f16") -> np.ndarray:
    """quant.ts:189-243: every weight fl(q * scale + bias) rounded once from
    double to f16 or f32."""
    G = m.cols // m.group_size
    if m.cols % m.group_size or m.scales.size != m.rows * G:
        raise ValueError(f"dequantizeMatrix: scales has {m.scales.size} values, want {m.rows} x {G}")
    if m.bits == 8 and m.data.size != m.rows * m.cols:
        raise ValueError(f"dequantizeMatrix: q8 data has {m.data.size} values, want {m.rows * m.cols}")
    if m.bits == 4:
        if m.biases is None or m.biases.size != m.rows * G:
            raise ValueError("dequantizeMatrix: q4 needs biases [rows, cols/groupSize]")
        if m.data.size * 2 != m.rows * m.cols:
            raise ValueError(f"dequantizeMatrix: q4 data has {m.data.size} bytes, want {m.rows * m.cols // 2}")
    q = _codes(m).astype(np.float64).reshape(m.rows, G, m.group_size)
    v = q * m.scales.astype(np.float64).reshape(m.rows, G, 1)
    if m.bits == 4:
        v = v + m.biases.astype(np.float64).reshape(m.rows, G, 1)
    return v.reshape(m.rows, m.cols).astype(np.float16 if dtype == "f16" else np.float32)


def host_quantized(m: QuantizedMatrix) -> HostQuantized:
    """weights.ts:71-83: q8 -> 8-bit symmetric, q4 -> 4-bit affine (views)."""
    G = m.cols // m.group_size
    return HostQuantized((m.rows, m.cols), m.bits, m.group_size, "symmetric" if m.bits == 8 else "affine",
                         m.data.view(np.uint8), HostTensor("f16", (m.rows, G), m.scales),
                         HostTensor("f16", (m.rows, G), m.biases) if m.biases is not None else None)


# ---------------------------------------------------------------- weight getters

def sanitize_name(name: str) -> str:
    """weights.ts:15-22: upstream PyTorch names -> laya-mlx names."""
    n = name.replace(".in_proj_weight", ".in_proj.weight").replace(".in_proj_bias", ".in_proj.bias")
    for prefix in ("scorer", "act_head"):
        if n.startswith(prefix + ".") and not n.startswith(prefix + ".layers."):
            n = prefix + ".layers." + n[len(prefix) + 1:]
    return n


class ConsumingWeights:
    """A one-shot weight getter: `get` hands a tensor out once and forgets
    it; `remaining()` lists what nobody asked for (weights.ts:24-51)."""

    def __init__(self, get: Callable, remaining: Callable):
        self.get = get
        self.remaining = remaining


def _host(name: str, t: RawTensor) -> HostTensor:
    d = DTYPES.get(t.dtype)
    if d is None:
        raise TypeError(f"laya: unsupported safetensors dtype {t.dtype} for {name}")
    data = t.data
    if d == "bool":
        data = (np.asarray(data) != 0).astype(np.uint8)
    return HostTensor(d, tuple(t.shape), data)


def consuming_weights(tensors: dict) -> ConsumingWeights:
    table = {}
    for name, t in tensors.items():
        key = sanitize_name(name)
        if key in table:
            raise ValueError(f"Duplicate checkpoint parameter after conversion: {key}")
        table[key] = t
    return ConsumingWeights(lambda name: table.pop(name, None), lambda: list(table))


def dequantizing_weights(raw: dict, dtype: str = "f16", keep_quantized: bool = False) -> ConsumingWeights:
    """weights.ts:86-131: quantized matrices stay packed until asked for; `get`
    dequantizes one to `dtype` (or, with keep_quantized, hands it out as a
    HostQuantized for the device path)."""
    quantized, plain = group_quantized(raw)
    q = {}
    for name, m in quantized.items():
        key = sanitize_name(name)
        if key in q:
            raise ValueError(f"Duplicate checkpoint parameter after conversion: {key}")
        q[key] = m
    rest = consuming_weights({name: _host(name, t) for name, t in plain.items()})
    for key in q:
        if key in rest.remaining():
            raise ValueError(f"Duplicate checkpoint parameter after conversion: {key}")

    def get(name):
        m = q.pop(name, None)
        if m is None:
            return rest.get(name)
        if keep_quantized:
            return host_quantized(m)
        return HostTensor(dtype, (m.rows, m.cols), dequantize_matrix(m, dtype))
    return ConsumingWeights(get, lambda: list(q) + rest.remaining())


def read_weights(source, dtype: Optional[str] = None, quantized: Optional[str] = None) -> ConsumingWeights:
    """weights.ts:145-161: a float checkpoint's tensors as they are; a
    quantized one's matrices dequantized to `dtype` (default f16) or, with
    quantized="device", kept packed."""
    f = read_safetensors(source)
    if quant_metadata(f.metadata) is None:
        return consuming_weights({n: _host(n, f.raw(n)) for n in f.names()})
    return dequantizing_weights({n: f.raw(n) for n in f.names()}, dtype or "f16", quantized == "device")


# ---------------------------------------------------------------- converter

def group_of(bits: int, cols: int, group_size=None) -> Optional[int]:
    """quant.ts:292-298."""
    g = DEFAULT_GROUP_SIZE if group_size is None else group_size
    size = cols if g == "row" else g
    if cols % size:
        return None
    if bits == 4 and (size % 2 or cols % 2):
        return None
    return size


def bits_of(name: str, bits: int, q8=()) -> int:
    """quant.ts:287-289: 8 for a q8-pattern tensor of a q4 checkpoint."""
    return 8 if bits == 4 and any(re.search(p, name) for p in q8) else bits


def should_quantize(name: str, dtype: str, shape, bits: int, group_size=None, embeddings: bool = True,
                    exclude=(), q8=()) -> bool:
    """quant.ts:276-284: the large 2-D float weights only."""
    if dtype not in ("F16", "BF16", "F32") or len(shape) != 2 or not name.endswith(".weight"):
        return False
    if re.search(r"(^|\.)(norm\d*|[a-z_]*norm)\.", name) or name == "type_emb.weight":
        return False
    if name.endswith("tok_embeddings.weight") and embeddings is False:
        return False
    if any(re.search(p, name) for p in exclude):
        return False
    rows, cols = shape
    if rows < 64:
        return False
    return group_of(bits_of(name, bits, q8), cols, group_size) is not None


def _to_f32(t: RawTensor) -> np.ndarray:
    a = np.asarray(t.data)
    if t.dtype == "BF16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def quantize_safetensors(source, bits: int, group_size=None, embeddings: bool = True, exclude=(), q8=(),
                         refine: bool = True, metadata: Optional[dict] = None) -> tuple:
    """quant.ts:314-360: a float checkpoint -> (quantized safetensors bytes,
    report).  Tensors are converted one at a time."""
    if bits not in (8, 4):
        raise ValueError(f"bits must be 8 or 4, got {bits}")
    g = DEFAULT_GROUP_SIZE if group_size is None else group_size
    if g != "row" and not (isinstance(g, int) and g > 0):
        raise ValueError(f'group size must be a positive integer or "row", got {g}')
    f = source if isinstance(source, SafetensorsFile) else read_safetensors(source)
    if quant_metadata(f.metadata) is not None:
        raise ValueError("laya quantize: the source checkpoint is already quantized")
    scheme = "q8" if bits == 8 else "q4"
    out = {}
    report = {"scheme": scheme, "group_size": g, "quantized": [], "promoted": [], "kept": [], "bytes_in": 0,
              "bytes_out": 0}
    dtypes = []
    for name in f.names():
        dt, shape = f.info(name)
        report["bytes_in"] += f.bytes(name).size
        m = re.match(r"^(.*)\.(scales|biases)$", name)
        if m and f.has(m.group(1)):
            raise ValueError(f"laya quantize: tensor name {name} collides with the quantization companions")
        if not should_quantize(name, dt, shape, bits, g, embeddings, exclude, q8):
            out[name] = RawTensor(dt, shape, f.array(name))
            report["kept"].append(name)
            continue
        if dt not in dtypes:
            dtypes.append(dt)
        rows, cols = shape
        b = bits_of(name, bits, q8)
        gs = group_of(b, cols, g)
        qv, s, z = quantize_matrix(_to_f32(f.raw(name)), rows, cols, b, gs, refine=(b == 4 and refine))
        G = cols // gs
        if b != bits:
            report["promoted"].append(name)
        if b == 8:
            out[name] = RawTensor("I8", (rows, cols), qv.astype(np.int8))
        else:
            qq = qv.astype(np.uint8)
            out[name] = RawTensor("U8", (rows, cols // 2), (qq[:, 0::2] | (qq[:, 1::2] << 4)).astype(np.uint8))
        out[name + ".scales"] = RawTensor("F16", (rows, G), s.astype(np.float16))
        if b == 4:
            out[name + ".biases"] = RawTensor("F16", (rows, G), z.astype(np.float16))
        report["quantized"].append(name)
    md = dict(metadata or {})
    md.update({"laya_quant": scheme, "group_size": str(g), "version": QUANT_FORMAT_VERSION,
               "laya_quant_source_dtype": ",".join(dtypes) or "none"})
    data = write_safetensors(out, md)
    report["bytes_out"] = len(data)
    return data, report
