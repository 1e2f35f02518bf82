"""Readers for the golden fixtures under tests/golden/.

The fixture files are copies of the reference's own test data (MIT /
Apache-2.0, laya-js): packages/tensor-backend/fixtures/{ops,ops-numerics,
ops-quantized}.json and packages/laya-fixtures/data/tiny/*.  The JSON
encoding is the one `decodeTensor` reads
(packages/tensor-backend/src/conformance.ts:58-86): base64 little-endian
element bytes, float dtypes always stored as f32.
"""
from __future__ import annotations

import base64
import json
import os
import struct

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

_NP = {"i32": np.int32, "bool": np.uint8, "u8": np.uint8, "i8": np.int8, "u16": np.uint16, "i16": np.int16,
       "u32": np.uint32, "u64": np.uint64, "i64": np.int64, "f64": np.float64}


def decode(e: dict | None):
    """EncodedTensor -> (dtype, numpy array)."""
    if e is None:
        return None
    raw = base64.b64decode(e["b64"])
    dt = _NP.get(e["dtype"], np.float32)
    a = np.frombuffer(raw, dtype=dt).reshape(e["shape"]).copy()
    return e["dtype"] if e["dtype"] in _NP else "f32", a


def arr(e: dict | None):
    d = decode(e)
    return None if d is None else d[1]


def load_cases(name: str = "ops.json") -> list[dict]:
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def case(name: str, file: str = "ops.json") -> dict:
    for c in load_cases(file):
        if c["name"] == name:
            return c
    raise KeyError(name)


def read_safetensors(path: str) -> dict[str, np.ndarray]:
    """Minimal safetensors reader for the tiny fixture checkpoint (F32/F16/I32)."""
    with open(path, "rb") as f:
        buf = f.read()
    n = struct.unpack("<Q", buf[:8])[0]
    header = json.loads(buf[8:8 + n])
    base = 8 + n
    out = {}
    dts = {"F32": np.float32, "F16": np.float16, "I32": np.int32, "I8": np.int8, "U8": np.uint8, "BF16": np.uint16}
    for k, v in header.items():
        if k == "__metadata__":
            continue
        s, e = v["data_offsets"]
        out[k] = np.frombuffer(buf[base + s:base + e], dtype=dts[v["dtype"]]).reshape(v["shape"]).copy()
    return out


def tiny():
    """(config json, encoder weights without the "encoder." prefix, activations json)."""
    with open(os.path.join(GOLDEN, "tiny", "encoder", "config.json")) as f:
        cfg = json.load(f)
    w = read_safetensors(os.path.join(GOLDEN, "tiny", "model.safetensors"))
    enc = {k[len("encoder."):]: v for k, v in w.items() if k.startswith("encoder.")}
    with open(os.path.join(GOLDEN, "tiny", "activations.json")) as f:
        act = json.load(f)
    return cfg, enc, act
