"""Replays the reference's conformance fixtures on a Backend, following
packages/tensor-backend/src/conformance.ts:117-320: every case in f32, then
in f16 and bf16 with inputs cast on the device and the tolerance floored at
2e-2 / 5e-2; optional ops through their compose helper; quantized cases
through upload_quantized."""
from __future__ import annotations

import numpy as np

from fixtures import decode
from laya_hip import compose as C
from laya_hip.host import HostQuantized, HostTensor, pack_quantized, to_f32, to_f64

REDUCED_TOLERANCE = {"f16": 2e-2, "bf16": 5e-2}
UNARY_NUMERICS = {"logicalNot", "sqrt", "rsqrt", "neg", "abs", "tanh", "sigmoid", "erf"}
BINARY_NUMERICS = {"equal", "notEqual", "less", "lessEqual", "greater", "greaterEqual", "logicalAnd", "logicalOr",
                   "pow"}
REDUCE_NUMERICS = {"argmax", "argmin", "mean", "min"}
QUANTIZED_CASE_OPS = {"quantizedLinear", "quantizedEmbedding"}
FOLLOWS_RUN = {"f32", "f16", "bf16"}


def host_of(e) -> HostTensor:
    dt, a = decode(e)
    return HostTensor(dt, tuple(a.shape), a)


def upload(b, h: HostTensor, dtype: str):
    if h.dtype != "f32" or dtype == "f32":
        return b.fromHost(h)
    f = b.fromHost(h)
    c = b.cast(f, dtype)
    b.dispose(f)
    return c


def case_quantized(c, first: int) -> HostQuantized:
    a = c["args"]
    q = host_of(c["inputs"][first])
    scales = host_of(c["inputs"][first + 1])
    bb = c["inputs"][first + 2]
    N, K = q.shape
    return HostQuantized((N, K), a["bits"], a["groupSize"], a["mode"], pack_quantized(q.data, a["bits"]), scales,
                         host_of(bb) if bb else None)


def run_quantized(b, c, dtype, owned):
    q = None
    try:
        if c["op"] == "quantizedLinear":
            x = upload(b, host_of(c["inputs"][0]), dtype)
            owned.append(x)
            bias = upload(b, host_of(c["inputs"][4]), dtype) if c["inputs"][4] else None
            if bias is not None:
                owned.append(bias)
            q = C.upload_quantized(b, case_quantized(c, 1), dtype)
            return C.quantized_linear(b, x, q, bias)
        ids = b.fromHost(host_of(c["inputs"][3]))
        owned.append(ids)
        q = C.upload_quantized(b, case_quantized(c, 0), dtype)
        return C.quantized_embedding(b, q, ids)
    finally:
        if q is not None:
            owned.extend([q.w, q.scales] + ([q.biases] if q.biases is not None else []))


def call_op(b, c, xs):
    a = c["args"]
    op = c["op"]
    x = xs[0]
    if op in UNARY_NUMERICS:
        return getattr(C, op)(b, x)
    if op in BINARY_NUMERICS:
        return getattr(C, op)(b, x, xs[1])
    if op in REDUCE_NUMERICS:
        return getattr(C, op)(b, x, a["axis"], a.get("keepDims", False))
    if op == "cumsum":
        return C.cumsum(b, x, a["axis"])
    if op in ("add", "sub", "mul", "div", "maximum"):
        return getattr(b, op)(x, xs[1])
    if op == "where":
        return b.where(x, xs[1], xs[2])
    if op == "scale":
        return b.scale(x, a["s"])
    if op in ("exp", "log", "relu", "gelu"):
        return getattr(b, op)(x)
    if op in ("sum", "max"):
        return getattr(b, op)(x, a["axis"], a.get("keepDims", False))
    if op in ("softmax", "sort"):
        return getattr(b, op)(x, a["axis"])
    if op == "matmul":
        return b.matmul(x, xs[1])
    if op == "linear":
        return b.linear(x, xs[1], xs[2])
    if op == "layerNorm":
        return b.layerNorm(x, xs[1], xs[2], a["eps"])
    if op == "embedding":
        return b.embedding(x, xs[1])
    if op == "gatherRows":
        return b.gatherRows(x, xs[1])
    if op == "rope":
        return b.rope(x, a["base"])
    if op == "sdpa":
        return b.sdpa(x, xs[1], xs[2], xs[3], a["scale"])
    if op == "reshape":
        return b.reshape(x, a["shape"])
    if op == "transpose":
        return b.transpose(x, a["perm"])
    if op == "slice":
        return b.slice(x, a["begin"], a["end"])
    if op == "split":
        return b.split(x, a["parts"], a["axis"])
    if op == "concat":
        return b.concat(xs, a["axis"])
    if op == "cast":
        return b.cast(x, a["dtype"])
    if op == "geglu":
        return C.geglu(b, x)
    if op == "meanPool":
        return C.mean_pool(b, x, xs[1])
    raise ValueError(f"conformance: unknown op {op}")


def close_report(got, want, atol, rtol):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    if got.shape != want.shape:
        return f"length {got.size} != {want.size}"
    if np.any(np.isnan(got) != np.isnan(want)):
        return "NaN mismatch"
    with np.errstate(invalid="ignore"):
        err = np.abs(got - want) - (atol + rtol * np.abs(want))
    err = np.nan_to_num(err, nan=0.0)
    i = int(np.argmax(err))
    if err[i] > 0:
        return f"[{i}] got {got[i]} want {want[i]} (atol {atol}, rtol {rtol})"
    return None


def applicable(b, c) -> bool:
    return not (c.get("nativeOnly") and c["op"] in C.NUMERICS_OPS and not C.has_native(b, c["op"]))


def case_supported(b, c) -> bool:
    fixed = [e["dtype"] for e in list(c["inputs"]) + list(c["outputs"]) if e and e["dtype"] not in FOLLOWS_RUN]
    if c["op"] == "cast" and c["args"].get("dtype") not in FOLLOWS_RUN:
        fixed.append(c["args"]["dtype"])
    return all(b.supports(d) for d in fixed)


def run_case(b, c, dtype):
    """Returns None on success or a failure message."""
    quantized = c["op"] in QUANTIZED_CASE_OPS
    xs = [] if quantized else [upload(b, host_of(e), dtype) if e else None for e in c["inputs"]]
    outs = []
    try:
        out = run_quantized(b, c, dtype, xs) if quantized else call_op(b, c, xs)
        outs = list(out) if isinstance(out, (list, tuple)) else [out]
        if len(outs) != len(c["outputs"]):
            return f"{c['name']}: {len(outs)} outputs, want {len(c['outputs'])}"
        tol = REDUCED_TOLERANCE.get(dtype, 0.0)
        for i, o in enumerate(outs):
            want = host_of(c["outputs"][i])
            got = b.read(o)
            if tuple(got.shape) != tuple(want.shape):
                return f"{c['name']}: shape {list(got.shape)} want {list(want.shape)}"
            if c["op"] in C.NUMERICS_OPS and want.dtype not in FOLLOWS_RUN and got.dtype != want.dtype:
                return f"{c['name']}[{i}] {dtype}: dtype {got.dtype} want {want.dtype}"
            conv = to_f64 if (want.dtype == "f64" or got.dtype == "f64") else to_f32
            msg = close_report(conv(got), conv(want), max(c["atol"], tol), max(c["rtol"], tol))
            if msg:
                return f"{c['name']}[{i}] {dtype}: {msg}"
        return None
    finally:
        for t in xs + outs:
            if t is not None:
                b.dispose(t)


def run_all(b, cases, dtype):
    failures = []
    ran = 0
    for c in cases:
        if dtype != "f32" and c.get("f32Only"):
            continue
        if not applicable(b, c) or not case_supported(b, c):
            continue
        ran += 1
        try:
            msg = run_case(b, c, dtype)
        except Exception as e:  # a thrown op error is a failure of that case
            msg = f"{c['name']} {dtype}: {type(e).__name__}: {e}"
        if msg:
            failures.append(msg)
    return ran, failures
