"""CPU oracle for the laya-js encoder path -- TEST INFRASTRUCTURE ONLY.

numpy/ctypes front end of ``oracle/cpu_ref.c``, a C restatement of the CPU
backend's arithmetic (backend-cpu = @johnhenry/math-plus-tensor-cpu@0.3.0,
packages/backend-cpu/src/index.ts:12-15): f32 storage, f64 accumulation.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, as the checker or as the timed CPU baseline.  The
product package (``laya-js_amd/laya_hip``) never imports it.

Every function here is pinned by a check in tests/test_oracle.py (fixture,
closed form or invariant); see the header of cpu_ref.c for the list.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libcpuref.so")
_lib = None

F32P = ctypes.POINTER(ctypes.c_float)
I64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compiles libcpuref.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "libcpuref.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.cr_f64_to_f16.restype = ctypes.c_uint16
        _lib.cr_f64_to_f16.argtypes = [ctypes.c_double]
        _lib.cr_f16_to_f64.restype = ctypes.c_double
        _lib.cr_f16_to_f64.argtypes = [ctypes.c_uint16]
        _lib.cr_num_threads.restype = ctypes.c_int
        _lib.cr_quantize_matrix.restype = ctypes.c_int
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def num_threads() -> int:
    return lib().cr_num_threads()


# ---------------------------------------------------------------- rounding

def f64_to_f16_bits(x: float) -> int:
    return int(lib().cr_f64_to_f16(float(x)))


def round_f16(x) -> np.ndarray:
    """Values rounded through binary16 storage (RNE), returned as f32."""
    y = _f32(x).copy()
    lib().cr_round_f16(_p(y), I64(y.size))
    return y


def f16_bits_to_f32(bits) -> np.ndarray:
    """IEEE binary16 bit patterns decoded exactly to f32."""
    h = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().cr_f16_bits_to_f32(_p(h), _p(out), I64(h.size))
    return out


def round_bf16(x) -> np.ndarray:
    """Values rounded through bfloat16 storage (RNE, NaN kept), as f32."""
    y = _f32(x).copy()
    lib().cr_round_bf16(_p(y), I64(y.size))
    return y


def round_to(x, dtype: str) -> np.ndarray:
    if dtype == "f16":
        return round_f16(x)
    if dtype == "bf16":
        return round_bf16(x)
    return _f32(x)


# ---------------------------------------------------------------- ops

def linear(x, w, b=None) -> np.ndarray:
    """y = x . w^T (+ b), f64 accumulation (tensor-backend/src/index.ts:211-215)."""
    x = _f32(x)
    w = _f32(w)
    K = x.shape[-1]
    N = w.shape[0]
    assert w.shape[1] == K
    M = x.size // K
    y = np.empty(x.shape[:-1] + (N,), np.float32)
    bb = _f32(b) if b is not None else None
    lib().cr_linear(_p(x), _p(w), _p(bb) if bb is not None else None, _p(y), I64(M), I64(N), I64(K))
    return y


def layer_norm(x, w=None, b=None, eps: float = 1e-5) -> np.ndarray:
    """LayerNorm over the last axis, f64 two-pass statistics (index.ts:216-217)."""
    x = _f32(x)
    D = x.shape[-1]
    y = np.empty_like(x)
    ww = _f32(w) if w is not None else None
    bb = _f32(b) if b is not None else None
    lib().cr_layernorm(_p(x), _p(ww) if ww is not None else None, _p(bb) if bb is not None else None, _p(y),
                       I64(x.size // D), I64(D), ctypes.c_double(eps))
    return y


def rope_table(L: int, D: int, base: float):
    c = np.empty((L, D // 2), np.float32)
    s = np.empty((L, D // 2), np.float32)
    lib().cr_rope_table(I64(L), I64(D), ctypes.c_double(base), _p(c), _p(s))
    return c, s


def rope(x, base: float) -> np.ndarray:
    """Split-half RoPE on x [..., L, D], positions 0..L-1 (index.ts:225-229)."""
    x = _f32(x)
    L, D = x.shape[-2], x.shape[-1]
    y = np.empty_like(x)
    lib().cr_rope(_p(x), _p(y), I64(x.size // (L * D)), I64(L), I64(D), ctypes.c_double(base))
    return y


def sdpa(q, k, v, mask, scale: float) -> np.ndarray:
    """Masked softmax attention, f64 softmax (index.ts:230-237); mask bool,
    broadcastable to [B, H, Lq, Lk]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, Lq, D = q.shape
    Lk = k.shape[2]
    o = np.empty_like(q)
    if mask is not None:
        m = np.ascontiguousarray(mask, dtype=np.uint8)
        while m.ndim < 4:
            m = m[None]
        strides = [0 if m.shape[i] == 1 else m.strides[i] for i in range(4)]
        ms = np.array(strides, np.int64)
        mp = _p(m)
    else:
        m = None
        ms = np.zeros(4, np.int64)
        mp = None
    lib().cr_sdpa(_p(q), _p(k), _p(v), mp, _p(ms), _p(o), I64(B), I64(H), I64(Lq), I64(Lk), I64(D),
                  ctypes.c_double(scale))
    return o


def gelu(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().cr_gelu(_p(x), _p(y), I64(x.size))
    return y


def erf(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().cr_erf(_p(x), _p(y), I64(x.size))
    return y


def geglu(x) -> np.ndarray:
    """gelu(value) * gate, [value, gate] = split(x, 2, -1) (compose.ts:86-93)."""
    x = _f32(x)
    F = x.shape[-1] // 2
    y = np.empty(x.shape[:-1] + (F,), np.float32)
    lib().cr_geglu(_p(x), _p(y), I64(x.size // (2 * F)), I64(F))
    return y


def embedding(table, ids) -> np.ndarray:
    table = _f32(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    V, D = table.shape
    out = np.empty(ids.shape + (D,), np.float32)
    lib().cr_embedding(_p(table), I64(V), I64(D), _p(ids), I64(ids.size), _p(out))
    return out


def mean_pool(x, mask) -> np.ndarray:
    x = _f32(x)
    m = np.ascontiguousarray(mask, dtype=np.uint8)
    B, L, D = x.shape
    out = np.empty((B, D), np.float32)
    lib().cr_meanpool(_p(x), _p(m), I64(B), I64(L), I64(D), _p(out))
    return out


# ---------------------------------------------------------------- quantized

def dequant_compose(q, scales, biases, group: int) -> np.ndarray:
    """compose.ts:379-398 dequantRows: f32(f32(q*s) + b)."""
    q = np.ascontiguousarray(q, dtype=np.int32)
    R, K = q.shape
    s = _f32(scales)
    b = _f32(biases) if biases is not None else None
    out = np.empty((R, K), np.float32)
    lib().cr_dequant_compose(_p(q), _p(s), _p(b) if b is not None else None, I64(R), I64(K), I64(group), _p(out))
    return out


def dequant_exact_f16(q, scales, biases, group: int) -> np.ndarray:
    """fl16(q*s + b) rounded once from the exact value (quant.ts:189-243), as f16 bits."""
    q = np.ascontiguousarray(q, dtype=np.int32)
    R, K = q.shape
    s = _f32(scales)
    b = _f32(biases) if biases is not None else None
    out = np.empty((R, K), np.uint16)
    lib().cr_dequant_exact_f16(_p(q), _p(s), _p(b) if b is not None else None, I64(R), I64(K), I64(group), _p(out))
    return out


def quantized_linear(x, q, scales, biases, group: int, bias=None, dtype: str = "f32") -> np.ndarray:
    """compose.ts:407-414: linear(x, dequantRows(...)) with the dequantized
    weight rounded once to x's dtype."""
    w = round_to(dequant_compose(q, scales, biases, group), dtype)
    return linear(x, w, bias)


def quantize_matrix(values, rows: int, cols: int, bits: int, group: int | None = None, refine: bool = True):
    """quantizeMatrix (laya/src/quant.ts:96-129) -> (q int32 [rows, cols],
    scales f16 bits [rows, G], biases f16 bits [rows, G] | None)."""
    group = cols if group is None else group
    v = _f32(values).reshape(rows, cols)
    G = cols // group
    q = np.empty((rows, cols), np.int32)
    s = np.empty((rows, G), np.uint16)
    b = np.empty((rows, G), np.uint16) if bits == 4 else None
    rc = lib().cr_quantize_matrix(_p(v), I64(rows), I64(cols), ctypes.c_int(bits), I64(group),
                                  ctypes.c_int(8 if refine else 0), _p(q), _p(s), _p(b) if b is not None else None)
    if rc != 0:
        raise ValueError(f"quantize_matrix: bad shape [{rows}, {cols}] bits {bits} group {group}")
    return q, s, b


def attention_masks(valid, B: int, L: int, window: int):
    """modernbert/src/index.ts:240-259 -> (full [B,1,1,L], sliding [B,1,L,L]) uint8."""
    v = np.ascontiguousarray(valid, dtype=np.uint8).reshape(B * L)
    full = np.empty((B, 1, 1, L), np.uint8)
    sliding = np.empty((B, 1, L, L), np.uint8)
    lib().cr_attention_masks(_p(v), I64(B), I64(L), I64(window), _p(full), _p(sliding))
    return full, sliding


# ---------------------------------------------------------------- encoder

@dataclass
class EncoderConfig:
    """The ModernBERT config fields the encoder path reads
    (modernbert/src/index.ts:58-110 defaults)."""
    hidden: int
    layers: int
    heads: int
    intermediate: int
    vocab: int
    local_attention: int = 128
    global_every: int = 3
    norm_eps: float = 1e-5
    global_theta: float = 160000.0
    local_theta: float = 10000.0
    layer_types: list = field(default_factory=list)

    def __post_init__(self):
        if not self.layer_types:
            self.layer_types = ["full_attention" if i % self.global_every == 0 else "sliding_attention"
                                for i in range(self.layers)]

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @staticmethod
    def from_json(j: dict) -> "EncoderConfig":
        return EncoderConfig(hidden=j["hidden_size"], layers=j["num_hidden_layers"], heads=j["num_attention_heads"],
                             intermediate=j["intermediate_size"], vocab=j["vocab_size"],
                             local_attention=j.get("local_attention", 128),
                             global_every=j.get("global_attn_every_n_layers", 3),
                             norm_eps=j.get("norm_eps", 1e-5),
                             global_theta=j.get("global_rope_theta", 160000.0),
                             local_theta=j.get("local_rope_theta", 10000.0),
                             layer_types=list(j.get("layer_types") or []))


def encoder_layer(cfg: EncoderConfig, W: dict, i: int, x: np.ndarray, mask: np.ndarray,
                  dtype: str = "f32") -> np.ndarray:
    """One pre-norm layer, op for op as modernbert/src/index.ts:342-357.
    ``dtype`` != "f32" rounds every op's result through that storage type,
    as a backend storing activations in f16/bf16 would."""
    r = lambda a: round_to(a, dtype)  # noqa: E731
    B, L, H = x.shape
    nh, hd = cfg.heads, cfg.head_dim
    p = f"layers.{i}."
    h = r(layer_norm(x, W.get(p + "attn_norm.weight"), None, cfg.norm_eps)) if (p + "attn_norm.weight") in W else x
    qkv = r(linear(h, W[p + "attn.Wqkv.weight"], W.get(p + "attn.Wqkv.bias")))
    qkv = qkv.reshape(B, L, 3, nh, hd).transpose(2, 0, 3, 1, 4)
    q, k, v = (np.ascontiguousarray(t) for t in qkv)
    kind = cfg.layer_types[i]
    base = cfg.global_theta if kind == "full_attention" else cfg.local_theta
    att = r(sdpa(r(rope(q, base)), r(rope(k, base)), v, mask, hd ** -0.5))
    merged = np.ascontiguousarray(att.transpose(0, 2, 1, 3)).reshape(B, L, H)
    x1 = r(x + r(linear(merged, W[p + "attn.Wo.weight"], W.get(p + "attn.Wo.bias"))))
    m = r(linear(r(layer_norm(x1, W[p + "mlp_norm.weight"], None, cfg.norm_eps)), W[p + "mlp.Wi.weight"],
                 W.get(p + "mlp.Wi.bias")))
    g = r(geglu(m))
    return r(x1 + r(linear(g, W[p + "mlp.Wo.weight"], W.get(p + "mlp.Wo.bias"))))


def encoder_forward(cfg: EncoderConfig, W: dict, ids: np.ndarray, valid: np.ndarray, dtype: str = "f32",
                    layers: int | None = None, stages: dict | None = None) -> np.ndarray:
    """embeddings -> layers -> final_norm (modernbert/src/index.ts:407-429).
    W maps names without the "encoder." prefix to f32 arrays (already rounded
    to ``dtype`` by the caller when simulating reduced storage)."""
    r = lambda a: round_to(a, dtype)  # noqa: E731
    B, L = ids.shape
    full, sliding = attention_masks(valid, B, L, cfg.local_attention)
    x = r(layer_norm(r(embedding(W["embeddings.tok_embeddings.weight"], ids)), W["embeddings.norm.weight"], None,
                     cfg.norm_eps))
    if stages is not None:
        stages["embeddings"] = x
    n = cfg.layers if layers is None else layers
    for i in range(n):
        mask = full if cfg.layer_types[i] == "full_attention" else sliding
        x = encoder_layer(cfg, W, i, x, mask, dtype)
        if stages is not None:
            stages[f"layers.{i}"] = x
    y = r(layer_norm(x, W["final_norm.weight"], None, cfg.norm_eps))
    if stages is not None:
        stages["final_norm"] = y
    return y


# ---------------------------------------------------------------- decision head

HEAD_EPS = 1e-5


def head_layer(W: dict, j: int, x: np.ndarray, mask: np.ndarray, heads: int) -> np.ndarray:
    """PyTorch pre-norm TransformerEncoderLayer with a ReLU FFN, op for op as
    laya/src/model.ts:124-138 (names as in laya-mlx checkpoints)."""
    B, L, D = x.shape
    hd = D // heads
    p = f"head.layers.{j}."
    h = layer_norm(x, W[p + "norm1.weight"], W[p + "norm1.bias"], HEAD_EPS)
    qkv = linear(h, W[p + "self_attn.in_proj.weight"], W[p + "self_attn.in_proj.bias"])
    qkv = qkv.reshape(B, L, 3, heads, hd).transpose(2, 0, 3, 1, 4)
    q, k, v = (np.ascontiguousarray(t) for t in qkv)
    att = sdpa(q, k, v, mask, hd ** -0.5)
    att = np.ascontiguousarray(att.transpose(0, 2, 1, 3)).reshape(B, L, D)
    x1 = x + linear(att, W[p + "self_attn.out_proj.weight"], W[p + "self_attn.out_proj.bias"])
    f = linear(np.maximum(linear(layer_norm(x1, W[p + "norm2.weight"], W[p + "norm2.bias"], HEAD_EPS),
                                 W[p + "linear1.weight"], W[p + "linear1.bias"]), np.float32(0)),
               W[p + "linear2.weight"], W[p + "linear2.bias"])
    return x1 + f


def softmax_rows(x) -> np.ndarray:
    """Softmax over the last axis in f64, stored f32."""
    z = np.asarray(x, np.float64)
    e = np.exp(z - z.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(np.float32)


def decision_forward(cfg: EncoderConfig, W: dict, head_layers: int, ids: np.ndarray, valid: np.ndarray,
                     qtype: np.ndarray, marker_pos: np.ndarray, marker_mask: np.ndarray,
                     stages: dict | None = None, enc_out: np.ndarray | None = None):
    """laya's DecisionModel.forwardCore (laya/src/model.ts:178-236) in f32
    storage: the encoder (``W`` names carry the "encoder." prefix), the type
    embedding, ``head_layers`` head layers, the marker scorer and the action
    head.  Returns (logits [B, M] f32 with masked slots -1e4, act [B, nAct]).
    ``enc_out`` skips the encoder with its precomputed final-norm output."""
    B, L = ids.shape
    M = marker_pos.shape[1]
    D = cfg.hidden
    if enc_out is None:
        encW = {k[len("encoder."):]: v for k, v in W.items() if k.startswith("encoder.")}
        enc_stages = {} if stages is not None else None
        enc_out = encoder_forward(cfg, encW, ids, valid, stages=enc_stages)
        if stages is not None:
            for k, v in enc_stages.items():
                stages["embeddings" if k == "embeddings" else f"encoder.{k}"] = v
    h = enc_out + embedding(W["type_emb.weight"], np.asarray(qtype, np.int32))[:, None, :]
    if stages is not None:
        stages["type_emb_added"] = h
    head_mask = (np.asarray(valid).reshape(B, 1, 1, L) != 0).astype(np.uint8)
    heads = max(1, D // 64)
    for j in range(head_layers):
        h = head_layer(W, j, h, head_mask, heads)
        if stages is not None:
            stages[f"head.layers.{j}"] = h
    pos = np.maximum(np.asarray(marker_pos, np.int64), 0)
    markers = np.ascontiguousarray(h[np.arange(B)[:, None], pos])
    s1 = gelu(linear(layer_norm(markers, W["scorer.layers.0.weight"], W["scorer.layers.0.bias"], HEAD_EPS),
                     W["scorer.layers.1.weight"], W["scorer.layers.1.bias"]))
    scored = linear(s1, W["scorer.layers.3.weight"], W["scorer.layers.3.bias"]).reshape(B, M)
    mm = np.asarray(marker_mask).reshape(B, M) != 0
    logits = np.where(mm, scored, np.float32(-1e4)).astype(np.float32)
    p = softmax_rows(logits)
    plogp = p * np.log(np.maximum(p, np.float32(1e-9)).astype(np.float64)).astype(np.float32)
    k = np.maximum(mm.sum(1), 2).astype(np.float32)
    entropy = (plogp.astype(np.float64).sum(-1).astype(np.float32) * np.float32(-1)) / \
        np.log(k.astype(np.float64)).astype(np.float32)
    top = np.sort(p, -1)[:, M - 2:]
    top2, top1 = top[:, 0:1], top[:, 1:2]
    features = np.concatenate([top1, top1 - top2, entropy.reshape(B, 1), k.reshape(B, 1) / np.float32(255)], -1)
    pooled = np.concatenate([h[:, 0, :], features], -1).astype(np.float32)
    act = linear(gelu(linear(pooled, W["act_head.layers.0.weight"], W["act_head.layers.0.bias"])),
                 W["act_head.layers.2.weight"], W["act_head.layers.2.bias"])
    if stages is not None:
        stages["logits"] = logits
        stages["act"] = act
    return logits, act
