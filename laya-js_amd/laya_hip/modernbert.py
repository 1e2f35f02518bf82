"""The ModernBERT encoder over `Backend` ops, restated from
packages/modernbert/src/index.ts so it runs unchanged on any backend: it
calls only contract ops and compose helpers.  This is the caller of the hot
path (`layer`, index.ts:342-357).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Optional

import numpy as np

from .compose import dispose_quantized, embedding_any, geglu, is_quantized, linear_any, mean_pool, upload_quantized
from .host import HostQuantized, HostTensor, to_f32

FLOATS = ("f32", "f16", "bf16")


@dataclass(frozen=True)
class ModernBertConfig:
    vocabSize: int
    hiddenSize: int
    intermediateSize: int
    numHiddenLayers: int
    numAttentionHeads: int
    headDim: int
    normEps: float
    normBias: bool
    attentionBias: bool
    mlpBias: bool
    localAttention: int
    globalAttnEveryNLayers: int
    maxPositionEmbeddings: int
    layerTypes: tuple
    ropeBase: dict = field(hash=False)
    modelType: str = "modernbert"
    hiddenActivation: str = "gelu"


def parseModernBertConfig(j: dict) -> ModernBertConfig:
    """index.ts:58-110 (EncoderConfig.from_dict with its validation)."""
    mt = j.get("model_type", "modernbert")
    if mt is None:
        mt = "modernbert"
    if mt != "modernbert":
        raise ValueError(f"Unsupported encoder: {mt!r}; expected modernbert")
    act = j.get("hidden_activation") or "gelu"
    if act != "gelu":
        raise ValueError(f"Unsupported encoder activation: {act!r}")

    def integer(name, fallback=None):
        v = j.get(name)
        if v is None and fallback is not None:
            return fallback
        if not isinstance(v, int) or isinstance(v, bool):
            raise TypeError(f"modernbert config: {name} must be an integer")
        return v

    def number(name, fallback):
        v = j.get(name)
        if v is None:
            return fallback
        if not isinstance(v, (int, float)) or isinstance(v, bool):
            raise TypeError(f"modernbert config: {name} must be a number")
        return float(v)

    H = integer("hidden_size")
    nh = integer("num_attention_heads")
    L = integer("num_hidden_layers")
    if nh <= 0 or H % nh or (H // nh) % 2:
        raise ValueError("ModernBERT requires an even, integral attention head dimension")
    every = integer("global_attn_every_n_layers", 3)
    lt = j.get("layer_types")
    if lt is None:
        lt = ["full_attention" if i % every == 0 else "sliding_attention" for i in range(L)]
    if not isinstance(lt, list) or len(lt) != L or any(k not in ("full_attention", "sliding_attention") for k in lt):
        raise ValueError("Invalid ModernBERT layer_types")
    rp = j.get("rope_parameters") or {}
    for kind in set(lt):
        if ((rp.get(kind) or {}).get("rope_type") or "default") != "default":
            raise ValueError("Only default (unscaled) ModernBERT RoPE is supported")
    gt = number("global_rope_theta", 160000.0)
    lth = number("local_rope_theta", 10000.0)
    base = {"full_attention": float((rp.get("full_attention") or {}).get("rope_theta") or gt),
            "sliding_attention": float((rp.get("sliding_attention") or {}).get("rope_theta") or lth)}
    return ModernBertConfig(
        vocabSize=integer("vocab_size"), hiddenSize=H, intermediateSize=integer("intermediate_size"),
        numHiddenLayers=L, numAttentionHeads=nh, headDim=H // nh, normEps=number("norm_eps", 1e-5),
        normBias=bool(j.get("norm_bias") or False), attentionBias=bool(j.get("attention_bias") or False),
        mlpBias=bool(j.get("mlp_bias") or False), localAttention=integer("local_attention", 128),
        globalAttnEveryNLayers=every, maxPositionEmbeddings=integer("max_position_embeddings", 8192),
        layerTypes=tuple(lt), ropeBase=base)


def attentionMasks(attention_mask: np.ndarray, B: int, L: int, window: int):
    """index.ts:240-259: full [B,1,1,L] = valid[b, j]; sliding [B,1,L,L] =
    (|i-j| <= window//2 OR query i padded) AND valid[b, j]."""
    m = np.asarray(attention_mask).reshape(B, L) != 0
    if m.size != B * L:
        raise ValueError(f"attentionMasks: mask has {m.size} values, want {B * L}")
    half = window // 2
    i = np.arange(L)
    near = np.abs(i[:, None] - i[None, :]) <= half
    pad_q = ~m[:, :, None]
    sliding = (near[None] | pad_q) & m[:, None, :]
    return (HostTensor("bool", (B, 1, 1, L), m.astype(np.uint8).reshape(B, 1, 1, L)),
            HostTensor("bool", (B, 1, L, L), sliding.astype(np.uint8).reshape(B, 1, L, L)))


def is_host_quantized(h) -> bool:
    return isinstance(h, HostQuantized)


def dispose_weight(b, w) -> None:
    if w is None:
        return
    if is_quantized(w):
        dispose_quantized(b, w)
    else:
        b.dispose(w)


def upload_as(b, h, dtype: str):
    """index.ts:175-188."""
    if is_host_quantized(h):
        if not b.supports(dtype):
            raise RuntimeError(f"{b.name} backend does not support {dtype}")
        return upload_quantized(b, h, dtype)
    if h.dtype not in FLOATS:
        return b.fromHost(h)
    if not b.supports(dtype):
        raise RuntimeError(f"{b.name} backend does not support {dtype}")
    src = h if (h.dtype == dtype or b.supports(h.dtype)) else HostTensor("f32", h.shape, to_f32(h))
    t = b.fromHost(src)
    if t.dtype == dtype:
        return t
    c = b.cast(t, dtype)
    b.dispose(t)
    return c


class ModernBert:
    def __init__(self, backend, config: ModernBertConfig, weights: dict, dtype: str):
        self.backend = backend
        self.config = config
        self.weights = weights
        self.dtype = dtype

    def embeddings(self, ids):
        """Token embeddings + LayerNorm (index.ts:336-339)."""
        b, w = self.backend, self.weights
        return b.scope(lambda: b.layerNorm(embedding_any(b, w["tok"], ids), w["emb_norm"], w.get("emb_norm_b"),
                                           self.config.normEps))

    def layer(self, i: int, x, mask):
        """One pre-norm encoder layer (index.ts:342-357)."""
        b, c, w = self.backend, self.config, self.weights["layers"][i]

        def f():
            B, L, H = x.shape
            nh, hd = c.numAttentionHeads, c.headDim
            h = b.layerNorm(x, w["attn_norm"], w.get("attn_norm_b"), c.normEps) if w["attn_norm"] is not None else x
            qkv = b.transpose(b.reshape(linear_any(b, h, w["Wqkv"], w.get("Wqkv_b")), [B, L, 3, nh, hd]),
                              [2, 0, 3, 1, 4])
            q, k, v = [b.reshape(t, [B, nh, L, hd]) for t in b.split(qkv, 3, 0)]
            base = c.ropeBase[w["kind"]]
            att = b.sdpa(b.rope(q, base), b.rope(k, base), v, mask, hd ** -0.5)
            merged = b.reshape(b.transpose(att, [0, 2, 1, 3]), [B, L, H])
            x1 = b.add(x, linear_any(b, merged, w["Wo"], w.get("Wo_b")))
            m = linear_any(b, b.layerNorm(x1, w["mlp_norm"], w.get("mlp_norm_b"), c.normEps), w["Wi"], w.get("Wi_b"))
            return b.add(x1, linear_any(b, geglu(b, m), w["WoMlp"], w.get("WoMlp_b")))
        return b.scope(f)

    def finalNorm(self, x):
        b, w = self.backend, self.weights
        return b.scope(lambda: b.layerNorm(x, w["final_norm"], w.get("final_norm_b"), self.config.normEps))

    def uploadInputs(self, input_ids: np.ndarray, attention_mask: np.ndarray, B: int, L: int) -> dict:
        """index.ts:369-381."""
        b, c = self.backend, self.config
        if np.asarray(input_ids).size != B * L:
            raise ValueError(f"modernbert: inputIds has {np.asarray(input_ids).size} values, want {B * L}")
        full, sliding = attentionMasks(attention_mask, B, L, c.localAttention)
        done = {}
        try:
            done["ids"] = b.fromHost(HostTensor("i32", (B, L), np.asarray(input_ids, np.int32).reshape(B, L)))
            done["mask"] = b.fromHost(HostTensor("bool", (B, L), np.asarray(attention_mask).reshape(B, L) != 0))
            if "full_attention" in c.layerTypes:
                done["full"] = b.fromHost(full)
            if "sliding_attention" in c.layerTypes:
                done["sliding"] = b.fromHost(sliding)
        except BaseException:
            for t in done.values():
                b.dispose(t)
            raise
        return {"ids": done["ids"], "mask": done["mask"],
                "masks": {"full_attention": done.get("full"), "sliding_attention": done.get("sliding")}}

    def disposeInputs(self, inp: dict) -> None:
        for t in (inp["ids"], inp["mask"], inp["masks"]["full_attention"], inp["masks"]["sliding_attention"]):
            if t is not None:
                self.backend.dispose(t)

    def forward(self, input_ids, attention_mask, B: int, L: int, onStage: Optional[Callable] = None):
        inp = self.uploadInputs(input_ids, attention_mask, B, L)
        try:
            return self.encode(inp, onStage)
        finally:
            self.disposeInputs(inp)

    def encode(self, inp: dict, onStage: Optional[Callable] = None):
        """index.ts:407-429: embeddings -> layers -> final norm; `onStage(name,
        t)` returning True takes ownership of a stage output."""
        b, c = self.backend, self.config
        kept = []

        def emit(name, t, last):
            if onStage is not None and onStage(name, t) is True and not last:
                kept.append(t)

        def f():
            masks = inp["masks"]
            x = self.embeddings(inp["ids"])
            emit("embeddings", x, False)
            for i in range(c.numHiddenLayers):
                nxt = self.layer(i, x, masks[c.layerTypes[i]])
                if not any(k is x for k in kept):
                    b.dispose(x)
                x = nxt
                emit(f"layers.{i}", x, False)
            y = self.finalNorm(x)
            if not any(k is x for k in kept):
                b.dispose(x)
            emit("final_norm", y, True)
            return [y, *kept]
        return b.scope(f)[0]

    def embed(self, input_ids, attention_mask, B: int, L: int):
        """Mean-pooled sentence vectors [B, H] f32 (index.ts:435-443)."""
        b = self.backend
        inp = self.uploadInputs(input_ids, attention_mask, B, L)
        try:
            return b.scope(lambda: mean_pool(b, self.encode(inp), inp["mask"]))
        finally:
            self.disposeInputs(inp)

    def dispose(self) -> None:
        b, w = self.backend, self.weights
        for k in ("tok", "emb_norm", "emb_norm_b", "final_norm", "final_norm_b"):
            dispose_weight(b, w.get(k))
        for lw in w["layers"]:
            for k, v in lw.items():
                if k != "kind":
                    dispose_weight(b, v)


def detectPrefix(get: Callable) -> str:
    for p in ("encoder.", "model.", ""):
        if get(f"{p}embeddings.tok_embeddings.weight") is not None:
            return p
    raise ValueError("modernbert: no embeddings.tok_embeddings.weight under prefixes encoder., model. or ''")


def loadModernBert(backend, config: ModernBertConfig, weights, dtype: str = "f32",
                   prefix: Optional[str] = None) -> ModernBert:
    """index.ts:498-559: validates names and shapes first, then uploads every
    tensor; a failure frees whatever was uploaded."""
    if not backend.supports(dtype):
        raise RuntimeError(f"{backend.name} backend does not support {dtype}")
    get = weights if callable(weights) else weights.get
    prefix = detectPrefix(get) if prefix is None else prefix
    H, I = config.hiddenSize, config.intermediateSize
    need = {}

    def req(name, shape, matrix=False):
        key = prefix + name
        h = get(key)
        if h is None:
            raise ValueError(f"modernbert: missing weight {key}")
        if tuple(h.shape) != tuple(shape):
            raise ValueError(f"modernbert: {key} has shape [{','.join(map(str, h.shape))}], "
                             f"want [{','.join(map(str, shape))}]")
        if not matrix and is_host_quantized(h):
            raise ValueError(f"modernbert: {key} cannot be quantized (only Linear weights and the token embedding)")
        need[key] = h
        return key

    tree = {"tok": req("embeddings.tok_embeddings.weight", (config.vocabSize, H), True),
            "emb_norm": req("embeddings.norm.weight", (H,)),
            "final_norm": req("final_norm.weight", (H,)), "layers": []}
    if config.normBias:
        tree["emb_norm_b"] = req("embeddings.norm.bias", (H,))
        tree["final_norm_b"] = req("final_norm.bias", (H,))
    for i in range(config.numHiddenLayers):
        p = f"layers.{i}."
        lw = {"kind": config.layerTypes[i],
              "attn_norm": None if i == 0 else req(p + "attn_norm.weight", (H,)),
              "Wqkv": req(p + "attn.Wqkv.weight", (3 * H, H), True), "Wo": req(p + "attn.Wo.weight", (H, H), True),
              "mlp_norm": req(p + "mlp_norm.weight", (H,)), "Wi": req(p + "mlp.Wi.weight", (2 * I, H), True),
              "WoMlp": req(p + "mlp.Wo.weight", (H, I), True)}
        if config.normBias:
            if i:
                lw["attn_norm_b"] = req(p + "attn_norm.bias", (H,))
            lw["mlp_norm_b"] = req(p + "mlp_norm.bias", (H,))
        if config.attentionBias:
            lw["Wqkv_b"] = req(p + "attn.Wqkv.bias", (3 * H,))
            lw["Wo_b"] = req(p + "attn.Wo.bias", (H,))
        if config.mlpBias:
            lw["Wi_b"] = req(p + "mlp.Wi.bias", (2 * I,))
            lw["WoMlp_b"] = req(p + "mlp.Wo.bias", (H,))
        tree["layers"].append(lw)
    uploaded = {}
    try:
        for key, h in need.items():
            uploaded[key] = upload_as(backend, h, dtype)
    except BaseException:
        for t in uploaded.values():
            dispose_weight(backend, t)
        raise

    def resolve(v):
        return uploaded[v] if isinstance(v, str) and v in uploaded else v
    w = {k: resolve(v) for k, v in tree.items() if k != "layers"}
    w["layers"] = [{k: (v if k == "kind" else resolve(v)) for k, v in lw.items()} for lw in tree["layers"]]
    return ModernBert(backend, config, w, dtype)
