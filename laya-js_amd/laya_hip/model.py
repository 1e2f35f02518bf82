"""laya's DecisionModel over `Backend` ops, restated from
packages/laya/src/model.ts so that it runs unchanged on any backend: the
ModernBERT encoder, the question-type embedding, PyTorch-style pre-norm
decision-head layers, the marker scorer and the action head.  It calls only
contract ops and compose helpers, like the encoder driver in modernbert.py.

Also `loadDecisionModel` (model.ts:283-338, the weight names and shapes of
buildHeadWeights :340-385) and `loadCheckpoint`, the part of laya's `load()`
(load.ts:45-92) that turns a local checkpoint directory into a model.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass
from typing import Callable, Optional

import numpy as np

from .compose import embedding_any, is_quantized, linear_any
from .host import HostTensor
from .modernbert import (ModernBertConfig, attentionMasks, dispose_weight, is_host_quantized, loadModernBert,
                         parseModernBertConfig, upload_as)

HEAD_EPS = 1e-5  # PyTorch / MLX nn.LayerNorm default (model.ts:30)


@dataclass
class Batch:
    """One collated batch (laya-core's `Batch`): ids and masks row-major
    [size, length], markers [size, markerCount]."""
    size: int
    length: int
    markerCount: int
    inputIds: np.ndarray
    attentionMask: np.ndarray
    markerPos: np.ndarray
    markerMask: np.ndarray
    qtype: np.ndarray


class DecisionModel:
    """model.ts:97-269."""

    def __init__(self, backend, encoder, weights: dict, dtype: str, nAct: int):
        self.backend = backend
        self.encoder = encoder
        self.weights = weights
        self.dtype = dtype
        self.nAct = nAct
        self.hiddenSize = encoder.config.hiddenSize
        self.headHeads = max(1, self.hiddenSize // 64)

    def headLayer(self, j: int, x, mask):
        """PyTorch pre-norm nn.TransformerEncoderLayer with a ReLU FFN; mask
        bool [B, 1, 1, L] (model.ts:124-138)."""
        b, w = self.backend, self.weights["head"][j]

        def f():
            B, L, D = x.shape
            nh = self.headHeads
            hd = D // nh
            h = b.layerNorm(x, w["norm1"], w["norm1_b"], HEAD_EPS)
            qkv = b.transpose(b.reshape(linear_any(b, h, w["inProj"], w["inProjBias"]), [B, L, 3, nh, hd]),
                              [2, 0, 3, 1, 4])
            q, k, v = [b.reshape(t, [B, nh, L, hd]) for t in b.split(qkv, 3, 0)]
            att = b.reshape(b.transpose(b.sdpa(q, k, v, mask, hd ** -0.5), [0, 2, 1, 3]), [B, L, D])
            x1 = b.add(x, linear_any(b, att, w["outProj"], w["outProjBias"]))
            n2 = b.layerNorm(x1, w["norm2"], w["norm2_b"], HEAD_EPS)
            f_ = linear_any(b, b.relu(linear_any(b, n2, w["linear1"], w["linear1Bias"])), w["linear2"],
                            w["linear2Bias"])
            return b.add(x1, f_)
        return b.scope(f)

    def uploadBatch(self, batch: Batch) -> dict:
        """Host -> device upload of one batch (model.ts:146-171): ids, both
        encoder masks, the head's key-padding mask, marker positions clamped
        to >= 0, the marker mask, qtype and k = max(#markers, 2) per row."""
        b = self.backend
        B, L, M = batch.size, batch.length, batch.markerCount
        if M < 2:
            raise ValueError("DecisionModel: markerCount must be >= 2 (collate pads to two slots)")
        full, sliding = attentionMasks(batch.attentionMask, B, L, self.encoder.config.localAttention)
        pos = np.maximum(np.asarray(batch.markerPos, np.int32).reshape(B, M), 0)
        mm = np.asarray(batch.markerMask).reshape(B, M) != 0
        k = np.maximum(mm.sum(1), 2).astype(np.float32)
        hosts = {
            "inputIds": HostTensor("i32", (B, L), np.asarray(batch.inputIds, np.int32).reshape(B, L)),
            "fullMask": full,
            "slidingMask": sliding,
            "headMask": HostTensor("bool", (B, 1, 1, L), np.asarray(batch.attentionMask).reshape(B, 1, 1, L) != 0),
            "qtype": HostTensor("i32", (B,), np.asarray(batch.qtype, np.int32).reshape(B)),
            "markerPos": HostTensor("i32", (B, M), pos),
            "markerMask": HostTensor("bool", (B, M), mm),
            "k": HostTensor("f32", (B,), k),
        }
        done = {}
        try:
            for name, h in hosts.items():
                done[name] = b.fromHost(h)
        except BaseException:
            for t in done.values():
                b.dispose(t)
            raise
        return done

    def disposeInputs(self, inp: dict) -> None:
        for t in inp.values():
            self.backend.dispose(t)

    def forwardCore(self, inp: dict, onStage: Optional[Callable] = None):
        """The decision forward as a function of device tensors
        (model.ts:178-236): returns (logits f32 [B, M] with masked slots
        -1e4, act f32 [B, nAct]).  `onStage(name, t)` returning True takes
        ownership of a stage output; the rest are freed."""
        b, w, enc = self.backend, self.weights, self.encoder
        B, L = inp["inputIds"].shape
        M = inp["markerPos"].shape[1]
        D = self.hiddenSize
        kept = []

        def emit(name, t) -> bool:
            own = onStage is not None and onStage(name, t) is True
            if own:
                kept.append(t)
            return own
        cst = w["constants"]

        def f():
            masks = {"full_attention": inp["fullMask"], "sliding_attention": inp["slidingMask"]}
            x = enc.embeddings(inp["inputIds"])
            owned = emit("embeddings", x)
            for i in range(enc.config.numHiddenLayers):
                nxt = enc.layer(i, x, masks[enc.config.layerTypes[i]])
                if not owned:
                    b.dispose(x)
                x = nxt
                owned = emit(f"encoder.layers.{i}", x)
            enc_out = enc.finalNorm(x)
            if not owned:
                b.dispose(x)
            emit("encoder.final_norm", enc_out)
            h = b.add(enc_out, b.reshape(embedding_any(b, w["typeEmb"], inp["qtype"]), [B, 1, D]))
            emit("type_emb_added", h)
            for j in range(len(w["head"])):
                h = self.headLayer(j, h, inp["headMask"])
                emit(f"head.layers.{j}", h)
            # markers = h[arange(B)[:, None], maximum(marker_pos, 0)]
            markers = b.gatherRows(h, inp["markerPos"])
            s = w["scorer"]
            scored = linear_any(b, b.gelu(linear_any(b, b.layerNorm(markers, s["norm"], s["norm_b"], HEAD_EPS),
                                                     s["w1"], s["b1"])), s["w2"], s["b2"])
            logits = b.where(inp["markerMask"], b.cast(b.reshape(scored, [B, M]), "f32"), cst["maskedLogit"])
            # action features [top1, top1 - top2, entropy / log(k), k / 255]
            p = b.softmax(logits, -1)
            plogp = b.mul(p, b.log(b.maximum(p, cst["probFloor"])))
            entropy = b.div(b.scale(b.sum(plogp, -1), -1), b.log(inp["k"]))
            top = b.slice(b.sort(p, -1), [0, M - 2], [B, M])
            top2 = b.slice(top, [0, 0], [B, 1])
            top1 = b.slice(top, [0, 1], [B, 2])
            k_scaled = b.div(b.reshape(inp["k"], [B, 1]), cst["kScale"])
            features = b.concat([top1, b.sub(top1, top2), b.reshape(entropy, [B, 1]), k_scaled], -1)
            cls = b.cast(b.reshape(b.slice(h, [0, 0, 0], [B, 1, D]), [B, D]), "f32")
            pooled = b.cast(b.concat([cls, features], -1), self.dtype)
            a = w["act"]
            act = b.cast(linear_any(b, b.gelu(linear_any(b, pooled, a["w1"], a["b1"])), a["w2"], a["b2"]), "f32")
            return [logits, act, *kept]
        out = b.scope(f)
        return out[0], out[1]

    _INPUTS = ("inputIds", "fullMask", "slidingMask", "headMask", "qtype", "markerPos", "markerMask", "k")

    def compiled(self) -> Optional[Callable]:
        """model.ts:250-275: a forwardTensors equivalent through
        `backend.compile` (recorded once per input shape signature); None
        when the backend has no compile.  No stage observation."""
        b = self.backend
        if getattr(b, "compile", None) is None:
            return None
        names = self._INPUTS
        fn = b.compile(lambda *ts: list(self.forwardCore(dict(zip(names, ts)))))

        def run(batch: Batch):
            inp = self.uploadBatch(batch)
            try:
                logits, act = fn(*(inp[n] for n in names))
                return logits, act
            finally:
                self.disposeInputs(inp)
        run.release = fn.release  # frees the recordings (HipBackend.compile)
        return run

    def forwardTensors(self, batch: Batch, onStage: Optional[Callable] = None):
        """model.ts:242-249: (logits, act) device tensors; caller disposes."""
        inp = self.uploadBatch(batch)
        try:
            return self.forwardCore(inp, onStage)
        finally:
            self.disposeInputs(inp)

    def readOutputs(self, r) -> dict:
        """model.ts:276-288: host f32 logits / act, and frees them."""
        logits, act = r
        b = self.backend
        try:
            b.flush(logits, act)
            lg = np.asarray(b.read(logits).data, np.float32).reshape(-1)
            ac = np.asarray(b.read(act).data, np.float32).reshape(-1)
            return {"logits": lg, "act": ac, "nAct": self.nAct}
        finally:
            b.dispose(logits)
            b.dispose(act)

    def forward(self, batch: Batch, onStage: Optional[Callable] = None) -> dict:
        return self.readOutputs(self.forwardTensors(batch, onStage))

    @property
    def quantizedOnDevice(self) -> bool:
        w = self.weights
        qs = [w["typeEmb"], w["scorer"]["w1"], w["scorer"]["w2"], w["act"]["w1"], w["act"]["w2"]]
        for lw in w["head"]:
            qs += [lw["inProj"], lw["outProj"], lw["linear1"], lw["linear2"]]
        enc = self.encoder.weights
        encq = [enc["tok"]] + [lw[k] for lw in enc["layers"] for k in ("Wqkv", "Wo", "Wi", "WoMlp")]
        return any(is_quantized(t) for t in qs + encq)

    def dispose(self) -> None:
        """Frees every weight, the encoder's and the constants included."""
        self.encoder.dispose()
        _dispose_head(self.backend, self.weights)


def _dispose_head(b, w: dict) -> None:
    for lw in w.get("head", []):
        for v in lw.values():
            dispose_weight(b, v)
    for key in ("scorer", "act", "constants"):
        for v in (w.get(key) or {}).values():
            dispose_weight(b, v)
    dispose_weight(b, w.get("typeEmb"))


def _head_names(D: int, head_layers: int, nAct: int) -> dict:
    """buildHeadWeights (model.ts:340-385): tree key -> (accepted names,
    shape, may be quantized)."""
    def seq(prefix, i, what):
        return [f"{prefix}.layers.{i}.{what}", f"{prefix}.{i}.{what}"]
    spec = {}
    for j in range(head_layers):
        p = f"head.layers.{j}"
        spec[("head", j, "norm1")] = ([f"{p}.norm1.weight"], (D,), False)
        spec[("head", j, "norm1_b")] = ([f"{p}.norm1.bias"], (D,), False)
        spec[("head", j, "norm2")] = ([f"{p}.norm2.weight"], (D,), False)
        spec[("head", j, "norm2_b")] = ([f"{p}.norm2.bias"], (D,), False)
        spec[("head", j, "inProj")] = ([f"{p}.self_attn.in_proj.weight", f"{p}.self_attn.in_proj_weight"],
                                       (3 * D, D), True)
        spec[("head", j, "inProjBias")] = ([f"{p}.self_attn.in_proj.bias", f"{p}.self_attn.in_proj_bias"],
                                           (3 * D,), False)
        spec[("head", j, "outProj")] = ([f"{p}.self_attn.out_proj.weight"], (D, D), True)
        spec[("head", j, "outProjBias")] = ([f"{p}.self_attn.out_proj.bias"], (D,), False)
        spec[("head", j, "linear1")] = ([f"{p}.linear1.weight"], (4 * D, D), True)
        spec[("head", j, "linear1Bias")] = ([f"{p}.linear1.bias"], (4 * D,), False)
        spec[("head", j, "linear2")] = ([f"{p}.linear2.weight"], (D, 4 * D), True)
        spec[("head", j, "linear2Bias")] = ([f"{p}.linear2.bias"], (D,), False)
    spec[("typeEmb",)] = (["type_emb.weight"], (3, D), True)
    spec[("scorer", "norm")] = (seq("scorer", 0, "weight"), (D,), False)
    spec[("scorer", "norm_b")] = (seq("scorer", 0, "bias"), (D,), False)
    spec[("scorer", "w1")] = (seq("scorer", 1, "weight"), (D, D), True)
    spec[("scorer", "b1")] = (seq("scorer", 1, "bias"), (D,), False)
    spec[("scorer", "w2")] = (seq("scorer", 3, "weight"), (1, D), True)
    spec[("scorer", "b2")] = (seq("scorer", 3, "bias"), (1,), False)
    spec[("act", "w1")] = (seq("act_head", 0, "weight"), (256, D + 4), True)
    spec[("act", "b1")] = (seq("act_head", 0, "bias"), (256,), False)
    spec[("act", "w2")] = (seq("act_head", 2, "weight"), (nAct, 256), True)
    spec[("act", "b2")] = (seq("act_head", 2, "bias"), (nAct,), False)
    return spec


def _shape_str(s) -> str:
    return ",".join(str(int(d)) for d in s)


def validateConfig(cfg, enc: ModernBertConfig) -> None:
    """`Agent.__init__`'s config check (agent.ts:96-105), run by load()
    before any weight is read (load.ts:53): the config names its encoder and
    head layers, and 4 < head_max_len < max_len <= the encoder's position
    limit (defaults 192 and 512).  Raises with the reference's messages."""
    if not isinstance(cfg, dict) or "encoder" not in cfg or "head_layers" not in cfg:
        raise ValueError("Laya config must specify encoder and head_layers")
    max_len = cfg.get("max_len")
    head_max_len = cfg.get("head_max_len")
    max_len = 512 if max_len is None else max_len
    head_max_len = 192 if head_max_len is None else head_max_len
    try:
        ok = 4 < head_max_len < max_len <= enc.maxPositionEmbeddings
    except TypeError:
        ok = False
    if not ok:
        raise ValueError("Expected 4 < head_max_len < max_len <= max_position_embeddings")


def loadDecisionModel(backend, encoderConfig, agentConfig: dict, weights, dtype: str = "f32") -> DecisionModel:
    """model.ts:283-338: loads the encoder (names under "encoder.") and the
    decision-head weights; every name and shape is checked before the
    head's uploads start, and a failure frees whatever was uploaded."""
    config = encoderConfig if isinstance(encoderConfig, ModernBertConfig) else parseModernBertConfig(encoderConfig)
    get = weights if callable(weights) else weights.get
    D = config.hiddenSize
    head_layers = agentConfig.get("head_layers")
    head_layers = 2 if head_layers is None else int(head_layers)
    nAct = len(agentConfig.get("act_costs") or {}) + 1
    nh = max(1, D // 64)
    if D % nh:
        raise ValueError("Decision head dimensions must be divisible by its head count")
    spec = _head_names(D, head_layers, nAct)
    hosts = {}
    chosen = {}
    encoder = loadModernBert(backend, config, get, dtype=dtype, prefix="encoder.")
    uploaded = {}
    try:
        for key, (names, shape, matrix) in spec.items():  # validate everything first (loadInBatch's first pass)
            for n in names:
                h = hosts.get(n)
                if h is None:
                    h = get(n)
                if h is None:
                    continue
                hosts[n] = h
                if tuple(h.shape) != tuple(shape):
                    raise ValueError(f"DecisionModel: {n} has shape [{_shape_str(h.shape)}], "
                                     f"want [{_shape_str(shape)}]")
                if not matrix and is_host_quantized(h):
                    raise ValueError(f"DecisionModel: {n} cannot be quantized (only Linear weights and type_emb)")
                chosen[key] = n
                break
            else:
                raise ValueError(f"DecisionModel: missing weight {names[0]}")
        for key, n in chosen.items():
            if n not in uploaded:
                uploaded[n] = upload_as(backend, hosts[n], dtype)
        consts = {}
        for name, v in (("maskedLogit", -1e4), ("probFloor", 1e-9), ("kScale", 255.0)):  # f32 whatever the dtype
            consts[name] = backend.fromHost(HostTensor("f32", (1,), np.array([v], np.float32)))
            uploaded["\0" + name] = consts[name]
    except BaseException:
        encoder.dispose()
        for t in uploaded.values():
            dispose_weight(backend, t)
        raise
    hosts.clear()
    tree = {"head": [{} for _ in range(head_layers)], "scorer": {}, "act": {}, "constants": consts}
    for key, n in chosen.items():
        t = uploaded[n]
        if key[0] == "head":
            tree["head"][key[1]][key[2]] = t
        elif key[0] == "typeEmb":
            tree["typeEmb"] = t
        else:
            tree[key[0]][key[1]] = t
    return DecisionModel(backend, encoder, tree, dtype, nAct)


def loadCheckpoint(backend, path: str, dtype: str = "f32", quantized: str = "device") -> DecisionModel:
    """The model half of laya's `load()` (load.ts:45-92) for a local
    checkpoint directory (model.safetensors, rl_agent_config.json,
    encoder/config.json): quantized checkpoints keep their matrices packed
    on the device (`quantized="device"`) or are dequantized to `dtype` while
    loading; parameters the model does not use are an error, except the
    `temperature` buffer."""
    from .checkpoint import read_weights
    if dtype not in ("f16", "f32"):
        raise ValueError('dtype must be one of ["f16", "f32"]')
    if quantized not in ("device", "dequantize"):
        raise ValueError('quantized must be "device" or "dequantize"')
    for f in ("model.safetensors", "rl_agent_config.json", os.path.join("encoder", "config.json")):
        if not os.path.exists(os.path.join(path, f)):
            raise FileNotFoundError(f"{path} is not a complete Laya checkpoint (missing {f})")
    with open(os.path.join(path, "rl_agent_config.json")) as fh:
        agent_cfg = json.load(fh)
    with open(os.path.join(path, "encoder", "config.json")) as fh:
        enc_cfg = json.load(fh)
    validateConfig(agent_cfg, parseModernBertConfig(enc_cfg))  # before reading weights (load.ts:53)
    weights = read_weights(os.path.join(path, "model.safetensors"), dtype=dtype, quantized=quantized)
    model = loadDecisionModel(backend, enc_cfg, agent_cfg, weights.get, dtype=dtype)
    extra = [n for n in weights.remaining() if n != "temperature"]
    if extra:
        model.dispose()
        raise ValueError(f"Received parameters not in model: {', '.join(sorted(extra))}")
    return model
