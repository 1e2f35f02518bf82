"""laya's DecisionModel (packages/laya/src/model.ts) running unchanged on
HipBackend.

- The tiny checkpoint, stage by stage, as laya/test/model.test.ts:26-79
  checks it on the CPU backend: every stage (encoder, type embedding, both
  head layers, logits, act) within 1e-5 abs + rel of the MLX activations in
  f32 and within the reference's f16 bar (0.02) in f16, valid and padded
  positions separately; masked logit slots exactly -1e4; the same argmax.
- `forward()` returns host logits / act and frees every intermediate
  (model.test.ts:81-103).
- `loadDecisionModel` rejects a missing weight and a wrong shape and frees
  every upload (model.test.ts:105-137).
- `loadCheckpoint` on the tiny checkpoint directory, float and quantized.
- The north_star bar at the ModernBERT-base shape: a 22-layer encoder with
  the decision head in f16 against the f32 oracle, logits within 1e-2
  absolute and the same argmax in every sequence.
"""
import json
import os

import numpy as np
import pytest

from fixtures import GOLDEN, arr, read_safetensors
from gpu_util import read32
from laya_hip.checkpoint import quantize_safetensors, read_weights
from laya_hip.host import HostTensor
from laya_hip.model import Batch, loadCheckpoint, loadDecisionModel
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu

TINY = os.path.join(GOLDEN, "tiny")


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _json(*p):
    with open(os.path.join(TINY, *p)) as f:
        return json.load(f)


def _tiny_batch(act, M=None):
    inp = {k: arr(v) for k, v in act["inputs"].items()}
    B, L = inp["input_ids"].shape
    return Batch(size=B, length=L, markerCount=M or inp["marker_pos"].shape[1], inputIds=inp["input_ids"],
                 attentionMask=inp["attention_mask"], markerPos=inp["marker_pos"], markerMask=inp["marker_mask"],
                 qtype=inp["qtype"])


def _err_stats(got, want, tol):
    d = np.abs(got.astype(np.float64) - want)
    return float(d.max()) if d.size else 0.0, float(np.max(d / (tol + tol * np.abs(want)))) if d.size else 0.0


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-5), ("f16", 2e-2)])
def test_tiny_decision_model_every_stage(b, dtype, tol):
    act = _json("activations.json")
    model = loadDecisionModel(b, _json("encoder", "config.json"), _json("rl_agent_config.json"),
                              read_weights(os.path.join(TINY, "model.safetensors")).get, dtype=dtype)
    batch = _tiny_batch(act)
    staged = {}
    logits, a = model.forwardTensors(batch, onStage=lambda n, t: (staged.__setitem__(n, t), True)[1])
    staged["logits"], staged["act"] = logits, a
    assert sorted(staged) == sorted(act["stages"]), "stage names"
    valid = batch.attentionMask.reshape(-1) != 0
    report = []
    for name, enc in act["stages"].items():
        want = arr(enc).astype(np.float64)
        got = read32(b, staged[name])
        assert got.shape == want.shape, name
        if want.ndim == 3:
            D = want.shape[-1]
            g2, w2 = got.reshape(-1, D), want.reshape(-1, D)
            (va, vw), (pa, pw) = _err_stats(g2[valid], w2[valid], tol), _err_stats(g2[~valid], w2[~valid], tol)
            report.append(f"{name:20s} valid maxAbs {va:.2e} | padded maxAbs {pa:.2e}")
            assert vw <= 1 and pw <= 1, f"{name}: valid {va:.2e} padded {pa:.2e} (tol {tol})"
        else:
            ma, w = _err_stats(got, want, tol)
            report.append(f"{name:20s} maxAbs {ma:.2e}")
            assert w <= 1, f"{name}: maxAbs {ma:.2e} (tol {tol})"
    lg = read32(b, logits)
    mm = batch.markerMask != 0
    assert np.all(lg[~mm] == np.float32(-1e4)), "masked logit slots are exactly -1e4"
    want_lg = arr(act["stages"]["logits"])
    assert np.array_equal(np.argmax(np.where(mm, lg, -np.inf), 1), np.argmax(np.where(mm, want_lg, -np.inf), 1))
    print(f"tiny decision model {dtype}:\n  " + "\n  ".join(report))
    for t in staged.values():
        b.dispose(t)
    model.dispose()


def test_forward_returns_host_outputs_and_frees_intermediates(b):
    act = _json("activations.json")
    model = loadDecisionModel(b, _json("encoder", "config.json"), _json("rl_agent_config.json"),
                              read_weights(os.path.join(TINY, "model.safetensors")).get)
    blocks = b.pool_stats()["live_blocks"]
    batch = _tiny_batch(act, M=3)
    out = model.forward(batch)
    assert out["nAct"] == 2
    assert out["logits"].size == batch.size * 3 and out["act"].size == batch.size * 2
    _, w = _err_stats(out["act"].reshape(batch.size, 2), arr(act["stages"]["act"]).astype(np.float64), 1e-5)
    assert w <= 1
    assert b.pool_stats()["live_blocks"] == blocks, "forward() leaves no tensor behind"
    model.dispose()


class _Counting:
    """The backend with a count of live uploads (model.test.ts:110-121)."""

    def __init__(self, be):
        self._be = be
        self.live = set()

    def fromHost(self, h):
        t = self._be.fromHost(h)
        self.live.add(id(t))
        return t

    def dispose(self, t):
        self.live.discard(id(t))
        self._be.dispose(t)

    def __getattr__(self, name):
        return getattr(self._be, name)


def test_load_rejects_missing_weights_and_wrong_shapes(b):
    W = read_safetensors(os.path.join(TINY, "model.safetensors"))
    get = lambda n: HostTensor("f32", W[n].shape, W[n].astype(np.float32)) if n in W else None  # noqa: E731
    enc_cfg = _json("encoder", "config.json")
    cb = _Counting(b)
    with pytest.raises(ValueError, match=r"missing weight head\.layers\.2"):
        loadDecisionModel(cb, enc_cfg, {"head_layers": 3}, get)
    assert not cb.live, "encoder uploads freed after a head validation error"
    with pytest.raises(ValueError, match=r"act_head\.layers\.2\.weight has shape \[2,256\], want \[3,256\]"):
        loadDecisionModel(cb, enc_cfg, {"head_layers": 2, "act_costs": {"a": 1, "b": 2}}, get)
    assert not cb.live
    ok = loadDecisionModel(cb, enc_cfg, _json("rl_agent_config.json"), get)
    assert cb.live
    ok.dispose()
    assert not cb.live, "dispose frees every weight and constant"


def test_load_checkpoint_directory_float_and_quantized(b, tmp_path):
    """load()'s model half on the tiny checkpoint directory; then the same
    checkpoint quantized (q8, group 32) and loaded with its matrices packed
    on the device or dequantized on the host: both give the same act."""
    act = _json("activations.json")
    batch = _tiny_batch(act)
    m = loadCheckpoint(b, TINY, dtype="f32")
    out = m.forward(batch)
    _, w = _err_stats(out["act"].reshape(batch.size, -1), arr(act["stages"]["act"]).astype(np.float64), 1e-5)
    assert w <= 1
    m.dispose()
    qdir = tmp_path / "q8"
    (qdir / "encoder").mkdir(parents=True)
    data, report = quantize_safetensors(os.path.join(TINY, "model.safetensors"), 8, 32)
    assert report["quantized"]
    (qdir / "model.safetensors").write_bytes(data)
    for p in ("rl_agent_config.json", os.path.join("encoder", "config.json")):
        with open(os.path.join(TINY, p)) as f:
            (qdir / p).write_text(f.read())
    outs = {}
    for mode in ("device", "dequantize"):
        m = loadCheckpoint(b, str(qdir), dtype="f16", quantized=mode)
        assert m.quantizedOnDevice == (mode == "device")
        outs[mode] = m.forward(batch)
        m.dispose()
    np.testing.assert_allclose(outs["device"]["act"], outs["dequantize"]["act"], atol=2e-3)
    np.testing.assert_allclose(outs["device"]["act"].reshape(batch.size, -1), arr(act["stages"]["act"]), atol=5e-2)


def _base_decision_weights(rng, H=768, I=1152, layers=22, V=50368, head_layers=2, nAct=3):
    """A ModernBERT-base encoder with laya's decision head, every matrix and
    bias random-init fp16 ~N(0, 0.02) (BASELINE's init), LayerNorm gamma = 1
    and the head's beta ~N(0, 0.02)."""
    n = lambda *s: rng.normal(0, 0.02, s)  # noqa: E731
    W = {"encoder.embeddings.tok_embeddings.weight": n(V, H), "encoder.embeddings.norm.weight": np.ones(H),
         "encoder.final_norm.weight": np.ones(H), "type_emb.weight": n(3, H)}
    for i in range(layers):
        p = f"encoder.layers.{i}."
        if i:
            W[p + "attn_norm.weight"] = np.ones(H)
        W[p + "attn.Wqkv.weight"] = n(3 * H, H)
        W[p + "attn.Wo.weight"] = n(H, H)
        W[p + "mlp_norm.weight"] = np.ones(H)
        W[p + "mlp.Wi.weight"] = n(2 * I, H)
        W[p + "mlp.Wo.weight"] = n(H, I)
    for j in range(head_layers):
        p = f"head.layers.{j}."
        for ln in ("norm1", "norm2"):
            W[p + ln + ".weight"] = np.ones(H)
            W[p + ln + ".bias"] = n(H)
        W[p + "self_attn.in_proj.weight"], W[p + "self_attn.in_proj.bias"] = n(3 * H, H), n(3 * H)
        W[p + "self_attn.out_proj.weight"], W[p + "self_attn.out_proj.bias"] = n(H, H), n(H)
        W[p + "linear1.weight"], W[p + "linear1.bias"] = n(4 * H, H), n(4 * H)
        W[p + "linear2.weight"], W[p + "linear2.bias"] = n(H, 4 * H), n(H)
    W["scorer.layers.0.weight"], W["scorer.layers.0.bias"] = np.ones(H), n(H)
    W["scorer.layers.1.weight"], W["scorer.layers.1.bias"] = n(H, H), n(H)
    W["scorer.layers.3.weight"], W["scorer.layers.3.bias"] = n(1, H), n(1)
    W["act_head.layers.0.weight"], W["act_head.layers.0.bias"] = n(256, H + 4), n(256)
    W["act_head.layers.2.weight"], W["act_head.layers.2.bias"] = n(nAct, 256), n(nAct)
    return {k: np.asarray(v, np.float16).astype(np.float32) for k, v in W.items()}


def test_base_decision_model_logits_and_argmax_match_oracle(b):
    """ModernBERT-base shape (22 layers, hidden 768) plus laya's decision
    head in f16, B = 4 sequences of up to 128 tokens with 2..8 markers,
    against the f32 oracle on the same f16-valued weights: logits within
    1e-2 absolute, masked slots exactly -1e4, the chosen marker (argmax)
    identical in every sequence, act within 1e-2."""
    rng = np.random.default_rng(7)
    W = _base_decision_weights(rng)
    enc_cfg = {"vocab_size": 50368, "hidden_size": 768, "intermediate_size": 1152, "num_hidden_layers": 22,
               "num_attention_heads": 12, "local_attention": 128}
    agent = {"head_layers": 2, "act_costs": {"escalate": 0.5, "defer": 0.25}}
    model = loadDecisionModel(b, enc_cfg, agent, lambda n: HostTensor("f16", W[n].shape, W[n].astype(np.float16))
                              if n in W else None, dtype="f16")
    B, L, M = 4, 128, 8
    lens = np.array([128, 97, 64, 120])
    ids = rng.integers(0, 50368, (B, L)).astype(np.int32)
    valid = (np.arange(L)[None, :] < lens[:, None]).astype(np.uint8)
    nmark = np.array([8, 5, 2, 7])
    pos = np.zeros((B, M), np.int32)
    mm = np.zeros((B, M), np.uint8)
    for r in range(B):
        pos[r, :nmark[r]] = np.sort(rng.choice(np.arange(1, lens[r]), nmark[r], replace=False))
        mm[r, :nmark[r]] = 1
    qtype = np.array([0, 1, 2, 1], np.int32)
    batch = Batch(B, L, M, ids, valid, pos, mm, qtype)
    out = model.forward(batch)
    logits, act = out["logits"].reshape(B, M), out["act"].reshape(B, -1)
    ref_lg, ref_act = cr.decision_forward(cr.EncoderConfig.from_json(enc_cfg), W, 2, ids, valid, qtype, pos, mm)
    err = float(np.max(np.abs(logits - ref_lg)))
    aerr = float(np.max(np.abs(act - ref_act)))
    gaps = [np.diff(np.sort(ref_lg[r, mm[r] != 0]))[-1] for r in range(B)]
    scale = float(np.max(np.abs(ref_lg[mm != 0])))
    print(f"base decision model f16: logits max abs err {err:.2e} (max |logit| {scale:.3f}, max-rel "
          f"{err / scale:.2e}), act {aerr:.2e}; oracle top-2 gaps {', '.join(f'{g:.4f}' for g in gaps)}")
    assert np.all(logits[mm == 0] == np.float32(-1e4))
    assert err <= 1e-2 and aerr <= 1e-2
    assert np.array_equal(np.argmax(np.where(mm != 0, logits, -np.inf), 1),
                          np.argmax(np.where(mm != 0, ref_lg, -np.inf), 1))
    model.dispose()


def _eager_and_compiled(model, batches):
    """Eager forward and the `compiled()` forward (model.ts:250-275) on each
    batch: (eager logits, eager act, compiled logits, compiled act) bits."""
    b = model.backend
    run = model.compiled()
    assert run is not None, "HipBackend has compile, so compiled() returns a function"
    out = []
    for batch in batches:
        e = model.forward(batch)
        lg, ac = run(batch)
        c = model.readOutputs((lg, ac))
        out.append((e["logits"], e["act"], c["logits"], c["act"]))
    run.release()
    return out


def test_compiled_tiny_decision_model_equals_eager_bits(b):
    """DecisionModel.compiled() on HipBackend (Backend.compile over
    HipBackend.capture): the first call records, later calls of the same
    shape copy their inputs into the recorded blocks and replay.  Every
    call gives the eager forward's bits, also after the batch's ids,
    markers and padding change; after release() and destroy of the model
    the pool holds no block of the model's calls."""
    act = _json("activations.json")
    model = loadDecisionModel(b, _json("encoder", "config.json"), _json("rl_agent_config.json"),
                              read_weights(os.path.join(TINY, "model.safetensors")).get)
    blocks = b.pool_stats()["live_blocks"]
    base = _tiny_batch(act, M=3)
    rng = np.random.default_rng(3)
    B, L = base.size, base.length
    other = Batch(B, L, 3, rng.integers(0, 128, (B, L)).astype(np.int32), base.attentionMask.copy(),
                  base.markerPos.copy(), base.markerMask.copy(), base.qtype.copy())
    other.attentionMask[0, L // 2:] = 0
    other.markerPos[0] = np.minimum(other.markerPos[0], L // 2 - 1)
    runs = _eager_and_compiled(model, [base, other, base])
    for i, (el, ea, cl, ca) in enumerate(runs):
        np.testing.assert_array_equal(cl.view(np.uint32), el.view(np.uint32), err_msg=f"logits, call {i}")
        np.testing.assert_array_equal(ca.view(np.uint32), ea.view(np.uint32), err_msg=f"act, call {i}")
    assert not np.array_equal(runs[0][0], runs[1][0])
    model.dispose()
    assert b.pool_stats()["live_blocks"] <= blocks


def test_compiled_base_decision_model_equals_eager_with_a_new_mask(b):
    """The compiled forward at the ModernBERT-base shape (22 layers, f16,
    B = 4, L = 128): the same bits as the eager forward on two batches of
    one shape whose padding (and so every attention mask and the mask
    summaries recorded into the graph) differs between the calls."""
    rng = np.random.default_rng(8)
    W = _base_decision_weights(rng)
    enc_cfg = {"vocab_size": 50368, "hidden_size": 768, "intermediate_size": 1152, "num_hidden_layers": 22,
               "num_attention_heads": 12, "local_attention": 128}
    agent = {"head_layers": 2, "act_costs": {"escalate": 0.5, "defer": 0.25}}
    model = loadDecisionModel(b, enc_cfg, agent, lambda n: HostTensor("f16", W[n].shape, W[n].astype(np.float16))
                              if n in W else None, dtype="f16")
    B, L, M = 4, 128, 8
    batches = []
    for lens in ([128, 97, 64, 120], [40, 128, 111, 77]):
        lens = np.array(lens)
        ids = rng.integers(0, 50368, (B, L)).astype(np.int32)
        valid = (np.arange(L)[None, :] < lens[:, None]).astype(np.uint8)
        pos = np.zeros((B, M), np.int32)
        mm = np.zeros((B, M), np.uint8)
        for r in range(B):
            nm = int(rng.integers(2, M + 1))
            pos[r, :nm] = np.sort(rng.choice(np.arange(1, lens[r]), nm, replace=False))
            mm[r, :nm] = 1
        batches.append(Batch(B, L, M, ids, valid, pos, mm, rng.integers(0, 3, B).astype(np.int32)))
    for i, (el, ea, cl, ca) in enumerate(_eager_and_compiled(model, batches)):
        print(f"compiled base decision model, call {i}: logits {cl.reshape(B, M)[:, :2].tolist()}")
        np.testing.assert_array_equal(cl.view(np.uint32), el.view(np.uint32), err_msg=f"logits, call {i}")
        np.testing.assert_array_equal(ca.view(np.uint32), ea.view(np.uint32), err_msg=f"act, call {i}")
    model.dispose()
