"""the ModernBERT-large-shape encoder (hidden 1024, 16
heads, GeGLU 2624, window 128 with a global layer every third, 256000-token
vocabulary) at B=16, T=2048, in fp16 and in laya's quantized format, ending in
a mean-pooled 1024 -> 8 classifier with softmax.

Three layers (one global, two local) keep the CPU oracle's share of the run
to seconds; every kernel shape of the 28-layer model is exercised by them
(K = 1024 and 2624, the ragged 2624-wide GeGLU output, 2048-token attention,
the 256000-row quantized embedding gather).  Checked:
- one full-length sequence against the f32 oracle (max abs <= 5e-2 on the
  hidden states, the reference's f16 parity bar for the encoder);
- batch independence: sequences encoded alone give the batched rows bit for
  bit (the M = 2048 and M = 32768 GEMM kernels agree);
- the classifier probabilities within 1e-2 of the oracle's and the same
  argmax wherever the oracle's top two are 1e-2 apart.
The quantized run uses q4 affine Linear weights from the format's own
quantizer (group 64, refit on) and q8 codes with f16 scales for the
embedding table; its oracle uses the same dequantized weights fl16(q*s + z).
"""
import numpy as np
import pytest

from gpu_util import read32
from laya_hip.host import HostQuantized, HostTensor, pack_quantized
from laya_hip.modernbert import loadModernBert, parseModernBertConfig
from laya_hip.quant import quantize_matrix
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu

H, I, NH, V = 1024, 2624, 16, 256000
LAYERS = 3
CFG = {"vocab_size": V, "hidden_size": H, "intermediate_size": I, "num_hidden_layers": LAYERS,
       "num_attention_heads": NH, "local_attention": 128}
B, T = 16, 2048


@pytest.fixture(scope="module")
def b():
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.destroy()


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def _weights(rng):
    """fp16 ~N(0, 0.02) matrices, LayerNorm gamma = 1 (names without the prefix)."""
    n = lambda *s: _f16(rng.standard_normal(s, dtype=np.float32) * 0.02)  # noqa: E731
    W = {"embeddings.tok_embeddings.weight": n(V, H), "embeddings.norm.weight": np.ones(H, np.float16),
         "final_norm.weight": np.ones(H, np.float16)}
    for i in range(LAYERS):
        p = f"layers.{i}."
        if i:
            W[p + "attn_norm.weight"] = np.ones(H, np.float16)
        W[p + "attn.Wqkv.weight"] = n(3 * H, H)
        W[p + "attn.Wo.weight"] = n(H, H)
        W[p + "mlp_norm.weight"] = np.ones(H, np.float16)
        W[p + "mlp.Wi.weight"] = n(2 * I, H)
        W[p + "mlp.Wo.weight"] = n(H, I)
    return W


def _inputs(rng):
    lens = rng.integers(256, T + 1, B)
    lens[0] = T
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    valid = (np.arange(T)[None, :] < lens[:, None]).astype(np.uint8)
    return lens, ids, valid


def _oracle_one(W32, ids_row, valid_row):
    """The f32 oracle on one sequence, with the embedding table cut to the
    rows that sequence uses (ids remapped)."""
    uniq, inv = np.unique(ids_row, return_inverse=True)
    Wo = dict(W32)
    Wo["embeddings.tok_embeddings.weight"] = W32["embeddings.tok_embeddings.weight"][uniq]
    ocfg = cr.EncoderConfig.from_json(dict(CFG, vocab_size=len(uniq)))
    return cr.encoder_forward(ocfg, Wo, inv.reshape(1, -1).astype(np.int32), valid_row[None, :])[0]


def _softmax(z):
    z = z - z.max(-1, keepdims=True)
    e = np.exp(z)
    return e / e.sum(-1, keepdims=True)


def _head(b, enc, ids, valid, Wc, bc):
    """meanPool -> 1024->8 linear (+ bias) -> softmax on the backend."""
    pooled = enc.embed(ids, valid, ids.shape[0], ids.shape[1])  # [n, H] f32
    Wt, Bt = b.fromHost(HostTensor("f32", Wc.shape, Wc)), b.fromHost(HostTensor("f32", bc.shape, bc))
    probs = b.softmax(b.linear(pooled, Wt, Bt), -1)
    out = read32(b, probs), read32(b, pooled)
    for t in (pooled, Wt, Bt, probs):
        b.dispose(t)
    return out


def _check_head(probs, pooled_ref, Wc, bc):
    ref = _softmax(pooled_ref @ Wc.T + bc)
    assert np.max(np.abs(probs - ref)) <= 1e-2
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 1e-2:
        assert int(np.argmax(probs)) == int(np.argmax(ref))


def test_config4_fp16_encoder_and_classifier(b):
    rng = np.random.default_rng(4)
    W = _weights(rng)
    lens, ids, valid = _inputs(rng)
    cfg = parseModernBertConfig(CFG)
    enc = loadModernBert(b, cfg, lambda nm: HostTensor("f16", W[nm[8:]].shape, W[nm[8:]])
                         if nm.startswith("encoder.") and nm[8:] in W else None, dtype="f16")
    print(f"config4 fp16: B={B} T={T} lens {lens.min()}..{lens.max()}", flush=True)
    full = read32(b, enc.forward(ids, valid, B, T))
    assert np.isfinite(full[valid != 0]).all()
    for i in (0, 7):
        one = read32(b, enc.forward(ids[i:i + 1], valid[i:i + 1], 1, T))
        n = lens[i]
        np.testing.assert_array_equal(one[0, :n], full[i, :n])
    W32 = {k: v.astype(np.float32) for k, v in W.items()}
    ref = _oracle_one(W32, ids[0], valid[0])
    err = float(np.max(np.abs(full[0] - ref)))
    print(f"config4 fp16: seq 0 (T={T}) max abs err vs f32 oracle {err:.3e}", flush=True)
    assert err <= 5e-2
    crng = np.random.default_rng(44)
    Wc = (crng.standard_normal((8, H)) * 0.5).astype(np.float32)
    bc = (crng.standard_normal(8) * 0.1).astype(np.float32)
    probs, pooled = _head(b, enc, ids[:1], valid[:1], Wc, bc)
    _check_head(probs[0], ref[valid[0] != 0].mean(0), Wc, bc)
    enc.dispose()


def test_config4_quantized_encoder_and_classifier(b):
    rng = np.random.default_rng(5)
    W = _weights(rng)
    Bq = 4  # M = 8192: the large-M quantized GEMM
    lens, ids, valid = _inputs(rng)
    ids, valid, lens = ids[:Bq], valid[:Bq], lens[:Bq]
    hosts, W32 = {}, {}
    for k, v in W.items():
        if k.endswith("Wqkv.weight") or k.endswith("Wo.weight") or k.endswith("Wi.weight"):
            N, K = v.shape
            q, s, z = quantize_matrix(v.astype(np.float32), N, K, 4, 64, refine=True)
            hosts[k] = HostQuantized((N, K), 4, 64, "affine", pack_quantized(q, 4), HostTensor("f16", s.shape, s),
                                     HostTensor("f16", z.shape, z))
            W32[k] = cr.dequant_exact_f16(q, s.astype(np.float32), z.astype(np.float32), 64) \
                .view(np.float16).astype(np.float32)
        elif k == "embeddings.tok_embeddings.weight":
            # q8 symmetric codes with f16 scales (group 64), drawn directly
            q = rng.integers(-127, 128, (V, H)).astype(np.int32)
            s = _f16(rng.uniform(1e-4, 3e-4, (V, H // 64)))
            hosts[k] = HostQuantized((V, H), 8, 64, "symmetric", pack_quantized(q, 8),
                                     HostTensor("f16", s.shape, s), None)
            W32[k] = (q.reshape(V, H // 64, 64) * s.astype(np.float32)[:, :, None]).reshape(V, H) \
                .astype(np.float16).astype(np.float32)
        else:
            hosts[k] = HostTensor("f16", v.shape, v)
            W32[k] = v.astype(np.float32)
    cfg = parseModernBertConfig(CFG)
    enc = loadModernBert(b, cfg, lambda nm: hosts.get(nm[8:]) if nm.startswith("encoder.") else None, dtype="f16")
    print(f"config4 quantized: B={Bq} T={T}", flush=True)
    full = read32(b, enc.forward(ids, valid, Bq, T))
    assert np.isfinite(full[valid != 0]).all()
    ref = _oracle_one(W32, ids[0], valid[0])
    err = float(np.max(np.abs(full[0] - ref)))
    print(f"config4 quantized: seq 0 max abs err vs f32 oracle on the dequantized weights {err:.3e}", flush=True)
    assert err <= 5e-2
    crng = np.random.default_rng(45)
    Wc = (crng.standard_normal((8, H)) * 0.5).astype(np.float32)
    bc = (crng.standard_normal(8) * 0.1).astype(np.float32)
    probs, _ = _head(b, enc, ids[:1], valid[:1], Wc, bc)
    _check_head(probs[0], ref[valid[0] != 0].mean(0), Wc, bc)
    enc.dispose()
