"""the ModernBERT-large-shape encoder (hidden 1024, 16
heads, GeGLU 2624, window 128 with a global layer every third, 256000-token
vocabulary) at B=16, T=2048, all 28 layers, in fp16 and in laya's quantized
format, ending in a mean-pooled 1024 -> 8 classifier with softmax.

Checked against the f32 oracle (the north_star bar: logits within 1e-2
absolute, the same argmax), every one of the 16 sequences:
- fp16, through all 28 layers: hidden states within 5e-2 absolute (the
  reference's f16 parity bar for the encoder), the classifier logits before
  the softmax within 1e-2 and the same argmax; batch independence
  (sequences encoded alone give the batched rows bit for bit: the M = 2048
  and M = 32768 GEMM kernels agree);
- quantized, the whole batch (M = 32768), against the oracle on the
  dequantized weights fl16(q*s + z), the same bars.
The quantized weights come from laya's quantizer (the oracle's restatement
of quantizeMatrix, laya/src/quant.ts:96-187) applied to the fp16 ~N(0, 0.02)
weights: q4 affine with group 64 and the least-squares refit for the
Linears, q8 symmetric with group 64 for the embedding table.  The oracle
runs each sequence on its valid tokens only (valid rows attend valid keys
only, so the padded tail does not change them).
"""
import concurrent.futures as cf

import numpy as np
import pytest

from gpu_util import read32
from laya_hip.host import HostQuantized, HostTensor, pack_quantized
from laya_hip.modernbert import loadModernBert, parseModernBertConfig
from oracle import cpu_ref as cr

pytestmark = pytest.mark.gpu

H, I, NH, V = 1024, 2624, 16, 256000
LAYERS = 28
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
    """The f32 oracle on one sequence's valid tokens ([n, H]), with the
    embedding table cut to the rows that sequence uses (ids remapped)."""
    n = int(np.count_nonzero(valid_row))
    uniq, inv = np.unique(ids_row[:n], return_inverse=True)
    Wo = dict(W32)
    Wo["embeddings.tok_embeddings.weight"] = W32["embeddings.tok_embeddings.weight"][uniq]
    ocfg = cr.EncoderConfig.from_json(dict(CFG, vocab_size=len(uniq)))
    return cr.encoder_forward(ocfg, Wo, inv.reshape(1, -1).astype(np.int32), np.ones((1, n), np.uint8))[0]


def _softmax(z):
    z = z - z.max(-1, keepdims=True)
    e = np.exp(z)
    return e / e.sum(-1, keepdims=True)


def _classifier(rng):
    return ((rng.standard_normal((8, H)) * 0.5).astype(np.float32), (rng.standard_normal(8) * 0.1).astype(np.float32))


def _head(b, enc, ids, valid, Wc, bc):
    """meanPool -> 1024->8 linear (+ bias) -> softmax on the backend;
    returns (logits before the softmax, probabilities, pooled)."""
    pooled = enc.embed(ids, valid, ids.shape[0], ids.shape[1])  # [n, H] f32
    Wt, Bt = b.fromHost(HostTensor("f32", Wc.shape, Wc)), b.fromHost(HostTensor("f32", bc.shape, bc))
    logits = b.linear(pooled, Wt, Bt)
    probs = b.softmax(logits, -1)
    out = read32(b, logits), read32(b, probs), read32(b, pooled)
    for t in (pooled, Wt, Bt, logits, probs):
        b.dispose(t)
    return out


def _check_seq(tag, full_row, valid_row, ref, logits, probs, Wc, bc):
    """Hidden states (valid rows; `ref` holds those rows) within 5e-2;
    classifier logits within 1e-2 and the same argmax; probabilities within
    1e-2."""
    v = valid_row != 0
    err = float(np.max(np.abs(full_row[v] - ref)))
    ref_logits = ref.astype(np.float64).mean(0) @ Wc.T.astype(np.float64) + bc
    lerr = float(np.max(np.abs(logits - ref_logits)))
    print(f"{tag}: {v.sum()} tokens, hidden max abs err {err:.3e}, logits max abs err {lerr:.3e}, "
          f"argmax {int(np.argmax(logits))} vs {int(np.argmax(ref_logits))}", flush=True)
    assert err <= 5e-2
    assert lerr <= 1e-2
    assert int(np.argmax(logits)) == int(np.argmax(ref_logits))
    assert float(np.max(np.abs(probs - _softmax(ref_logits)))) <= 1e-2


def test_config4_fp16_encoder_and_classifier(b):
    rng = np.random.default_rng(4)
    W = _weights(rng)
    lens, ids, valid = _inputs(rng)
    cfg = parseModernBertConfig(CFG)
    enc = loadModernBert(b, cfg, lambda nm: HostTensor("f16", W[nm[8:]].shape, W[nm[8:]])
                         if nm.startswith("encoder.") and nm[8:] in W else None, dtype="f16")
    print(f"config4 fp16: B={B} T={T} {LAYERS} layers, lens {lens.min()}..{lens.max()}", flush=True)
    full = read32(b, enc.forward(ids, valid, B, T))
    assert np.isfinite(full[valid != 0]).all()
    for i in (0, 7):
        one = read32(b, enc.forward(ids[i:i + 1], valid[i:i + 1], 1, T))
        n = lens[i]
        np.testing.assert_array_equal(one[0, :n], full[i, :n])
    Wc, bc = _classifier(np.random.default_rng(44))
    logits, probs, _ = _head(b, enc, ids, valid, Wc, bc)
    W32 = {k: v.astype(np.float32) for k, v in W.items()}
    for i in range(B):
        ref = _oracle_one(W32, ids[i], valid[i])
        _check_seq(f"config4 fp16 seq {i}", full[i], valid[i], ref, logits[i], probs[i], Wc, bc)
    enc.dispose()


def _quantize(w16, bits):
    """laya's quantizeMatrix (group 64; q4 affine with the refit, q8
    symmetric) of an fp16 matrix -> (HostQuantized, dequantized f32 weights
    fl16(q*s + z))."""
    N, K = w16.shape
    q, s, z = cr.quantize_matrix(w16.astype(np.float32), N, K, bits, 64)
    sh = HostTensor("f16", s.shape, s.view(np.float16))
    zh = HostTensor("f16", z.shape, z.view(np.float16)) if z is not None else None
    h = HostQuantized((N, K), bits, 64, "affine" if bits == 4 else "symmetric", pack_quantized(q, bits), sh, zh)
    w = cr.dequant_exact_f16(q, s.view(np.float16).astype(np.float32),
                             z.view(np.float16).astype(np.float32) if z is not None else None, 64)
    return h, w.view(np.float16).astype(np.float32)


def test_config4_quantized_encoder_and_classifier(b):
    rng = np.random.default_rng(5)
    W = _weights(rng)
    lens, ids, valid = _inputs(rng)
    hosts, W32 = {}, {}
    qnames = [k for k in W if k.endswith(("Wqkv.weight", "Wo.weight", "Wi.weight"))]
    qnames.append("embeddings.tok_embeddings.weight")
    with cf.ThreadPoolExecutor(8) as ex:  # the C quantizer releases the GIL
        jobs = {k: ex.submit(_quantize, W[k], 8 if k.startswith("embeddings") else 4) for k in qnames}
        for k, j in jobs.items():
            hosts[k], W32[k] = j.result()
    for k, v in W.items():
        if k not in hosts:
            hosts[k] = HostTensor("f16", v.shape, v)
            W32[k] = v.astype(np.float32)
    del W
    cfg = parseModernBertConfig(CFG)
    enc = loadModernBert(b, cfg, lambda nm: hosts.get(nm[8:]) if nm.startswith("encoder.") else None, dtype="f16")
    print(f"config4 quantized: B={B} T={T} {LAYERS} layers (M = {B * T})", flush=True)
    full = read32(b, enc.forward(ids, valid, B, T))
    assert np.isfinite(full[valid != 0]).all()
    Wc, bc = _classifier(np.random.default_rng(45))
    logits, probs, _ = _head(b, enc, ids, valid, Wc, bc)
    for i in range(B):
        ref = _oracle_one(W32, ids[i], valid[i])
        _check_seq(f"config4 quantized seq {i}", full[i], valid[i], ref, logits[i], probs[i], Wc, bc)
    enc.dispose()
