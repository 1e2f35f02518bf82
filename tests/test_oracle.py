"""Pins the CPU oracle (oracle/cpu_ref.*) before anything is compared to it.

Each oracle function is checked against the reference's own golden vectors
(tests/golden, copied from packages/tensor-backend/fixtures and
packages/laya-fixtures/data/tiny) at the reference's tolerances
(`assertClose`, packages/tensor-backend/src/conformance.ts:223-233), and
against what the mathematics fixes (closed forms, invariants, brute force),
chosen so that a plausible slip -- a dropped term, a wrong sign, a transposed
operand -- fails at least one check.  The "planted mistake" tests perturb the
ORACLE's inputs on the CPU and show the fixture check notices.
"""
import math

import numpy as np
import pytest

from fixtures import arr, case, load_cases, tiny
from oracle import cpu_ref as cr


def assert_close(got, want, atol, rtol, label=""):
    """conformance.ts:223-233: |v - e| <= atol + rtol |e| everywhere."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    assert got.shape == want.shape, label
    assert not np.any(np.isnan(got) != np.isnan(want)), f"{label}: NaN mismatch"
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    i = int(np.argmax(err))
    assert err[i] <= 0, f"{label}: [{i}] got {got[i]} want {want[i]} (atol {atol}, rtol {rtol})"


def close(got, want, atol, rtol):
    try:
        assert_close(got, want, atol, rtol)
        return True
    except AssertionError:
        return False


# ------------------------------------------------------------------ linear

@pytest.mark.parametrize("name", ["linear/bias", "linear/nobias"])
def test_linear_fixture(name):
    c = case(name)
    x, w, b = (arr(e) for e in c["inputs"])
    assert_close(cr.linear(x, w, b), arr(c["outputs"][0]), c["atol"], c["rtol"], name)


def test_linear_bruteforce_and_transpose_sensitivity():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((37, 45)).astype(np.float32)
    w = rng.standard_normal((70, 45)).astype(np.float32)
    b = rng.standard_normal(70).astype(np.float32)
    ref = np.array([[sum(float(x[i, k]) * float(w[n, k]) for k in range(45)) + float(b[n]) for n in range(70)]
                    for i in range(37)])
    assert_close(cr.linear(x, w, b), ref, 1e-5, 1e-6)
    # planted mistake: a transposed weight of a square problem must fail
    ws = rng.standard_normal((45, 45)).astype(np.float32)
    good = cr.linear(x, ws)
    assert not close(cr.linear(x, ws.T.copy()), good, 1e-4, 1e-4)


# ------------------------------------------------------------------ layerNorm

@pytest.mark.parametrize("name", ["layerNorm/wb", "layerNorm/w", "layerNorm/none"])
def test_layernorm_fixture(name):
    c = case(name)
    x, w, b = (arr(e) for e in c["inputs"])
    assert_close(cr.layer_norm(x, w, b, c["args"]["eps"]), arr(c["outputs"][0]), c["atol"], c["rtol"], name)


def test_layernorm_closed_form_and_biased_variance():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((9, 768)) * 3 + 5).astype(np.float32)
    w = rng.standard_normal(768).astype(np.float32)
    xd = x.astype(np.float64)
    mu = xd.mean(-1, keepdims=True)
    var = ((xd - mu) ** 2).mean(-1, keepdims=True)  # biased (1/D), as LayerNorm
    ref = (xd - mu) / np.sqrt(var + 1e-5) * w
    assert_close(cr.layer_norm(x, w, None, 1e-5), ref, 1e-5, 1e-5)
    # planted mistake: the unbiased (1/(D-1)) variance differs measurably at D=64
    c = case("layerNorm/none")
    xf = arr(c["inputs"][0]).astype(np.float64)
    m = xf.mean(-1, keepdims=True)
    bad = (xf - m) / np.sqrt(((xf - m) ** 2).sum(-1, keepdims=True) / (xf.shape[-1] - 1) + 1e-5)
    assert not close(bad, arr(c["outputs"][0]), c["atol"], c["rtol"])


# ------------------------------------------------------------------ rope

@pytest.mark.parametrize("name", ["rope/base10000", "rope/base160000"])
def test_rope_fixture(name):
    c = case(name)
    x = arr(c["inputs"][0])
    assert_close(cr.rope(x, c["args"]["base"]), arr(c["outputs"][0]), c["atol"], c["rtol"], name)


def test_rope_invariants_and_sensitivity():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 50, 64)).astype(np.float32)
    y = cr.rope(x, 10000.0)
    # position 0 is the identity; every (j, j+D/2) pair keeps its norm
    np.testing.assert_allclose(y[:, :, 0], x[:, :, 0], rtol=0, atol=0)
    n0 = x[..., :32] ** 2 + x[..., 32:] ** 2
    n1 = y[..., :32] ** 2 + y[..., 32:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=2e-6, atol=1e-6)
    # angle rule: theta(l, i) = l * base^(-i/half), checked in f64 for a few entries
    c, s = cr.rope_table(50, 64, 10000.0)
    for l, i in [(1, 0), (7, 5), (49, 31)]:
        th = l * 10000.0 ** (-i / 32)
        assert abs(c[l, i] - math.cos(th)) < 2e-6 and abs(s[l, i] - math.sin(th)) < 2e-6
    # planted mistake: the wrong base fails the fixture
    cf = case("rope/base10000")
    xf = arr(cf["inputs"][0])
    assert not close(cr.rope(xf, 160000.0), arr(cf["outputs"][0]), cf["atol"], cf["rtol"])


# ------------------------------------------------------------------ sdpa

@pytest.mark.parametrize("name", ["sdpa/full_attention", "sdpa/sliding_attention", "sdpa/nomask"])
def test_sdpa_fixture(name):
    c = case(name)
    q, k, v, m = (arr(e) for e in c["inputs"])
    assert_close(cr.sdpa(q, k, v, m, c["args"]["scale"]), arr(c["outputs"][0]), c["atol"], c["rtol"], name)


def test_sdpa_closed_forms():
    rng = np.random.default_rng(4)
    B, H, L, D = 2, 3, 17, 16
    k = rng.standard_normal((B, H, L, D)).astype(np.float32)
    v = rng.standard_normal((B, H, L, D)).astype(np.float32)
    valid = rng.random((B, L)) > 0.3
    valid[:, 0] = True
    mask = valid[:, None, None, :].astype(np.uint8)
    # q = 0: uniform weights over visible keys = masked mean of v
    o = cr.sdpa(np.zeros_like(k), k, v, mask, 0.25)
    for b in range(B):
        mean = v[b][:, valid[b]].mean(axis=1)
        np.testing.assert_allclose(o[b], np.broadcast_to(mean[:, None, :], (H, L, D)), rtol=1e-5, atol=1e-6)
    # one visible key: output is exactly that key's value row
    m1 = np.zeros((B, 1, L, L), np.uint8)
    m1[..., 5] = 1
    o1 = cr.sdpa(rng.standard_normal((B, H, L, D)).astype(np.float32), k, v, m1, 0.25)
    np.testing.assert_allclose(o1, np.broadcast_to(v[:, :, 5:6, :], o1.shape), rtol=1e-6, atol=1e-6)
    # planted mistake: dropping the scale fails the fixture
    c = case("sdpa/full_attention")
    q, kk, vv, m = (arr(e) for e in c["inputs"])
    assert not close(cr.sdpa(q, kk, vv, m, 1.0), arr(c["outputs"][0]), c["atol"], c["rtol"])


def test_attention_masks_match_fixture_masks():
    """modernbert/test/modernbert.test.ts:52-63: the sdpa fixtures' masks are
    attentionMasks(valid, B, L, 16)."""
    full = arr(case("sdpa/full_attention")["inputs"][3])
    sliding = arr(case("sdpa/sliding_attention")["inputs"][3])
    B, L = full.shape[0], full.shape[3]
    f, s = cr.attention_masks(full.reshape(B, L), B, L, 16)
    np.testing.assert_array_equal(f, full)
    np.testing.assert_array_equal(s, sliding)


# ------------------------------------------------------------------ gelu / geglu

def test_gelu_fixture_and_libm_values():
    c = case("gelu/erf")
    assert_close(cr.gelu(arr(c["inputs"][0])), arr(c["outputs"][0]), c["atol"], c["rtol"])
    # backend-cpu/test/backend.test.ts:56-73 (Python math.erf values)
    xs = np.array([0.5, 1, 2.4, 3, -4.5, 6], np.float32)
    want = [0.5204998778130465, 0.8427007929497148, 0.999311486103355, 0.9999779095030015, -0.9999999998033839, 1.0]
    got = cr.erf(xs)
    for g, w in zip(got, want):
        assert g == np.float32(w)
    g1 = cr.gelu(np.array([0.0, -10.0, 1.0], np.float32))
    assert g1[0] == 0 and abs(g1[1]) < 1e-20 and g1[2] == np.float32(0.8413447460685429)


def test_geglu_fixture_and_split_order():
    c = case("geglu")
    x = arr(c["inputs"][0])
    assert_close(cr.geglu(x), arr(c["outputs"][0]), c["atol"], c["rtol"])
    # planted mistake: swapping value and gate halves fails
    F = x.shape[-1] // 2
    swapped = np.concatenate([x[..., F:], x[..., :F]], -1)
    assert not close(cr.geglu(swapped), arr(c["outputs"][0]), c["atol"], c["rtol"])


# ------------------------------------------------------------------ gathers

def test_embedding_and_meanpool_fixtures():
    c = case("embedding")
    assert_close(cr.embedding(arr(c["inputs"][0]), arr(c["inputs"][1])), arr(c["outputs"][0]), c["atol"], c["rtol"])
    c = case("meanPool")
    assert_close(cr.mean_pool(arr(c["inputs"][0]), arr(c["inputs"][1])), arr(c["outputs"][0]), c["atol"], c["rtol"])


# ------------------------------------------------------------------ quantized

QCASES = load_cases("ops-quantized.json")


@pytest.mark.parametrize("c", QCASES, ids=[c["name"] for c in QCASES])
def test_quantized_fixture(c):
    a = c["args"]
    if c["op"] == "quantizedLinear":
        x, q, s, b, bias = (arr(e) for e in c["inputs"])
        got = cr.quantized_linear(x, q, s, b, a["groupSize"], bias)
    else:
        q, s, b, ids = (arr(e) for e in c["inputs"])
        w = cr.dequant_compose(q, s, b, a["groupSize"])
        got = cr.embedding(w, ids)
    assert_close(got, arr(c["outputs"][0]), c["atol"], c["rtol"], c["name"])


def test_dequant_exact_is_fl16_of_exact_value():
    """quant.test.ts:107-160 / QUANTIZATION.md: host dequantization is
    fl16(q*s + b) rounded once.  Checked against numpy's float16 cast of the
    f64 value (numpy rounds f64 -> f16 correctly), subnormals included."""
    rng = np.random.default_rng(5)
    q = rng.integers(0, 16, (64, 128)).astype(np.int32)
    s = np.float16(rng.uniform(1e-6, 0.02, (64, 2))).astype(np.float32)
    b = np.float16(rng.uniform(-0.1, 0.1, (64, 2))).astype(np.float32)
    s[0, 0] = np.float32(np.float16(3e-7))  # subnormal scale
    got = cr.dequant_exact_f16(q, s, b, 64)
    exact = q.astype(np.float64) * np.repeat(s, 64, 1).astype(np.float64) + np.repeat(b, 64, 1).astype(np.float64)
    want = exact.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_f16_rounding_matches_numpy():
    rng = np.random.default_rng(6)
    x = np.concatenate([rng.standard_normal(10000) * 10.0 ** rng.integers(-9, 6, 10000),
                        [65504.0, 65519.0, 65520.0, 6e-8, 3e-8, 2.98e-8, -0.0, 1e-10]])
    got = np.array([cr.f64_to_f16_bits(v) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------------ quantizeMatrix

def _weights(rows, cols, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)


def _deq(q, s, b, g):
    sf = s.view(np.float16).astype(np.float64)
    bf = b.view(np.float16).astype(np.float64) if b is not None else 0 * sf
    return q * np.repeat(sf, g, 1) + np.repeat(bf, g, 1)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("g", [64, 32])
def test_quantize_range_fit_bound_and_refit_monotone(bits, g):
    """laya/test/quant.test.ts:47-74."""
    rows, cols = 96, 192
    w = _weights(rows, cols, bits * g)
    q, s, b = cr.quantize_matrix(w, rows, cols, bits, g, refine=False)
    d = _deq(q, s, b, g)
    wd = w.reshape(rows, cols).astype(np.float64)
    sf = np.repeat(s.view(np.float16).astype(np.float64), g, 1)
    eps16 = np.abs(wd) * 2.0 ** -11 + 2.0 ** -24
    assert np.all(np.abs(wd - d) <= sf / 2 + eps16 * 2 + 1e-7)
    lo, hi = (-127, 127) if bits == 8 else (0, 15)
    assert q.min() >= lo and q.max() <= hi
    q2, s2, b2 = cr.quantize_matrix(w, rows, cols, bits, g, refine=True)
    assert ((wd - _deq(q2, s2, b2, g)) ** 2).sum() <= ((wd - d) ** 2).sum()


def test_quantize_zero_rows_and_nibble_layout():
    """laya/test/quant.test.ts:76-97."""
    w = _weights(64, 128, 7)
    w[:128] = 0
    q, s, _ = cr.quantize_matrix(w, 64, 128, 8)
    assert s[0, 0] == 0 and np.all(q[0] == 0)
    d = _deq(q, s, None, 128)
    wd = w.reshape(64, 128)
    assert math.sqrt(((wd - d) ** 2).sum() / (wd.astype(np.float64) ** 2).sum()) < 0.05
    levels = [0, 15, 1, 14, 2, 13, 3, 12, 4, 11, 5, 10, 6, 9, 7, 8]
    w16 = np.array([lv * 0.5 - 1 for lv in levels], np.float32)
    q, s, b = cr.quantize_matrix(w16, 1, 16, 4, 16)
    assert s.view(np.float16)[0, 0] == 0.5 and b.view(np.float16)[0, 0] == -1
    np.testing.assert_array_equal(q[0], levels)
    np.testing.assert_array_equal(_deq(q, s, b, 16)[0], w16)


def test_quantize_round_half_up():
    """Math.round ties go toward +inf (quant.ts:139): a value exactly halfway
    between two q8 levels rounds up, also for negative values."""
    s16 = float(np.float16(1.0 / 127))
    w = np.zeros(64, np.float32)
    w[0] = 1.0                      # sets amax -> scale = f16(1/127)
    w[1] = np.float32(2.5 * s16)    # -> 3 (not banker's 2)
    w[2] = np.float32(-2.5 * s16)   # -> -2 (JS rounds -2.5 to -2)
    q, s, _ = cr.quantize_matrix(w, 1, 64, 8, 64, refine=False)
    assert float(s.view(np.float16)[0, 0]) == s16
    assert q[0, 1] == 3 and q[0, 2] == -2


# ------------------------------------------------------------------ encoder

def test_tiny_encoder_stages_match_golden():
    """modernbert/test/modernbert.test.ts:65-117: every stage within 1e-5
    (abs + rel) of the MLX fp32 activations."""
    cfg_json, W, act = tiny()
    cfg = cr.EncoderConfig.from_json(cfg_json)
    assert cfg.layer_types == act["layer_types"]
    ids = arr(act["inputs"]["input_ids"])
    valid = arr(act["inputs"]["attention_mask"])
    stages = {}
    cr.encoder_forward(cfg, W, ids, valid, stages=stages)
    names = {"embeddings": "embeddings", "final_norm": "encoder.final_norm"}
    names.update({f"layers.{i}": f"encoder.layers.{i}" for i in range(cfg.layers)})
    for ours, theirs in names.items():
        assert_close(stages[ours], arr(act["stages"][theirs]), 1e-5, 1e-5, ours)
    # embed(): masked mean of final_norm
    pooled = cr.mean_pool(stages["final_norm"], valid)
    fin = arr(act["stages"]["encoder.final_norm"]).astype(np.float64)
    for b in range(ids.shape[0]):
        np.testing.assert_allclose(pooled[b], fin[b][valid[b] != 0].mean(0), atol=1e-5)


# ------------------------------------------------------------------ 16-bit storage formats

def _bits32(x) -> np.ndarray:
    return np.asarray(x, np.float32).view(np.uint32)


def test_bf16_rounding_pinned_by_the_format():
    """round_bf16 from what the format fixes, not from a formula: every
    bfloat16 value (all 65,536 patterns) comes back unchanged; a value
    exactly halfway between two neighbours goes to the one with an even
    last bit; one f32 ulp either side of that halfway point goes to the
    nearer neighbour; halfway above the largest finite value overflows to
    +-inf.  torch's bfloat16 conversion (its own RNE) agrees on 200k random
    values across the exponent range."""
    import torch
    hi = np.arange(65536, dtype=np.uint32)
    vals = (hi << 16).view(np.float32)
    nan = np.isnan(vals)
    got = _bits32(cr.round_bf16(vals))
    np.testing.assert_array_equal(got[~nan], (hi << 16)[~nan])
    assert np.all(np.isnan(got.view(np.float32)[nan]))
    # finite bf16 values below the largest: halfway points and one ulp either side
    fin = hi[~nan & ~np.isinf(vals) & ((hi & 0x7fff) < 0x7f7f)]
    mid = (fin << 16) | 0x8000
    up = fin + 1  # the next bf16 in magnitude, for either sign
    even = np.where(fin & 1, up, fin)
    np.testing.assert_array_equal(_bits32(cr.round_bf16(mid.view(np.float32))) >> 16, even)
    np.testing.assert_array_equal(_bits32(cr.round_bf16((mid - 1).view(np.float32))) >> 16, fin)
    np.testing.assert_array_equal(_bits32(cr.round_bf16((mid + 1).view(np.float32))) >> 16, up)
    big = np.array([0x7f7f8000, 0x7f7fffff, 0xff7f8000, 0x7f7f7fff], np.uint32).view(np.float32)
    np.testing.assert_array_equal(_bits32(cr.round_bf16(big)) >> 16, [0x7f80, 0x7f80, 0xff80, 0x7f7f])
    rng = np.random.default_rng(16)
    x = (rng.standard_normal(200000) * 10.0 ** rng.integers(-38, 38, 200000)).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(_bits32(cr.round_bf16(x)), _bits32(want))


def test_f16_decode_and_encode_every_pattern():
    """All 65,536 binary16 patterns decode to numpy's float16 values (NaN to
    NaN), and every non-NaN value rounds back through f16 storage to itself
    (subnormals, +-0 and +-inf included)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = cr.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(_bits32(got[~nan]), _bits32(want[~nan]))
    back = np.array([cr.f64_to_f16_bits(float(v)) for v in got[~nan]], np.uint16)
    np.testing.assert_array_equal(back, h[~nan])
    np.testing.assert_array_equal(_bits32(cr.round_f16(got[~nan])), _bits32(got[~nan]))


def test_reduced_storage_encoder_rounds_every_op():
    """encoder_forward(dtype="f16"), the model of a backend that stores every
    activation in f16: (1) layer 0 equals the oracle's pinned ops composed
    with an f16 rounding after each op, bit for bit; (2) every stage holds
    f16 values only; (3) every stage is within the reference's f16 parity
    bar (0.02, docs/RESULTS.md) of the MLX f32 activations and differs from
    the f32 path, so the rounding is really applied."""
    cfg_json, W, act = tiny()
    cfg = cr.EncoderConfig.from_json(cfg_json)
    ids = arr(act["inputs"]["input_ids"])
    valid = arr(act["inputs"]["attention_mask"])
    W16 = {k: cr.round_f16(v) for k, v in W.items()}
    st16 = {}
    cr.encoder_forward(cfg, W16, ids, valid, dtype="f16", stages=st16)
    # (1) layer 0 op by op (a global layer: no attn_norm in layer 0)
    r = cr.round_f16
    full, _ = cr.attention_masks(valid, *ids.shape, cfg.local_attention)
    x = st16["embeddings"]
    B, L, H = x.shape
    nh, hd = cfg.heads, cfg.head_dim
    qkv = r(cr.linear(x, W16["layers.0.attn.Wqkv.weight"])).reshape(B, L, 3, nh, hd).transpose(2, 0, 3, 1, 4)
    q, k, v = (np.ascontiguousarray(t) for t in qkv)
    att = r(cr.sdpa(r(cr.rope(q, cfg.global_theta)), r(cr.rope(k, cfg.global_theta)), v, full, hd ** -0.5))
    merged = np.ascontiguousarray(att.transpose(0, 2, 1, 3)).reshape(B, L, H)
    x1 = r(x + r(cr.linear(merged, W16["layers.0.attn.Wo.weight"])))
    m = r(cr.linear(r(cr.layer_norm(x1, W16["layers.0.mlp_norm.weight"], None, cfg.norm_eps)),
                    W16["layers.0.mlp.Wi.weight"]))
    y = r(x1 + r(cr.linear(r(cr.geglu(m)), W16["layers.0.mlp.Wo.weight"])))
    np.testing.assert_array_equal(_bits32(st16["layers.0"]), _bits32(y))
    st32 = {}
    cr.encoder_forward(cfg, W, ids, valid, stages=st32)
    for name, t in st16.items():
        np.testing.assert_array_equal(_bits32(r(t)), _bits32(t))  # (2)
        theirs = "embeddings" if name == "embeddings" else f"encoder.{name}"
        assert_close(t, arr(act["stages"][theirs]), 2e-2, 2e-2, name)  # (3)
        assert not np.array_equal(t, st32[name]), name


# ------------------------------------------------------------------ decision head

def _tiny_decision():
    import json
    import os
    from fixtures import GOLDEN, read_safetensors
    W = {k: v.astype(np.float32) for k, v in read_safetensors(os.path.join(GOLDEN, "tiny", "model.safetensors")).items()}
    with open(os.path.join(GOLDEN, "tiny", "rl_agent_config.json")) as f:
        agent = json.load(f)
    cfg_json, _, act = tiny()
    return cr.EncoderConfig.from_json(cfg_json), W, agent, act


def test_decision_head_stages_match_golden():
    """laya/test/model.test.ts:26-79 on the oracle: every stage (encoder,
    type embedding, both head layers, logits, act) within 1e-5 (abs + rel)
    of the MLX activations, and masked logit slots exactly -1e4."""
    cfg, W, agent, act = _tiny_decision()
    inp = {k: arr(v) for k, v in act["inputs"].items()}
    st = {}
    logits, a = cr.decision_forward(cfg, W, agent["head_layers"], inp["input_ids"], inp["attention_mask"],
                                    inp["qtype"], inp["marker_pos"], inp["marker_mask"], stages=st)
    assert sorted(st) == sorted(act["stages"])
    for name, e in act["stages"].items():
        assert_close(st[name], arr(e), 1e-5, 1e-5, name)
    mm = inp["marker_mask"] != 0
    assert np.all(logits[~mm] == np.float32(-1e4))
    assert a.shape == (inp["input_ids"].shape[0], len(agent["act_costs"]) + 1)


@pytest.mark.parametrize("slip", ["in_proj_bias", "relu", "sort"])
def test_decision_head_planted_mistakes_fail(slip):
    """A dropped attention in-projection bias in the head, the ReLU left out
    of its FFN, or
    the top-two features taken from an unsorted row each break the fixture
    check (the mistake is planted in the oracle's inputs or ops, on the CPU)."""
    cfg, W, agent, act = _tiny_decision()
    inp = {k: arr(v) for k, v in act["inputs"].items()}
    W = dict(W)
    saved = None
    if slip == "in_proj_bias":
        W["head.layers.0.self_attn.in_proj.bias"] = np.zeros_like(W["head.layers.0.self_attn.in_proj.bias"])
    elif slip == "relu":
        saved = np.maximum
        np.maximum = lambda a, b, *x, **k: a if np.ndim(b) == 0 and float(b) == 0 else saved(a, b, *x, **k)
    else:
        saved = np.sort
        np.sort = lambda a, axis=-1, **k: a
    try:
        st = {}
        cr.decision_forward(cfg, W, agent["head_layers"], inp["input_ids"], inp["attention_mask"], inp["qtype"],
                            inp["marker_pos"], inp["marker_mask"], stages=st)
    finally:
        if slip == "relu":
            np.maximum = saved
        elif slip == "sort":
            np.sort = saved
    name = "act" if slip == "sort" else "head.layers.0"
    assert not close(st[name], arr(act["stages"][name]), 1e-5, 1e-5)
