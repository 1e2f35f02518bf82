"""Benchmark: ModernBERT-base encode tokens/s at B=32, T=512 on one MI355X.

One step = one full encoder forward (embeddings + 22 layers + final norm)
over a new batch of 32 sequences of 512 tokens (lengths uniform in [64, 512],
right-padded), through HipBackend, the laya-js `Backend`
contract on libhipbackend.so, driven by the unchanged encoder code.  Every
step encodes a batch of its own (token ids and masks, all resident on the GPU
before the timed region), so each step also builds its masks' tile summaries,
and each step launches its whole output, the final LayerNorm included.  Weights
are random-init fp16 ~N(0, 0.02) with LayerNorm gamma = 1; ids uniform in
[0, 50368).

Prints ONE JSON line on stdout.  `value` comes from a clean timed region
(HIP events around K steps, nothing else instrumented).  Also reported:
- roofline of the dominant kernel, the large-M linear GEMM
  (gemm_mfma_arow, f16, plain epilogue: Wqkv, attn Wo and mlp Wo of every
  layer): a second timed region of K steps with HIP events around each
  linear launch on the backend's stream gives its average launch time;
  achieved = algorithmic 2*M*N*K per launch / that time.  `traffic` is the
  HBM bytes per launch read from the rocprofv3 FETCH_SIZE / WRITE_SIZE
  summary committed in profiles/ (null when absent);
- cpu_baseline: the CPU oracle (a C restatement of the reference's CPU
  backend, OpenMP over the host cores) on a bounded sample of the same
  workload.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
  python bench.py --mode gemm    # isolated config-1/2 GEMM sweep (stderr table + JSON lines)
  python bench.py --mode copy    # the library's contiguous copy kernel (HBM counter calibration)
  python bench.py --mode config4 # BASELINE config 4 (ModernBERT-large shape, B=16, T=2048), fp16 and quantized
  python bench.py --mode config0 # BASELINE config 0 (B=1, T=128): ms per forward, CPU oracle beside it
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "laya-js_amd"))

PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA (spec)
PEAK_HBM_GBS = 8000.0

BASE = {"vocab_size": 50368, "hidden_size": 768, "intermediate_size": 1152, "num_hidden_layers": 22,
        "num_attention_heads": 12, "local_attention": 128}
METRIC = "ModernBERT-base encode tokens/s at B=32,T=512; linear-layer MFMA util %"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_weights(cfg: dict, seed: int = 0) -> dict:
    """Random-init fp16 encoder weights (names without the 'encoder.' prefix)."""
    rng = np.random.default_rng(seed)
    H, I, V, Lr = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_hidden_layers"]

    def n(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * 0.02).astype(np.float16)
    W = {"embeddings.tok_embeddings.weight": n(V, H), "embeddings.norm.weight": np.ones(H, np.float16),
         "final_norm.weight": np.ones(H, np.float16)}
    for i in range(Lr):
        p = f"layers.{i}."
        if i:
            W[p + "attn_norm.weight"] = np.ones(H, np.float16)
        W[p + "attn.Wqkv.weight"] = n(3 * H, H)
        W[p + "attn.Wo.weight"] = n(H, H)
        W[p + "mlp_norm.weight"] = np.ones(H, np.float16)
        W[p + "mlp.Wi.weight"] = n(2 * I, H)
        W[p + "mlp.Wo.weight"] = n(H, I)
    return W


def linear_flops_per_forward(cfg: dict, M: int) -> float:
    H, I, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    per_layer = 2 * M * (3 * H * H + H * H + 2 * I * H + H * I)
    return float(per_layer * L)


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "gemm_mfma_arow_config3_hbm_counters.md")


def _is_dominant(key: str) -> bool:
    """linear[M=..,N=..,K=..] launches served by the large-M f16 kernel with a
    plain epilogue (not GeGLU, not the fused q / k / v projection)."""
    return (key.startswith("linear[") and "geglu" not in key and ",qkv" not in key
            and int(key.split("M=")[1].split(",")[0]) >= 4096)


def _key_flops(key: str) -> float:
    """2*M*N*K of one linear launch.  The key's N is the launch's output
    width; a GeGLU launch computes twice that many columns (value and gate)
    before its epilogue halves them."""
    f = dict(kv.split("=") for kv in key[key.index("[") + 1:key.index("]")].split(",") if "=" in kv)
    n = int(f["N"]) * (2 if "geglu" in key else 1)
    return 2.0 * int(f["M"]) * n * int(f["K"])


def _profiled_traffic():
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 counter summary (line `hbm_bytes_per_launch: <n>`), or None."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            for line in f:
                if line.strip().startswith("hbm_bytes_per_launch:"):
                    return float(line.split(":", 1)[1].strip().split()[0])
    except OSError:
        pass
    return None


def make_batches(n: int, B: int, T: int, seed: int) -> list:
    """n synthetic config-3 batches: ids uniform in [0, 50368), lengths
    uniform in [64, T], right-padded."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        lens = rng.integers(64, T + 1, B)
        ids = rng.integers(0, BASE["vocab_size"], (B, T)).astype(np.int32)
        out.append((ids, (np.arange(T)[None, :] < lens[:, None]).astype(np.uint8)))
    return out


def run_encode(args) -> dict:
    from laya_hip.backend import HipBackend
    from laya_hip.host import HostTensor
    from laya_hip.modernbert import loadModernBert, parseModernBertConfig

    B, T = 32, 512
    cfg = parseModernBertConfig(BASE)
    W = make_weights(BASE)

    be = HipBackend(0, fuse_qkv=args.fuse_qkv)
    info = be.device_info()
    log(f"device: {info}")
    t0 = time.time()
    enc = loadModernBert(be, cfg, lambda nm: HostTensor("f16", W[nm[8:]].shape, W[nm[8:]])
                         if nm.startswith("encoder.") and nm[8:] in W else None, dtype="f16")
    # one batch per step, all resident before anything is timed: every step
    # encodes new inputs, so it also summarises its own attention masks
    batches = make_batches(args.warmup + 2 * args.steps, B, T, seed=1)
    inputs = [enc.uploadInputs(ids, valid, B, T) for ids, valid in batches]
    be.flush()
    log(f"weights + {len(inputs)} batches of inputs resident in {time.time() - t0:.1f}s")
    cursor = iter(range(len(inputs)))

    def step():
        i = next(cursor)
        y = enc.encode(inputs[i])
        be.flush(y, wait=False)  # the whole forward, final LayerNorm included, is launched inside the step
        be.dispose(y)
        return i

    for _ in range(args.warmup):
        step()
    be.flush()

    def timed(n):
        ev0, ev1 = be.event(), be.event()
        be.flush()
        wall0 = time.perf_counter()
        be.record(ev0)
        used = [step() for _ in range(n)]
        be.record(ev1)
        be.flush()
        return be.elapsed_ms(ev0, ev1), time.perf_counter() - wall0, used

    gpu_ms, wall, used = timed(args.steps)
    ms_per_step = gpu_ms / args.steps
    tokens = B * T
    valid_tokens = float(np.mean([batches[i][1].sum() for i in used]))
    log(f"timed {args.steps} steps (one new batch each): {gpu_ms:.2f} ms on the stream ({wall * 1e3:.2f} ms wall) "
        f"-> {ms_per_step:.3f} ms/step")

    # second timed region: HIP events around every linear launch (on the
    # backend's stream) -> per-launch GPU time by shape
    be.startProfiling(only={"hb_linear", "hb_linear_qkv"})
    gpu_ms2, _, _ = timed(args.steps)
    prof = be.stopProfiling()
    log(f"instrumented region: {gpu_ms2 / args.steps:.3f} ms/step")
    dom = {k: v for k, v in prof.items() if _is_dominant(k)}
    dom_n = sum(n for n, t in dom.values())
    dom_ms = sum(t for n, t in dom.values())
    dom_flops = sum(n * _key_flops(k) for k, (n, t) in dom.items())
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    lin_ms = sum(t for n, t in prof.values()) / args.steps
    lin_launches = sum(n for n, t in prof.values()) // args.steps
    lin_flops = linear_flops_per_forward(BASE, tokens)
    log("linear launches per forward:")
    for k, (n, t) in sorted(prof.items(), key=lambda kv: -kv[1][1]):
        log(f"  {k:44s} launches {n // args.steps:4d}  avg {t / n * 1e3:8.1f} us  "
            f"{_key_flops(k) / (t / n * 1e-3) / 1e12:7.1f} TFLOP/s")
    log(f"dominant kernel: {dom_n // args.steps} launches/forward, avg {dom_ms / dom_n * 1e3:.1f} us, "
        f"{achieved:.1f} TFLOP/s")
    traffic = _profiled_traffic()
    for inp in inputs:
        enc.disposeInputs(inp)

    # host-to-host rate, never `value`: host mask build, uploads over PCIe,
    # the encode, and the [B, T, 768] f16 output read back; each part timed
    ids, valid = batches[0]
    parts = {"masks_ms": 0.0, "upload_ms": 0.0, "encode_ms": 0.0, "read_ms": 0.0}
    reps = 3
    from laya_hip.modernbert import attentionMasks
    w0 = time.perf_counter()
    for _ in range(reps):
        a = time.perf_counter()
        attentionMasks(valid, B, T, cfg.localAttention)
        parts["masks_ms"] += time.perf_counter() - a
        a = time.perf_counter()
        inp2 = enc.uploadInputs(ids, valid, B, T)  # builds the masks again, then uploads
        be.flush()
        parts["upload_ms"] += time.perf_counter() - a
        a = time.perf_counter()
        y = enc.encode(inp2)
        be.flush(y)
        parts["encode_ms"] += time.perf_counter() - a
        a = time.perf_counter()
        out = be.read(y)
        parts["read_ms"] += time.perf_counter() - a
        be.dispose(y)
        enc.disposeInputs(inp2)
    pcie_ms = (time.perf_counter() - w0) / reps * 1e3
    parts = {k: v / reps * 1e3 for k, v in parts.items()}
    parts["upload_ms"] -= parts["masks_ms"]  # uploadInputs' own mask build
    log(f"host-to-host (build masks, upload ids/masks, encode, read [{B},{T},768] f16 back): {pcie_ms:.2f} ms/step "
        f"= " + ", ".join(f"{k} {v:.2f}" for k, v in parts.items()))

    inp = enc.uploadInputs(ids, valid, B, T)
    y = enc.encode(inp)
    out = be.read(y)
    be.dispose(y)
    finite = bool(np.isfinite(out.data.astype(np.float32)).all())
    enc.disposeInputs(inp)
    enc.dispose()
    be.destroy()

    res = {
        "metric": METRIC,
        "value": tokens / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (random-init fp16 weights ~N(0,0.02), ids U[0,50368), lengths U[64,512] right-padded)",
        "config": {
            "workload": "BASELINE config 3: ModernBERT-base-shape encoder forward, B=32, T=512, 22 layers, "
                        "hidden 768, 12 heads, GeGLU 1152, local window 128 / global every 3rd layer",
            "global_batch": B, "seq_len": T, "parallelism": "single GPU", "fuse_qkv": bool(args.fuse_qkv),
            "padded_tokens_per_step": tokens, "valid_tokens_per_step": valid_tokens,
            "valid_tokens_per_s": valid_tokens / (ms_per_step * 1e-3),
            "linear_tflop_per_step": lin_flops / 1e12,
            "linear_ms_per_step": lin_ms, "linear_launches_per_step": lin_launches,
            "linear_tflops": lin_flops / (lin_ms * 1e-3) / 1e12,
            "linear_mfma_util_pct": 100.0 * lin_flops / (lin_ms * 1e-3) / 1e12 / PEAK_F16_TFLOPS,
            "output_finite": finite, "device": info.get("name") or info.get("arch"),
            "host_to_host_ms_per_step": pcie_ms, "host_to_host_parts_ms": parts,
        },
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_F16_TFLOPS, "traffic": traffic,
                     "kernel": "gemm_mfma_arow (f16, plain epilogue): Wqkv 16384x2304x768, attn Wo "
                               "16384x768x768 and mlp Wo 16384x768x1152 of every layer; algorithmic 2*M*N*K = "
                               f"{dom_flops / dom_n / 1e9:.2f} GFLOP per launch on average over "
                               f"{dom_n // args.steps} launches per forward; avg launch {dom_ms / dom_n * 1e3:.1f} us",
                     "avg_launch_us": dom_ms / dom_n * 1e3},
    }
    return res


LARGE = {"vocab_size": 256000, "hidden_size": 1024, "intermediate_size": 2624, "num_hidden_layers": 28,
         "num_attention_heads": 16, "local_attention": 128}


def run_config4(args) -> None:
    """the ModernBERT-large-shape encoder (hidden 1024, 28
    layers, 16 heads, GeGLU 2624, window 128 / global every third layer,
    256000-token vocabulary) at B = 16, T = 2048 (full-length sequences),
    then the pooled 1024 -> 8 classifier with softmax; fp16 weights, then
    laya's quantized format (q4 affine Linears, group 64, and a q8 symmetric
    embedding table).  The quantized codes, scales and zeros are drawn at
    random in the format's ranges (the kernels' time does not depend on the
    values; tests/test_gpu_config4.py checks the numerics).  One JSON line
    per weight format."""
    from laya_hip.backend import HipBackend
    from laya_hip.compose import mean_pool
    from laya_hip.host import HostQuantized, HostTensor, pack_quantized
    from laya_hip.modernbert import loadModernBert, parseModernBertConfig

    B, T, C = 16, 2048, 8
    H, I, V = LARGE["hidden_size"], LARGE["intermediate_size"], LARGE["vocab_size"]
    cfg = parseModernBertConfig(LARGE)
    rng = np.random.default_rng(4)
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    valid = np.ones((B, T), np.uint8)
    be = HipBackend(0)
    Wc = be.fromHost(HostTensor("f32", (C, H), (rng.standard_normal((C, H)) * 0.5).astype(np.float32)))
    bc = be.fromHost(HostTensor("f32", (C,), (rng.standard_normal(C) * 0.1).astype(np.float32)))
    t0 = time.time()
    W = make_weights(LARGE, seed=4)
    log(f"config4: fp16 weights generated in {time.time() - t0:.1f}s")

    def quantized(name):
        v = W[name]
        N, K = v.shape
        if name == "embeddings.tok_embeddings.weight":
            q = rng.integers(-127, 128, (N, K), dtype=np.int64)
            s = rng.uniform(1e-4, 3e-4, (N, K // 64)).astype(np.float16)
            return HostQuantized((N, K), 8, 64, "symmetric", pack_quantized(q, 8), HostTensor("f16", s.shape, s), None)
        q = rng.integers(0, 16, (N, K), dtype=np.int64)
        s = rng.uniform(2e-3, 6e-3, (N, K // 64)).astype(np.float16)
        z = (-7.5 * s.astype(np.float32)).astype(np.float16)
        return HostQuantized((N, K), 4, 64, "affine", pack_quantized(q, 4), HostTensor("f16", s.shape, s),
                             HostTensor("f16", z.shape, z))

    def getter(fmt):
        def get(nm):
            if not nm.startswith("encoder.") or nm[8:] not in W:
                return None
            k = nm[8:]
            if fmt == "quantized" and (k.endswith(("Wqkv.weight", "Wo.weight", "Wi.weight")) or
                                        k == "embeddings.tok_embeddings.weight"):
                return quantized(k)
            return HostTensor("f16", W[k].shape, W[k])
        return get

    for fmt in ("fp16", "quantized"):
        t0 = time.time()
        enc = loadModernBert(be, cfg, getter(fmt), dtype="f16")
        inp = enc.uploadInputs(ids, valid, B, T)
        be.flush()
        log(f"config4 {fmt}: weights + inputs resident in {time.time() - t0:.1f}s")

        def step():
            def f():
                pooled = mean_pool(be, enc.encode(inp), inp["mask"])
                return be.softmax(be.linear(pooled, Wc, bc), -1)
            return be.scope(f)

        for _ in range(args.warmup):
            be.dispose(step())
        ev0, ev1 = be.event(), be.event()
        be.flush()
        be.record(ev0)
        for _ in range(args.steps):
            be.dispose(step())
        be.record(ev1)
        be.flush()
        ms = be.elapsed_ms(ev0, ev1) / args.steps
        print(json.dumps({"mode": "config4", "metric": "ModernBERT-large encode + pooled classifier tokens/s at "
                          "B=16,T=2048", "weights": fmt, "value": B * T / (ms * 1e-3), "unit": "tokens/s",
                          "ms_per_step": ms, "steps": args.steps, "warmup": args.warmup, "dtype": "f16",
                          "data": "synthetic (random-init weights, ids U[0,256000), full-length sequences)",
                          "config": {"workload": "BASELINE config 4", "global_batch": B, "seq_len": T,
                                     "layers": LARGE["num_hidden_layers"], "hidden": H, "intermediate": I,
                                     "vocab": V}}), flush=True)
        enc.disposeInputs(inp)
        enc.dispose()
    be.dispose(Wc)
    be.dispose(bc)
    be.destroy()


def run_config0(args) -> None:
    """the ModernBERT-base-shape encoder at batch 1, seq
    128, no padding (the reference's CPU-runnable case): GPU ms per forward
    (inputs resident) through the Backend ops, the same forward recorded
    once and replayed (`replay_ms`), the same forward through Backend.compile
    (`compile_ms`: input copies, replay and output copy per call), and the
    CPU oracle on that forward."""
    from laya_hip.backend import HipBackend
    from laya_hip.host import HostTensor
    from laya_hip.modernbert import loadModernBert, parseModernBertConfig
    from oracle import cpu_ref as cr

    B, T = 1, 128
    cfg = parseModernBertConfig(BASE)
    W = make_weights(BASE)
    rng = np.random.default_rng(0)
    ids = rng.integers(0, BASE["vocab_size"], (B, T)).astype(np.int32)
    valid = np.ones((B, T), np.uint8)
    be = HipBackend(0)
    enc = loadModernBert(be, cfg, lambda nm: HostTensor("f16", W[nm[8:]].shape, W[nm[8:]])
                         if nm.startswith("encoder.") and nm[8:] in W else None, dtype="f16")
    inp = enc.uploadInputs(ids, valid, B, T)
    for _ in range(args.warmup):
        be.dispose(enc.encode(inp))
    ev0, ev1 = be.event(), be.event()
    be.flush()
    be.record(ev0)
    for _ in range(args.steps):
        be.dispose(enc.encode(inp))
    be.record(ev1)
    be.flush()
    ms = be.elapsed_ms(ev0, ev1) / args.steps
    # the same forward recorded once and replayed (HipBackend.capture): no
    # per-op host work in the timed region
    g = be.capture(lambda: enc.encode(inp))
    for _ in range(args.warmup):
        g.run()
    be.flush()
    be.record(ev0)
    for _ in range(args.steps):
        g.run()
    be.record(ev1)
    be.flush()
    replay_ms = be.elapsed_ms(ev0, ev1) / args.steps
    out = g.out
    g.destroy()
    be.dispose(out)
    # the same forward through Backend.compile (the contract member laya's
    # DecisionModel.compiled() uses): each call copies its inputs into the
    # recorded blocks, replays, and returns a fresh copy of the output
    fn = be.compile(lambda i_, m_, f_, s_: enc.encode({"ids": i_, "mask": m_, "masks": {
        "full_attention": f_, "sliding_attention": s_}}))
    ins = (inp["ids"], inp["mask"], inp["masks"]["full_attention"], inp["masks"]["sliding_attention"])
    for _ in range(max(1, args.warmup)):
        be.dispose(fn(*ins))
    be.flush()
    be.record(ev0)
    for _ in range(args.steps):
        be.dispose(fn(*ins))
    be.record(ev1)
    be.flush()
    compile_ms = be.elapsed_ms(ev0, ev1) / args.steps
    fn.release()
    enc.disposeInputs(inp)
    enc.dispose()
    be.destroy()
    cfg0 = cr.EncoderConfig.from_json(BASE)
    W32 = {k: v.astype(np.float32) for k, v in W.items()}
    t0 = time.perf_counter()
    y = cr.encoder_forward(cfg0, W32, ids, valid)
    cpu_ms = (time.perf_counter() - t0) * 1e3
    assert np.isfinite(y).all()
    print(json.dumps({"mode": "config0", "metric": "ModernBERT-base encode ms per forward at B=1,T=128",
                      "value": ms, "unit": "ms", "higher_is_better": False, "tokens_per_s": B * T / (ms * 1e-3),
                      "replay_ms": replay_ms, "replay_tokens_per_s": B * T / (replay_ms * 1e-3),
                      "compile_ms": compile_ms, "compile_tokens_per_s": B * T / (compile_ms * 1e-3),
                      "steps": args.steps, "warmup": args.warmup, "dtype": "f16",
                      "data": "synthetic (random-init fp16 weights ~N(0,0.02), ids U[0,50368), no padding)",
                      "config": {"workload": "BASELINE config 0", "global_batch": B, "seq_len": T},
                      "cpu_baseline": {"value": cpu_ms, "unit": "ms", "cores": cr.num_threads(), "kind": "port",
                                       "sample": "the same forward on the CPU oracle (f32 storage, f64 "
                                                 "accumulation)"}}), flush=True)


def cpu_baseline(sample_b: int = 8) -> dict:
    """The CPU oracle (C, OpenMP, f64 accumulation) on `sample_b` of the 32
    sequences at T=512, all 22 layers; reported as tokens/s of that sample."""
    from oracle import cpu_ref as cr
    sys.path.insert(0, ROOT)
    B, T = sample_b, 512
    W = {k: v.astype(np.float32) for k, v in make_weights(BASE).items()}
    rng = np.random.default_rng(1)
    lens = rng.integers(64, T + 1, 32)[:B]
    ids = rng.integers(0, BASE["vocab_size"], (32, T)).astype(np.int32)[:B]
    valid = (np.arange(T)[None, :] < lens[:, None]).astype(np.uint8)
    cfg = cr.EncoderConfig.from_json(BASE)
    t0 = time.perf_counter()
    y = cr.encoder_forward(cfg, W, ids, valid)
    dt = time.perf_counter() - t0
    assert np.isfinite(y).all()
    cpu = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": B * T / dt, "unit": "tokens/s", "cores": cr.num_threads(), "kind": "port",
            "sample": f"{B} of the 32 sequences (T=512, padded, all 22 layers) in {dt:.1f}s on {cpu}; "
                      "C restatement of the reference CPU backend (f32 storage, f64 accumulation)"}


def run_gemm_sweep(args) -> None:
    """BASELINE configs 1 and 2: isolated linears at M in {128..16384}."""
    from laya_hip import compose as C
    from laya_hip.backend import HipBackend
    from laya_hip.host import HostQuantized, HostTensor, pack_quantized
    from laya_hip.quant import quantize_matrix

    be = HipBackend(0)
    rng = np.random.default_rng(0)
    shapes = [("Wqkv", 2304, 768, False), ("Wo", 768, 768, False), ("Wi+GeGLU", 2304, 768, True),
              ("WoMlp", 768, 1152, False)]
    log(f"{'shape':10s} {'M':>6s} {'kind':>5s} {'us':>9s} {'TFLOP/s':>8s} {'%peak':>6s}")
    for name, N, K, geglu in shapes:
        w = (rng.standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float16)
        Wt = be.fromHost(HostTensor("f16", (N, K), w))
        quants = {}
        for bits in (8, 4):
            q, s, z = quantize_matrix(w.astype(np.float32), N, K, bits, 64, refine=bits == 4)
            h = HostQuantized((N, K), bits, 64, "symmetric" if bits == 8 else "affine", pack_quantized(q, bits),
                              HostTensor("f16", s.shape, s), HostTensor("f16", z.shape, z) if z is not None else None)
            quants[bits] = C.upload_quantized(be, h, "f16")
        for M in (128, 512, 2048, 8192, 16384):
            X = be.fromHost(HostTensor("f16", (M, K), rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)))
            kinds = [("f16", lambda: be.linear(X, Wt))]
            if M in (512, 2048, 8192):
                kinds += [(f"q{b}", (lambda b=b: C.quantized_linear(be, X, quants[b]))) for b in (8, 4)]
            for kind, fn in kinds:
                def launch():
                    y = fn()
                    return be._ready(be.geglu(y) if geglu else y)  # launched now, not left pending
                for _ in range(3):
                    be.dispose(launch())
                reps = max(5, int(2e11 / (2 * M * N * K)))
                a, b = be.event(), be.event()
                be.flush()
                be.record(a)
                for _ in range(reps):
                    be.dispose(launch())
                be.record(b)
                ms = be.elapsed_ms(a, b) / reps
                tf = 2 * M * N * K / (ms * 1e-3) / 1e12
                log(f"{name:10s} {M:6d} {kind:>5s} {ms * 1e3:9.1f} {tf:8.1f} {100 * tf / PEAK_F16_TFLOPS:6.1f}")
                print(json.dumps({"shape": name, "M": M, "N": N, "K": K, "kind": kind, "us": ms * 1e3,
                                  "tflops": tf, "mfma_util_pct": 100 * tf / PEAK_F16_TFLOPS}), flush=True)
            be.dispose(X)
    be.destroy()


def run_copy(args) -> None:
    """The library's contiguous copy kernel (copy_bytes_kernel via hb_unary
    COPY) over a buffer of known size: reference for the HBM counters."""
    from laya_hip import ffi as F
    from laya_hip.backend import HipBackend
    be = HipBackend(0)
    nbytes = args.copy_mib << 20
    src, dst = be._malloc(nbytes), be._malloc(nbytes)
    n = nbytes // 2
    shape, xs = F.i64s([n]), F.i64s([1])

    def launch():
        be.n.call("copy", "hb_unary", be.ctx, F.HB_UN_COPY, F.HB_F16, src.ptr, xs, F.HB_F16, dst.ptr, None, shape,
                  1, 0.0)
    for _ in range(3):
        launch()
    a, b = be.event(), be.event()
    be.flush()
    be.record(a)
    for _ in range(args.steps):
        launch()
    be.record(b)
    ms = be.elapsed_ms(a, b) / args.steps
    print(json.dumps({"mode": "copy", "kernel": "copy_bytes_kernel", "bytes_read_per_launch": nbytes,
                      "bytes_written_per_launch": nbytes, "us_per_launch": ms * 1e3,
                      "GB_per_s": 2 * nbytes / (ms * 1e-3) / 1e9}), flush=True)
    be.destroy()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", choices=["encode", "gemm", "copy", "config0", "config4"], default="encode")
    ap.add_argument("--copy-mib", type=int, default=512, help="buffer size for --mode copy")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--fuse-qkv", action="store_true",
                    help="encode with HipBackend(fuse_qkv=True): the q / k / v projection written head-major with "
                         "RoPE in its epilogue (hb_linear_qkv)")
    ap.add_argument("--cpu-sample", type=int, default=8, help="sequences in the CPU-baseline sample")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the encoder is "
              "data-parallel over sequences: N GPUs would each encode B/N of the batch rows with the same "
              "weights, with no collective on the path", file=sys.stderr)
        sys.exit(2)
    if args.mode == "config4":
        run_config4(args)
        return
    if args.mode == "config0":
        run_config0(args)
        return
    if args.mode == "gemm":
        run_gemm_sweep(args)
        return
    if args.mode == "copy":
        run_copy(args)
        return
    res = run_encode(args)
    if not args.no_cpu:
        log("timing the CPU baseline ...")
        res["cpu_baseline"] = cpu_baseline(args.cpu_sample)
        log(f"cpu baseline: {res['cpu_baseline']}")
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
