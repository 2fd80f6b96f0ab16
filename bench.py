#!/usr/bin/env python3
"""Decode throughput of the 3B AR model at batch 1, KV length 4096, on one GPU.

Workload: the 3B AR decoder (hidden 3072, 24/8 heads, head_dim 128, FFN 8192,
28 layers, vocab 83968, RMSNorm eps 1e-5, RoPE theta 5e5), random-init bf16
weights N(0, 0.02) with unit norm gains, a random prompt prefilled so that the
timed steps are centred on KV length 4096, then greedy decoding. A step is one
token: the device sampler (argmax) followed by the whole decode step (28 x
[QKV GEMV, split-K attention, O GEMV, gate/up GEMV, down GEMV], lm_head GEMV),
replayed as one hipGraph per token with no host sync between tokens, one
kernel per op. Inputs (weights, KV cache, logits) are resident in HBM when the
timed region starts.

Other workloads of the same model (one JSON line each, not the headline):
  --config cfg     CFG as batch 2 (cond + uncond 512-token prompts), scale 1.5,
                   T 1.0 / top-k 50 / top-p 0.93, 1024 tokens through the
                   request driver (yuear_generate_tokens): output tokens/s.
  --config long    3000-token prefill (TFLOP/s against the bf16 MFMA peak),
                   then batch-1 decode until KV 8192: ms/token per 512 steps.
  --config batch8  8 independent sequences, prompts U[128, 2048], capacity
                   6144, 512 greedy steps each: aggregate tokens/s.

Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "yue2-mlx_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

CONFIG = dict(hidden_size=3072, intermediate_size=8192, num_hidden_layers=28,
              num_attention_heads=24, num_key_value_heads=8, head_dim=128, vocab_size=83968,
              max_position_embeddings=24576, rms_norm_eps=1e-5, rope_theta=500000.0,
              qk_norm=True)
PEAK_HBM = 8.0e12  # MI355X HBM3E, bytes/s
PEAK_BF16 = 2.5e15  # MI355X dense bf16 MFMA, flop/s
KV_BYTES_PER_POS = 2 * 8 * 128 * 2 * 28  # K and V, Hkv * D * bf16 * layers


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def bytes_per_weight(bits):
    """HBM bytes per linear weight: bf16, or affine group-64 codes plus one
    bf16 scale and one bf16 bias per 64 weights."""
    return 2.0 if not bits else bits / 8 + 4 / 64


def precision_bits(args):
    return {"bf16": 0, "8bit": 8, "4bit": 4}[args.precision]


def weight_bytes(c, bits=0):
    H, F, V, L = c["hidden_size"], c["intermediate_size"], c["vocab_size"], c["num_hidden_layers"]
    qd, kd = c["num_attention_heads"] * 128, c["num_key_value_heads"] * 128
    per_layer = (qd + 2 * kd) * H + H * qd + 2 * F * H + H * F  # linear weights
    # + lm_head (the embedding row gather is 6 KiB)
    return int(bytes_per_weight(bits) * (L * per_layer + V * H))


def kernel_bytes(c, kernel, kv_len, bits=0):
    """Algorithmic HBM bytes of one launch (weights + activations + KV)."""
    H, F, V = c["hidden_size"], c["intermediate_size"], c["vocab_size"]
    qd, kd = c["num_attention_heads"] * 128, c["num_key_value_heads"] * 128
    w = bytes_per_weight(bits)
    return int({
        "qkv": w * (qd + 2 * kd) * H + 2 * (H + (qd + 2 * kd)),
        "attention": kv_len * 2 * kd * 2 + 2 * (qd + 2 * kd + qd) + 2 * 2 * kd,
        "o_proj": w * H * qd + 2 * (qd + 2 * H),
        "gate_up": w * 2 * F * H + 2 * (H + F),
        "down": w * H * F + 2 * (F + 2 * H),
        "lm_head": w * V * H + 2 * (H + V),
    }[kernel])


def gemv_shape(c, kernel):
    """(weight rows, K) of a decode projection."""
    H, F, V = c["hidden_size"], c["intermediate_size"], c["vocab_size"]
    qd, kd = c["num_attention_heads"] * 128, c["num_key_value_heads"] * 128
    return {"qkv": (qd + 2 * kd, H), "o_proj": (H, qd), "gate_up": (2 * F, H),
            "down": (H, F), "lm_head": (V, H)}[kernel]


def traffic_from_profiles(kernel):
    """Measured HBM bytes per launch, if a PMC summary has been committed."""
    name = f"gemv_{kernel}_3b_pmc.md"
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def host_cpu():
    """The CPU the baseline runs on: model name, logical CPUs of the host, and
    the threads used -- every CPU this process may run on, capped by the
    per-GPU CPU share the environment grants (OMP_NUM_THREADS)."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    share = int(os.environ.get("OMP_NUM_THREADS", usable))
    threads = max(1, min(usable, share))
    note = (f"all {threads} CPUs granted to this process" if threads == usable else
            f"{threads} threads: the CPU share per GPU (OMP_NUM_THREADS) of a host with "
            f"{usable} usable CPUs")
    return {"model": model, "nproc": nproc, "threads": threads, "note": note}


def lin_params(c):
    H, F = c["hidden_size"], c["intermediate_size"]
    qd, kd = c["num_attention_heads"] * 128, c["num_key_value_heads"] * 128
    return (qd + 2 * kd) * H + H * qd + 2 * F * H + H * F


def prefill_flops(c, T):
    """Linear layers for T tokens, lm_head for the last one, causal attention."""
    L, V, H = c["num_hidden_layers"], c["vocab_size"], c["hidden_size"]
    return (2 * T * L * lin_params(c) + 2 * V * H
            + L * 4 * c["num_attention_heads"] * 128 * T * (T + 1) // 2)


def run_cfg(args, engine, c):
    import numpy as np
    rng = np.random.default_rng(args.seed + 3)
    cond = rng.integers(0, c["vocab_size"], size=512).tolist()
    uncond = rng.integers(0, c["vocab_size"], size=512).tolist()
    sampling = dict(temperature=1.0, top_p=0.93, top_k=50, repetition_penalty=1.0,
                    penalty_window=50, min_tokens=0, max_tokens=1024)
    engine.generate_tokens(cond, dict(sampling, max_tokens=16), args.seed, negative=uncond,
                           cfg_scale=1.5)  # warm: graphs, code objects
    tokens, timing, _ = engine.generate_tokens(cond, sampling, args.seed, negative=uncond,
                                               cfg_scale=1.5)
    decode_s = timing["seconds"] - timing["prefill_seconds"]
    tps = (len(tokens) - 1) / decode_s
    L = 512 + len(tokens) / 2  # mean per-branch KV length
    step_bytes = weight_bytes(c, precision_bits(args)) + 2 * L * KV_BYTES_PER_POS
    log(f"[bench] cfg: {len(tokens)} tokens, prefill {timing['prefill_seconds']:.3f}s, "
        f"decode {tps:.1f} tok/s")
    return {"metric": "CFG decode tokens/sec (batch 2 cond+uncond, scale 1.5, top-k 50 / "
                      "top-p 0.93, T 1.0)",
            "value": round(tps, 2), "unit": "tokens/s", "n_gpus": 1,
            "higher_is_better": True, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "3B decoder, CFG pair, 512 + 512 prompt ids, 1024 tokens",
                       "driver": "yuear_generate_tokens (host loop, pipelined)"},
            "prefill_seconds": round(timing["prefill_seconds"], 4),
            "step_roofline": {"bytes_per_step": int(step_bytes),
                              "frac": round(step_bytes * tps / PEAK_HBM, 4)},
            "tokens": len(tokens)}


def run_long(args, engine, c):
    import numpy as np
    import torch
    T, end = 3000, 8192
    rng = np.random.default_rng(args.seed + 4)
    s = engine.session(1, end + 8)
    warm = engine.session(1, 2048 + 8)
    warm.prefill(0, rng.integers(0, c["vocab_size"], size=2048).tolist())  # code objects
    warm.close()
    torch.cuda.synchronize()
    t = time.perf_counter()
    s.prefill(0, rng.integers(0, c["vocab_size"], size=T).tolist())
    torch.cuda.synchronize()
    pre_s = time.perf_counter() - t
    flops = prefill_flops(c, T)
    log(f"[bench] long: prefill {T} tokens {pre_s * 1e3:.1f} ms, "
        f"{flops / pre_s / 1e12:.1f} TFLOP/s")
    greedy = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                  penalty_window=50, min_tokens=0, max_tokens=end)
    curve, reset = [], True
    while s.position(0) + 512 <= end:
        L0 = s.position(0)
        ms, _ = s.time_generate(greedy, args.seed, 512, reset=reset)
        reset = False
        curve.append({"kv_from": L0 + 1, "kv_to": L0 + 512, "ms_per_token": round(ms, 4),
                      "tokens_per_s": round(1e3 / ms, 1)})
        log(f"[bench] long: KV {L0 + 1}-{L0 + 512}: {ms:.4f} ms/token")
    return {"metric": "prefill TFLOP/s (3000 tokens) and decode ms/token vs KV length",
            "value": round(flops / pre_s / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
            "higher_is_better": True, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "3B decoder, 3000-token prefill then decode to KV 8192"},
            "prefill_ms": round(pre_s * 1e3, 2), "prefill_flops": flops,
            "mfma_frac": round(flops / pre_s / PEAK_BF16, 4), "decode_curve": curve}


def run_prefill(args, engine, c):
    """Profiling mode: `--prefills` prefills of `--prefill-tokens` (3000: the
    prefill half of the long-context workload) tokens on the 3B model, timed
    one by one."""
    import numpy as np
    import torch
    T = args.prefill_tokens
    rng = np.random.default_rng(args.seed + 4)
    times = []
    for i in range(args.prefills + 1):  # the first call loads code objects
        s = engine.session(1, T + 8)
        prompt = rng.integers(0, c["vocab_size"], size=T).tolist()
        torch.cuda.synchronize()
        t = time.perf_counter()
        s.prefill(0, prompt)
        torch.cuda.synchronize()
        if i:
            times.append(time.perf_counter() - t)
        s.close()
        log(f"[bench] prefill {i}: {(time.perf_counter() - t) * 1e3:.2f} ms")
    flops = prefill_flops(c, T)
    best = min(times)
    return {"metric": f"prefill TFLOP/s ({T} tokens)", "value": round(flops / best / 1e12, 2),
            "unit": "TFLOP/s", "n_gpus": 1, "higher_is_better": True, "dtype": "bf16",
            "data": "synthetic", "config": {"workload": f"3B decoder, {T}-token prefill"},
            "prefill_ms": [round(t * 1e3, 3) for t in times], "prefill_flops": flops,
            "mfma_frac": round(flops / best / PEAK_BF16, 4)}


def run_nar(args):
    """The acoustic-model attention (nar_attention.cpp:63-218) at the 3B head
    shape: a 512-frame chunk attending over 3000 conditioning keys plus its
    own (non-causal), and the causal form over 3000 tokens."""
    import torch
    import yuear
    Hq, Hkv, D = 24, 8, 128
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    out = {}
    for name, Lq, Lk, causal in (("chunk", 512, 3512, False), ("causal", 3000, 3000, True)):
        q = torch.randn(1, Hq, Lq, D, device="cuda", generator=g).to(torch.bfloat16)
        k = torch.randn(1, Hkv, Lk, D, device="cuda", generator=g).to(torch.bfloat16)
        v = torch.randn(1, Hkv, Lk, D, device="cuda", generator=g).to(torch.bfloat16)
        ws = torch.empty(yuear.lib.yuear_nar_attention_workspace_bytes(1, Hkv, Lk) // 2,
                         dtype=torch.bfloat16, device="cuda")
        stream = torch.cuda.current_stream()
        for _ in range(3):
            yuear.nar_attention(q, k, v, causal, workspace=ws, stream=stream.cuda_stream)
        reps = 20
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            yuear.nar_attention(q, k, v, causal, workspace=ws, stream=stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        pairs = Lq * (Lq + 1) // 2 if causal else Lq * Lk  # visible (query, key) pairs
        flops = 4 * pairs * D * Hq
        out[name] = {"q_len": Lq, "kv_len": Lk, "causal": causal, "ms": round(ms, 4),
                     "TFLOPs": round(flops / (ms / 1e3) / 1e12, 1),
                     "frac_bf16_peak": round(flops / (ms / 1e3) / PEAK_BF16, 4)}
        log(f"[bench] nar {name}: {Lq} x {Lk} causal={causal} {ms:.3f} ms "
            f"{flops / (ms / 1e3) / 1e12:.1f} TFLOP/s")
    return {"metric": "acoustic-model attention TFLOP/s (nar_attention, 3B heads 24/8)",
            "value": out["chunk"]["TFLOPs"], "unit": "TFLOP/s", "n_gpus": 1,
            "higher_is_better": True, "dtype": "bf16 (fp32 softmax and P.V)",
            "data": "synthetic N(0,1) q/k/v",
            "config": {"workload": "nar_attention: 512-query chunk over 3512 keys; causal 3000"},
            "roofline": {"bound": "mfma", "achieved": out["chunk"]["TFLOPs"],
                         "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                         "frac": out["chunk"]["frac_bf16_peak"], "traffic": None},
            "shapes": out}


def run_batch8(args, engine, c):
    import numpy as np
    import torch
    B, steps, cap = 8, 512, 6144
    rng = np.random.default_rng(args.seed + 5)
    lens = rng.integers(128, 2049, size=B)
    s = engine.session(B, cap)
    for b, n in enumerate(lens):
        s.prefill(b, rng.integers(0, c["vocab_size"], size=int(n)).tolist())
    greedy = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                  penalty_window=50, min_tokens=0, max_tokens=steps + 16)
    s.time_generate(greedy, args.seed, 8, reset=True)  # warm (captures the graph)
    torch.cuda.synchronize()
    t = time.perf_counter()
    dev_ms, _ = s.time_generate(greedy, args.seed, steps, reset=False)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t
    agg = B * steps / wall
    mean_kv = float(np.mean(lens)) + 8 + steps / 2
    step_bytes = weight_bytes(c, precision_bits(args)) + B * mean_kv * KV_BYTES_PER_POS
    # per-kernel device time at batch 8; the projections run on MFMA
    # (v_mfma_f32_16x16x32_bf16, 8 of 16 columns live), so their MFMA
    # utilisation is the useful flops over the dense bf16 peak
    kernels = {}
    pos = [s.position(b) for b in range(B)]
    for name in ("qkv", "attention", "o_proj", "gate_up", "down", "lm_head"):
        ms = s.time_kernel(name, 56 if name != "lm_head" else 8)
        if name == "attention":
            nbytes = sum(kernel_bytes(c, name, p + 1) for p in pos)
            flops = None
        else:
            n, k = gemv_shape(c, name)
            nbytes = kernel_bytes(c, name, 0) + (B - 1) * (kernel_bytes(c, name, 0) - 2 * n * k)
            flops = 2 * B * n * k
        kernels[name] = {"us": round(ms * 1e3, 2), "bytes": int(nbytes),
                         "GBps": round(nbytes / (ms / 1e3) / 1e9, 1)}
        if flops:
            kernels[name]["mfma_util"] = round(flops / (ms / 1e3) / PEAK_BF16, 5)
        log(f"[bench] batch8 {name:9s} {ms * 1e3:8.2f} us  {nbytes / 1e6:8.2f} MB  "
            f"{nbytes / (ms / 1e3) / 1e9:7.1f} GB/s")
    log(f"[bench] batch8: {agg:.1f} tok/s aggregate ({wall / steps * 1e3:.3f} ms/step)")
    return {"metric": "aggregate decode tokens/sec, 8 independent sequences",
            "value": round(agg, 2), "unit": "tokens/s", "n_gpus": 1,
            "higher_is_better": True, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "3B decoder, batch 8, prompts U[128,2048], capacity 6144, "
                                   "512 greedy steps", "prompt_lengths": [int(x) for x in lens]},
            "ms_per_step": round(wall / steps * 1e3, 4),
            "step_roofline": {"bytes_per_step": int(step_bytes),
                              "frac": round(step_bytes / (wall / steps) / PEAK_HBM, 4)},
            "kernels": kernels}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--kv", type=int, default=4096)
    ap.add_argument("--precision", choices=("bf16", "8bit", "4bit"), default="bf16",
                    help="linear weights: bf16 (the headline metric) or affine group-64 "
                         "quantized (the reference's 8bit / 4bit checkpoints)")
    ap.add_argument("--seed", type=int, default=20251201)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-launches", type=int, default=112)
    ap.add_argument("--prefills", type=int, default=3,
                    help="--config prefill: number of timed prefills")
    ap.add_argument("--prefill-tokens", type=int, default=3000,
                    help="--config prefill: prompt length of each prefill")
    ap.add_argument("--config", choices=("decode", "cfg", "long", "batch8", "nar", "prefill"),
                    default="decode",
                    help="workload (decode: the headline batch-1 KV-4096 line)")
    ap.add_argument("--kernel-only", default=None,
                    help="profiling mode: only time these decode kernels, comma-separated "
                         "(qkv, attention, o_proj, gate_up, down, lm_head), in that order")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="profiling mode: one device-to-device copy of MIB MiB (counter scale)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path; the decode "
              "step of one sequence runs on a single GPU", file=sys.stderr)
        sys.exit(2)
    if not 1 <= args.prefill_tokens <= 24576 - 8:
        ap.error("--prefill-tokens must lie in [1, 24568] (the 3B context is 24576)")

    import numpy as np
    import torch
    import yuear

    if args.copy_calibration:
        # HBM counter calibration: a plain copy of known size (read N, write N)
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n}), flush=True)
        return

    t_start = time.perf_counter()
    if args.config == "nar":
        print(json.dumps(run_nar(args)), flush=True)
        return
    c = CONFIG
    bits = precision_bits(args)
    log(f"[bench] generating 3B weights on host ({weight_bytes(c) / 1e9:.2f} GB) ...")
    weights = yuear.random_weights(c, args.seed)
    if bits:
        weights = yuear.quantized_weights(weights, bits)
    log(f"[bench] weights ready {time.perf_counter() - t_start:.1f}s; uploading")
    engine = yuear.Engine(c, weights, bits=bits)
    if args.config != "decode":
        line = {"cfg": run_cfg, "long": run_long, "batch8": run_batch8,
                "prefill": run_prefill}[args.config](
            args, engine, c)
        print(json.dumps(line), flush=True)
        log(f"[bench] total {time.perf_counter() - t_start:.1f}s")
        return
    W, K = args.warmup, args.steps
    prefill = args.kv - 1 - W - (K - 1) // 2  # timed steps centred on KV length kv
    step_launches = 16
    capacity = prefill + W + K + step_launches + 8
    session = engine.session(1, capacity)
    rng = np.random.default_rng(args.seed)
    if args.kernel_only:
        # the decode line's prompt length, so the attention reads its KV length
        session.prefill(0, rng.integers(0, c["vocab_size"], size=prefill).tolist())
        for name in args.kernel_only.split(","):
            ms = session.time_kernel(name, args.kernel_launches)
            print(json.dumps({"kernel": name, "launches": args.kernel_launches,
                              "us": ms * 1e3}), flush=True)
        return
    prompt = rng.integers(0, c["vocab_size"], size=prefill).tolist()
    t = time.perf_counter()
    session.prefill(0, prompt)
    torch.cuda.synchronize()
    log(f"[bench] prefill {prefill} tokens {time.perf_counter() - t:.2f}s")

    greedy = dict(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.0,
                  penalty_window=50, min_tokens=0, max_tokens=K + W + 8)
    session.time_generate(greedy, args.seed, W, reset=True)  # warmup (captures the graph)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dev_ms, tokens = session.time_generate(greedy, args.seed, K, reset=False)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / K
    value = K / wall
    mean_kv = prefill + W + (K - 1) / 2 + 1
    step_bytes = weight_bytes(c, bits) + mean_kv * KV_BYTES_PER_POS
    log(f"[bench] decode {K} steps: {ms_per_step:.4f} ms/token wall, {dev_ms:.4f} ms device, "
        f"{value:.1f} tok/s, step roofline {step_bytes / (ms_per_step / 1e3) / PEAK_HBM:.3f}")

    # per-kernel device time (HIP events on the session stream)
    kernels = {}
    for name in ("qkv", "attention", "o_proj", "gate_up", "down", "lm_head"):
        launches = args.kernel_launches if name != "lm_head" else max(8, args.kernel_launches // 8)
        ms = session.time_kernel(name, launches)
        nbytes = kernel_bytes(c, name, session.position(0) + 1, bits)
        kernels[name] = {"us": round(ms * 1e3, 3), "bytes": nbytes,
                         "GBps": round(nbytes / (ms / 1e3) / 1e9, 1)}
        log(f"[bench] {name:9s} {ms * 1e3:8.2f} us  {nbytes / 1e6:8.2f} MB  "
            f"{nbytes / (ms / 1e3) / 1e9:7.1f} GB/s")
    dom = kernels["gate_up"]
    achieved = dom["bytes"] / (dom["us"] / 1e6) / 1e9
    name = ("gemv_kernel<1,6,2,SwiGLU> (gate/up 16384x3072" if not bits else
            f"qgemv_kernel<1,{bits},{64 if bits == 8 else 32},3,2> (gate/up 16384x3072, "
            f"{bits}-bit codes")
    roofline = {"kernel": f"{name} + RMSNorm + SwiGLU)",
                "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM / 1e9,
                "unit": "GB/s", "frac": round(achieved / (PEAK_HBM / 1e9), 4),
                "traffic": traffic_from_profiles("gate_up")}

    cpu = None
    if not args.no_cpu:
        import cpu_ref
        host = host_cpu()
        threads = host["threads"]
        cpu_ref.lib().oracle_set_threads(threads)
        model = cpu_ref.Model(c, weights, bits=bits)
        L0 = args.kv - 1
        cap = 256  # steps at most; --cpu-seconds ends the sample first on a 16-thread host
        cache = model.cache(L0 + cap + 1)
        for layer in range(c["num_hidden_layers"]):
            k, v = session.read_kv(layer, 0, L0)
            cache.keys(layer)[:, :L0] = k
            cache.values(layer)[:, :L0] = v
        cache.offset = L0
        token, n = int(tokens[-1]), 0
        t = time.perf_counter()
        while n < cap and (n < 2 or time.perf_counter() - t < args.cpu_seconds):
            logits = model.step(token, cache)
            token = int(cpu_ref.bf16_to_f32(logits).argmax())
            n += 1
        elapsed = time.perf_counter() - t
        cpu = {"value": round(n / elapsed, 4), "unit": "tokens/s", "cores": threads,
               "kind": "port", "host_cpus": host["nproc"], "cpu_model": host["model"],
               "threads_note": host["note"],
               "sample": f"{n} greedy decode steps of the same 3B model on the same weights, "
                         f"KV {L0 + 1}..{L0 + n} copied from the GPU run "
                         f"(CPU restatement of the reference graph, {elapsed:.1f} s)"}
        log(f"[bench] cpu oracle {n} steps {elapsed:.1f}s -> {n / elapsed:.3f} tok/s "
            f"({threads} threads)")

    line = {
        "metric": ("decode tokens/sec @ batch 1, 3B bf16, KV 4096; % of HBM roofline" if not bits
                   else f"decode tokens/sec @ batch 1, 3B {args.precision} (affine group 64), "
                        f"KV 4096; % of HBM roofline"),
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if not bits else f"u{bits} codes x bf16 (fp32 accumulate)",
        "data": "synthetic: random-init N(0,0.02) bf16 weights, unit norm gains, random prompt ids"
                + ("" if not bits else f"; linears quantized to {bits} bits (affine, group 64)"),
        "config": {"workload": "3B bf16 AR decoder (H3072/F8192/28L/24:8 heads/V83968), "
                               "greedy decode at batch 1 centred on KV length 4096",
                   "batch": 1, "kv_len": args.kv, "prefill_tokens": prefill,
                   "mean_kv_len": mean_kv, "decode": "kernels",
                   "parallelism": "single-gpu"},
        "step_roofline": {"bytes_per_step": int(step_bytes),
                          "achieved_GBps": round(step_bytes / (ms_per_step / 1e3) / 1e9, 1),
                          "frac": round(step_bytes / (ms_per_step / 1e3) / PEAK_HBM, 4),
                          "device_ms_per_step": round(dev_ms, 5)},
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    log(f"[bench] total {time.perf_counter() - t_start:.1f}s")


if __name__ == "__main__":
    main()
