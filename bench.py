#!/usr/bin/env python3
"""Decode throughput of the 3B-class YuE2-style AR decoder on one MI355X.

Workload (the reference's token loop, sampling::generate src/sampling.rs:222-294):
  28 layers, hidden 3072, 24 q heads / 8 KV heads, head_dim 128, SwiGLU 8192,
  vocab 84000; random-init BF16 weights ~N(0, 0.02) (synthetic: the real
  checkpoint is not available offline); seed-0 2048-token prompt (the
  unconditional row: seed-1 prompt); sampling T 0.9, top-k 50, top-p 0.93,
  repetition penalty 1.2 over 50 tokens; CFG batch 2 with guidance 1.5.
A step is one loop iteration: CFG mix + choose() + one token through all 28
layers for both rows + LM head, all on the device as one hipGraph launch;
only the token id comes back.  Weights, KV caches and prompts are resident in
HBM before the timed region.  The batch-1 line (no CFG) is measured the same
way on its own cache.

The prompts are prefilled on the matrix cores (yue2_hip_prefill_mfma:
BF16 MFMA GEMMs + causal flash attention; --prefill exact uses the
bit-exact decode-order kernels instead); the prefill's own rate is reported
beside the decode line.

--workload long: the long-context run on the same model -- 24000-token
prompts for both CFG rows, then CFG batch-2 decode to the full 24576-token
context, reporting ms/token as the context grows and the step kernel's
roofline at the last position (24576 attended keys).

--workload yue2: the same loop on the YuE2 shape (the reference's Config
defaults, src/model.rs:35-44: hidden 2048, 28 layers, 16 q / 8 KV heads,
head_dim 128, SwiGLU 6144, vocab 184704, RoPE theta 1e6) in the semantic
phase of Pipeline::generate_semantic: the LM head reads the 32768 codec rows
and MUSIC_END (project_phase, src/model.rs:478-507); min_tokens keeps the
end token out until the timed steps are done.

--workload any: the same loop on a shape with no step kernel of its own
(--shape 1b: hidden 2048, 16 layers, 32 q / 8 KV heads, head_dim 64, SwiGLU
8192; --shape 8b: hidden 4096, 32 layers, 32 q / 8 KV heads, head_dim 128,
SwiGLU 14336; vocab 128256): the generic step kernel of its head_dim
(--step-kernel 0: the per-phase kernels).

Prints one JSON line.  Progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

METRIC = "AR decode tokens/s @1 GPU (bs1 & CFG bs2) + % of HBM roofline; p50 ms/token"
HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def weight_bytes(c, head_rows=None) -> int:
    """Every layer's weights and norms, the final norm and the LM head rows
    one step reads (all of them, or a phase's rows and its stop row)."""
    H, D, I, V = c.hidden_size, c.head_dim, c.intermediate_size, c.vocab_size
    q, kv = c.num_attention_heads * D, c.num_key_value_heads * D
    per_layer = 2 * (H * (q + 2 * kv) + q * H + 3 * H * I) + 4 * (2 * H + 2 * D)
    return c.num_hidden_layers * per_layer + 2 * (V if head_rows is None else head_rows) * H + 4 * H


def kv_bytes_per_position(c) -> int:
    return c.num_hidden_layers * 2 * c.num_key_value_heads * c.head_dim * 2


def step_bytes(c, rows: int, context: float, head_rows=None) -> float:
    """Algorithmic HBM bytes of one step: every weight once, each row's KV for
    `context` attended positions plus the new token's K/V, its embedding row."""
    return weight_bytes(c, head_rows) + rows * (kv_bytes_per_position(c) * (context + 1) + 2 * c.hidden_size)


def measure(y2, model, caches, first, sampling, scale, warmup, steps, c, phase=0, head_rows=None):
    dec = y2.Decoder(model, caches[0], caches[1] if len(caches) > 1 else None, sampling=sampling, seed=0,
                     scale=scale, phase=phase)
    dec.run(warmup, first_logits=first)
    ctx0 = caches[0].length
    y2.synchronize()
    t0 = time.perf_counter()
    tokens, ms = dec.run(steps, timing=True)
    y2.synchronize()
    wall = time.perf_counter() - t0
    assert len(tokens) == steps
    rows = len(caches)
    ctx = [ch.length for ch in caches]
    mean_ctx = np.mean([(ctx0 + steps / 2.0) for _ in caches])
    return dec, {
        "wall_s": wall,
        "ms_per_step": 1000.0 * wall / steps,
        "tokens_per_s": steps / wall,
        "p50_ms": float(np.percentile(ms, 50)),
        "p90_ms": float(np.percentile(ms, 90)),
        "mean_event_ms": float(np.mean(ms)),
        "context_start": int(ctx0),
        "context_end": [int(x) for x in ctx],
        "hbm_roofline_frac": step_bytes(c, rows, mean_ctx, head_rows) / (wall / steps) / HBM_PEAK,
        "bytes_per_step": step_bytes(c, rows, mean_ctx, head_rows),
    }


MFMA_BF16_PEAK = 2.5e15  # MI355X dense BF16 matrix FLOP/s


def prefill_flops(c, n: int) -> float:
    """Algorithmic FLOPs of prefilling n tokens: every layer linear once per
    token, the causal attention (QK^T and PV over 1..n keys per query head),
    the LM head of the last row."""
    H, D, I, V = c.hidden_size, c.head_dim, c.intermediate_size, c.vocab_size
    q, kv = c.num_attention_heads * D, c.num_key_value_heads * D
    linear = 2.0 * n * c.num_hidden_layers * (H * (q + 2 * kv) + q * H + 3 * H * I)
    attention = c.num_hidden_layers * c.num_attention_heads * 4.0 * D * n * (n + 1) / 2.0
    return linear + attention + 2.0 * V * H


def prefill(y2, model, c, ids, cap, mode):
    """(cache, last-row logits, seconds) of one prompt."""
    y2.synchronize()
    t = time.perf_counter()
    if mode == "mfma":
        cache, logits = model.prefill_mfma(ids, cap)
    else:
        cache, logits = model.prefill_phase(ids, cap)
    y2.synchronize()
    return cache, logits, time.perf_counter() - t


def prefill_report(c, n, seconds, mode):
    fl = prefill_flops(c, n)
    return {"mode": mode, "tokens": n, "s": round(seconds, 4), "tokens_per_s": round(n / seconds, 1),
            "TFLOP_s": round(fl / seconds / 1e12, 2), "mfma_frac": round(fl / seconds / MFMA_BF16_PEAK, 4),
            "flops": fl}


def measured_traffic(context, profile="step_kernel_3b_cfg_traffic.md"):
    """HBM bytes per launch of the CFG step kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (calibrated against a plain copy)
    of the bench's own timing loop, when they were measured at this context;
    otherwise None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", profile)
    try:
        text = open(path).read()
    except OSError:
        return None
    vals = dict(re.findall(r"^(traffic_bytes_per_launch|context): (\d+)$", text, re.M))
    if int(vals.get("context", -1)) != context:
        return None
    return int(vals["traffic_bytes_per_launch"])


def host_cpu():
    """(model name, logical CPUs) of this host."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count() or 1


def native_oracle():
    """Build the oracle for this host's CPU (-O3 -march=native) into a
    temporary directory and point the oracle binding at it; the prebuilt
    portable library (-O2 x86-64-v3) stays in use if that fails."""
    import subprocess
    import tempfile
    from oracle import oracle as O
    src = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle", "oracle.c")
    out = os.path.join(tempfile.mkdtemp(prefix="y2o_"), "liboracle_native.so")
    cmd = ["gcc", "-O3", "-march=native", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-fopenmp", "-shared",
           src, "-o", out, "-lm"]
    try:
        subprocess.run(cmd, check=True, capture_output=True, timeout=120)
    except (OSError, subprocess.SubprocessError):
        return "-O2 -march=x86-64-v3 (prebuilt)"
    O._lib = None
    O.LIB = __import__("pathlib").Path(out)
    return "-O3 -march=native"


def cpu_baseline(ckpt, c, prompt_len, scale, sampling, threads, budget_s, max_steps):
    """The oracle's CFG step on the host cores: both rows' forward over a
    synthetic BF16 KV cache of prompt_len positions, CFG mix and choose()."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    flags = native_oracle()
    from oracle import oracle as O

    O.set_threads(threads)
    om = O.Model(ckpt)
    caches = [O.Cache(om, prompt_len + max_steps + 1) for _ in range(2)]
    for i, ch in enumerate(caches):
        ch.fill_random(prompt_len, seed=100 + i)
    rng = O.Generator(0)
    ids = [1, 2]
    logits = [om.forward([ids[i]], caches[i]) for i in range(2)]
    history = []
    t0 = time.perf_counter()
    steps = 0
    while steps < max_steps and (steps == 0 or time.perf_counter() - t0 < budget_s):
        mixed = O.cfg_mix(logits[0], logits[1], scale)
        tok = O.choose(mixed, sampling, history, steps, O.PHASE_NONE, False, rng)
        history.append(tok)
        logits = [om.forward([tok], caches[i]) for i in range(2)]
        steps += 1
    wall = time.perf_counter() - t0
    model, nproc = host_cpu()
    return {"value": steps / wall, "unit": "tokens/s", "cores": threads, "kind": "port",
            "ms_per_step": 1000.0 * wall / steps, "cpu_model": model, "nproc": nproc, "build": flags,
            "sample": f"{steps} CFG batch-2 steps of the C oracle (restated reference CPU token step, "
                      f"portable DOT order in place of Accelerate; gcc {flags}) at context {prompt_len}, "
                      f"synthetic BF16 KV, {threads} threads (one GPU's share of the host's CPUs) of {nproc} "
                      f"logical CPUs ({model})"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--scale", type=float, default=1.5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--kernel-iters", type=int, default=112)
    ap.add_argument("--step-kernel", type=int, default=1, choices=[0, 1],
                    help="1 (default): one persistent kernel per token; 0: one kernel per phase")
    ap.add_argument("--prefill", default="mfma", choices=["mfma", "exact"],
                    help="mfma (default): matrix-core prefill; exact: decode-order (bit-exact) prefill")
    ap.add_argument("--workload", default="decode", choices=["decode", "long", "yue2", "any"],
                    help="decode (default): 2048-token prompts; long: 24000-token prompts decoded to 24576; "
                         "yue2: the YuE2 shape in the semantic phase; any: a 1B-class shape on the generic "
                         "step kernel")
    ap.add_argument("--shape", default="1b", choices=["1b", "8b"], help="--workload any: the shape")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (--gpus must be 1)",
              file=sys.stderr)
        return 2

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import yue2_rs_amd as y2
    from yue2_rs_amd import synthetic

    if not y2.available():
        print("no gfx950 device available", file=sys.stderr)
        return 1
    if args.workload == "yue2":
        return shape_workload(args, y2, synthetic, synthetic.YUE2, y2.PHASE_SEMANTIC, 32768 + 1,
                              "YuE2-shape AR decode loop, semantic phase",
                              "YuE2 shape: 28 layers + semantic-phase LM head + sampler")
    if args.workload == "any" and args.shape == "1b":
        return shape_workload(args, y2, synthetic, synthetic.CLASS_1B_ANY, y2.PHASE_NONE, None,
                              "1B-class AR decode loop (no shape-specific step kernel)",
                              "1B-class shape: 16 layers + LM head + sampler, the generic head_dim-64 kernel")
    if args.workload == "any":
        return shape_workload(args, y2, synthetic, synthetic.CLASS_8B_ANY, y2.PHASE_NONE, None,
                              "8B-class AR decode loop (no shape-specific step kernel)",
                              "8B-class shape: 32 layers + LM head + sampler, the generic head_dim-128 kernel")
    c = synthetic.CLASS_3B
    log("generating synthetic 3B-class weights")
    t = time.perf_counter()
    ckpt = synthetic.checkpoint(c, seed=0, threads=16)
    log(f"weights ready in {time.perf_counter() - t:.1f}s; uploading")
    model = y2.Model.open(ckpt)
    step_kernel = model.set_step_kernel(bool(args.step_kernel))
    if args.workload == "long":
        return long_context(args, y2, synthetic, c, ckpt, model, step_kernel)
    W, K, P = args.warmup, args.steps, args.prompt
    cond_ids = synthetic.prompt(P, c.vocab_size, seed=0)
    neg_ids = synthetic.prompt(P, c.vocab_size, seed=1)
    cap = P + W + K + 1
    sampling = y2.Sampling(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                           min_tokens=0, max_tokens=W + K + 1)
    log(f"prefilling 3 x {P} tokens ({args.prefill})")
    c_bs1, l_bs1, _ = prefill(y2, model, c, cond_ids, cap, args.prefill)
    c_pos, l_pos, t_pos = prefill(y2, model, c, cond_ids, cap, args.prefill)
    c_neg, l_neg, t_neg = prefill(y2, model, c, neg_ids, cap, args.prefill)
    pre = prefill_report(c, P, min(t_pos, t_neg), args.prefill)
    log(f"prefill: {pre['tokens_per_s']:.0f} tokens/s, {pre['TFLOP_s']:.1f} TFLOP/s")

    # Dominant kernel at a context that does not depend on --steps/--warmup:
    # the CFG decoder takes one step (both caches reach P + 1 positions) and
    # its step kernel is launched again at that position, timed with HIP
    # events on the decoder's stream (or, on the per-phase path, its gate/up
    # + SwiGLU GEMV, the largest weight read of a layer).
    d0 = y2.Decoder(model, c_pos, c_neg, sampling=sampling, seed=0, scale=args.scale)
    d0.run(1, first_logits=np.concatenate([l_pos, l_neg]))
    context = c_pos.length
    if step_kernel:
        dom_ms, dom_b = d0.time_kernel("step", args.kernel_iters)
        dom_name = "step_kernel<2, 128, 3, 6, 6, 16> (whole CFG batch-2 token: 28 layers + LM head + sampler)"
        traffic = measured_traffic(context)
    else:
        dom_ms, dom_b = d0.time_kernel("gate_up", args.kernel_iters)
        dom_name = "gemv_kernel<2, EPI_SWIGLU, 6, true> (RMSNorm + gate/up + SwiGLU of one layer)"
        traffic = None
    l_pos, l_neg = [row.copy() for row in d0.logits()]
    d0.close()

    log(f"batch 1: {W} warmup + {K} timed steps")
    d1, bs1 = measure(y2, model, [c_bs1], l_bs1, sampling, 1.0, W, K, c)
    d1.close()
    log(f"batch 1: {bs1['tokens_per_s']:.1f} tokens/s, p50 {bs1['p50_ms']:.3f} ms")
    log(f"CFG batch 2: {W} warmup + {K} timed steps")
    d2, cfg = measure(y2, model, [c_pos, c_neg], np.concatenate([l_pos, l_neg]), sampling, args.scale, W, K, c)
    log(f"CFG batch 2: {cfg['tokens_per_s']:.1f} steps/s, p50 {cfg['p50_ms']:.3f} ms")

    # the per-phase GEMV kernels of the phase-kernel path, for reference
    others = {}
    for name in ("gate_up", "down", "qkv", "o", "lm_head"):
        ms, by = d2.time_kernel(name, args.kernel_iters if name != "lm_head" else 16)
        others[name] = {"launch_ms": round(ms, 5), "GB_s": round(by / (ms * 1e-3) / 1e9, 1)}
    d2.close()
    achieved = dom_b / (dom_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                "frac": round(achieved / 8000.0, 4), "traffic": traffic, "kernel": dom_name,
                "launch_ms": round(dom_ms, 5), "bytes_per_launch": int(dom_b), "context": context}

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (oracle on host cores)")
        threads = min(16, os.cpu_count() or 1)  # one GPU's share of the host's CPUs
        cpu = cpu_baseline(ckpt, c, P, args.scale, sampling, threads, args.cpu_budget, 512)
        log(f"CPU baseline: {cpu['value']:.3f} steps/s with {threads} threads")

    out = {
        "metric": METRIC,
        "value": round(cfg["tokens_per_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(cfg["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "3B-class AR decode loop, CFG batch 2 (guidance 1.5), T 0.9 / top-k 50 / "
                               f"top-p 0.93 / penalty 1.2, {P}-token prompts, {K} steps",
                   "layers": c.num_hidden_layers, "hidden": c.hidden_size, "heads": c.num_attention_heads,
                   "kv_heads": c.num_key_value_heads, "head_dim": c.head_dim,
                   "intermediate": c.intermediate_size, "vocab": c.vocab_size, "prompt": P,
                   "global_batch": 2, "parallelism": "none (1 GPU)",
                   "execution": "persistent step kernel" if step_kernel else "one kernel per phase"},
        "p50_ms": round(cfg["p50_ms"], 4),
        "p90_ms": round(cfg["p90_ms"], 4),
        "hbm_roofline_frac": round(cfg["hbm_roofline_frac"], 4),
        "bytes_per_step": int(cfg["bytes_per_step"]),
        "row_tokens_per_s": round(2 * cfg["tokens_per_s"], 2),
        "bs1": {"tokens_per_s": round(bs1["tokens_per_s"], 2), "ms_per_step": round(bs1["ms_per_step"], 4),
                "p50_ms": round(bs1["p50_ms"], 4), "p90_ms": round(bs1["p90_ms"], 4),
                "hbm_roofline_frac": round(bs1["hbm_roofline_frac"], 4),
                "bytes_per_step": int(bs1["bytes_per_step"])},
        "roofline": roofline,
        "prefill": pre,
        "phase_kernels": others,
        "cpu_baseline": cpu,
        "norm_fallbacks": model.norm_fallbacks(),
    }
    print(json.dumps(out), flush=True)
    return 0


def shape_workload(args, y2, synthetic, c, phase, head_rows, name, kernel_desc):
    """The decode loop on another shape (c) in a phase of the LM head
    (head_rows: the rows that phase reads, None for all): CFG batch 2 and
    batch 1 after 2048-token prompts (matrix-core prefill), the step kernel
    timed alone one position past the prompts."""
    log(f"generating synthetic weights: {name}")
    ckpt = synthetic.checkpoint(c, seed=0, threads=16)
    model = y2.Model.open(ckpt)
    step_kernel = model.set_step_kernel(bool(args.step_kernel))
    W, K, P = args.warmup, args.steps, args.prompt
    cond_ids = synthetic.prompt(P, c.vocab_size, seed=0)
    neg_ids = synthetic.prompt(P, c.vocab_size, seed=1)
    cap = P + W + K + 1
    sampling = y2.Sampling(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                           min_tokens=W + K + 2, max_tokens=W + K + 2)
    log(f"prefilling 3 x {P} tokens ({args.prefill})")
    def pre(ids):
        y2.synchronize()
        t = time.perf_counter()
        if args.prefill == "mfma":
            cache, logits = model.prefill_mfma(ids, cap, phase)
        else:
            cache, logits = model.prefill_phase(ids, cap, phase)
        y2.synchronize()
        return cache, logits, time.perf_counter() - t
    c_bs1, l_bs1, _ = pre(cond_ids)
    c_pos, l_pos, t_pos = pre(cond_ids)
    c_neg, l_neg, t_neg = pre(neg_ids)
    prep = prefill_report(c, P, min(t_pos, t_neg), args.prefill)
    d0 = y2.Decoder(model, c_pos, c_neg, sampling=sampling, seed=0, scale=args.scale, phase=phase)
    d0.run(1, first_logits=np.concatenate([l_pos, l_neg]))
    context = c_pos.length
    dom_ms, dom_b = d0.time_kernel("step", args.kernel_iters) if step_kernel else (None, None)
    l_pos, l_neg = [row.copy() for row in d0.logits()]
    d0.close()
    log(f"batch 1: {W} warmup + {K} timed steps")
    d1, bs1 = measure(y2, model, [c_bs1], l_bs1, sampling, 1.0, W, K, c, phase, head_rows)
    d1.close()
    log(f"CFG batch 2: {W} warmup + {K} timed steps")
    d2, cfg = measure(y2, model, [c_pos, c_neg], np.concatenate([l_pos, l_neg]), sampling, args.scale, W, K, c,
                      phase, head_rows)
    d2.close()
    log(f"CFG batch 2: {cfg['tokens_per_s']:.1f} steps/s, p50 {cfg['p50_ms']:.3f} ms")
    roofline = None
    if step_kernel:
        achieved = dom_b / (dom_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                    "frac": round(achieved / 8000.0, 4), "traffic": None,
                    "kernel": f"step_kernel (whole CFG batch-2 token of the {kernel_desc})",
                    "launch_ms": round(dom_ms, 5), "bytes_per_launch": int(dom_b), "context": context}
    out = {
        "metric": METRIC,
        "value": round(cfg["tokens_per_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(cfg["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{name}, CFG batch 2 (guidance 1.5), T 0.9 / "
                               f"top-k 50 / top-p 0.93 / penalty 1.2, {P}-token prompts, {K} steps",
                   "layers": c.num_hidden_layers, "hidden": c.hidden_size, "heads": c.num_attention_heads,
                   "kv_heads": c.num_key_value_heads, "head_dim": c.head_dim,
                   "intermediate": c.intermediate_size, "vocab": c.vocab_size, "head_rows": head_rows,
                   "prompt": P, "global_batch": 2, "parallelism": "none (1 GPU)",
                   "execution": "persistent step kernel" if step_kernel else "per-phase kernels"},
        "p50_ms": round(cfg["p50_ms"], 4),
        "p90_ms": round(cfg["p90_ms"], 4),
        "hbm_roofline_frac": round(cfg["hbm_roofline_frac"], 4),
        "bytes_per_step": int(cfg["bytes_per_step"]),
        "bs1": {"tokens_per_s": round(bs1["tokens_per_s"], 2), "ms_per_step": round(bs1["ms_per_step"], 4),
                "p50_ms": round(bs1["p50_ms"], 4), "hbm_roofline_frac": round(bs1["hbm_roofline_frac"], 4),
                "bytes_per_step": int(bs1["bytes_per_step"])},
        "roofline": roofline,
        "prefill": prep,
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)
    return 0


def long_context(args, y2, synthetic, c, ckpt, model, step_kernel):
    """24000-token prompts for both CFG rows (matrix-core prefill), then CFG
    batch-2 decode to the full 24576-token context in segments of 64 steps,
    each segment's per-step HIP-event times giving ms/token at its context.
    The step kernel is timed alone at the last free position (24575: 24576
    attended keys) before the final step fills it."""
    P, full = 24000, c.max_position_embeddings
    steps = full - P
    cond_ids = synthetic.prompt(P, c.vocab_size, seed=0)
    neg_ids = synthetic.prompt(P, c.vocab_size, seed=1)
    sampling = y2.Sampling(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                           min_tokens=0, max_tokens=steps + 1)
    log(f"prefilling 2 x {P} tokens ({args.prefill})")
    c_pos, l_pos, t_pos = prefill(y2, model, c, cond_ids, full, args.prefill)
    log(f"conditional row prefilled in {t_pos:.2f}s")
    c_neg, l_neg, t_neg = prefill(y2, model, c, neg_ids, full, args.prefill)
    pre = prefill_report(c, P, min(t_pos, t_neg), args.prefill)
    log(f"prefill: {pre['tokens_per_s']:.0f} tokens/s, {pre['TFLOP_s']:.1f} TFLOP/s")
    dec = y2.Decoder(model, c_pos, c_neg, sampling=sampling, seed=0, scale=args.scale)
    curve, times = [], []
    first = np.concatenate([l_pos, l_neg])
    y2.synchronize()
    t0 = time.perf_counter()
    done = 0
    while done < steps - 1:
        n = min(64, steps - 1 - done)
        ctx = c_pos.length
        toks, ms = dec.run(n, first_logits=first if done == 0 else None, timing=True)
        assert len(toks) == n, "decode stopped early"
        times.extend(ms)
        curve.append({"context": int(ctx), "steps": n, "p50_ms": round(float(np.percentile(ms, 50)), 4),
                      "mean_ms": round(float(np.mean(ms)), 4)})
        log(f"context {ctx}..{ctx + n}: p50 {curve[-1]['p50_ms']:.3f} ms/token")
        done += n
    y2.synchronize()
    wall = time.perf_counter() - t0
    context = c_pos.length
    if step_kernel:
        dom_ms, dom_b = dec.time_kernel("step", 32)
        dom_name = "step_kernel<2, 128, 3, 6, 6, 16> (whole CFG batch-2 token: 28 layers + LM head + sampler)"
    else:
        dom_ms, dom_b = dec.time_kernel("gate_up", args.kernel_iters)
        dom_name = "gemv_kernel<2, EPI_SWIGLU, 6, true> (RMSNorm + gate/up + SwiGLU of one layer)"
    toks, ms = dec.run(1, timing=True)
    times.extend(ms)
    assert c_pos.length == full and c_neg.length == full
    dec.close()
    achieved = dom_b / (dom_ms * 1e-3) / 1e9
    traffic = measured_traffic(context, "step_kernel_3b_cfg_context24575_traffic.md") if step_kernel else None
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                "frac": round(achieved / 8000.0, 4), "traffic": traffic, "kernel": dom_name,
                "launch_ms": round(dom_ms, 5), "bytes_per_launch": int(dom_b), "context": context}
    cpu = None
    if not args.no_cpu:
        log("CPU baseline (oracle on host cores)")
        threads = min(16, os.cpu_count() or 1)
        cpu = cpu_baseline(ckpt, c, P, args.scale, sampling, threads, args.cpu_budget, 64)
        log(f"CPU baseline: {cpu['value']:.3f} steps/s with {threads} threads")
    timed = steps - 1
    out = {
        "metric": METRIC,
        "value": round(timed / wall, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": timed,
        "warmup": 0,
        "ms_per_step": round(1000.0 * wall / timed, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"3B-class long-context CFG batch-2 decode, {P}-token prompts decoded to "
                               f"{full} positions, T 0.9 / top-k 50 / top-p 0.93 / penalty 1.2",
                   "prompt": P, "context_end": full, "global_batch": 2, "parallelism": "none (1 GPU)",
                   "execution": "persistent step kernel" if step_kernel else "one kernel per phase"},
        "p50_ms": round(float(np.percentile(times, 50)), 4),
        "ms_per_token_vs_context": curve,
        "roofline": roofline,
        "prefill": pre,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
