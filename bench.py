#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X: the five seeded workloads, HBM-resident inputs.

Prints ONE JSON line.  ``value`` is the prefill throughput of the BF16 layer with 128 tokens
(H 2048, 128 experts, top-8, I 768); every workload's tokens/s, HBM and MFMA fractions and CPU
baseline are listed under ``all_configs``.  ``roofline`` describes the dominant kernel of the
headline workload, its duration measured with HIP events on the stream it runs on.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs a,b] [--cpu-seconds S]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer decode tok/s + % HBM peak; prefill tok/s + % MFMA peak, 1 GPU"
HBM_PEAK = 8.0e12                                            # B/s
MFMA_PEAK = {"bf16": 2.5e15, "fp8": 5.0e15, "fp4": 10.1e15}  # dense FLOP/s
HEADLINE = ("c2_bf16_prefill", 128)
RUNS = [("c1_bf16_decode", 1), ("c2_bf16_prefill", 128), ("c3_mxfp4_decode", 1),
        ("c3_mxfp4_decode", 32), ("c4_mxfp8", 1), ("c4_mxfp8", 512),
        ("c5_mxfp4_zipf_prefill", 1024)]
MALL_BYTES = 256 << 20   # Infinity Cache: rotate enough layer copies to stream past it


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="all",
                    help="comma list of name:tokens (default: all seven runs; the "
                         "MX-activation variants c4_mxfp8_mx_activation and "
                         "c5_mxfp4_mx_activation run when named)")
    ap.add_argument("--cpu-seconds", type=float, default=3.0,
                    help="CPU-baseline budget per run (the headline run gets 4x)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-steps", type=int, default=5)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run a device-to-device copy of this many MiB (a known-size "
                         "kernel for calibrating HBM byte counters)")
    return ap.parse_args()


def layer_bytes(spec, C, tokens, distinct):
    """Algorithmic HBM bytes of one layer call: distinct experts' weights, the shared expert,
    the router and BF16 activations in and out."""
    return (distinct * C.expert_bytes(spec) + C.shared_bytes(spec)
            + spec.n_experts * spec.hidden * 2 + tokens * spec.hidden * 2 * 2)


def layer_flops(spec, tokens):
    H, I, E, k, Is = spec.hidden, spec.intermediate, spec.n_experts, spec.top_k, \
        spec.shared_intermediate
    return 2 * tokens * (E * H + k * 3 * H * I + 3 * H * Is)


def stage_bytes(spec, C, stage, tokens, distinct):
    """Algorithmic HBM bytes of one launch of a stage (weights touched once, f32 activations)."""
    H, I, E, k, Is = spec.hidden, spec.intermediate, spec.n_experts, spec.top_k, \
        spec.shared_intermediate
    eb = lambda fmt, r, c: sum(C.matrix_bytes(fmt, r, c))
    ef = spec.expert_format
    if stage == "gate_up":
        return distinct * 2 * eb(ef, I, H) + tokens * H * 4 + tokens * k * I * 4
    if stage == "down":
        return distinct * eb(ef, H, I) + tokens * k * I * 4 + tokens * k * H * 4
    if stage == "shared_gate_up":
        return 2 * eb(spec.shared_format, Is, H) + tokens * H * 4 + tokens * Is * 4
    if stage == "shared_down":
        return eb(spec.shared_format, H, Is) + tokens * Is * 4 + tokens * H * 4
    if stage == "router":
        return E * H * 2 + tokens * H * 4 + tokens * E * 4
    if stage == "combine":
        return tokens * k * H * 4 + tokens * H * 4 * (2 if Is else 1)
    return tokens * k * 16


def measured_traffic(workload, tokens, stage):
    """HBM bytes per launch of a stage's kernel from the committed counter measurement
    (profiles/hbm_traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by
    what the counter reads for a device copy of known size), or None when none matches."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            m = json.load(f)
    except (OSError, ValueError):
        return None
    for e in m.get("measurements", []):
        if (e.get("workload"), e.get("tokens"), e.get("stage")) == (workload, tokens, stage):
            return e.get("bytes_per_launch")
    return None


def cpu_baseline(name, spec, C, dev, x, budget_s, threads, tok=None):
    """The CPU oracle (a C++ restatement of the reference's CPU path) timed on a bounded
    sample of the same workload's tokens, one worker per core."""
    import numpy as np
    from oracle import oracle as O
    T = x.shape[0]
    host = dev.to_host()
    xs = x.cpu().numpy()
    ts = None if tok is None else tok.cpu().numpy().astype(np.uint32)

    def call(n):
        O.moe_forward(spec, host.experts, host.router_weight, xs[:n], host.correction_bias,
                      host.shared, threads=threads, shared_expert_gate=host.shared_expert_gate,
                      token_ids=None if ts is None else ts[:n], hash_experts=host.hash_experts)
    call(1)  # warm pool and page cache
    t0 = time.perf_counter()
    call(1)
    one = time.perf_counter() - t0
    # tokens per call: the whole batch when a call fits the budget, else a prefix that does;
    # whole calls repeat until the budget is spent
    n = int(max(1, min(T, budget_s / max(one, 1e-6))))
    reps = 0
    t0 = time.perf_counter()
    while True:
        call(n)
        reps += 1
        if time.perf_counter() - t0 >= budget_s or reps >= 5000:
            break
    dt = (time.perf_counter() - t0) / reps
    return {"value": n / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{name}: first {n} of {T} tokens x{reps}, {dt * 1e3:.1f} ms per call, "
                      f"C++ restatement of the reference CPU path, {threads} threads"}


def run_one(name, T, args, want_cpu, cpu_budget):
    import numpy as np
    import torch
    from urbilateria_amd import configs as C
    from urbilateria_amd import moe

    w = C.workload(name)
    spec = w.spec
    bias = None
    if w.zipf_s:
        from urbilateria_amd import synth
        # logit std of a BF16 N(0, 0.02) router row on N(0, 1) inputs is 0.02 * sqrt(H)
        std = np.full(spec.n_experts, 0.02 * math.sqrt(spec.hidden))
        beta = C.calibrate_zipf_beta(spec.n_experts, spec.top_k, w.zipf_s, std,
                                     router=spec.router)
        bias = C.zipf_bias(spec.n_experts, w.zipf_s, beta)
    table = tok = None
    if w.hash_vocab:
        from urbilateria_amd import synth
        # a synthetic tid2eid table and uniform token ids
        table = torch.from_numpy(C.hash_table(w.hash_vocab, spec.n_experts, spec.top_k)).cuda()
        ids_tok = synth.splitmix64(synth.stream_seed("bench.tokens"), 0, T) % np.uint64(
            w.hash_vocab)
        tok = torch.from_numpy(ids_tok.astype(np.int32)).cuda()

    def synthesize():
        d = moe.DeviceLayer.synthesize(spec, correction_bias=bias)
        d.hash_experts = table
        return d
    first = synthesize()
    x = moe.synth_activations(T, spec.hidden)
    probe = moe.MoeLayer(first, max_tokens=T)
    _, ids, _ = probe.forward(x, token_ids=tok)
    ids_np = ids.cpu().numpy()
    distinct = len(np.unique(ids_np))
    counts = np.bincount(ids_np.ravel(), minlength=spec.n_experts)
    touched = layer_bytes(spec, C, T, distinct)
    copies = max(1, min(8, math.ceil(3 * MALL_BYTES / touched)))
    full = C.expert_bytes(spec) * spec.n_experts + C.shared_bytes(spec)
    layers, devs = [probe], [first]
    for _ in range(copies - 1):
        d = synthesize()
        devs.append(d)
        layers.append(moe.MoeLayer(d, max_tokens=T))
    y = torch.empty((T, spec.hidden), dtype=torch.float32, device="cuda")
    idb = torch.empty((T, spec.top_k), dtype=torch.int32, device="cuda")
    wb = torch.empty((T, spec.top_k), dtype=torch.float32, device="cuda")
    for i in range(args.warmup):
        layers[i % copies].forward_into(x, y, idb, wb, token_ids=tok)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        layers[i % copies].forward_into(x, y, idb, wb, token_ids=tok)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    for l in layers:
        l.sync()
    # per-stage spans (a separate pass: spans wait for each call)
    for l in layers:
        l.profile(True)
    for i in range(args.profile_steps * copies):
        layers[i % copies].forward_into(x, y, idb, wb, token_ids=tok)
    torch.cuda.synchronize()
    stages = {}
    for l in layers:
        for k, (tms, n) in l.profile_read().items():
            a = stages.setdefault(k, [0.0, 0])
            a[0] += tms
            a[1] += n
        l.profile(False)
    stage_rows = {}
    for k, (tms, n) in stages.items():
        if n:
            avg = tms / n
            b = stage_bytes(spec, C, k, T, distinct)
            stage_rows[k] = {"avg_us": avg * 1e3, "bytes": b, "GBps": b / (avg * 1e-3) / 1e9}
    dom = max(stage_rows, key=lambda k: stage_rows[k]["avg_us"]) if stage_rows else None
    flops = layer_flops(spec, T)
    fmt = C.FORMAT_NAMES[spec.expert_format]
    mfma_dtype = {"bf16": "bf16", "mxfp8": "fp8", "mxfp4": "fp4"}[fmt]
    rec = {
        "workload": name, "tokens": T, "description": w.description,
        "ms_per_call": ms, "tokens_per_s": T / (ms * 1e-3),
        "algorithmic_bytes": touched, "GBps": touched / (ms * 1e-3) / 1e9,
        "hbm_frac": touched / (ms * 1e-3) / HBM_PEAK,
        "flops": flops, "TFLOPs": flops / (ms * 1e-3) / 1e12,
        "mfma_frac_bf16": flops / (ms * 1e-3) / MFMA_PEAK["bf16"],
        "mfma_frac_native": flops / (ms * 1e-3) / MFMA_PEAK[mfma_dtype],
        "mfma_ceiling_at_hbm_roofline_bf16": min(1.0, flops / (touched / HBM_PEAK) / MFMA_PEAK["bf16"]),
        "distinct_experts": distinct, "max_tokens_per_expert": int(counts.max()),
        "layer_copies_rotated": copies, "stages": stage_rows, "dominant_stage": dom,
    }
    if w.zipf_s:
        rec["zipf_bias_beta"] = float(beta)
    cpu_job = None
    if want_cpu:
        # run after every GPU measurement, so no GPU timing follows seconds of host-only work
        threads = min(16, os.cpu_count() or 1)
        cpu_job = (lambda dev=first, xx=x, tt=tok:
                   cpu_baseline(name, spec, C, dev, xx, cpu_budget, threads, tt))
    for l in layers:
        l.close()
    del layers, devs, first, x, y
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return rec, cpu_job


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested); the MoE layer "
              "here is built and measured on one MI355X.", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_probe_mib:
        n = args.copy_probe_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {args.copy_probe_mib} MiB device-to-device")
        del src, dst
    runs = RUNS if args.configs == "all" else [
        (c.split(":")[0], int(c.split(":")[1])) for c in args.configs.split(",")]
    results, jobs = [], []
    for name, T in runs:
        log(f"run {name} T={T}")
        head = (name, T) == HEADLINE
        budget = args.cpu_seconds * (4.0 if head else 1.0)
        rec, job = run_one(name, T, args, not args.no_cpu, budget)
        jobs.append((rec, job))
        log(f"  {rec['tokens_per_s']:.1f} tok/s, {rec['ms_per_call']:.3f} ms, "
            f"{rec['GBps']:.0f} GB/s ({100 * rec['hbm_frac']:.1f}% HBM), dominant "
            f"{rec['dominant_stage']}")
        results.append(rec)
    for rec, job in jobs:
        if job is not None:
            log(f"cpu baseline {rec['workload']} T={rec['tokens']}")
            rec["cpu_baseline"] = job()
            log(f"  {rec['cpu_baseline']['value']:.1f} tokens/s on "
                f"{rec['cpu_baseline']['cores']} threads")
    head = next((r for r in results if (r["workload"], r["tokens"]) == HEADLINE), results[0])
    dom = head["stages"].get(head["dominant_stage"], {})
    line = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_call"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if "bf16" in head["workload"] else "f32-accumulated MX",
        "data": "synthetic (seeded SplitMix64 weights and activations)",
        "config": {"workload": f"{head['workload']}: {head['description']}",
                   "tokens": head["tokens"], "parallelism": "single GPU"},
        "hbm_frac": head["hbm_frac"],
        "mfma_frac": head["mfma_frac_bf16"],
        "roofline": {
            "kernel": head["dominant_stage"], "bound": "hbm",
            "achieved": dom.get("GBps"), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": (dom.get("GBps") or 0) / (HBM_PEAK / 1e9),
            "traffic": measured_traffic(head["workload"], head["tokens"], head["dominant_stage"]),
            "bytes_per_launch": dom.get("bytes"), "avg_launch_us": dom.get("avg_us"),
        },
        "cpu_baseline": head.get("cpu_baseline"),
        "all_configs": results,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
