#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X: the five seeded workloads, HBM-resident inputs.

Prints ONE JSON line.  ``value`` is the prefill throughput of the largest workload, the Kimi-scale
MXFP4 layer with 1024 tokens and Zipf(1.1)-skewed routing (H 7168, 384 experts, top-8, I 2048,
BF16 shared expert).  Every workload's tokens/s, HBM and MFMA fractions, its own ``roofline``
block and its CPU baseline are listed under ``all_configs``.  A ``roofline`` block describes the
workload's dominant kernel: algorithmic bytes per launch over its average duration, measured
with HIP events on the stream the kernel runs on, and the HBM bytes the rocprofv3 counters
measured for it (profiles/hbm_traffic.json).

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
HEADLINE = ("c5_mxfp4_zipf_prefill", 1024)
RUNS = [("c1_bf16_decode", 1), ("c2_bf16_prefill", 128), ("c3_mxfp4_decode", 1),
        ("c3_mxfp4_decode", 32), ("c4_mxfp8", 1), ("c4_mxfp8", 512),
        ("c5_mxfp4_zipf_prefill", 1024), ("c5_mxfp4_zipf_flat", 1024),
        ("c5_mxfp4_zipf_hot", 1024)]
# The projection stages a roofline block may name (routing kernels are latency-bound).  The
# routed projections always run on the caller's stream, on the critical path.  The shared
# expert's run there too for one token and for batches of SHARED_INLINE_TOKENS or more in the
# f32-activation compositions; other batches run them on a side stream beside the routing, where
# their spans include the time they wait for CUs, so they are not candidates then.
PROJECTIONS = ("gate_up", "down")
SHARED_PROJECTIONS = ("shared_gate_up", "shared_down")
SHARED_INLINE_TOKENS = 256
MALL_BYTES = 256 << 20   # Infinity Cache: rotate enough layer copies to stream past it


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="all",
                    help="comma list of name:tokens (default: all nine runs; the "
                         "MX-activation variants c4_mxfp8_mx_activation and "
                         "c5_mxfp4_mx_activation run when named)")
    ap.add_argument("--cpu-seconds", type=float, default=3.0,
                    help="CPU-baseline budget per run (the headline run gets 4x)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-steps", type=int, default=5)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run a device-to-device copy of this many MiB (a known-size "
                         "kernel for calibrating HBM byte counters)")
    ap.add_argument("--pack-cost", action="store_true",
                    help="instead of the layer runs, time the ingest conversion of checkpoint "
                         "matrices into the panel layout (urb_pack_matrix, HBM to HBM) and a "
                         "pinned host-to-HBM copy of the same bytes; prints one JSON line")
    return ap.parse_args()


def pack_cost(steps):
    """The cost of converting checkpoint-layout expert matrices into the panel layout at ingest:
    urb_pack_matrix on one [2048, 7168] projection per format (an expert matrix of the c3 and c5
    workloads), HBM to HBM, against a pinned host-to-HBM copy of the same checkpoint bytes (the
    copy every ingest makes anyway)."""
    import torch
    from urbilateria_amd import configs as C
    from urbilateria_amd import moe
    rows, cols = 2048, 7168
    out = []
    for fmt, name in ((C.FMT_BF16, "bf16"), (C.FMT_MXFP4, "mxfp4"), (C.FMT_MXFP8, "mxfp8")):
        nbytes = rows * cols * 2 if fmt == C.FMT_BF16 else rows * cols // (2 if fmt == C.FMT_MXFP4 else 1)
        # any bytes: the conversion moves bytes without decoding them (E8M0 scales 127 = 1.0)
        data = torch.randint(0, 120, (nbytes,), dtype=torch.uint8, device="cuda")
        scales = (None if fmt == C.FMT_BF16 else
                  torch.full((rows * cols // 32,), 127, dtype=torch.uint8, device="cuda"))
        total = nbytes + (0 if scales is None else scales.numel())
        for _ in range(3):
            moe.pack_matrix(fmt, data, scales, rows, cols)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            moe.pack_matrix(fmt, data, scales, rows, cols)
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / steps
        host = torch.empty(total, dtype=torch.uint8, pin_memory=True)
        dev = torch.empty(total, dtype=torch.uint8, device="cuda")
        dev.copy_(host, non_blocking=True)
        torch.cuda.synchronize()
        t0.record()
        for _ in range(steps):
            dev.copy_(host, non_blocking=True)
        t1.record()
        torch.cuda.synchronize()
        h2d = t0.elapsed_time(t1) * 1e3 / steps
        out.append({"format": name, "rows": rows, "cols": cols, "checkpoint_bytes": total,
                    "pack_us": us, "pack_GBps": total / (us * 1e-6) / 1e9,
                    "h2d_pinned_us": h2d, "h2d_pinned_GBps": total / (h2d * 1e-6) / 1e9,
                    "pack_over_h2d": us / h2d})
        log(f"pack {name} [{rows}, {cols}]: {us:.1f} us ({total / (us * 1e-6) / 1e9:.0f} GB/s); "
            f"pinned H2D {h2d:.1f} us ({total / (h2d * 1e-6) / 1e9:.1f} GB/s)")
    print(json.dumps({"pack_cost": out}), flush=True)


def layer_bytes(spec, C, tokens, distinct):
    """Algorithmic HBM bytes of one layer call: distinct experts' weights, the shared expert,
    the router and BF16 activations in and out."""
    return (distinct * C.expert_bytes(spec) + C.shared_bytes(spec)
            + spec.n_experts * spec.hidden * 2 + tokens * spec.hidden * 2 * 2)


def layer_flops(spec, tokens):
    H, I, E, k, Is = spec.hidden, spec.intermediate, spec.n_experts, spec.top_k, \
        spec.shared_intermediate
    return 2 * tokens * (E * H + k * 3 * H * I + 3 * H * Is)


def stage_flops(spec, stage, tokens):
    """FLOPs of one launch of a projection stage (2 per multiply-add)."""
    from urbilateria_amd import configs as C
    H, I, k, Is = spec.hidden, spec.intermediate, spec.top_k, spec.shared_intermediate
    f = {"gate_up": 2 * tokens * k * 2 * H * I, "down": 2 * tokens * k * H * I,
         "shared_gate_up": 2 * tokens * 2 * H * Is,
         "shared_down": 2 * tokens * H * Is}.get(stage, 0)
    if (stage == "gate_up" and tokens == 1 and Is
            and spec.composition in (C.COMPOSE_GLM, C.COMPOSE_QWEN36)):
        f += 2 * H * Is  # the shared down projection runs in the same launch
    return f


def stage_bytes(spec, C, stage, tokens, distinct):
    """Algorithmic HBM bytes of one launch of a stage: weights touched once, the token rows at
    the width the gate/up reads them (a GLM batch's BF16 copy from the MFMA router, as the
    synthetic rows are BF16-valued; f32 otherwise), and the
    SwiGLU rows between gate/up and down at the width the path stores them (f16 where the down
    projection runs on f16 MFMAs, f32 otherwise)."""
    H, I, E, k, Is = spec.hidden, spec.intermediate, spec.n_experts, spec.top_k, \
        spec.shared_intermediate
    eb = lambda fmt, r, c: sum(C.matrix_bytes(fmt, r, c))
    ef = spec.expert_format
    glm = spec.composition == C.COMPOSE_GLM
    # batches of a GLM layer with MX experts: f16 SwiGLU rows (urb_moe_host.cpp, down_f16)
    act_w = 2 if glm and ef != C.FMT_BF16 and tokens > 1 else 4
    # in-line batches of a GLM layer's BF16 shared expert: f16 SwiGLU rows (shared16)
    sact_w = 2 if (glm and spec.shared_format == C.FMT_BF16 and tokens > 1
                   and shared_in_line(spec, C, tokens)) else 4
    # the routed gate+up of a GLM batch reads the MFMA router's BF16 copy of the token rows
    # (urb_moe_host.cpp, Workspace::xb; the other compositions route with the 8-lane tree or
    # read quantized rows)
    x_w = 2 if glm and tokens > 1 else 4
    if stage == "gate_up":
        routed = distinct * 2 * eb(ef, I, H) + tokens * H * x_w + tokens * k * I * act_w
        if tokens == 1 and Is and spec.composition in (C.COMPOSE_GLM, C.COMPOSE_QWEN36):
            # one token: the shared expert's down projection runs in the routed gate+up launch
            routed += stage_bytes(spec, C, "shared_down", tokens, distinct)
        return routed
    if stage == "down":
        return distinct * eb(ef, H, I) + tokens * k * I * act_w + tokens * k * H * 4
    if stage == "shared_gate_up":
        return 2 * eb(spec.shared_format, Is, H) + tokens * H * 4 + tokens * Is * sact_w
    if stage == "shared_down":
        return eb(spec.shared_format, H, Is) + tokens * Is * sact_w + tokens * H * 4
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


def host_disclosure(workers):
    """The CPU the baseline ran on: model, sockets, physical cores and logical CPUs of the
    allowed set, AVX2/FMA (which select the reference's BF16 and MXFP8 kernels), workers."""
    from oracle import oracle as O
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    allowed = sorted(os.sched_getaffinity(0))
    packages = set()
    for c in allowed:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id") as f:
                packages.add(int(f.read()))
        except (OSError, ValueError):
            pass
    return {"cpu_model": model, "sockets": len(packages), "physical_cores": O.physical_cores(),
            "logical_cpus": len(allowed), "avx2": "avx2" in flags, "fma": "fma" in flags,
            "workers": workers, "pinned": "physical-core-first, one worker per core"}


def cpu_workers():
    """One worker per physical core of the allowed CPU set (src/execution.rs:254-263), capped
    at the CPU share this process is given (OMP_NUM_THREADS on a shared GPU host)."""
    from oracle import oracle as O
    physical = max(1, O.physical_cores())
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return min(physical, share) if share > 0 else physical


def cpu_baseline(name, spec, C, dev, x, budget_s, tok=None):
    """The CPU oracle (a C++ restatement of the reference's CPU path) timed on a bounded
    sample of the same workload's tokens, with the reference's execution contract: one worker
    per physical core, pinned physical-core-first (src/execution.rs:254-394)."""
    import numpy as np
    from oracle import oracle as O
    T = x.shape[0]
    host = dev.to_host()
    xs = x.cpu().numpy()
    ts = None if tok is None else tok.cpu().numpy().astype(np.uint32)
    threads = cpu_workers()
    prev = O.set_pinning(True)

    def call(n):
        O.moe_forward(spec, host.experts, host.router_weight, xs[:n], host.correction_bias,
                      host.shared, threads=threads, shared_expert_gate=host.shared_expert_gate,
                      token_ids=None if ts is None else ts[:n], hash_experts=host.hash_experts)
    try:
        call(1)  # warm pool and page cache
        t0 = time.perf_counter()
        call(1)
        one = time.perf_counter() - t0
        # tokens per call: the whole batch when a call fits the budget, else a prefix that
        # does; whole calls repeat until the budget is spent
        n = int(max(1, min(T, budget_s / max(one, 1e-6))))
        reps = 0
        t0 = time.perf_counter()
        while True:
            call(n)
            reps += 1
            if time.perf_counter() - t0 >= budget_s or reps >= 5000:
                break
        dt = (time.perf_counter() - t0) / reps
    finally:
        O.set_pinning(prev)
    return {"value": n / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{name}: first {n} of {T} tokens x{reps}, {dt * 1e3:.1f} ms per call, "
                      f"C++ restatement of the reference CPU path, {threads} pinned workers",
            "host": host_disclosure(threads)}


def shared_in_line(spec, C, tokens):
    """Whether the layer call runs the shared expert on the caller's stream (urb_moe_host.cpp,
    shared_stream): one token, or f32-activation batches of SHARED_INLINE_TOKENS or more."""
    mx = spec.composition in (C.COMPOSE_HY4, C.COMPOSE_DSV41, C.COMPOSE_DSV4)
    return bool(spec.shared_intermediate) and (tokens == 1 or
                                               (not mx and tokens >= SHARED_INLINE_TOKENS))


def committed_trace(workload, tokens, stage):
    """The committed rocprofv3 kernel-trace statistics of a stage's kernel
    (profiles/kernel_traces.json: kernel name, calls, average/min/max duration and the command),
    or None."""
    path = os.path.join(ROOT, "profiles", "kernel_traces.json")
    try:
        with open(path) as f:
            m = json.load(f)
    except (OSError, ValueError):
        return None
    for e in m.get("traces", []):
        if (e.get("workload"), e.get("tokens"), e.get("stage")) == (workload, tokens, stage):
            return e
    return None


def roofline_block(rec, spec, C, workload, tokens):
    """The dominant projection kernel of a run: algorithmic bytes per launch over its average
    launch duration (HIP events on its stream), against 8 TB/s; its MFMA rate against the
    dense BF16 peak; the counter-measured HBM bytes per launch when profiles/ holds them; and
    the same kernel's average duration and fraction in the committed rocprofv3 kernel trace."""
    stages = rec["stages"]
    names = PROJECTIONS + (SHARED_PROJECTIONS if shared_in_line(spec, C, tokens) else ())
    cands = [k for k in names if k in stages]
    if not cands:
        return None
    dom = max(cands, key=lambda k: stages[k]["avg_us"])
    st = stages[dom]
    achieved = st["bytes"] / (st["avg_us"] * 1e-6) / 1e9
    block = {"kernel": dom, "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK / 1e9,
             "unit": "GB/s", "frac": achieved / (HBM_PEAK / 1e9),
             "traffic": measured_traffic(workload, tokens, dom),
             "bytes_per_launch": st["bytes"], "avg_launch_us": st["avg_us"],
             "mfma_frac_bf16": st.get("flops", 0) / (st["avg_us"] * 1e-6) / MFMA_PEAK["bf16"]}
    tr = committed_trace(workload, tokens, dom)
    if tr:
        block["trace"] = {"kernel_name": tr["kernel"], "avg_us": tr["avg_us"],
                          "frac": st["bytes"] / (tr["avg_us"] * 1e-6) / HBM_PEAK,
                          "file": "profiles/kernel_traces.json"}
    return block


def run_one(name, T, args, want_cpu, cpu_budget):
    import numpy as np
    import torch
    from urbilateria_amd import configs as C
    from urbilateria_amd import moe

    w = C.workload(name)
    spec = w.spec
    zipf, bias = C.workload_bias(w)
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
            stage_rows[k] = {"avg_us": avg * 1e3, "bytes": b, "GBps": b / (avg * 1e-3) / 1e9,
                             "flops": stage_flops(spec, k, T)}
    # the longest span on the caller's stream (the shared expert's spans overlap the others')
    main = [k for k in stage_rows if not k.startswith("shared_")]
    dom = max(main, key=lambda k: stage_rows[k]["avg_us"]) if main else None
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
    if zipf:
        rec["zipf_bias"] = zipf
    rec["roofline"] = roofline_block(rec, spec, C, name, T)
    cpu_job = None
    if want_cpu:
        # run after every GPU measurement, so no GPU timing follows seconds of host-only work
        cpu_job = (lambda dev=first, xx=x, tt=tok:
                   cpu_baseline(name, spec, C, dev, xx, cpu_budget, tt))
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
    if args.pack_cost:
        pack_cost(args.steps)
        return
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
    fmt = head["workload"]
    dtype = ("bf16 weights x f32 activations" if "bf16" in fmt else
             "mxfp8 weights x f32 activations" if "mxfp8" in fmt else
             "mxfp4 weights x f32 activations") + " (bf16 MFMA, f32 accumulation)"
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
        "dtype": dtype,
        "data": "synthetic (seeded SplitMix64 weights and activations)",
        "config": {"workload": f"{head['workload']}: {head['description']}",
                   "tokens": head["tokens"], "parallelism": "single GPU"},
        "hbm_frac": head["hbm_frac"],
        "mfma_frac": head["mfma_frac_bf16"],
        "roofline": head.get("roofline"),
        "cpu_baseline": head.get("cpu_baseline"),
        "all_configs": results,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
