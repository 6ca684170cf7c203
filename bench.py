#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X through the C ABI (libqmoe.so).

Default workload: the Qwen3-30B-A3B-shaped MoE layer (H=2048, E=128, top-8,
I=768, bf16 weights ~ N(0, 0.02)) at decode, T=1 token per step, true top-8 of
128 (selection scope C=E), x ~ N(0, 1).  One step = one forward of the layer
over one batch of T tokens whose x already sits in HBM.

Honest bandwidth: the layer's weights are uploaded into several distinct copies
and the steps rotate through them, so each round of copies reads more than
2 x 256 MB (the Infinity Cache) of weights.

The default run (--workload decode) also measures the metric's other half,
the same layer at prefill T=2048 (router x4, skewed tokens), and reports it in
a nested "prefill" object of the same JSON line, and the block's neighbours in
a "neighbours" object: the LM head GEMV (151936 x 2048 bf16, T = 1, bit-exact
sequential sums) with its CPU baseline, and the decode step with the
post-attention norm and the residual add folded in against the block alone.

Also reported on the same JSON line:
  roofline      the dominant kernel's algorithmic bytes per launch divided by
                its average duration, timed with HIP events recorded on the
                kernel's own stream during the timed region;
  cpu_baseline  the CPU oracle (a C restatement of model/moe.go, the Go
                reference cannot run here) on a bounded sample of the same
                workload on this host's cores.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen-go_amd"))

import qmoe  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

WORKLOADS = {
    # name: (config key, T, scope, description)
    "decode": ("qwen3_30b_a3b", 1, "E", "qwen3-30b-a3b moe layer decode T=1, bf16 weights, top-8 of 128"),
    "decode8": ("qwen3_30b_a3b", 8, "E", "qwen3-30b-a3b moe layer decode T=8, bf16 weights, top-8 of 128"),
    "prefill": ("qwen3_30b_a3b", 2048, "E",
                "qwen3-30b-a3b moe layer prefill T=2048, bf16 weights, router x4, skewed tokens, top-8 of 128"),
    "prefill_firstk": ("qwen3_30b_a3b", 2048, "k",
                       "qwen3-30b-a3b moe layer prefill T=2048, bf16 weights, first-8 of 128 "
                       "(the reference's selection: every token on experts 0..7)"),
    "int8_decode": ("qwen3_30b_a3b_int8", 1, "E",
                    "qwen3-30b-a3b moe layer decode T=1, int8 group-32 experts, top-8 of 128"),
    "int8_prefill": ("qwen3_30b_a3b_int8", 512, "E",
                     "qwen3-30b-a3b moe layer prefill T=512, int8 group-32 experts, top-8 of 128"),
    "next_decode": ("qwen3_next", 1, "E",
                    "qwen3-next moe layer decode T=1, int4 group-32 experts + gated shared expert, top-10 of 512"),
    "next_prefill": ("qwen3_next", 4096, "E",
                     "qwen3-next moe layer prefill T=4096, int4 group-32 experts + gated shared expert, top-10 of 512"),
    "toy": ("toy", 16, "k", "toy moe layer T=16, f32, first-2 of 8 (reference selection)"),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="decode", choices=sorted(WORKLOADS) + ["lm_head"],
                    help="lm_head: the LM head GEMV alone (its own JSON line)")
    ap.add_argument("--copies", type=int, default=0, help="weight copies to rotate (0 = auto)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prefill-steps", type=int, default=100,
                    help="decode workload: steps of the prefill half of the metric (T=2048) on the same line")
    ap.add_argument("--prefill-warmup", type=int, default=10)
    ap.add_argument("--no-prefill", action="store_true",
                    help="decode workload: leave out the prefill half of the metric")
    ap.add_argument("--no-neighbours", action="store_true",
                    help="decode workload: leave out the LM head and norm+residual measurements")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--skew", type=float, default=10.0,
                    help="prefill: target ratio of the busiest expert's load to the median load")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB, 5 times (the calibration "
                         "kernel for rocprofv3 FETCH_SIZE / WRITE_SIZE), and exit")
    return ap.parse_args()


def copy_probe(mib):
    """A plain copy kernel of known size: reads and writes mib MiB per launch."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n * 4, "launches": 5}))


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary for this workload (profiles/traffic_<workload>.txt: FETCH_SIZE and
    WRITE_SIZE, each scaled by the copy kernel's calibration), or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) >= 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
            return int(float(parts[2]))
    return None


# prefill workloads: router weights x4 and tokens pulled along one direction
ROUTER_SCALE = {"prefill": 4.0}


def stage_bytes(cfg, T, ids):
    """Algorithmic HBM bytes of each kernel for one forward with routing ids."""
    H, E, k, I, Is = cfg.hidden, cfg.n_experts, cfg.top_k, cfg.moe_inter, cfg.shared_inter
    touched = len(np.unique(ids))
    wb = qmoe.weight_bytes
    b = {
        qmoe.STAGE_ROUTER: wb(cfg.router_fmt, E, H) + T * H * 4 + T * E * 4,
        qmoe.STAGE_SELECT: T * E * 4 + T * k * 8,
        # batched path: weights + bf16 x rows in + bf16 SwiGLU rows out
        qmoe.STAGE_GATE_UP: touched * wb(cfg.expert_fmt, 2 * I, H) + T * H * 2 + T * k * I * 2,
        # weights + bf16 SwiGLU rows in + f32 weighted rows out
        qmoe.STAGE_DOWN: touched * wb(cfg.expert_fmt, H, I) + T * k * I * 2 + T * k * H * 4,
        # x in, bf16 x out, ids/weights in, slot tables out
        qmoe.STAGE_DISPATCH: T * H * 4 + T * H * 2 + T * k * 8 + T * k * 12,
        # f32 weighted rows in, out
        qmoe.STAGE_COMBINE: T * k * H * 4 + T * H * 4,
    }
    if Is:
        b[qmoe.STAGE_SHARED_GATE_UP] = 2 * wb(cfg.shared_fmt, Is, H) + T * H * 2 + T * Is * 2
        b[qmoe.STAGE_DOWN] += wb(cfg.shared_fmt, H, Is) + T * Is * 2 + T * H * 4
        b[qmoe.STAGE_DISPATCH] += H * 4
        b[qmoe.STAGE_COMBINE] += T * H * 4
    # decode: one kernel reads the routed (and shared) gate_up and down weights,
    # x and the router partials, and accumulates out
    b[qmoe.STAGE_FUSED] = (touched * (wb(cfg.expert_fmt, 2 * I, H) + wb(cfg.expert_fmt, H, I)) + T * H * 4
                           + T * E * 16 + T * H * 4)
    if Is:
        b[qmoe.STAGE_FUSED] += 2 * wb(cfg.shared_fmt, Is, H) + wb(cfg.shared_fmt, H, Is) + H * 4
    return b


def stage_flops(cfg, T):
    """MFMA flops of the batched GEMMs for one forward of T tokens."""
    H, k, I, Is = cfg.hidden, cfg.top_k, cfg.moe_inter, cfg.shared_inter
    f = {qmoe.STAGE_GATE_UP: 2 * T * k * 2 * I * H, qmoe.STAGE_DOWN: 2 * T * k * H * I}
    if Is:
        f[qmoe.STAGE_SHARED_GATE_UP] = 2 * T * 2 * Is * H
        f[qmoe.STAGE_DOWN] += 2 * T * H * Is
    return f


def host_cpu():
    """(nproc, CPU model name) of this host."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return nproc, model


def cpu_baseline(hw, cfg, T, scope, xs, budget_s):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    nproc, model = host_cpu()
    threads = min(nproc, 8)
    ol = oracle.OracleLayer(hw, scope=scope, threads=threads)
    # per-token cost is independent of T (one forward per token, model.go:508-514):
    # a bounded slice of at most 32 tokens per call
    Tc = min(T, 32)
    x = xs[0][:Tc]
    t0 = time.perf_counter()
    ol.forward(x)
    one = time.perf_counter() - t0
    reps = max(2, min(400, int(budget_s / max(one, 1e-6))))
    t0 = time.perf_counter()
    for i in range(reps):
        ol.forward(xs[i % len(xs)][:Tc])
    dt = time.perf_counter() - t0
    return {
        "value": round(reps * Tc / dt, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": (f"{reps} forwards of T={Tc} ({reps * Tc} tokens) of the same layer and routing, "
                   f"C restatement of model/moe.go (gcc -O2 -ffp-contract=off), one call per token as "
                   f"decodeLayers does; router/shared bf16 GEMVs on {threads} threads "
                   f"(GOMAXPROCS-equivalent min(nproc,8)), expert GEMVs single-threaded; Go is not "
                   f"installed on the box"),
        "seconds": round(dt, 2),
        "nproc": nproc, "cpu_model": model, "gomaxprocs_equivalent": threads, "expert_gemv_threads": 1,
    }


def main():
    args = parse()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              f"(the MoE block is built and measured on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "lm_head":
        print(json.dumps(measure_lm_head(args, steps=args.steps)))
        return
    result = measure(args, args.workload, args.steps, args.warmup, args.cpu_seconds)
    if args.workload == "decode" and not args.no_prefill:
        # the metric's other half on the same line: the same layer at T=2048
        pre = measure(args, "prefill", args.prefill_steps, args.prefill_warmup, args.cpu_seconds / 2)
        result["prefill"] = {k: pre[k] for k in ("value", "unit", "ms_per_step", "steps", "warmup", "dtype", "config",
                                                  "roofline", "mfma", "layer_roofline", "cpu_baseline") if k in pre}
    if args.workload == "decode" and not args.no_neighbours:
        result["neighbours"] = {"lm_head": measure_lm_head(args), "norm_residual": measure_norm_residual(args)}
    print(json.dumps(result))


def _time_us(fn, steps, warmup):
    """Average µs of fn() over steps calls, HIP events on torch's current
    stream (every call here launches on that stream)."""
    import torch
    for _ in range(warmup):
        fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / steps


def measure_lm_head(args, rows=151936, cols=2048, steps=200):
    """The LM head (model/model.go:519-525): y = x @ W^T, W (151936, 2048) bf16,
    T = 1, through qmoe_linear_forward_device; bytes = W + x + y (622 MB, more
    than the Infinity Cache holds).  CPU baseline: the oracle's matvec, bf16
    rows fanned out on min(nproc, 8) threads as linear.matvec does."""
    import torch
    rng = np.random.default_rng(args.seed + 7)
    w = qmoe.f32_to_bf16_bits(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
    lin = qmoe.Linear(rows, cols, qmoe.BF16)
    try:
        lin.set(w)
        x = torch.from_numpy(rng.standard_normal((1, cols), dtype=np.float32)).cuda()
        y = torch.empty((1, rows), dtype=torch.float32, device="cuda")
        sptr = torch.cuda.current_stream().cuda_stream
        us = _time_us(lambda: lin.forward_device(x.data_ptr(), 1, y.data_ptr(), sptr), steps, 20)
        tok = torch.empty(1, dtype=torch.int32, device="cuda")
        us_argmax = _time_us(lambda: lin.argmax_device(y.data_ptr(), 1, rows, tok.data_ptr(), sptr), steps, 20)
    finally:
        lin.close()
    nbytes = qmoe.weight_bytes(qmoe.BF16, rows, cols) + 4 * (rows + cols)
    gbs = nbytes / us / 1e3
    out = {"value": round(1e6 / us, 1), "unit": "calls/s", "us_per_call": round(us, 2),
           "argmax_us": round(us_argmax, 2), "dtype": "f32 (bf16 weights)",
           "config": {"workload": f"lm head GEMV ({rows}, {cols}) bf16, T=1, outputs bit-exact"},
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 3), "algorithmic_bytes": nbytes}}
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        nproc, model = host_cpu()
        threads = min(nproc, 8)
        xh = x.cpu().numpy()[0]
        reps, t0 = 0, time.perf_counter()
        while reps < 3 or (time.perf_counter() - t0 < 4.0 and reps < 50):
            oracle.matvec(oracle.BF16, w, None, xh, rows, cols, threads=threads)
            reps += 1
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(reps / dt, 2), "unit": "calls/s", "cores": threads, "kind": "port",
                               "sample": f"{reps} full LM-head matvecs, C restatement of linear.matvec "
                                         f"(model/model.go:131-176), bf16 rows on {threads} threads",
                               "nproc": nproc, "cpu_model": model}
    return out


def measure_norm_residual(args, steps=400):
    """decodeLayers' MLP step with the post-attention norm and the residual
    add on the device (qmoe_forward_residual_device) against the block alone
    (qmoe_forward_device), Qwen3-30B-A3B bf16 layer, T = 1, one weight copy
    for both (the difference is what the folding costs)."""
    import torch
    cfg = qmoe.CONFIGS["qwen3_30b_a3b"].with_(select_scope=128)
    hw = qmoe.synthetic_weights(cfg, args.seed)
    L = qmoe.MoeLayer(cfg)
    try:
        hw.upload(L)
        L.set_post_norm(np.random.default_rng(args.seed).standard_normal(cfg.hidden).astype(np.float32) * 0.2, 1e-6)
        x = torch.from_numpy(qmoe.synthetic_tokens(cfg, 1, args.seed + 3) * np.float32(8.0)).cuda()
        out = torch.empty_like(x)
        sptr = torch.cuda.current_stream().cuda_stream
        plain = _time_us(lambda: L.forward_device(x.data_ptr(), 1, out.data_ptr(), None, None, sptr), steps, 40)
        res = _time_us(lambda: L.forward_residual_device(x.data_ptr(), 1, out.data_ptr(), None, None, sptr),
                       steps, 40)
    finally:
        L.close()
    return {"block_us": round(plain, 2), "norm_block_residual_us": round(res, 2),
            "overhead_us": round(res - plain, 2),
            "config": {"workload": "qwen3-30b-a3b moe layer decode T=1 bf16, top-8 of 128, one weight copy"}}


def measure(args, workload, steps, warmup, cpu_seconds):
    """One workload: warmup, `steps` timed forwards, roofline and CPU baseline."""
    import torch

    key, T, scope_kind, desc = WORKLOADS[workload]
    cfg = qmoe.CONFIGS[key]
    scope = cfg.n_experts if scope_kind == "E" else cfg.top_k
    cfg = cfg.with_(select_scope=scope)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream

    t_gen = time.perf_counter()
    hw = qmoe.synthetic_weights(cfg, args.seed, router_scale=ROUTER_SCALE.get(workload, 1.0))
    lb = qmoe.layer_bytes(cfg)
    layer_total = lb["router"] + cfg.n_experts * lb["per_expert"] + lb["shared"]
    step_bytes_est = lb["router"] + min(cfg.n_experts, T * cfg.top_k) * lb["per_expert"] + lb["shared"]
    copies = args.copies or max(1, min(32, math.ceil(2 * 256e6 / step_bytes_est) + 1))
    layers = []
    for _ in range(copies):
        L = qmoe.MoeLayer(cfg)
        hw.upload(L)
        layers.append(L)
    gen_s = time.perf_counter() - t_gen

    n_x = max(2, min(64, (1 << 24) // (T * cfg.hidden)))
    skew = None
    if workload in ROUTER_SCALE:
        xs_host, stats = [], []
        for i in range(n_x):
            x, st = qmoe.skewed_tokens(cfg, hw, T, args.seed + 1000 + i, args.skew)
            xs_host.append(x)
            stats.append(st)
        skew = {"target_max_over_median": args.skew, "per_x": stats}
    else:
        xs_host = [qmoe.synthetic_tokens(cfg, T, args.seed + 1000 + i) for i in range(n_x)]
    d_x = torch.from_numpy(np.stack(xs_host)).to(dev).contiguous()   # (n_x, T, H)
    d_out = torch.empty((T, cfg.hidden), dtype=torch.float32, device=dev)
    d_ids = torch.empty((n_x, T, cfg.top_k), dtype=torch.int32, device=dev)
    d_w = torch.empty((n_x, T, cfg.top_k), dtype=torch.float32, device=dev)
    xstride = T * cfg.hidden * 4
    kstride = T * cfg.top_k * 4

    def step(s, L=None):
        i = s % n_x
        (L or layers[s % copies]).forward_device(d_x.data_ptr() + i * xstride, T, d_out.data_ptr(),
                                                 d_ids.data_ptr() + i * kstride, d_w.data_ptr() + i * kstride,
                                                 sptr)

    # routing of every x in the pool (same for every copy)
    for i in range(n_x):
        step(i, layers[0])
    torch.cuda.synchronize()
    ids_all = d_ids.cpu().numpy()
    per_x_bytes = [stage_bytes(cfg, T, ids_all[i]) for i in range(n_x)]

    # warmup, all stages profiled to find the dominant kernel
    all_stages = list(range(qmoe.STAGE_COUNT))
    for L in layers:
        L.profile_enable(all_stages)
        L.profile_read(reset=True)
    for s in range(warmup):
        step(s)
    torch.cuda.synchronize()
    tot_ms = np.zeros(qmoe.STAGE_COUNT)
    tot_n = np.zeros(qmoe.STAGE_COUNT, np.int64)
    for L in layers:
        ms, n = L.profile_read(reset=True)
        tot_ms += ms
        tot_n += n
    stage_avg_us = {qmoe.STAGE_NAMES[s]: round(1e3 * tot_ms[s] / max(tot_n[s], 1), 3)
                    for s in all_stages if tot_n[s]}
    if tot_n[qmoe.STAGE_FUSED] and not tot_n[qmoe.STAGE_ROUTER]:
        # T = 1: the expert kernel computes the router partials itself and reads the router
        for b in per_x_bytes:
            b[qmoe.STAGE_FUSED] += b[qmoe.STAGE_ROUTER] - T * cfg.n_experts * 4
            b[qmoe.STAGE_ROUTER] = 0
    # dominant HBM-bound kernel: the one with the most time among the weight-streaming stages
    weight_stages = [qmoe.STAGE_GATE_UP, qmoe.STAGE_DOWN, qmoe.STAGE_FUSED]
    dom = max(weight_stages, key=lambda s: tot_ms[s])

    # timed region: only the dominant kernel carries events, and only on the
    # first weight copy (every `copies`-th step) -- a launch with events costs
    # the host about 20 us more, which would otherwise make a decode step
    # host-bound
    for i, L in enumerate(layers):
        L.profile_enable([dom] if i == 0 else [])
        L.profile_read(reset=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        step(s)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    dom_ms = 0.0
    dom_n = 0
    for L in layers:
        ms, n = L.profile_read(reset=True)
        dom_ms += ms[dom]
        dom_n += int(n[dom])
    dom_avg_s = dom_ms / 1e3 / max(dom_n, 1)
    dom_bytes = float(np.mean([per_x_bytes[s % n_x][dom] for s in range(0, steps, copies)]))
    achieved = dom_bytes / dom_avg_s / 1e9
    mfma_path = layers[0].forward_path(T) == qmoe.PATH_MFMA
    dom_flops = stage_flops(cfg, T).get(dom, 0) if mfma_path else 0
    mfma_tflops = dom_flops / dom_avg_s / 1e12
    # the binding roof of the dominant kernel: its flops at the dense bf16
    # MFMA peak take longer than its bytes at the HBM peak (only when the
    # selection concentrates every token on k experts)
    mfma_bound = dom_flops / (MFMA_BF16_PEAK_TFLOPS * 1e12) > dom_bytes / (HBM_PEAK_GBS * 1e9)

    # whole-layer roofline: all algorithmic bytes / measured step time
    def layer_step_bytes(bmap):
        if tot_n[qmoe.STAGE_FUSED]:
            return bmap[qmoe.STAGE_ROUTER] + bmap[qmoe.STAGE_FUSED]
        return sum(v for st, v in bmap.items() if st != qmoe.STAGE_FUSED and tot_n[st])
    layer_bytes_step = float(np.mean([layer_step_bytes(per_x_bytes[s % n_x]) for s in range(steps)]))
    ms_per_step = 1e3 * elapsed / steps
    layer_gbs = layer_bytes_step / (elapsed / steps) / 1e9

    result = {
        "metric": "MoE-layer tokens/s (decode T=1, prefill T=2048) + % of HBM/MFMA roofline",
        "value": round(T * steps / elapsed, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if mfma_path else "f32",
        "data": "synthetic",
        "config": {
            "workload": desc, "tokens_per_step": T, "hidden": cfg.hidden, "n_experts": cfg.n_experts,
            "top_k": cfg.top_k, "moe_inter": cfg.moe_inter, "shared_inter": cfg.shared_inter,
            "select_scope": scope, "router_fmt": qmoe.FORMAT_NAMES[cfg.router_fmt],
            "expert_fmt": qmoe.FORMAT_NAMES[cfg.expert_fmt], "weight_copies": copies,
            "weight_bytes_per_copy": layer_total, "x_pool": n_x, "seed": args.seed,
            "path": "mfma" if mfma_path else "gemv",
        },
        "roofline": ({
            "bound": "mfma", "kernel": qmoe.STAGE_NAMES[dom], "achieved": round(mfma_tflops, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(mfma_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": measured_traffic(workload, qmoe.STAGE_NAMES[dom]),
            "flops_per_launch": int(dom_flops), "bytes_per_launch": int(dom_bytes),
            "avg_launch_us": round(dom_avg_s * 1e6, 3),
        } if mfma_bound else {
            "bound": "hbm", "kernel": qmoe.STAGE_NAMES[dom], "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(workload, qmoe.STAGE_NAMES[dom]),
            "bytes_per_launch": int(dom_bytes), "avg_launch_us": round(dom_avg_s * 1e6, 3),
        }),
        "mfma": ({"kernel": qmoe.STAGE_NAMES[dom], "flops_per_launch": int(dom_flops),
                  "achieved_tflops": round(mfma_tflops, 1), "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                  "util": round(mfma_tflops / MFMA_BF16_PEAK_TFLOPS, 4)} if mfma_path else None),
        "layer_roofline": {
            "bytes_per_step": int(layer_bytes_step), "achieved_gbs": round(layer_gbs, 1),
            "frac": round(layer_gbs / HBM_PEAK_GBS, 4), "stage_avg_us": stage_avg_us,
        },
    }
    fb = sum(L.router_fallbacks() for L in layers)
    rescued = sum(L.router_rescues() for L in layers)
    result["layer_roofline"]["router_fallbacks"] = {
        "tokens": int(fb), "rescued": int(rescued), "of_tokens": int(T * (n_x + warmup + steps)),
        "note": "tokens the certified decode router could not certify: rescued = settled by exact logits of "
                "the candidates in doubt; tokens = routed by the full exact path"}
    if skew:
        result["config"]["skew"] = {"target_max_over_median": skew["target_max_over_median"],
                                    "c": skew["per_x"][0]["c"], "max_load": skew["per_x"][0]["max_load"],
                                    "median_load": skew["per_x"][0]["median_load"],
                                    "experts_used": skew["per_x"][0]["experts_used"]}
    if not args.no_cpu_baseline:
        scope_for_oracle = scope
        result["cpu_baseline"] = cpu_baseline(hw, cfg, T, scope_for_oracle, xs_host, cpu_seconds)
    print(f"# {workload}: setup {gen_s:.1f}s, {copies} copies x {layer_total / 1e9:.2f} GB", file=sys.stderr)
    for L in layers:
        L.close()
    del layers, d_x, d_out, d_ids, d_w
    torch.cuda.empty_cache()
    return result


if __name__ == "__main__":
    main()
