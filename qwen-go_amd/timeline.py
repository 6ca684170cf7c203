#!/usr/bin/env python3
"""Phase timeline of the decode kernel (T = 1) from the instrumented library.

Build it first (make -C qwen-go_amd libqmoe_timeline.so): the same sources with
-DQMOE_TIMELINE, where every workgroup of the decode kernel records
s_memrealtime (100 MHz) at fixed points.  This script loads that library in
place of libqmoe.so, runs the named layers at decode with their weights in
several rotated copies (as bench.py does), and prints, per point, the median /
min / max over workgroups of the time since the earliest workgroup started,
averaged over a few calls.

  python qwen-go_amd/timeline.py [qwen3_30b_a3b qwen3_30b_a3b_int8 qwen3_next]
"""
import ctypes
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

STAMPS = 16
MAX_BLOCKS = 4096
POINTS = {
    0: "start (wave 0)", 1: "start (wave 1)", 2: "router partials published (wave 1)",
    3: "all router words seen (control wave)", 4: "selection certified (control wave)",
    5: "first tentative expert known (wave 1)", 12: "first tentative expert known (wave 7)",
    6: "burst rows landed (wave 1)", 13: "burst rows landed (wave 7)",
    7: "rows done (wave 1)", 14: "rows done (wave 7)",
    8: "out initialised everywhere (control wave)", 9: "block barrier (control wave)",
    10: "atomics into out done (control wave)",
}


def run(key, samples=20, warmup=50):
    import torch
    import qmoe
    cfg = qmoe.CONFIGS[key].with_(select_scope=qmoe.CONFIGS[key].n_experts)
    hw = qmoe.synthetic_weights(cfg, 2026)
    lb = qmoe.layer_bytes(cfg)
    step_bytes = lb["router"] + cfg.top_k * lb["per_expert"] + lb["shared"]
    copies = max(1, min(32, math.ceil(2 * 256e6 / step_bytes) + 1))
    layers = []
    for _ in range(copies):
        L = qmoe.MoeLayer(cfg)
        hw.upload(L)
        layers.append(L)
    x = torch.from_numpy(qmoe.synthetic_tokens(cfg, 1, 3026)).cuda()
    out = torch.empty_like(x)
    sptr = torch.cuda.current_stream().cuda_stream
    lib = qmoe.load_library()
    lib.qmoe_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.qmoe_timeline_read.restype = ctypes.c_int
    buf = np.zeros(MAX_BLOCKS * STAMPS, np.uint64)
    for s in range(warmup):
        layers[s % copies].forward_device(x.data_ptr(), 1, out.data_ptr(), None, None, sptr)
    torch.cuda.synchronize()
    acc = {i: [] for i in POINTS}
    kernel_us = []
    for s in range(samples):
        L = layers[s % copies]
        L.profile_enable([qmoe.STAGE_FUSED])
        L.profile_read(reset=True)
        L.forward_device(x.data_ptr(), 1, out.data_ptr(), None, None, sptr)
        torch.cuda.synchronize()
        ms, n = L.profile_read(reset=True)
        L.profile_enable([])
        kernel_us.append(1e3 * ms[qmoe.STAGE_FUSED] / max(n[qmoe.STAGE_FUSED], 1))
        if lib.qmoe_timeline_read(buf.ctypes.data, buf.size) != 0:
            raise RuntimeError("qmoe_timeline_read failed")
        st = buf.reshape(MAX_BLOCKS, STAMPS).astype(np.int64)
        s0 = st[:, 0]
        latest = s0.max()
        valid = s0 >= latest - 10000  # this call's workgroups (stamps of 100 us back at most)
        t0 = s0[valid].min()
        for i in POINTS:
            v = st[valid, i]
            ok = (v >= s0[valid]) & (v <= s0[valid] + 100000)
            if ok.any():
                us = (v[ok] - t0) / 100.0
                acc[i].append((np.median(us), us.min(), us.max(), int(ok.sum())))
    for L in layers:
        L.close()
    res = {"kernel_us": round(float(np.mean(kernel_us)), 2), "copies": copies, "samples": samples, "phases_us": {}}
    for i, name in POINTS.items():
        if acc[i]:
            a = np.array(acc[i])
            res["phases_us"][name] = {"p50": round(float(a[:, 0].mean()), 2), "min": round(float(a[:, 1].mean()), 2),
                                      "max": round(float(a[:, 2].mean()), 2), "workgroups": int(a[:, 3].mean())}
    return res


def main(argv):
    import torch
    torch.cuda.init()  # torch's HIP runtime before the library loads
    import qmoe
    path = os.path.join(HERE, "libqmoe_timeline.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} is missing: make -C qwen-go_amd libqmoe_timeline.so")
    qmoe.load_library(path)
    keys = argv or ["qwen3_30b_a3b", "qwen3_30b_a3b_int8", "qwen3_next"]
    for key in keys:
        r = run(key)
        print(f"== {key}: decode kernel {r['kernel_us']} us (mean of {r['samples']} calls, {r['copies']} weight copies)")
        print(f"   {'point':44s} {'p50':>7s} {'min':>7s} {'max':>7s}  workgroups  (us since the first start)")
        for name, v in sorted(r["phases_us"].items(), key=lambda kv: kv[1]["p50"]):
            print(f"   {name:44s} {v['p50']:7.2f} {v['min']:7.2f} {v['max']:7.2f}  {v['workgroups']:10d}")
        print(json.dumps({key: r}), file=sys.stderr)
        sys.stdout.flush()


if __name__ == "__main__":
    main(sys.argv[1:])
