#!/usr/bin/env python3
"""Benchmark of the gfx950 verify path on one MI355X.

Workload: one layer's int4 g128 projection set -- QKV-like 7168x5120,
O 5120x6144, fused gate/up 34816x5120, down 5120x17408, fp16 scale/min -- scored against
M = 8 verify rows (1 committed + 7 drafts), bf16 x ~ N(0, 1), synthetic seeded data.
A "step" is one pass over the layer set: 4 GEMM launches, each captured in a hipGraph.
Steps cycle through enough distinct weight copies (>= 1 GiB) that every step reads its
weights from HBM, not from the 256 MB MALL.

value = whole-job algorithmic bytes / wall time of the timed steps (GB/s), bytes per GEMM
  N*K/2 + 4*N*K/128 + 2*M*K + 2*M*N.
roofline: the dominant kernel (gate/up) -- its algorithmic bytes / its average duration
  measured with HIP events on the launch stream inside the timed region, vs 8 TB/s.
cpu_baseline: the CPU oracle (numpy dequantize + matmul, the reference's torch path
  restated) on one layer set at M = 8, single thread, on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "token-rush_amd"))

HBM_PEAK_GBS = 8000.0
LAYER_SET = [("qkv", 7168, 5120), ("o", 5120, 6144), ("gate_up", 34816, 5120), ("down", 5120, 17408)]
M_VERIFY = 8


def algo_bytes(N, K, M, out_bytes=2):
    return N * K // 2 + 4 * N * K // 128 + 2 * M * K + out_bytes * M * N


def make_layer_set(torch, gen, dev):
    ws = []
    for name, N, K in LAYER_SET:
        q = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=gen)
        s = (torch.rand(N, K // 128, device=dev, generator=gen) * 0.018 + 0.002).half()
        m = (torch.rand(N, K // 128, device=dev, generator=gen) * 0.14 - 0.15).half()
        ws.append((name, N, K, q, s, m))
    return ws


def time_config(torch, gfx950, copies, M, steps, warmup, dev, gen):
    """Returns (wall seconds for `steps` steps, {name: mean kernel ms}, bytes per step)."""
    xs = {K: torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16) for _, _, K in LAYER_SET}
    graphs = []         # graphs[c][i]: copy c, projection i
    for ws in copies:
        row = []
        for name, N, K, B, s, m in ws:
            y = gfx950.mul(xs[K], B, s, m)               # warm + allocate outside capture
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                y2 = gfx950.mul(xs[K], B, s, m)
            row.append((name, g, y2))
        graphs.append(row)
    torch.cuda.synchronize()
    C = len(graphs)
    for i in range(warmup):
        for _, g, _ in graphs[i % C]:
            g.replay()
    torch.cuda.synchronize()
    nproj = len(LAYER_SET)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(nproj + 1)] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        row = graphs[i % C]
        ev[i][0].record()
        for j, (_, g, _) in enumerate(row):
            g.replay()
            ev[i][j + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = {}
    for j, (name, _, _) in enumerate(graphs[0]):
        per[name] = sum(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(steps)) / steps
    step_bytes = sum(algo_bytes(N, K, M) for _, N, K in LAYER_SET)
    return wall, per, step_bytes


def cpu_baseline(M=M_VERIFY):
    """Oracle (numpy, single thread) dequantize + matmul over one layer set at M rows."""
    import numpy as np
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:     # pragma: no cover
        threadpool_limits = None
    sys.path.insert(0, ROOT)
    from oracle import int4 as o
    total_bytes, total_s = 0, 0.0
    ctx = threadpool_limits(1) if threadpool_limits else None
    try:
        for i, (name, N, K) in enumerate(LAYER_SET):
            p, s, m = o.make_weights(N, K, seed=300 + i, dtype="fp16")
            x = o.make_x(M, K, seed=400 + i)
            t0 = time.perf_counter()
            y = o.gemm_dequant(x, p, s, m, "fp16")
            total_s += time.perf_counter() - t0
            total_bytes += algo_bytes(N, K, M)
            del p, s, m, y
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    return {"value": round(total_bytes / total_s / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"one config-2 layer set (4 projections) at M={M}, numpy dequantize (two fp16 roundings) "
                      f"+ fp64 matmul, {total_s:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the verify path shards "
              "column/row-parallel by design, but only the one-GPU kernel is built and measured)", file=sys.stderr)
        sys.exit(2)

    import torch
    from tokenrush_amd import gfx950
    gfx950.ext()                                   # fail loudly if the library is missing
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    copy_bytes = sum(N * K // 2 + 4 * N * K // 128 for _, N, K in LAYER_SET)
    n_copies = max(2, -(-(1 << 30) // copy_bytes))  # >= 1 GiB of distinct weights
    copies = []
    for _ in range(n_copies):
        ws = make_layer_set(torch, gen, dev)
        copies.append([(name, N, K) + gfx950.pack(q, s, m) for name, N, K, q, s, m in ws])
        del ws
    torch.cuda.synchronize()

    wall8, per8, bytes8 = time_config(torch, gfx950, copies, M_VERIFY, a.steps, a.warmup, dev, gen)
    wall1, per1, bytes1 = time_config(torch, gfx950, copies, 1, a.steps, a.warmup, dev, gen)
    value = bytes8 * a.steps / wall8 / 1e9
    ms_step = wall8 * 1e3 / a.steps
    gu = dict((n, (N, K)) for n, N, K in LAYER_SET)["gate_up"]
    achieved = algo_bytes(gu[0], gu[1], M_VERIFY) / (per8["gate_up"] * 1e-3) / 1e9
    kern8 = sum(per8.values())
    kern1 = sum(per1.values())
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gate_up_m8_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
    out = {
        "metric": "int4 verify GEMM HBM GB/s (% of peak) at M=1,8; verify+accept step latency us",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4 weights x bf16 -> fp32 acc (fp16 scale/min), bf16 out", "data": "synthetic",
        "config": {"workload": "BASELINE config 2: one layer set (qkv 7168x5120, o 5120x6144, gate_up 34816x5120, "
                               "down 5120x17408) at M=8, weights cycled over %d copies" % n_copies,
                   "M": M_VERIFY, "parallelism": "none (1 GPU)"},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "kernel_us_m8": {k: round(v * 1e3, 2) for k, v in per8.items()},
        "kernel_us_m1": {k: round(v * 1e3, 2) for k, v in per1.items()},
        "kernel_gbs_m8": {n: round(algo_bytes(N, K, 8) / (per8[n] * 1e-3) / 1e9, 1) for n, N, K in LAYER_SET},
        "kernel_gbs_m1": {n: round(algo_bytes(N, K, 1) / (per1[n] * 1e-3) / 1e9, 1) for n, N, K in LAYER_SET},
        "value_m1": round(bytes1 * a.steps / wall1 / 1e9, 2),
        "m8_over_m1_kernel_time": round(kern8 / kern1, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "int4_gemm_kernel gate_up 34816x5120 M=8"},
    }
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
