#!/usr/bin/env python3
"""Benchmark of the gfx950 verify path on one MI355X.

Workload (benchmark config 2): one layer's int4 g128 projection set -- QKV-like 7168x5120,
O 5120x6144, fused gate/up 34816x5120, down 5120x17408, fp16 scale/min -- scored against
M = 8 verify rows (1 committed + 7 drafts), bf16 x ~ N(0, 1), synthetic seeded data. As in the
reference engine (weights.py:163-174, model.py:211-260), the hidden-sized outputs (O, down) are
produced as fp32 split-K partials (QLinear.partials) and the others as bf16 (QLinear.__call__).
A "step" is one pass over the layer set: 4 kernel launches captured in one hipGraph. Steps
cycle through enough distinct weight copies (>= 1 GiB) that every step reads its weights from
HBM, not from the 256 MB MALL.

value       whole-job algorithmic bytes / wall time of the timed steps (GB/s); bytes per GEMM
            N*K/2 + 4*N*K/128 + 2*M*K + (2*M*N bf16 out | 4*S*M*N fp32 partials).
roofline    the dominant kernel (gate/up, 53% of the bytes): its algorithmic bytes / its mean
            duration, measured with HIP events around a graph of back-to-back launches of that
            kernel alone over all weight copies, on the launch stream; vs 8 TB/s.
config1     benchmark config 1: a single 5120x5120 GEMV at M = 1 over >= 1 GiB of weight copies,
            mean us per launch, GB/s and % of 8 TB/s.
accept      on-device accept latency (benchmark config 3 and 4): mean per launch over a graph of
            back-to-back calls.
config5     one verify step of the random-init 64-layer hybrid at M = 8 (257 int4 GEMMs, split-K
            partial consumers, 48 GDN steps, 16 FP8 attention layers over 8192 live tokens, lm_head,
            greedy accept) captured as one hipGraph; time per replay and weight bytes / time.
config4     a seeded 32-node draft tree verified through the same model (tree mixers, M = 32
            GEMMs, lm_head, tree accept and commit), one hipGraph; time per replay.
cpu_baseline  the reference's CPU path restated in torch (unpack, in-place dequant, F.linear) on
            one layer set at M = 8, OMP_NUM_THREADS host cores, median of >= 5 passes
            (about 10 s).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "token-rush_amd"))

HBM_PEAK_GBS = 8000.0
# (name, N, K, partial): partial = the reference computes this projection as split-K partials
LAYER_SET = [("qkv", 7168, 5120, False), ("o", 5120, 6144, True), ("gate_up", 34816, 5120, False),
             ("down", 5120, 17408, True)]
M_VERIFY = 8
V = 248320


def algo_bytes(N, K, M, slots=None):
    out = 4 * slots * M * N if slots else 2 * M * N
    return N * K // 2 + 4 * N * K // 128 + 2 * M * K + out


def make_layer_set(torch, gfx950, gen, dev):
    ws = []
    for name, N, K, partial in LAYER_SET:
        q = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=gen)
        s = (torch.rand(N, K // 128, device=dev, generator=gen) * 0.018 + 0.002).half()
        m = (torch.rand(N, K // 128, device=dev, generator=gen) * 0.14 - 0.15).half()
        B, sv, _ = gfx950.pack(q, s, m)
        gfx950.workspaces(N, dev, K)
        ws.append((name, N, K, partial, B, sv))
        del q, s, m
    return ws


def call(gfx950, x, w):
    name, N, K, partial, B, sv = w
    return gfx950.mul_partial(x, B, sv) if partial else gfx950.mul(x, B, sv)


def graph_of(torch, fn):
    fn()                                           # warm up + allocate outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def timed_graph(torch, g, reps=3):
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e-3      # seconds per replay


def run_steps(torch, gfx950, copies, M, steps, warmup, gen, dev):
    """Wall seconds of `steps` layer-set steps, round robin over the weight copies, and of the same
    steps launched one graph per step. The steps are captured a pass over the copies at a time
    (C steps, 4 C launches, one hipGraph), as a serving loop captures many launches in one graph;
    steps beyond the last whole pass run from the one-step graphs."""
    xs = {K: torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16) for _, _, K, _ in LAYER_SET}
    graphs = [graph_of(torch, lambda c=c: [call(gfx950, xs[w[2]], w) for w in c]) for c in copies]
    C = len(graphs)
    gpass = graph_of(torch, lambda: [call(gfx950, xs[w[2]], w) for c in copies for w in c])

    def timed(passes):
        for i in range(warmup):
            graphs[i % C].replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        done = 0
        if passes:
            for _ in range(steps // C):
                gpass.replay()
            done = steps // C * C
        for i in range(done, steps):
            graphs[i % C].replay()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    wall_each = timed(False)
    wall = timed(True)
    del gpass
    return wall, wall_each, xs


def kernel_means(torch, gfx950, copies, xs, reps=4):
    """Mean seconds per launch of each projection: a graph of reps x copies back-to-back launches."""
    out = {}
    for j, (name, N, K, partial) in enumerate(LAYER_SET):
        g = graph_of(torch, lambda j=j, K=K: [call(gfx950, xs[K], c[j]) for _ in range(reps) for c in copies])
        out[name] = timed_graph(torch, g) / (reps * len(copies))
        del g
    return out


def config1_gemv(torch, gfx950, dev, reps=4):
    """benchmark config 1: one 5120x5120 int4 g128 GEMV at M = 1 (fp16 scale/min, x ~ N(0, 1)),
    cycled over >= 1 GiB of distinct weight copies so every launch reads HBM: mean microseconds per
    launch over a graph of back-to-back launches, GB/s of its algorithmic bytes, % of 8 TB/s."""
    N = K = 5120
    gen = torch.Generator(device=dev)
    gen.manual_seed(101)
    per = N * K // 2 + 4 * N * K // 128
    n_copies = -(-(1 << 30) // per)
    ws = []
    for _ in range(n_copies):
        q = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=gen)
        s = (torch.rand(N, K // 128, device=dev, generator=gen) * 0.018 + 0.002).half()
        m = (torch.rand(N, K // 128, device=dev, generator=gen) * 0.14 - 0.15).half()
        B, sv, _ = gfx950.pack(q, s, m)
        ws.append((B, sv))
    x = torch.randn(1, K, device=dev, generator=gen).to(torch.bfloat16)
    g = graph_of(torch, lambda: [gfx950.mul(x, B, sv) for _ in range(reps) for B, sv in ws])
    t = timed_graph(torch, g) / (reps * n_copies)
    del g, ws
    nbytes = algo_bytes(N, K, 1)
    return {"us": round(t * 1e6, 3), "GBps": round(nbytes / t / 1e9, 1),
            "pct_of_hbm_peak": round(100 * nbytes / t / 1e9 / HBM_PEAK_GBS, 2), "bytes": nbytes,
            "copies": n_copies, "note": "5120x5120 M=1 fp16 scale/min; mean per launch over a graph of "
                                        "%d back-to-back launches (launch gap included)" % (reps * n_copies)}


def accept_latency(torch, dev):
    """Mean microseconds per launch of the accept kernels at benchmark configs 3 and 4."""
    from tokenrush_amd.accept import AcceptState, accept_greedy, accept_residual, accept_sampled, accept_tree
    from tokenrush_amd.sample import SamplingParams, workspace
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    res = {}
    lg8 = (torch.randn(8, V, device=dev, generator=gen) * 2).to(torch.bfloat16)
    lg32 = (torch.randn(32, V, device=dev, generator=gen) * 2).to(torch.bfloat16)
    spec = torch.randint(0, V, (32,), device=dev, generator=gen)
    q = torch.softmax(torch.randn(7, V, device=dev, generator=gen) * 2, -1).contiguous()
    u = torch.rand(32, device=dev, generator=gen)
    parent = torch.tensor([-1] + [max(0, (i - 1) // 4) for i in range(1, 32)], dtype=torch.int32, device=dev)
    p = SamplingParams(dev)
    p.set(temperature=1.0, top_p=0.95, top_k=64)
    st8, st32 = AcceptState(8, dev), AcceptState(32, dev)
    workspace(32, V, dev)
    cases = {
        "greedy_m8": lambda: accept_greedy(lg8, spec, st8),
        "sampled_m8": lambda: accept_sampled(lg8, spec, p, st8, u[:8]),
        "residual_m8": lambda: accept_residual(lg8, q, spec, u[:8], st8),
        "tree_m32": lambda: accept_tree(lg32, spec, parent, st32),
    }
    reps = 20
    for name, fn in cases.items():
        g = graph_of(torch, lambda fn=fn: [fn() for _ in range(reps)])
        res[name] = round(timed_graph(torch, g) / reps * 1e6, 2)
        del g
    return res


def lm_head_accept(torch, dev, M=M_VERIFY, reps=8):
    """The verify tail of config 5: the 248320x5120 int4 lm_head at M rows with the accept, as
    (a) the greedy accept in the GEMM's epilogue, (b) the GEMM writing logits followed by the
    sampled accept kernel (temperature 1, top_p 0.95, top_k 64). Microseconds per call over a
    graph of back-to-back calls (launch gaps included)."""
    from tokenrush_amd.accept import AcceptState, accept_sampled, lm_head_greedy
    from tokenrush_amd.quant import QLinear
    from tokenrush_amd.sample import SamplingParams
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    K = 5120
    q = torch.randint(0, 256, (V, K // 2), dtype=torch.uint8, device=dev, generator=gen)
    s = (torch.rand(V, K // 128, device=dev, generator=gen) * 0.018 + 0.002).to(torch.bfloat16)
    m = (torch.rand(V, K // 128, device=dev, generator=gen) * 0.14 - 0.15).to(torch.bfloat16)
    lm = QLinear(q, s, m)
    del q, s, m
    hidden = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
    spec = torch.randint(0, V, (M,), device=dev, generator=gen)
    u = torch.rand(M, device=dev, generator=gen)
    p = SamplingParams(dev)
    p.set(temperature=1.0, top_p=0.95, top_k=64)
    st = AcceptState(M, dev)
    cases = {"greedy_fused": lambda: lm_head_greedy(lm, hidden, spec, st, keep_logits=True),
             "sampled": lambda: accept_sampled(lm(hidden), spec, p, st, u)}
    out = {}
    for name, fn in cases.items():
        g = graph_of(torch, lambda fn=fn: [fn() for _ in range(reps)])
        out[name] = round(timed_graph(torch, g) / reps * 1e6, 2)
        del g
    del lm
    torch.cuda.empty_cache()
    return out


def config5_step(torch, dev, M=M_VERIFY, reps=10, tree=True):
    """benchmark config 5: one verify step of the random-init 64-layer hybrid (48 GDN + 16 attention
    layers, int4 g128 weights, GDN steps and FP8 attention over 8192 live tokens) + lm_head + greedy
    accept/commit, captured as one hipGraph (tokenrush_amd.step). Returns the replay time and the
    weight-streaming rate; with tree, also config 4 through the same model (config4_tree_step)."""
    from tokenrush_amd.accept import AcceptState
    from tokenrush_amd.step import StepConfig, VerifyModel, prepare
    t0 = time.perf_counter()
    model = VerifyModel(StepConfig(tree_nodes=32 if tree else 0), device=dev, seed=5)
    prepare(model, M)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    x0 = torch.randn(M, model.cfg.hidden, device=dev, generator=gen).to(torch.bfloat16)
    spec = torch.randint(0, model.cfg.vocab, (M,), device=dev, generator=gen)
    st = AcceptState(M, dev)
    st.pos.fill_(model.cfg.live)               # the cache holds `live` tokens; the accept advances pos
    st.slot.zero_()
    g = graph_of(torch, lambda: model.step(x0, spec, st))
    build_s = time.perf_counter() - t0
    # each replay advances pos by at most M: the replays below stay inside the cache's headroom
    assert (reps + 3) * M <= model.cfg.headroom
    st.pos.fill_(model.cfg.live)
    t = timed_graph(torch, g, reps=reps)
    nbytes, state_bytes, live = model.nbytes(), model.state.nbytes(), model.cfg.live
    n_attn = sum(1 for li in range(model.cfg.n_layers) if model.cfg.is_attention(li))
    launches = (model.cfg.n_layers - n_attn) * 7 + n_attn * 9 + 2
    del g
    c4 = config4_tree_step(torch, dev, model, reps=reps) if tree else None
    del model
    torch.cuda.empty_cache()
    return c4, {"ms_per_step": round(t * 1e3, 3), "weights_GB": round(nbytes / 1e9, 3),
            "weight_GBps": round(nbytes / t / 1e9, 1), "launches": launches, "M": M, "replays": reps,
            "build_s": round(build_s, 1),
            "state_GB": round(state_bytes / 1e9, 3), "live_tokens": live,
            "note": "one hipGraph: 257 int4 GEMMs (the 64 gate/up with silu_mul in the epilogue), 129 add_rmsnorm "
                    "(split-K partial consumers), 48 GDN steps (conv ring, delta rule, 8 snapshot slots, gated norm), "
                    "16 attention layers (prep + FP8 flash-decoding split + combine) over 8192 live tokens, lm_head "
                    "248320x5120 with the greedy accept/commit in its epilogue"}


def _random_parent(n, seed, max_branch=4, max_depth=7):
    """A seeded draft tree: node 0 the root (-1); each later node hangs off a random earlier node
    with fewer than max_branch children and depth below max_depth."""
    import random
    rng = random.Random(seed)
    parent, depth, kids = [-1], [0], [0]
    for i in range(1, n):
        j = rng.choice([k for k in range(i) if kids[k] < max_branch and depth[k] < max_depth])
        parent.append(j)
        depth.append(depth[j] + 1)
        kids.append(0)
        kids[j] += 1
    return parent


def config4_tree_step(torch, dev, model, reps=10, M=32):
    """benchmark config 4 through the config-5 model: a seeded 32-node draft tree (branching <= 4,
    depth <= 7) verified by the 64-layer step with the tree mixers (ancestor-masked attention,
    per-node GDN states), M = 32 GEMMs, lm_head, tree accept and commit (KV rows, scales, conv
    rings), one hipGraph (VerifyModel.step_tree). The node tokens are planted from a first eager
    pass so that the deepest root path is accepted (its nodes hold their parents' argmax, every
    other node a different token): each timed replay then commits a real path. Each replay starts
    from the same restored decode state and is timed alone with HIP events on the launch stream."""
    import numpy as np
    from tokenrush_amd.accept import AcceptState
    from tokenrush_amd.step import prepare
    prepare(model, M)
    gen = torch.Generator(device=dev)
    gen.manual_seed(8)
    x0 = torch.randn(M, model.cfg.hidden, device=dev, generator=gen).to(torch.bfloat16)
    parent_l = _random_parent(M, seed=4)
    parent = torch.tensor(parent_l, dtype=torch.int32, device=dev)
    st = AcceptState(M, dev)
    snap = model.state.snapshot()

    def reset():
        model.state.restore(snap)
        st.pos.fill_(model.cfg.live)
        st.slot.zero_()

    reset()
    pred = model.lm_head(model.hidden(x0, st.pos, st.slot, parent)).float().argmax(-1).cpu().numpy()
    depth = [0] * M
    for i in range(1, M):
        depth[i] = depth[parent_l[i]] + 1
    node, path = int(np.argmax(depth)), []
    while node >= 0:
        path.append(node)
        node = parent_l[node]
    V = model.cfg.vocab
    toks_l = [7] + [(int(pred[parent_l[i]]) + 1) % V for i in range(1, M)]
    for i in path[:-1]:
        toks_l[i] = int(pred[parent_l[i]])
    toks = torch.tensor(toks_l, dtype=torch.int64, device=dev)
    reset()
    g = graph_of(torch, lambda: model.step_tree(x0, toks, parent, st))
    times, accepted = [], []
    stream = torch.cuda.current_stream()
    for _ in range(reps + 1):
        reset()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e-3)
        accepted.append(int(st.n_accepted))
    times, accepted = times[1:], accepted[1:]          # the first replay warms up
    del g, snap
    t = sum(times) / len(times)
    return {"ms_per_step": round(t * 1e3, 3), "M": M, "replays": reps,
            "accepted_depth": sorted(set(accepted)), "planted_depth": len(path) - 1,
            "note": "one hipGraph: 257 int4 GEMMs at M=32 (the 64 gate/up GEMMs then slot_sum_kernel for their two K slots and silu), tree GDN steps (per-node state, 32 snapshot slots), "
                    "ancestor-masked FP8 attention over 8192 live tokens, lm_head 248320x5120 writing logits, tree "
                    "accept, commit of KV rows/scales (4 launches) and conv rings (1 launch); node tokens planted "
                    "along the deepest root path, each replay from the same restored state"}


TL_MARKS = {0: "entry", 1: "launch constants", 21: "activation loads issued", 22: "past the ordering barrier",
            3: "first two strips issued", 2: "activations staged",
            4: "prologue end", 5: "strip 0 MACs", 6: "strip 1 MACs", 7: "strip 2 MACs", 8: "strip 3 MACs",
            9: "strip 4 MACs", 10: "strip 5 MACs", 16: "batch reduced (last)", 20: "strip loop exit",
            19: "slot-sum arrival (K slots > 1)", 23: "slot sum done (last arriver)"}


def gemm_timeline(torch, gfx950, dev, name, M=M_VERIFY, launches=6):
    """The in-kernel timeline of one projection's GEMM (a -DTR_TIMELINE build of the library,
    named by TOKENRUSH_HIP_LIB): s_memrealtime stamps per wave at fixed points, one launch at a time
    on weights not read before (HBM, not cache). Returns per-mark percentiles (0, 10, 50, 90, 100)
    over the launch's waves, in us from the launch's first wave entry."""
    import ctypes
    import numpy as np
    from tokenrush_amd import _lib
    lib = _lib.lib()
    if not hasattr(lib, "tr_gemm_timeline"):
        raise SystemExit("--timeline needs TOKENRUSH_HIP_LIB=token-rush_amd/tokenrush_amd/libtrhip_timeline.so "
                         "(make -C token-rush_amd/csrc timeline)")
    lib.tr_gemm_timeline.restype = ctypes.c_void_p
    lib.tr_gemm_timeline.argtypes = [ctypes.POINTER(ctypes.c_size_t)]
    nbytes = ctypes.c_size_t(0)
    buf = lib.tr_gemm_timeline(ctypes.byref(nbytes))
    hip = ctypes.CDLL("libamdhip64.so")
    j = [n for n, _, _, _ in LAYER_SET].index(name)
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    copies = [make_layer_set(torch, gfx950, gen, dev)[j] for _ in range(launches + 1)]
    x = torch.randn(M, LAYER_SET[j][2], device=dev, generator=gen).to(torch.bfloat16)
    call(gfx950, x, copies[-1])                      # first call: workspaces, code load
    torch.cuda.synchronize()
    host = np.zeros(nbytes.value // 8, dtype=np.uint64)
    stamps = {k: [] for k in TL_MARKS}
    spans = []
    for c in copies[:launches]:
        hip.hipMemset(ctypes.c_void_p(buf), 0, ctypes.c_size_t(nbytes.value))
        hip.hipDeviceSynchronize()
        call(gfx950, x, c)
        torch.cuda.synchronize()
        hip.hipMemcpy(ctypes.c_void_p(host.ctypes.data), ctypes.c_void_p(buf), ctypes.c_size_t(nbytes.value), 2)
        t = host.reshape(-1, 16, 24).astype(np.int64)
        live = t[:, :, 0] > 0
        t0 = t[:, :, 0][live].min()
        for k in TL_MARKS:
            v = t[:, :, k][live & (t[:, :, k] > 0)]
            stamps[k].extend(((v - t0) / 100.0).tolist())
        spans.append((t[:, :, 20][live].max() - t0) / 100.0)
    pct = {TL_MARKS[k]: [round(float(q), 2) for q in np.percentile(v, [0, 10, 50, 90, 100])]
           for k, v in stamps.items() if v}
    return {"timeline": name, "M": M, "launches": launches, "workgroups_x_waves": int(len(stamps[0]) / launches),
            "us_from_first_entry_p0_p10_p50_p90_p100": pct, "last_wave_exit_us": [round(s_, 2) for s_ in spans],
            "note": "one launch at a time on weights not read before; stamps by lane 0 of each wave (100 MHz)"}


def cpu_baseline(M=M_VERIFY, min_reps=5, budget_s=10.0):
    """The reference's CPU path restated (oracle.int4.torch_dequant_linear: torch unpack, in-place
    fp16 dequant, F.linear in bf16) over one layer set at M rows on the host's CPU share; median of
    the timed passes (at least `min_reps`, then until `budget_s` seconds) after one warm-up pass."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import int4 as o
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)   # the host's CPU share
    torch.set_num_threads(cores)
    layers = []
    for i, (name, N, K, partial) in enumerate(LAYER_SET):
        p, s, m = o.make_weights(N, K, seed=300 + i, dtype="fp16")
        x = o.make_x(M, K, seed=400 + i)
        layers.append((torch.from_numpy(x).to(torch.bfloat16), torch.from_numpy(p),
                       torch.from_numpy(s).half(), torch.from_numpy(m).half(), algo_bytes(N, K, M)))
    total_bytes = sum(L[-1] for L in layers)
    times, r = [], 0
    while r <= min_reps or sum(times) < budget_s:
        t0 = time.perf_counter()
        for x, p, s, m, _ in layers:
            o.torch_dequant_linear(x, p, s, m)
        if r:
            times.append(time.perf_counter() - t0)
        r += 1
    t = float(np.median(times))
    return {"value": round(total_bytes / t / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"one config-2 layer set (4 projections, 178 MB int4 weights) at M={M}: torch CPU "
                      f"unpack + in-place fp16 dequant + bf16 F.linear on {cores} threads, median of {len(times)} "
                      f"passes ({t * 1e3:.0f} ms each, {sum(times):.1f} s timed)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-config5", action="store_true", help="skip the 64-layer verify-step graph (config 5)")
    ap.add_argument("--rows", type=int, default=M_VERIFY,
                    help="profiling aid: the verify rows M of --only <projection | layer_set> (1..32)")
    ap.add_argument("--only", choices=[n for n, _, _, _ in LAYER_SET] + ["layer_set", "config5", "config4", "config1",
                                                                       "lm_head", "accept"],
                    help="profiling aid: run just this projection's launches (M=8), or the config-5 step graph, and exit")
    ap.add_argument("--timeline", choices=[n for n, _, _, _ in LAYER_SET],
                    help="profiling aid: the in-kernel timeline of this projection's GEMM at M=8 (needs the "
                         "TR_TIMELINE build named by TOKENRUSH_HIP_LIB)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="profiling aid: run a plain 1 GiB device copy (read 1 GiB, write 1 GiB) and exit")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (how the verify path would "
              "shard is a design note; only the one-GPU kernels are built and measured)", file=sys.stderr)
        sys.exit(2)

    import torch
    from tokenrush_amd import gfx950
    gfx950.ext()                                   # fail loudly if the library is missing
    dev = torch.device("cuda:0")
    if a.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4}))
        return
    if a.timeline:
        print(json.dumps(gemm_timeline(torch, gfx950, dev, a.timeline)))
        return
    if a.only == "accept":
        print(json.dumps({"accept_us": accept_latency(torch, dev)}))
        return
    if a.only == "lm_head":
        print(json.dumps({"lm_head_accept_us_m8": lm_head_accept(torch, dev)}))
        return
    if a.only == "config1":
        print(json.dumps({"config1_gemv_m1": config1_gemv(torch, gfx950, dev)}))
        return
    if a.only in ("config5", "config4"):
        c4, c5 = config5_step(torch, dev, reps=max(1, a.steps // 30), tree=a.only == "config4")
        print(json.dumps({"config5_verify_step": c5, "config4_tree_step": c4}))
        return
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    copy_bytes = sum(N * K // 2 + 4 * N * K // 128 for _, N, K, _ in LAYER_SET)
    n_copies = max(2, -(-(1 << 30) // copy_bytes))  # >= 1 GiB of distinct weights
    copies = [make_layer_set(torch, gfx950, gen, dev) for _ in range(n_copies)]
    torch.cuda.synchronize()

    if a.only:
        if not 1 <= a.rows <= 32:
            raise SystemExit("--rows must be 1..32")
        js = range(len(LAYER_SET)) if a.only == "layer_set" else [[n for n, _, _, _ in LAYER_SET].index(a.only)]
        xs = {K: torch.randn(a.rows, K, device=dev, generator=gen).to(torch.bfloat16) for _, _, K, _ in LAYER_SET}
        for _ in range(max(1, a.steps // n_copies)):
            for c in copies:
                for j in js:
                    call(gfx950, xs[LAYER_SET[j][2]], c[j])
        torch.cuda.synchronize()
        print(json.dumps({"only": a.only, "rows": a.rows, "launches": max(1, a.steps // n_copies) * n_copies * len(js)}))
        return

    slots = {name: (gfx950.partial_slots(N, K, M_VERIFY) if partial else None) for name, N, K, partial in LAYER_SET}
    step_bytes = {M: sum(algo_bytes(N, K, M, slots[n]) for n, N, K, _ in LAYER_SET) for M in (1, 8)}

    wall8, wall8_each, xs8 = run_steps(torch, gfx950, copies, M_VERIFY, a.steps, a.warmup, gen, dev)
    k8 = kernel_means(torch, gfx950, copies, xs8)
    wall1, _, xs1 = run_steps(torch, gfx950, copies, 1, a.steps, a.warmup, gen, dev)
    k1 = kernel_means(torch, gfx950, copies, xs1)
    sweep = {}
    for M in (2, 4, 16, 32):
        xsM = {K: torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16) for _, _, K, _ in LAYER_SET}
        sweep[M] = round(sum(kernel_means(torch, gfx950, copies, xsM, reps=2).values()) * 1e6, 2)
    acc = accept_latency(torch, dev)
    del copies
    torch.cuda.empty_cache()
    c1 = config1_gemv(torch, gfx950, dev)
    lmh = lm_head_accept(torch, dev)
    torch.cuda.empty_cache()
    c4, c5 = (None, None) if a.no_config5 else config5_step(torch, dev)

    value = step_bytes[8] * a.steps / wall8 / 1e9
    gu = dict((n, (N, K)) for n, N, K, _ in LAYER_SET)["gate_up"]
    achieved = algo_bytes(gu[0], gu[1], M_VERIFY) / k8["gate_up"] / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gate_up_m8_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
    busy = {}
    bpath = os.path.join(ROOT, "profiles", "gate_up_m8_mfma_valu.json")
    if os.path.exists(bpath):   # rocprofv3 MfmaUtil / VALUBusy of the same kernel (a separate counter run)
        busy = {k: v for k, v in json.load(open(bpath)).items() if k.endswith("_pct")}
    out = {
        "metric": "int4 verify GEMM HBM GB/s (% of peak) at M=1,8; verify+accept step latency us",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(wall8 * 1e3 / a.steps, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4 x bf16 -> fp32 acc (fp16 scale/min)", "data": "synthetic",
        "config": {"workload": "benchmark config 2: one layer set (qkv 7168x5120, o 5120x6144 partials, gate_up "
                               "34816x5120, down 5120x17408 partials), M=8, weights cycled over %d copies (%.2f GB)"
                               % (n_copies, n_copies * copy_bytes / 1e9), "M": M_VERIFY, "parallelism": "none"},
        "launch": "steps captured %d at a time (one pass over the weight copies) in one hipGraph" % n_copies,
        "ms_per_step_one_graph_each": round(wall8_each * 1e3 / a.steps, 5),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "value_m1": round(step_bytes[1] * a.steps / wall1 / 1e9, 2),
        "kernel_us_m8": {k: round(v * 1e6, 2) for k, v in k8.items()},
        "kernel_us_m1": {k: round(v * 1e6, 2) for k, v in k1.items()},
        "kernel_gbs_m8": {n: round(algo_bytes(N, K, 8, slots[n]) / k8[n] / 1e9, 1) for n, N, K, _ in LAYER_SET},
        "m8_over_m1": round(sum(k8.values()) / sum(k1.values()), 4),
        "layer_set_us_by_M": {1: round(sum(k1.values()) * 1e6, 2), 8: round(sum(k8.values()) * 1e6, 2), **sweep},
        "accept_us": acc,
        "verify_accept_us_m8": round(sum(k8.values()) * 1e6 + acc["greedy_m8"], 2),
        # one layer set's GEMMs at the config's M plus its accept: configs 3 (M = 8, greedy /
        # sampled / residual) and 4 (M = 32 tree)
        "verify_accept_us": {"greedy_m8": round(sum(k8.values()) * 1e6 + acc["greedy_m8"], 2),
                             "sampled_m8": round(sum(k8.values()) * 1e6 + acc["sampled_m8"], 2),
                             "residual_m8": round(sum(k8.values()) * 1e6 + acc["residual_m8"], 2),
                             "tree_m32": round(sweep.get(32, float("nan")) + acc["tree_m32"], 2)},
        "config1_gemv_m1": c1,
        "lm_head_accept_us_m8": lmh,
        "config5_verify_step": c5,
        "config4_tree_step": c4,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "int4_gemm_kernel gate_up 34816x5120 M=8 (%.2f us)" % (k8["gate_up"] * 1e6), **busy},
    }
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
