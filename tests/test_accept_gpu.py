"""Parity of the on-device accept/commit kernels with the CPU oracle (oracle/accept.py), called
through the C-ABI (tokenrush_amd.sample / tokenrush_amd.accept -> libtrhip.so). Token ids,
accepted lengths, positions and commit indices must be bit-exact. Covers benchmark configs 3-4
at full size (V = 248320), ragged and tiny vocabularies, ties, every draft prefix length,
graph replay and repeated calls (the workspace counters reset themselves)."""
import numpy as np
import pytest
import torch

from oracle import accept as oa
from oracle.int4 import f32_to_bf16_bits

pytestmark = pytest.mark.gpu
F = np.float32
V_FULL = 248320


def say(*a):
    print(*a, flush=True)


def dev_logits(lg: np.ndarray) -> torch.Tensor:
    bits = f32_to_bf16_bits(lg).view(np.int16)
    return torch.from_numpy(bits).to("cuda:0").view(torch.bfloat16)


def state(M, pos=0):
    from tokenrush_amd.accept import AcceptState
    st = AcceptState(M, "cuda:0")
    st.pos.fill_(pos)
    return st


def check_state(st, ref, M):
    torch.cuda.synchronize()
    n = ref["n"]
    assert int(st.n_accepted) == n, (int(st.n_accepted), n)
    assert int(st.tok) == ref["tok"] and int(st.pos) == ref["pos"] and int(st.slot) == ref["slot"]
    toks = st.tokens.cpu().tolist()
    com = st.commit.cpu().tolist()
    assert toks[:n + 1] == ref["tokens"] and all(t == -1 for t in toks[n + 1:M])
    assert com[:n + 1] == ref["commit"] and all(c == -1 for c in com[n + 1:M])


@pytest.mark.parametrize("M,V", [(8, V_FULL), (32, V_FULL), (3, 1000), (1, 64), (5, 4097), (2, 262144)])
def test_argmax_rows(dev, M, V):
    from tokenrush_amd import _lib
    from tokenrush_amd.sample import workspace
    say(f"argmax M={M} V={V}")
    lg = oa.planted_logits(M, V, seed=M + V)
    lg[0, V // 3] = lg[0, V // 2] = lg[0].max() + 4              # tie: first index wins
    x = dev_logits(lg)
    pred = torch.empty(M, dtype=torch.long, device=dev)
    ws = workspace(M, V, dev)
    for _ in range(3):
        _lib.check(_lib.lib().tr_argmax_rows(_lib.ptr(x), M, V, _lib.ptr(ws), ws.numel(), _lib.ptr(pred),
                                             _lib.stream_of(x)), "argmax")
        assert np.array_equal(pred.cpu().numpy(), oa.argmax_rows(lg))


@pytest.mark.parametrize("prefix", range(8))
def test_accept_greedy_config3(dev, prefix):
    """benchmark config 3 greedy: 7 drafts, argmax planted on a prefix of length 0..7."""
    from tokenrush_amd.accept import accept_greedy
    say(f"greedy prefix={prefix}")
    rng = np.random.default_rng(prefix)
    spec = rng.integers(0, V_FULL, 8).astype(np.int64)
    lg = oa.planted_logits(8, V_FULL, seed=100 + prefix, drafts_from=spec, prefix=prefix)
    st = state(8, pos=1000)
    accept_greedy(dev_logits(lg), torch.from_numpy(spec).to(dev), st)
    check_state(st, oa.verify_chain(oa.argmax_rows(lg), spec, pos=1000), 8)
    assert np.array_equal(st.pred.cpu().numpy(), oa.argmax_rows(lg))


@pytest.mark.parametrize("T,top_p,top_k", [(0.0, 1.0, 64), (1.0, 1.0, 64), (0.7, 0.9, 64), (1.5, 0.95, 40),
                                           (1.0, 1.0, 3), (0.05, 1.0, 64)])
def test_sample_config3_rows(dev, T, top_p, top_k):
    from tokenrush_amd.sample import SamplingParams, sample
    say(f"sample T={T} top_p={top_p} top_k={top_k}")
    lg = oa.planted_logits(8, V_FULL, seed=7)                    # bf16 N(0, 4): many ties in the top 64
    x = dev_logits(lg)
    p = SamplingParams(dev)
    p.set(temperature=T, top_p=top_p, top_k=top_k)
    rng = np.random.default_rng(8)
    for trial in range(6):
        u = rng.random(8).astype(F)
        got = sample(x, p, torch.from_numpy(u).to(dev)).cpu().numpy()
        assert np.array_equal(got, oa.sample(lg, T, top_p, top_k, u)), trial


def test_sample_heavy_ties_full_vocab(dev):
    """Integer-valued logits at V = 248320: thousands of equal values around every chunk's and
    row's 64th largest, so the threshold selects overflow and both exact fallbacks (the radix
    select per chunk, the bitonic list merge per row) run; a second set mixes a tied row with
    continuous ones."""
    from tokenrush_amd.sample import SamplingParams, sample
    say("sample heavy ties")
    rng = np.random.default_rng(31)
    lg = np.round(rng.standard_normal((8, V_FULL))).astype(F)
    lg[4:] = oa.planted_logits(4, V_FULL, seed=32)
    x = dev_logits(lg)
    p = SamplingParams(dev)
    for T, top_p, top_k in ((1.0, 1.0, 64), (0.8, 0.9, 50), (0.0, 1.0, 64)):
        p.set(temperature=T, top_p=top_p, top_k=top_k)
        u = rng.random(8).astype(F)
        got = sample(x, p, torch.from_numpy(u).to(dev)).cpu().numpy()
        assert np.array_equal(got, oa.sample(lg, T, top_p, top_k, u)), (T, top_p, top_k)


def test_sample_small_and_peaked(dev):
    """The reference's test_sample.py:75-88 rows plus a vocabulary smaller than a chunk."""
    from tokenrush_amd.sample import SamplingParams, sample
    say("sample small")
    lg = np.zeros((4, 1000), F)
    lg[0, 5] = lg[1, 7] = lg[2, 9] = lg[3, 11] = 20.0
    x = dev_logits(lg)
    p = SamplingParams(dev)
    for T in (1.0, 0.0):
        p.set(temperature=T)
        assert sample(x, p, torch.rand(4, device=dev)).tolist() == [5, 7, 9, 11]
    lg2 = oa.planted_logits(3, 700, seed=9)
    u = np.array([0.1, 0.5, 0.999], F)
    p.set(temperature=1.0, top_p=0.8, top_k=20)
    assert np.array_equal(sample(dev_logits(lg2), p, torch.from_numpy(u).to(dev)).cpu().numpy(),
                          oa.sample(lg2, 1.0, 0.8, 20, u))


@pytest.mark.parametrize("T", [0.0, 1.0])
def test_accept_sampled_chain(dev, T):
    """Engine._verify_step with sampling (model.py:302-312): pred = sample(), leading matches."""
    from tokenrush_amd.accept import accept_sampled
    from tokenrush_amd.sample import SamplingParams
    say(f"accept sampled T={T}")
    p = SamplingParams(dev)
    p.set(temperature=T, top_p=1.0, top_k=64)
    for seed in range(4):
        rng = np.random.default_rng(seed)
        spec = rng.integers(0, V_FULL, 8).astype(np.int64)
        lg = oa.planted_logits(8, V_FULL, seed=200 + seed, drafts_from=spec, prefix=2 * seed)
        for i in range(2 * seed):                                  # make the planted token dominant
            lg[i, spec[i + 1]] = 60.0
        u = rng.random(8).astype(F)
        st = state(8, pos=50)
        accept_sampled(dev_logits(lg), torch.from_numpy(spec).to(dev), p, st, torch.from_numpy(u).to(dev))
        pred = oa.sample(lg, T, 1.0, 64, u)
        check_state(st, oa.verify_chain(pred, spec, pos=50), 8)
        assert np.array_equal(st.pred.cpu().numpy(), pred)


def _draft_probs(K, V, seed):
    rng = np.random.default_rng(seed)
    ql = rng.standard_normal((K, V)) * 2.0
    e = np.exp(ql - ql.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(F)


@pytest.mark.parametrize("seed", range(6))
def test_accept_residual_config3(dev, seed):
    """benchmark config 3 stochastic: 7 drafts, q = softmax of N(0, 4) logits, u [8] given."""
    from tokenrush_amd.accept import accept_residual
    say(f"residual seed={seed}")
    rng = np.random.default_rng(300 + seed)
    K = 7
    q = _draft_probs(K, V_FULL, seed)
    spec = rng.integers(0, V_FULL, K + 1).astype(np.int64)
    lg = oa.planted_logits(K + 1, V_FULL, seed=400 + seed, drafts_from=spec, prefix=seed)
    for i in range(seed):                                          # make drafts likely under p
        lg[i, spec[i + 1]] = 30.0
    u = rng.random(K + 1).astype(F)
    ref = oa.residual_accept(lg, q, spec[1:], u, pos=7)
    st = state(8, pos=7)
    accept_residual(dev_logits(lg), torch.from_numpy(q).to(dev), torch.from_numpy(spec).to(dev),
                    torch.from_numpy(u).to(dev), st)
    check_state(st, ref, 8)


def test_accept_residual_config3_drafts_from_q(dev):
    """240 draws at the full vocabulary (V = 248320): q a perturbed copy of the target's own
    distribution, drafts drawn from q, uniforms drawn fresh, so acceptance, rejection near the
    u q < p boundary and the residual resample all run at full width (every accepted length
    0..7 occurs)."""
    from tokenrush_amd.accept import accept_residual
    say("residual config 3, drafts drawn from q")
    K, V = 7, V_FULL
    rng = np.random.default_rng(77)
    lg = oa.planted_logits(K + 1, V, seed=78)
    z = lg[:K].astype(np.float64) + rng.standard_normal((K, V)) * 0.7
    e = np.exp(z - z.max(-1, keepdims=True))
    q = (e / e.sum(-1, keepdims=True)).astype(F)
    cdf = np.cumsum(q.astype(np.float64), -1)
    x, qd = dev_logits(lg), torch.from_numpy(q).to(dev)
    cache, seen = {}, set()
    st = state(8, pos=0)
    for trial in range(240):
        spec = np.zeros(K + 1, np.int64)
        spec[0] = trial
        spec[1:] = [min(int(np.searchsorted(cdf[i], rng.random() * cdf[i, -1])), V - 1) for i in range(K)]
        u = rng.random(K + 1).astype(F)
        st.pos.fill_(trial)
        st.slot.fill_(0)
        accept_residual(x, qd, torch.from_numpy(spec).to(dev), torch.from_numpy(u).to(dev), st)
        ref = oa.residual_accept(lg, q, spec[1:], u, pos=trial, cache=cache)
        check_state(st, ref, 8)
        seen.add(ref["n"])
    assert seen == set(range(K + 1)), seen


def test_accept_residual_small_vocab_many_draws(dev):
    """Many draws on a small vocabulary (bonus row, residual rows, p == q edge) against the oracle."""
    from tokenrush_amd.accept import accept_residual
    say("residual small")
    V, K = 3000, 3
    rng = np.random.default_rng(11)
    lg = oa.planted_logits(K + 1, V, seed=12)
    q = _draft_probs(K, V, 13)
    x, qd = dev_logits(lg), torch.from_numpy(q).to(dev)
    for trial in range(40):
        spec = rng.integers(0, V, K + 1).astype(np.int64)
        if trial % 4 == 0:
            spec[1:] = oa.argmax_rows(lg)[:K]                      # drafts the target likes
        u = rng.random(K + 1).astype(F)
        st = state(4, pos=trial)
        accept_residual(x, qd, torch.from_numpy(spec).to(dev), torch.from_numpy(u).to(dev), st)
        check_state(st, oa.residual_accept(lg, q, spec[1:], u, pos=trial), 4)


@pytest.mark.parametrize("seed", range(5))
def test_accept_tree_config4(dev, seed):
    """benchmark config 4: 32-node tree (branching <= 4, depth <= 7), logits [32, V]."""
    from tokenrush_amd.accept import accept_tree
    say(f"tree seed={seed}")
    parent = oa.random_tree(32, seed=seed)
    rng = np.random.default_rng(500 + seed)
    toks = rng.integers(0, V_FULL, 32).astype(np.int64)
    lg = oa.planted_logits(32, V_FULL, seed=600 + seed)
    # plant a path: pick a deep node, make each ancestor row predict the next node's token
    depth = oa.tree_depths(parent)
    node = int(np.argmax(depth)) if seed % 2 == 0 else int(rng.integers(1, 32))
    j = node
    while j > 0:
        lg[parent[j], toks[j]] = 50.0
        j = parent[j]
    st = state(32, pos=123)
    accept_tree(dev_logits(lg), torch.from_numpy(toks).to(dev), torch.from_numpy(parent).to(dev), st)
    ref = oa.tree_accept(oa.argmax_rows(lg), toks, parent, pos=123)
    check_state(st, ref, 32)
    assert ref["n"] >= depth[node]


@pytest.mark.parametrize("M", [1, 2, 5, 17, 32])
@pytest.mark.parametrize("shape", ["chain", "star", "random"])
def test_accept_tree_shapes(dev, M, shape):
    """Tree accept over shapes the config-4 trees do not reach: a chain M - 1 deep (all
    accepted, and cut at a random node), a star (depth-1 ties: the lowest index wins) and random
    trees where most nodes are accepted (many equal-depth accepted leaves)."""
    from tokenrush_amd.accept import accept_tree
    V = 4096
    rng = np.random.default_rng(1000 * M + len(shape))
    for trial in range(6):
        say(f"tree {shape} M={M} trial={trial}")
        if shape == "chain":
            parent = np.arange(-1, M - 1, dtype=np.int64)
        elif shape == "star":
            parent = np.array([-1] + [0] * (M - 1), dtype=np.int64)
        else:
            parent = np.array([-1] + [int(rng.integers(0, i)) for i in range(1, M)], dtype=np.int64)
        lg = oa.planted_logits(M, V, seed=2000 + 10 * M + trial)
        pred = oa.argmax_rows(lg)
        toks = rng.integers(0, V, M).astype(np.int64)
        for i in range(1, M):  # accept most nodes: node i's token is its parent's prediction
            if rng.random() < (0.9 if trial % 2 == 0 else 0.6):
                toks[i] = pred[parent[i]]
        st = state(M, pos=7 + trial)
        accept_tree(dev_logits(lg), torch.from_numpy(toks).to(dev), torch.from_numpy(parent.astype(np.int32)).to(dev), st)
        check_state(st, oa.tree_accept(pred, toks, parent, pos=7 + trial), M)


def test_commit_rows_tree(dev):
    """Tree commit moves the accepted path's rows to consecutive positions in every plane."""
    from tokenrush_amd.accept import accept_tree, commit_rows
    say("commit rows")
    parent = np.array([-1, 0, 0, 1, 2, 3, 3, 5], np.int32)          # path 0-1-3-5 (depth 3) to plant
    toks = np.array([0, 11, 12, 13, 14, 15, 16, 17], np.int64)
    V = 4096
    lg = oa.planted_logits(8, V, seed=1)
    for a, b in [(0, 1), (1, 3), (3, 5)]:
        lg[a, toks[b]] = 40.0
    st = state(8, pos=20)
    kv = torch.randint(0, 255, (4, 2, 64, 256), dtype=torch.uint8, device=dev)     # [layers, heads, len, dim] fp8
    sc = torch.rand(4, 2, 64, device=dev)                                          # per-(head, pos) scale
    kv0, sc0 = kv.clone(), sc.clone()
    accept_tree(dev_logits(lg), torch.from_numpy(toks).to(dev), torch.from_numpy(parent).to(dev), st)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    commit_rows(kv, st, "rows", status=status)
    commit_rows(sc, st, "scalars", status=status)
    torch.cuda.synchronize()
    assert int(status) == 0
    ref = oa.tree_accept(oa.argmax_rows(lg), toks, parent, pos=20)
    assert ref["commit"] == [0, 1, 3, 5]
    exp_kv, exp_sc = kv0.clone(), sc0.clone()
    for t, node in enumerate(ref["commit"]):
        exp_kv[:, :, 20 + t] = kv0[:, :, 20 + node]
        exp_sc[:, :, 20 + t] = sc0[:, :, 20 + node]
    assert torch.equal(kv, exp_kv) and torch.equal(sc, exp_sc)
    # a per-layer cache [kv_heads, max_len, head_dim] (one StepState.k[a]) commits the same way
    one = kv0[1].clone()
    commit_rows(one, st, "rows", status=status)
    torch.cuda.synchronize()
    assert torch.equal(one, exp_kv[1]) and int(status) == 0
    # more rows than max_n, or rows past the cache's end: nothing moves and status reads 1
    before = kv.clone()
    commit_rows(kv, st, "rows", max_n=2, status=status)
    torch.cuda.synchronize()
    assert int(status) == 1 and torch.equal(kv, before)
    status.zero_()
    short = kv0[:, :, :22].contiguous()                  # max_len 22: rows 20 + 5 are outside
    short0 = short.clone()
    commit_rows(short, st, "rows", status=status)
    torch.cuda.synchronize()
    assert int(status) == 1 and torch.equal(short, short0)


def test_accept_in_graph_replays(dev):
    """GEMM-free verify tail captured in one graph: accept + position advance replayed with
    changing inputs and eager work in between; every replay matches the oracle."""
    from tokenrush_amd.accept import AcceptState, accept_sampled
    from tokenrush_amd.sample import SamplingParams, workspace
    say("accept graph")
    M = 8
    p = SamplingParams(dev)
    p.set(temperature=1.0)
    logits = torch.zeros(M, V_FULL, dtype=torch.bfloat16, device=dev)
    spec = torch.zeros(M, dtype=torch.long, device=dev)
    u = torch.zeros(M, device=dev)
    st = AcceptState(M, dev)
    workspace(M, V_FULL, dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        accept_sampled(logits, spec, p, st, u)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        accept_sampled(logits, spec, p, st, u)
    pos = 0
    st.pos.zero_()
    for r in range(4):
        rng = np.random.default_rng(r)
        sp = rng.integers(0, V_FULL, M).astype(np.int64)
        lg = oa.planted_logits(M, V_FULL, seed=700 + r, drafts_from=sp, prefix=r + 1)
        for i in range(r + 1):
            lg[i, sp[i + 1]] = 60.0
        uu = rng.random(M).astype(F)
        logits.copy_(dev_logits(lg))
        spec.copy_(torch.from_numpy(sp))
        u.copy_(torch.from_numpy(uu))
        g.replay()
        torch.cuda.synchronize()
        ref = oa.verify_chain(oa.sample(lg, 1.0, 1.0, 64, uu), sp, pos=pos)
        check_state(st, ref, M)
        pos = ref["pos"]
        _ = torch.randn(1000, device=dev).sum()                     # eager work between replays


@pytest.mark.parametrize("V,M", [(248320, 8), (4096, 1), (4096, 16), (40960, 24)])
def test_lm_head_greedy_fused(dev, V, M):
    """lm_head + greedy accept in one launch == lm_head then tr_accept_greedy, bit for bit, and
    pred == the oracle's argmax of the same logits (M = 24 takes the two-launch path)."""
    from tokenrush_amd.accept import AcceptState, accept_greedy, lm_head_greedy
    from tokenrush_amd.quant import QLinear
    print(f"lm_head_greedy V={V} M={M}", flush=True)
    K = 5120
    g = torch.Generator(device="cuda:0").manual_seed(V + M)
    q = torch.randint(0, 256, (V, K // 2), dtype=torch.uint8, device="cuda:0", generator=g)
    s = (torch.rand(V, K // 128, device="cuda:0", generator=g) * 0.018 + 0.002).to(torch.bfloat16)
    m = (torch.rand(V, K // 128, device="cuda:0", generator=g) * 0.14 - 0.15).to(torch.bfloat16)
    lin = QLinear(q, s, m)
    del q
    h = torch.randn(M, K, device="cuda:0", generator=g).to(torch.bfloat16)
    ref_logits = lin(h)
    pred = ref_logits.float().argmax(-1)
    spec = torch.randint(0, V, (M,), device="cuda:0", generator=g)
    spec[1:min(M, 4)] = pred[:min(M, 4) - 1]                        # a planted accepted prefix
    st_ref, st = AcceptState(M, "cuda:0"), AcceptState(M, "cuda:0")
    st_ref.pos.fill_(50)
    st.pos.fill_(50)
    accept_greedy(ref_logits, spec, st_ref)
    logits = lm_head_greedy(lin, h, spec, st, keep_logits=True)
    torch.cuda.synchronize()
    assert torch.equal(logits, ref_logits)
    for name in ("pred", "n_accepted", "tok", "pos", "slot", "tokens", "commit"):
        assert torch.equal(getattr(st, name), getattr(st_ref, name)), name
    lg = ref_logits.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(st.pred.cpu().numpy(), oa.argmax_rows(oa.logits_f32(lg)))
    st2 = AcceptState(M, "cuda:0")
    assert lm_head_greedy(lin, h, None, st2) is None                 # argmax only, no logits written
    torch.cuda.synchronize()
    assert torch.equal(st2.pred, st.pred)
