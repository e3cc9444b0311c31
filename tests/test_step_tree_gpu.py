"""The draft-tree verify step (VerifyModel.step_tree; benchmark config 4's 32-node trees through
the real layers): tree mixers, lm_head, the tree accept and its commit.

* On a chain tree the tree step is the chain step: logits, accept outputs and the decode state
  after the commit equal the greedy chain step's, bit for bit (ring columns of rejected rows
  aside: the chain step writes them, the tree commit leaves them, and both are dead).
* On a random 32-node tree (branching <= 4, depth <= 7) with drafts planted along the deepest
  path, the accept equals oracle.accept.tree_accept on the step's own logits. After the commit the
  conv rings, the continued-from recurrent state and the KV rows 0..pos+n equal, bit for bit, those
  of a tree holding the same path as nodes 0..n (the small hybrid's only attention layer is its
  last, so every mixer input before it is bit-identical), whose path logits agree within 1e-2
  (the attention sums the same keys in another order); a chain step over the path (M = n + 1, a
  GEMM of another row class) agrees within rounding (2e-2 logits, 1e-2 state).
* The step captured as one hipGraph reproduces the eager step on repeated replays, at the small
  and at full size (64 layers, vocab 248320, 8192 live tokens).
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import accept as oa
from oracle import gdn as og

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


@pytest.fixture(scope="module")
def tree_model(dev):
    from tokenrush_amd.step import SMALL, VerifyModel
    m = VerifyModel(dataclasses.replace(SMALL, tree_nodes=32), seed=4)
    m.initial_state = m.state.snapshot()
    return m


def _reset(m, st):
    m.state.restore(m.initial_state)
    st.pos.fill_(m.cfg.live)
    st.slot.zero_()


def _planted(m, x0, parent, st):
    """Node tokens accepted exactly along the deepest root path (lowest index among equals): each
    path node holds its parent row's argmax, every other node a different token."""
    par = torch.from_numpy(parent).to(DEV)
    _reset(m, st)
    pred = m.lm_head(m.hidden(x0, st.pos, st.slot, par)).float().argmax(-1).cpu().numpy()
    depth = oa.tree_depths(parent)
    best = int(np.argmax(depth))
    path = og.root_path(parent, best)
    V = m.cfg.vocab
    toks = np.array([7] + [(int(pred[parent[i]]) + 1) % V for i in range(1, len(parent))], dtype=np.int64)
    for i in path[1:]:
        toks[i] = pred[parent[i]]
    return torch.from_numpy(toks).to(DEV), par, path


def _state_after(m):
    S = m.state
    return [t.clone() for t in (S.ring, S.rec, S.k, S.v, S.k_scale, S.v_scale)]


def test_tree_step_on_a_chain_is_the_chain_step(tree_model):
    from tokenrush_amd.accept import AcceptState
    print("tree step on a chain vs chain step", flush=True)
    m, M = tree_model, 8
    g = torch.Generator(device=DEV).manual_seed(21)
    x0 = torch.randn(M, m.cfg.hidden, device=DEV, generator=g).to(torch.bfloat16)
    st = AcceptState(M, DEV)
    parent = np.arange(-1, M - 1, dtype=np.int32)
    _reset(m, st)
    pred = m.body(x0).float().argmax(-1).cpu().numpy()
    spec = np.array([7] + list(pred[:3]) + [(int(p) + 1) % m.cfg.vocab for p in pred[3:7]], dtype=np.int64)
    spec_t = torch.from_numpy(spec).to(DEV)
    _reset(m, st)
    lg_c = m.step(x0, spec_t, st)
    torch.cuda.synchronize()
    chain = [t.clone() for t in (st.n_accepted, st.tok, st.pos, st.slot, st.tokens)]
    state_c = _state_after(m)
    assert int(st.n_accepted) == 3
    _reset(m, st)
    lg_t = m.step_tree(x0, spec_t, torch.from_numpy(parent).to(DEV), st)
    torch.cuda.synchronize()
    assert torch.equal(lg_t, lg_c)
    for a, b in zip((st.n_accepted, st.tok, st.pos, st.slot, st.tokens), chain):
        assert torch.equal(a, b)
    assert st.commit.cpu().tolist()[:4] == [0, 1, 2, 3]
    after = _state_after(m)
    # rings: the chain step wrote every row's column, the tree commit only the accepted path's;
    # the columns of rejected rows are dead (the next step overwrites them before reading)
    from tokenrush_amd.gdn import RING
    live = m.cfg.live
    dead = [(live + d) % RING for d in range(4, M)]
    keep = torch.tensor([c for c in range(RING) if c not in dead], device=DEV)
    assert torch.equal(after[0][..., keep], state_c[0][..., keep])
    for a, b in zip(after[1:], state_c[1:]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("seed", [1, 2, "deep"])
def test_tree_step_accept_commit_and_chain_equivalence(tree_model, seed):
    """seed "deep": branch parents at depths 8-10, deeper than the GDN kernel's state stack."""
    from tokenrush_amd.accept import AcceptState
    print(f"tree step random tree seed={seed}", flush=True)
    m, M = tree_model, 32
    parent = oa.deep_branch_tree(M) if seed == "deep" else oa.random_tree(M, seed)
    seed = 3 if seed == "deep" else seed
    g = torch.Generator(device=DEV).manual_seed(40 + seed)
    x0 = torch.randn(M, m.cfg.hidden, device=DEV, generator=g).to(torch.bfloat16)
    st = AcceptState(M, DEV)
    toks, par, path = _planted(m, x0, parent, st)
    n = len(path) - 1
    live = m.cfg.live
    _reset(m, st)
    lg = m.step_tree(x0, toks, par, st)
    torch.cuda.synchronize()
    lg_np = lg.view(torch.int16).cpu().numpy().view(np.uint16)
    want = oa.tree_accept(oa.argmax_rows(oa.logits_f32(lg_np)), toks.cpu().numpy(), parent, pos=live)
    assert want["n"] == n >= 2 and want["commit"] == path
    pad = [-1] * (M - n - 1)
    assert int(st.n_accepted) == n and int(st.tok) == want["tok"] and int(st.pos) == want["pos"]
    assert int(st.slot) == want["slot"] and st.tokens.cpu().tolist() == want["tokens"] + pad
    assert st.commit.cpu().tolist() == want["commit"] + pad
    tree_state = _state_after(m)
    best = want["slot"]
    rows = live + n + 1

    # The same path as nodes 0..n of another 32-node tree (the other nodes hang off the root):
    # the same GEMM row class (M = 32) and the same per-node mixer arithmetic, so everything the
    # commit keeps is the same bits; only the attention sums its keys in another order.
    others = [t for t in range(M) if t not in path]
    order = path + others
    parent2 = np.array([-1] + list(range(n)) + [0] * len(others), np.int32)
    idx = torch.tensor(order, device=DEV)
    _reset(m, st)
    lg2 = m.step_tree(x0[idx].contiguous(), toks[idx].contiguous(), torch.from_numpy(parent2).to(DEV), st)
    torch.cuda.synchronize()
    assert int(st.n_accepted) == n and int(st.slot) == n and int(st.pos) == want["pos"]
    assert rel(lg2[:n + 1], lg[torch.tensor(path, device=DEV)]) < 1e-2
    S = m.state
    assert torch.equal(tree_state[0], S.ring)                                     # rings
    assert torch.equal(tree_state[1][best], S.rec[n])                            # state continued from
    for a, b in zip(tree_state[2:4], (S.k, S.v)):
        assert torch.equal(a[:, :, :rows].view(torch.uint8), b[:, :, :rows].view(torch.uint8))
    for a, b in zip(tree_state[4:], (S.k_scale, S.v_scale)):
        assert torch.equal(a[:, :, :rows], b[:, :, :rows])

    # a chain step over the accepted path (M = n + 1, another GEMM row class): the same within
    # rounding; chain steps take at most 8 rows
    if n + 1 > 8:
        return
    st_c = AcceptState(n + 1, DEV)
    _reset(m, st_c)
    pidx = torch.tensor(path, device=DEV)
    lg_c = m.lm_head(m.hidden(x0[pidx].contiguous(), st_c.pos, st_c.slot))
    torch.cuda.synchronize()
    assert rel(lg_c, lg[pidx]) < 2e-2
    assert rel(S.ring, tree_state[0]) < 1e-2 and rel(S.rec[n], tree_state[1][best]) < 1e-2


def _graph_check(m, x0, toks, par, st, reps=3):
    def reset():
        _reset(m, st)

    reset()
    lg = m.step_tree(x0, toks, par, st)
    torch.cuda.synchronize()
    eager = [t.clone() for t in (lg, st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit)]
    eager_state = _state_after(m)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        reset()
        m.step_tree(x0, toks, par, st)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        lg_g = m.step_tree(x0, toks, par, st)
    for rep in range(reps):
        reset()
        st.n_accepted.fill_(-1)
        st.commit.fill_(-9)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (lg_g, st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit)
        for name, a, b in zip(("logits", "n", "tok", "pos", "slot", "tokens", "commit"), got, eager):
            assert torch.equal(a, b), (rep, name)
        for a, b in zip(_state_after(m), eager_state):
            assert torch.equal(a, b), rep
        _ = m.body(x0[:8])                                 # eager work between replays
        torch.cuda.synchronize()
    del graph
    return eager


def test_tree_step_graph_replay(tree_model):
    from tokenrush_amd.accept import AcceptState
    print("tree step graph (small)", flush=True)
    m, M = tree_model, 32
    parent = oa.random_tree(M, 9)
    g = torch.Generator(device=DEV).manual_seed(9)
    x0 = torch.randn(M, m.cfg.hidden, device=DEV, generator=g).to(torch.bfloat16)
    st = AcceptState(M, DEV)
    toks, par, path = _planted(m, x0, parent, st)
    eager = _graph_check(m, x0, toks, par, st)
    assert int(eager[1]) == len(path) - 1


def test_full_size_tree_step(dev):
    """Config 4 through the config-5 model: a 32-node tree (branching <= 4, depth <= 7) verified
    by the 64-layer step; accept vs the oracle on the step's own logits, graph == eager."""
    from tokenrush_amd.accept import AcceptState
    from tokenrush_amd.step import StepConfig, VerifyModel, prepare
    print("building the config-5 model with tree room", flush=True)
    M = 32
    m = VerifyModel(StepConfig(tree_nodes=M), seed=6)
    prepare(m, M)
    m.initial_state = m.state.snapshot()
    try:
        parent = oa.random_tree(M, 4)
        g = torch.Generator(device=DEV).manual_seed(4)
        x0 = torch.randn(M, m.cfg.hidden, device=DEV, generator=g).to(torch.bfloat16)
        st = AcceptState(M, DEV)
        toks, par, path = _planted(m, x0, parent, st)
        print("config-4 tree step: eager accept vs oracle, graph replays", flush=True)
        eager = _graph_check(m, x0, toks, par, st, reps=2)
        lg_np = eager[0].view(torch.int16).cpu().numpy().view(np.uint16)
        want = oa.tree_accept(oa.argmax_rows(oa.logits_f32(lg_np)), toks.cpu().numpy(), parent, pos=m.cfg.live)
        assert want["commit"] == path and int(eager[1]) == want["n"] == len(path) - 1
        assert int(eager[2]) == want["tok"] and int(eager[3]) == want["pos"] and int(eager[4]) == want["slot"]
    finally:
        del m
        torch.cuda.empty_cache()
