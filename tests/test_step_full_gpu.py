"""The config-5 verify step at full size: the random-init 64-layer hybrid (48 GDN + 16 attention
layers, hidden 5120, MLP 17408, vocab 248320, int4 g128 weights) over an FP8 cache with 8192 live
tokens, M = 8 verify rows.

* one GDN layer and one attention layer of the model, run by the step's own kernels at full
  hidden size, against the float reference (exact int4 weights, fp32 matmuls, the oracle's GDN
  step and FP8 attention) -- the same pieces test_step_gpu.py chains over the small hybrid;
* the greedy accept of the full step against oracle.verify_chain on the step's own logits, with
  drafts planted from an eager pass so that at least 3 are accepted (reference
  tokenrush/model.py:293-312);
* the step captured as one hipGraph reproducing the eager step bit for bit (logits, n_accepted,
  tok, pos, slot, tokens, commit) over several replays from a restored decode state, with eager
  work between the replays."""
import numpy as np
import pytest
import torch

from oracle import accept as oa
from test_step_gpu import _bf, _ref_lin, _ref_mixer, _ref_norm, _RefState

pytestmark = pytest.mark.gpu
M = 8


def rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


@pytest.fixture(scope="module")
def full_model(dev):
    from tokenrush_amd.step import StepConfig, VerifyModel, prepare
    print("building the config-5 model", flush=True)
    m = VerifyModel(StepConfig(), seed=5)
    prepare(m, M)
    m.initial_state = m.state.snapshot()
    torch.cuda.synchronize()
    yield m
    del m.initial_state
    torch.cuda.empty_cache()


@pytest.mark.parametrize("li", [0, 3])
def test_full_size_layer_matches_float_reference(full_model, li):
    """Layer 0 (GDN) and layer 3 (attention): projection, mixer and the out projection's partials
    at hidden 5120 against the float reference on the same normed rows and decode state."""
    from tokenrush_amd.fused import add_rmsnorm
    m = full_model
    L = m.layers[li]
    print(f"config-5 layer {li} ({'attention' if L.attention else 'GDN'})", flush=True)
    assert L.attention == (li == 3)
    m.state.restore(m.initial_state)
    g = torch.Generator(device="cuda:0").manual_seed(40 + li)
    x = torch.randn(M, m.cfg.hidden, device="cuda:0", generator=g).to(torch.bfloat16)
    rs = _RefState(m)                                   # the state before the kernels update it
    if L.attention:
        rs.attn_layer(m.attn_index[li])
    else:
        rs.gdn_layer(m.gdn_index[li])
    _, n = add_rmsnorm(x, None, L.ln1, m.cfg.eps)
    u = L.proj(n)
    y = m.mixer(li, L, n, m.state.pos, m.state.slot)
    h = L.out.partials(y)
    torch.cuda.synchronize()
    assert rel(n.float(), _ref_norm(x.float(), L.ln1, m.cfg.eps)) < 4e-3
    u_ref, y_ref = _ref_mixer(m, li, L, n.float(), rs)
    assert rel(u, u_ref) < 4e-3
    assert rel(y, y_ref) < 1e-2, rel(y, y_ref)
    h_ref = _ref_lin(L.out, _bf(y.float()))
    assert rel(h.sum(0), h_ref) < 4e-3
    if not L.attention:                                 # the committed recurrent state, all 8 slots
        rec_ref = torch.from_numpy(rs.gdn[m.gdn_index[li]][1]).to("cuda:0")
        assert rel(m.state.rec[:, m.gdn_index[li]], rec_ref) < 1e-3


def test_full_size_step_accept_and_graph_replay(full_model):
    from tokenrush_amd.accept import AcceptState
    m = full_model
    print("config-5 step: eager accept vs oracle, graph replays", flush=True)
    g = torch.Generator(device="cuda:0").manual_seed(11)
    x0 = torch.randn(M, m.cfg.hidden, device="cuda:0", generator=g).to(torch.bfloat16)
    st = AcceptState(M, "cuda:0")
    live, V = m.cfg.live, m.cfg.vocab

    def reset():
        m.state.restore(m.initial_state)
        st.pos.fill_(live)
        st.slot.zero_()

    reset()
    pred = m.body(x0).float().argmax(-1).cpu().numpy()
    spec = np.zeros(M, dtype=np.int64)
    spec[0] = 7
    spec[1:5] = pred[0:4]                              # 4 drafts the target agrees with
    spec[5:] = (pred[4:7] + 1) % V                     # then wrong ones
    spec_t = torch.from_numpy(spec).to("cuda:0")
    reset()
    lg = m.step(x0, spec_t, st)
    torch.cuda.synchronize()
    lg_np = lg.view(torch.int16).cpu().numpy().view(np.uint16)
    want = oa.verify_chain(oa.argmax_rows(oa.logits_f32(lg_np)), spec, pos=live)
    assert want["n"] == 4
    assert int(st.n_accepted) == want["n"] and int(st.tok) == want["tok"] and int(st.pos) == want["pos"]
    pad = [-1] * (M - want["n"] - 1)
    assert int(st.slot) == want["n"] and st.tokens.cpu().tolist() == want["tokens"] + pad
    assert st.commit.cpu().tolist() == want["commit"] + pad
    eager = [t.clone() for t in (lg, st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit)]
    eager_state = [t.clone() for t in m.state.tensors()[2:4]]      # ring and recurrent slots after the step

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        reset()
        m.step(x0, spec_t, st)                         # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        lg_g = m.step(x0, spec_t, st)
    for rep in range(3):
        reset()
        st.n_accepted.fill_(-1)
        st.tokens.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (lg_g, st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit)
        for name, a, b in zip(("logits", "n", "tok", "pos", "slot", "tokens", "commit"), got, eager):
            assert torch.equal(a, b), (rep, name)
        for a, b in zip(m.state.tensors()[2:4], eager_state):
            assert torch.equal(a, b), rep
        _ = m.body(x0)                                  # eager work between replays
        torch.cuda.synchronize()
    del graph


def _capture_and_replay(m, reset, run, st, eager, x0, reps=3):
    """Capture run() as one graph, replay it from the restored state `reps` times (eager work in
    between) and compare logits and accept outputs with the eager step bit for bit."""
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        reset()
        run()                                           # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        lg_g = run()
    for rep in range(reps):
        reset()
        st.n_accepted.fill_(-1)
        st.tokens.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (lg_g, st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit)
        for name, a, b in zip(("logits", "n", "tok", "pos", "slot", "tokens", "commit"), got, eager):
            assert torch.equal(a, b), (rep, name)
        _ = m.body(x0)                                  # eager work between replays
        torch.cuda.synchronize()
    del graph


def _check_accept(st, want):
    pad = [-1] * (M - want["n"] - 1)
    assert int(st.n_accepted) == want["n"] and int(st.tok) == want["tok"] and int(st.pos) == want["pos"]
    assert int(st.slot) == want["n"] and st.tokens.cpu().tolist() == want["tokens"] + pad
    assert st.commit.cpu().tolist() == want["commit"] + pad


def test_full_size_sampled_step_in_one_graph(full_model):
    """The reference's sampled verify (model.py:306: pred = sample(logits, params, u)) inside the
    step graph: device SamplingParams, uniforms supplied; drafts planted from an eager pass so 3
    are accepted; the accept against oracle.sample + verify_chain on the step's own logits."""
    from tokenrush_amd.accept import AcceptState
    from tokenrush_amd.sample import SamplingParams
    m = full_model
    print("config-5 sampled step", flush=True)
    g = torch.Generator(device="cuda:0").manual_seed(12)
    x0 = torch.randn(M, m.cfg.hidden, device="cuda:0", generator=g).to(torch.bfloat16)
    st, live, V = AcceptState(M, "cuda:0"), m.cfg.live, m.cfg.vocab
    params = SamplingParams("cuda:0")
    params.set(temperature=0.8, top_p=0.95, top_k=40)
    u = torch.rand(M, device="cuda:0", generator=g)

    def reset():
        m.state.restore(m.initial_state)
        st.pos.fill_(live)
        st.slot.zero_()

    def logits_np(lg):
        return oa.logits_f32(lg.view(torch.int16).cpu().numpy().view(np.uint16))

    reset()
    lg0 = logits_np(m.body(x0))
    pred = oa.sample(lg0, 0.8, 0.95, 40, u.cpu().numpy())
    spec = np.zeros(M, dtype=np.int64)
    spec[0] = 3
    spec[1:4] = pred[0:3]
    spec[4:] = (pred[3:7] + 1) % V
    spec_t = torch.from_numpy(spec).to("cuda:0")
    reset()
    lg = m.step(x0, spec_t, st, params=params, u=u)
    torch.cuda.synchronize()
    want = oa.verify_chain(oa.sample(logits_np(lg), 0.8, 0.95, 40, u.cpu().numpy()), spec, pos=live)
    assert want["n"] == 3
    _check_accept(st, want)
    eager = [t.clone() for t in (lg, st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit)]
    _capture_and_replay(m, reset, lambda: m.step(x0, spec_t, st, params=params, u=u), st, eager, x0)


def test_full_size_residual_step_in_one_graph(full_model):
    """Residual rejection sampling after the full step (draft probabilities q [7, V], uniforms
    supplied): the accept against oracle.residual_accept on the step's own logits; the step with
    it captured as one graph reproduces the eager step bit for bit."""
    from tokenrush_amd.accept import AcceptState
    m = full_model
    print("config-5 residual step", flush=True)
    g = torch.Generator(device="cuda:0").manual_seed(13)
    x0 = torch.randn(M, m.cfg.hidden, device="cuda:0", generator=g).to(torch.bfloat16)
    st, live, V = AcceptState(M, "cuda:0"), m.cfg.live, m.cfg.vocab
    reset_state = lambda: (m.state.restore(m.initial_state), st.pos.fill_(live), st.slot.zero_())
    reset_state()
    lg0 = m.body(x0).float()
    # drafts 1..3 are the target's argmax with q = the target's own distribution (accepted for
    # any u < 1); the rest are random tokens under a random draft distribution
    q = torch.softmax(torch.randn(M - 1, V, device="cuda:0", generator=g) * 2, -1)
    q[:3] = torch.softmax(lg0[:3], -1)
    q = q.contiguous()
    spec = torch.randint(0, V, (M,), device="cuda:0", generator=g)
    spec[1:4] = lg0[:3].argmax(-1)
    u = torch.rand(M, device="cuda:0", generator=g) * 0.9
    reset_state()
    lg = m.step(x0, spec, st, q=q, u=u)
    torch.cuda.synchronize()
    lg_np = oa.logits_f32(lg.view(torch.int16).cpu().numpy().view(np.uint16))
    want = oa.residual_accept(lg_np, q.cpu().numpy(), spec[1:].cpu().numpy(), u.cpu().numpy(), pos=live)
    assert want["n"] >= 3
    _check_accept(st, want)
    eager = [t.clone() for t in (lg, st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit)]
    _capture_and_replay(m, reset_state, lambda: m.step(x0, spec, st, q=q, u=u), st, eager, x0)


def test_full_size_verify_from_token_ids_in_one_graph(full_model):
    """The reference's _verify_step whole (model.py:293-312): token ids embedded on the device
    (model.py:215), body, lm_head, greedy accept, with spec_logits[:M] and spec_hidden[:M] kept
    (model.py:300-301). Eager verify() equals step() on torch's embedding rows bit for bit; the
    captured graph reproduces spec_x, spec_hidden, spec_logits and the accept over replays."""
    from tokenrush_amd.accept import AcceptState
    m = full_model
    print("config-5 verify from token ids", flush=True)
    g = torch.Generator(device="cuda:0").manual_seed(14)
    st, live, V = AcceptState(M, "cuda:0"), m.cfg.live, m.cfg.vocab
    spec = torch.randint(0, V, (M,), device="cuda:0", generator=g)

    def reset():
        m.state.restore(m.initial_state)
        st.pos.fill_(live)
        st.slot.zero_()

    reset()
    pred = m.body(m.embed[spec]).float().argmax(-1)
    spec[1:4] = pred[0:3]                              # 3 drafts the target agrees with
    spec[4:] = (pred[3:7] + 1) % V
    reset()
    lg_ref = m.step(m.embed[spec].contiguous(), spec, st).clone()
    hid_ref = m.spec_hidden[:M].clone()
    acc_ref = [t.clone() for t in (st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit)]
    assert int(st.n_accepted) == 3
    reset()
    m.embed_status.zero_()
    lg = m.verify(spec, st)
    torch.cuda.synchronize()
    assert int(m.embed_status) == 0
    assert torch.equal(m.spec_x[:M], m.embed[spec])
    assert torch.equal(lg, lg_ref) and torch.equal(m.spec_logits[:M], lg_ref)
    assert torch.equal(m.spec_hidden[:M], hid_ref)
    for a, b in zip((st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit), acc_ref):
        assert torch.equal(a, b)

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        reset()
        m.verify(spec, st)                             # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        m.verify(spec, st)
    for rep in range(2):
        reset()
        m.spec_hidden.zero_()
        m.spec_logits.zero_()
        m.spec_x.zero_()
        st.n_accepted.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(m.spec_x[:M], m.embed[spec]), rep
        assert torch.equal(m.spec_hidden[:M], hid_ref), rep
        assert torch.equal(m.spec_logits[:M], lg_ref), rep
        for a, b in zip((st.n_accepted, st.tok, st.pos, st.slot, st.tokens, st.commit), acc_ref):
            assert torch.equal(a, b), rep
        _ = m.body(m.embed[spec])                      # eager work between replays
        torch.cuda.synchronize()
    del graph
