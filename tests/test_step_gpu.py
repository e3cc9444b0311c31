"""The verify-step driver (tokenrush_amd/step.py) on a small hybrid config (3 GDN layers and one
attention layer with the config-5 head geometry, 300 live cache rows): the body against a float
reference built from the same weights and state (exact int4 weights, fp32 matmuls, the oracle's
GDN step and FP8 attention), the greedy accept against the oracle on the step's own logits
(bit-exact), and the whole step captured as one hipGraph reproducing the eager step bit-for-bit on
repeated replays from the same state."""
import numpy as np
import pytest
import torch

from oracle import accept as oa
from oracle import attn as oat
from oracle import gdn as og
from tokenrush_amd.attn import NSPLIT

pytestmark = pytest.mark.gpu


def _ref_body(model, x0):
    """Float reference of VerifyModel.body: exact weights q * s + m, fp32 matmuls, the same bf16
    rounding points as the kernels (projection outputs, residual stream, norm outputs)."""
    cfg = model.cfg
    bf = lambda t: t.to(torch.bfloat16).float()

    def lin(L, v):
        q, s, m = L.nibbles()                       # exact weight q * s + m (what the GEMM folds)
        codes = torch.stack([q & 0xF, q >> 4], -1).view(q.shape[0], -1).float()
        G = s.shape[1]
        W = codes.view(q.shape[0], G, -1) * s.float()[..., None] + m.float()[..., None]
        return v @ W.view(q.shape[0], -1).t()

    def norm(x, w):
        return bf(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.eps) * (1.0 + w.float()))

    def silu_mul(u):
        F = u.shape[1] // 2
        gg, v = u[:, :F], u[:, F:2 * F]
        return bf(gg / (1 + torch.exp(-gg)) * v)

    st = model.state
    npf = lambda t: t.float().cpu().numpy()
    pos, slot = int(st.pos), int(st.slot)
    ring, rec = npf(st.ring), npf(st.rec)
    kc, vc = st.k.view(torch.uint8).cpu().numpy(), st.v.view(torch.uint8).cpu().numpy()
    ks, vs, cos, sin = npf(st.k_scale), npf(st.v_scale), npf(st.cos), npf(st.sin)
    g = cfg.gdn
    x = x0.float()
    h = None
    for li, L in enumerate(model.layers):
        if h is not None:
            x = bf(x + bf(h))
        n = norm(x, L.ln1)
        u = bf(lin(L.proj, n))
        if L.attention:
            a = model.attn_index[li]
            q, kc[a], vc[a], ks[a], vs[a] = oat.attn_prep(npf(u), npf(L.q_norm_w), npf(L.k_norm_w), cos, sin, pos,
                                                          kc[a], vc[a], ks[a], vs[a], cfg.n_heads, cfg.n_kv_heads,
                                                          cfg.head_dim, cfg.rotary_dim, cfg.eps)
            y = oat.attn_decode(q, npf(u), kc[a], vc[a], ks[a], vs[a], pos, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                nsplit=NSPLIT)
        else:
            k = model.gdn_index[li]
            y, ring[k], rec_k = og.gdn_step(npf(u), npf(n), npf(L.in_ba), ring[k], npf(L.conv_w), npf(L.A),
                                            npf(L.dt_bias), rec[:, k], slot, npf(L.norm_w), pos, g.gdn_k_heads,
                                            g.gdn_v_heads, g.gdn_k_dim, g.gdn_v_dim, cfg.eps)
            rec[:, k] = rec_k
        h = lin(L.out, torch.from_numpy(y).to(x.device))
        x = bf(x + bf(h))
        n = norm(x, L.ln2)
        a = silu_mul(bf(lin(L.gate_up, n)))
        h = lin(L.down, a)
    x = bf(x + bf(h))
    n = norm(x, model.final_norm)
    return lin(model.lm_head, n)


@pytest.fixture(scope="module")
def small_model(dev):
    from tokenrush_amd.step import SMALL, VerifyModel
    m = VerifyModel(SMALL, seed=3)
    m.initial_state = m.state.snapshot()
    return m


@pytest.mark.parametrize("M", [1, 8])
def test_body_matches_float_reference(small_model, M):
    print(f"step body M={M}", flush=True)
    m = small_model
    g = torch.Generator(device="cuda:0").manual_seed(M)
    x0 = torch.randn(M, m.cfg.hidden, device="cuda:0", generator=g).to(torch.bfloat16)
    m.state.restore(m.initial_state)
    ref = _ref_body(m, x0)
    got = m.body(x0).float()
    rel = ((got - ref).norm() / ref.norm()).item()
    assert rel < 2e-2, rel


def test_step_accept_and_graph_replay(small_model):
    from tokenrush_amd.accept import AcceptState
    print("step graph", flush=True)
    m = small_model
    M = 8
    g = torch.Generator(device="cuda:0").manual_seed(11)
    x0 = torch.randn(M, m.cfg.hidden, device="cuda:0", generator=g).to(torch.bfloat16)
    st = AcceptState(M, "cuda:0")
    live = m.cfg.live

    def reset():
        m.state.restore(m.initial_state)
        st.pos.fill_(live)
        st.slot.zero_()

    # drafts: the target's own argmax on a prefix of 3, then a wrong token
    reset()
    logits = m.body(x0)
    pred = logits.float().argmax(-1).cpu().numpy()
    spec = np.zeros(M, dtype=np.int64)
    spec[0] = 7
    spec[1:4] = pred[0:3]
    spec[4:] = (pred[3:7] + 1) % m.cfg.vocab
    spec_t = torch.from_numpy(spec).to("cuda:0")
    reset()
    lg = m.step(x0, spec_t, st)
    torch.cuda.synchronize()
    lg_np = lg.view(torch.int16).cpu().numpy().view(np.uint16)
    want = oa.verify_chain(oa.argmax_rows(oa.logits_f32(lg_np)), spec, pos=live)
    assert int(st.n_accepted) == want["n"] >= 3 and int(st.tok) == want["tok"] and int(st.pos) == want["pos"]
    eager = (lg.clone(), st.n_accepted.clone(), st.tok.clone(), st.slot.clone(), st.tokens.clone(), st.commit.clone())

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        reset()
        m.step(x0, spec_t, st)                     # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        lg_g = m.step(x0, spec_t, st)
    for rep in range(3):
        reset()
        st.n_accepted.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _ = m.body(x0)                              # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(lg_g, eager[0]), rep
        assert torch.equal(st.n_accepted, eager[1]) and torch.equal(st.tok, eager[2]), rep
        assert torch.equal(st.slot, eager[3]) and torch.equal(st.tokens, eager[4]) and torch.equal(st.commit, eager[5])
        assert int(st.pos) == want["pos"]


def test_checkpoint_round_trip(small_model, tmp_path):
    """The model written in the packed checkpoint format (weights.py:60-102) and loaded back
    (weights.py:238-254): same engine-packed nibbles for every matrix, same small tensors, and the
    same step output bit for bit from the same decode state."""
    from tokenrush_amd.step import VerifyModel
    print("checkpoint round trip", flush=True)
    m = small_model
    info = m.save_checkpoint(str(tmp_path))
    assert "lm_head.weight" in info["quantized"] and "layers.0.mlp.gate_proj.weight" in info["quantized"]
    m2 = VerifyModel.from_checkpoint(str(tmp_path), device="cuda:0", live=m.cfg.live, headroom=m.cfg.headroom)
    for L, L2 in zip(m.layers, m2.layers):
        assert L.attention == L2.attention
        for a in ("proj", "out", "gate_up", "down"):
            for t, t2 in zip(getattr(L, a).nibbles(), getattr(L2, a).nibbles()):
                assert torch.equal(t, t2), a
        small = ("q_norm_w", "k_norm_w") if L.attention else ("in_ba", "conv_w", "A", "dt_bias", "norm_w")
        for a in small + ("ln1", "ln2"):
            assert torch.equal(getattr(L, a), getattr(L2, a)), a
    m2.state.restore(m.initial_state)
    m.state.restore(m.initial_state)
    g = torch.Generator(device="cuda:0").manual_seed(4)
    x0 = torch.randn(8, m.cfg.hidden, device="cuda:0", generator=g).to(torch.bfloat16)
    assert torch.equal(m.body(x0), m2.body(x0))
