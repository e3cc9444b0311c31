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


def _bf(t):
    return t.to(torch.bfloat16).float()


def _ref_lin(L, v):
    """v @ W^T with the exact weight q * s + m (what the GEMM folds), fp32."""
    q, s, m = L.nibbles()
    codes = torch.stack([q & 0xF, q >> 4], -1).view(q.shape[0], -1).float()
    G = s.shape[1]
    W = codes.view(q.shape[0], G, -1) * s.float()[..., None] + m.float()[..., None]
    return v @ W.view(q.shape[0], -1).t()


def _ref_norm(x, w, eps):
    return _bf(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w.float()))


def _ref_silu_mul(u):
    F = u.shape[1] // 2
    gg, v = u[:, :F], u[:, F:2 * F]
    return _bf(gg / (1 + torch.exp(-gg)) * v)


def _npf(t):
    return t.float().cpu().numpy()


class _RefState:
    """numpy copies of the decode state the float reference reads and updates, per layer on
    demand (the full-size state is too large to copy whole)."""

    def __init__(self, model):
        st = model.state
        self.model, self.pos, self.slot = model, int(st.pos), int(st.slot)
        self.cos, self.sin = _npf(st.cos), _npf(st.sin)
        self.gdn, self.attn = {}, {}

    def gdn_layer(self, k):
        if k not in self.gdn:
            st = self.model.state
            self.gdn[k] = [_npf(st.ring[k]), _npf(st.rec[:, k])]
        return self.gdn[k]

    def attn_layer(self, a):
        if a not in self.attn:
            st = self.model.state
            self.attn[a] = [st.k[a].view(torch.uint8).cpu().numpy(), st.v[a].view(torch.uint8).cpu().numpy(),
                            _npf(st.k_scale[a]), _npf(st.v_scale[a])]
        return self.attn[a]


def _ref_mixer(model, li, L, n, rs):
    """The layer's mixer on normed rows n (fp32 [M, hidden]) -> (u, y): the bf16 projection and the
    mixer output, the GDN step or FP8 attention restated by the oracle."""
    cfg = model.cfg
    u = _bf(_ref_lin(L.proj, n))
    if L.attention:
        kc, vc, ks, vs = rs.attn_layer(model.attn_index[li])
        q, kc[:], vc[:], ks[:], vs[:] = oat.attn_prep(_npf(u), _npf(L.q_norm_w), _npf(L.k_norm_w), rs.cos, rs.sin,
                                                      rs.pos, kc, vc, ks, vs, cfg.n_heads, cfg.n_kv_heads,
                                                      cfg.head_dim, cfg.rotary_dim, cfg.eps)
        y = oat.attn_decode(q, _npf(u), kc, vc, ks, vs, rs.pos, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                            nsplit=NSPLIT)
    else:
        g = cfg.gdn
        ring, rec = rs.gdn_layer(model.gdn_index[li])
        y, ring[:], rec_k = og.gdn_step(_npf(u), _npf(n), _npf(L.in_ba), ring, _npf(L.conv_w), _npf(L.A),
                                        _npf(L.dt_bias), rec, rs.slot, _npf(L.norm_w), rs.pos, g.gdn_k_heads,
                                        g.gdn_v_heads, g.gdn_k_dim, g.gdn_v_dim, cfg.eps)
        rec[:] = rec_k
    return u, torch.from_numpy(np.ascontiguousarray(y)).to(n.device)


def _ref_body(model, x0):
    """Float reference of VerifyModel.body: exact weights q * s + m, fp32 matmuls, the same bf16
    rounding points as the kernels (projection outputs, residual stream, norm outputs)."""
    cfg = model.cfg
    rs = _RefState(model)
    x = x0.float()
    h = None
    for li, L in enumerate(model.layers):
        if h is not None:
            x = _bf(x + _bf(h))
        n = _ref_norm(x, L.ln1, cfg.eps)
        _, y = _ref_mixer(model, li, L, n, rs)
        h = _ref_lin(L.out, y)
        x = _bf(x + _bf(h))
        n = _ref_norm(x, L.ln2, cfg.eps)
        a = _ref_silu_mul(_bf(_ref_lin(L.gate_up, n)))
        h = _ref_lin(L.down, a)
    x = _bf(x + _bf(h))
    n = _ref_norm(x, model.final_norm, cfg.eps)
    return _ref_lin(model.lm_head, n)


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
