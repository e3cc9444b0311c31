"""Draft-tree verify through the mixers on the GPU (csrc/gdn.hip tr_gdn_tree_step /
tr_gdn_tree_commit, csrc/attn.hip tr_attn_prep_tree / tr_attn_decode_tree) at the config-5 layer
geometry, for the 32-node trees of benchmark config 4 (branching <= 4, depth <= 7).

Oracles: oracle.gdn.gdn_tree_step / tree_commit and oracle.attn.attn_tree, which define node t
as the last token of a chain step over its root path (pinned by reduction to the chain oracles,
tests/test_oracle_gdn.py and tests/test_oracle_attn.py). Tolerances are the chain tests':
GDN states 1e-4 and outputs 5e-3 relative Frobenius; attention outputs 5e-3; q and cache codes
equal except at rounding ties. On a chain tree the tree kernels equal the chain kernels bit for bit.
"""
import numpy as np
import pytest
import torch

from oracle import accept as oa
from oracle import attn as oat
from oracle import gdn as og
from tokenrush_amd.accept import AcceptState
from tokenrush_amd.attn import AttnConfig, attn_decode_fused, attn_prep, rope_table
from tokenrush_amd.gdn import RING, GDNConfig, gdn_step_fused, tree_commit

pytestmark = pytest.mark.gpu
G = GDNConfig()
H, HV, K, V, HID = G.gdn_k_heads, G.gdn_v_heads, G.gdn_k_dim, G.gdn_v_dim, G.hidden
C = G.conv_dim
A_CFG = AttnConfig()
HQ, HKV, D, RD = A_CFG.n_heads, A_CFG.n_kv_heads, A_CFG.head_dim, A_CFG.rotary_dim
QKV = HQ * 2 * D + 2 * HKV * D
F8 = torch.float8_e4m3fn
NSLOT = 32


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def _np(t):
    return t.float().cpu().numpy()


def _codes(t):
    return t.view(torch.uint8).cpu().numpy()


def _tree(kind, M, seed):
    if kind == "chain":
        return np.arange(-1, M - 1, dtype=np.int32)
    if kind == "star":
        p = np.zeros(M, np.int32)
        p[0] = -1
        return p
    if kind == "deep":
        return oa.deep_branch_tree(M)
    return oa.random_tree(M, seed)


# ------------------------------------------------------------------ GDN

def _gdn_inputs(dev, seed, M):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    bf = torch.bfloat16
    w = dict(ba_w=(torch.randn(2 * HV, HID, device=dev, generator=gen) * 0.02).to(bf),
             conv_w=(torch.randn(C, 4, device=dev, generator=gen) * 0.3).to(bf),
             A=-torch.exp(torch.randn(HV, device=dev, generator=gen)),
             dt_bias=torch.randn(HV, device=dev, generator=gen),
             norm_w=(1 + 0.5 * torch.randn(V, device=dev, generator=gen)).to(bf))
    qkvz = torch.randn(M, C + HV * V, device=dev, generator=gen).to(bf)
    x = torch.randn(M, HID, device=dev, generator=gen).to(bf)
    ring = torch.randn(C, RING, device=dev, generator=gen).to(bf)
    rec = torch.randn(NSLOT, HV, K, V, device=dev, generator=gen) * 0.1
    return w, qkvz, x, ring, rec


def _gdn_tree(w, qkvz, x, ring, rec, slot, pos, parent_np, dev):
    M = qkvz.shape[0]
    node_in = torch.empty(M, C, device=dev, dtype=torch.bfloat16)
    par = torch.from_numpy(parent_np).to(dev)
    y = gdn_step_fused(qkvz, x, w["ba_w"], ring, w["conv_w"], w["A"], w["dt_bias"], rec,
                       torch.tensor([slot], device=dev), w["norm_w"], torch.tensor([pos], device=dev), G, 1e-6,
                       parent=par, node_in=node_in)
    torch.cuda.synchronize()
    return y, node_in


@pytest.mark.parametrize("kind,M,pos,slot", [("random", 32, 1000, 5), ("random", 17, 2, 31), ("star", 9, 40, 0),
                                             ("chain", 32, 77, 3), ("deep", 32, 500, 6), ("deep", 24, 3, 30)])
def test_gdn_tree_matches_oracle(dev, kind, M, pos, slot):
    print(f"gdn tree {kind} M={M} pos={pos} slot={slot}", flush=True)
    parent = _tree(kind, M, 100 + M)
    w, qkvz, x, ring, rec = _gdn_inputs(dev, 30 + M, M)
    ring0, rec0 = ring.clone(), _np(rec)
    y, node_in = _gdn_tree(w, qkvz, x, ring, rec, slot, pos, parent, dev)
    ry, rrec = og.gdn_tree_step(_np(qkvz), _np(x), _np(w["ba_w"]), _np(ring0), _np(w["conv_w"]), _np(w["A"]),
                                _np(w["dt_bias"]), rec0, slot, _np(w["norm_w"]), pos, parent, H, HV, K, V, 1e-6)
    assert torch.equal(ring, ring0), "a tree step leaves the ring alone"
    assert torch.equal(node_in, qkvz[:, :C]), "node_in holds the nodes' conv inputs"
    got = _np(rec)
    for t in range(M):
        assert rel(got[t], rrec[t]) < 1e-4, (t, rel(got[t], rrec[t]))
    assert np.array_equal(got[M:], rec0[M:]), "slots >= M untouched"
    gy = _np(y)
    assert np.isfinite(gy).all()
    for t in range(M):
        assert rel(gy[t], ry[t]) < 5e-3, (t, rel(gy[t], ry[t]))


def test_gdn_tree_on_a_chain_equals_the_chain_kernel(dev):
    """parent[t] = t - 1 at M = 8: the tree kernel's outputs and snapshots are the chain kernel's
    bits, and committing the whole path leaves the chain kernel's ring."""
    M, pos, slot = 8, 45, 2
    w, qkvz, x, ring, rec = _gdn_inputs(dev, 7, M)
    ring_c, rec_c = ring.clone(), rec.clone()
    y_c = gdn_step_fused(qkvz, x, w["ba_w"], ring_c, w["conv_w"], w["A"], w["dt_bias"], rec_c,
                         torch.tensor([slot], device=dev), w["norm_w"], torch.tensor([pos], device=dev), G, 1e-6)
    ring_t, rec_t = ring.clone(), rec.clone()
    y_t, node_in = _gdn_tree(w, qkvz, x, ring_t, rec_t, slot, pos, _tree("chain", M, 0), dev)
    assert torch.equal(y_t, y_c)
    assert torch.equal(rec_t[:M], rec_c[:M])
    st = AcceptState(M, dev)
    st.pos.fill_(pos + M)          # as the tree accept leaves it after accepting all M - 1 drafts
    st.n_accepted.fill_(M - 1)
    st.commit.copy_(torch.arange(M, device=dev))
    tree_commit(ring_t, node_in, st)
    torch.cuda.synchronize()
    assert torch.equal(ring_t, ring_c)


@pytest.mark.parametrize("seed", [1, 2])
def test_gdn_tree_commit_matches_oracle_and_chain(dev, seed):
    """After the tree accept names a path, the committed ring is the oracle's and the chain
    kernel's over the path's tokens; the next chain step from (pos, slot) equals a chain step
    that ran over the path."""
    M, pos, slot = 32, 300 + seed, 4
    parent = _tree("random", M, seed)
    w, qkvz, x, ring, rec = _gdn_inputs(dev, 50 + seed, M)
    ring0 = ring.clone()
    rec_tree = rec.clone()
    _, node_in = _gdn_tree(w, qkvz, x, ring, rec_tree, slot, pos, parent, dev)
    depth = oa.tree_depths(parent)
    best = int(np.argmax(depth))
    path = og.root_path(parent, best)
    n = len(path) - 1
    st = AcceptState(M, dev)
    st.pos.fill_(pos + n + 1)
    st.n_accepted.fill_(n)
    st.commit.fill_(-1)
    st.commit[:n + 1] = torch.tensor(path, device=dev)
    st.slot.fill_(best)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    tree_commit(ring, node_in, st, status)
    torch.cuda.synchronize()
    assert int(status) == 0
    want = og.tree_commit(_np(ring0), _np(node_in), path, pos)
    assert np.array_equal(_np(ring), want)
    # the chain kernel over the path's rows leaves the same ring and the same final state
    ring_c, rec_c = ring0.clone(), rec.clone()
    idx = torch.tensor(path, device=dev)
    gdn_step_fused(qkvz[idx].contiguous(), x[idx].contiguous(), w["ba_w"], ring_c, w["conv_w"], w["A"], w["dt_bias"],
                   rec_c, torch.tensor([slot], device=dev), w["norm_w"], torch.tensor([pos], device=dev), G, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(ring, ring_c)
    assert rel(_np(rec_tree[best]), _np(rec_c[n])) < 1e-5
    # a bad path (node past M) commits nothing and raises the status
    st.commit[1] = M + 3
    ring_b = ring.clone()
    tree_commit(ring, node_in, st, status)
    torch.cuda.synchronize()
    assert int(status) == 1 and torch.equal(ring, ring_b)


# ------------------------------------------------------------------ attention

def _attn_inputs(dev, seed, M, pos):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    maxlen = pos + M + 16
    qkv = torch.randn(M, QKV, device=dev, generator=gen).to(torch.bfloat16)
    qw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    kw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    cos, sin = rope_table(maxlen, RD, A_CFG.rope_theta, dev)
    k = torch.randn(HKV, pos, D, device=dev, generator=gen).to(torch.bfloat16).float()
    v = torch.randn(HKV, pos, D, device=dev, generator=gen).to(torch.bfloat16).float()
    kc = torch.zeros(HKV, maxlen, D, device=dev, dtype=F8)
    vc = torch.zeros_like(kc)
    ks, vs = torch.ones(HKV, maxlen, device=dev), torch.ones(HKV, maxlen, device=dev)
    if pos:
        ks[:, :pos] = k.abs().amax(-1).clamp(min=1e-6) / 448.0
        vs[:, :pos] = v.abs().amax(-1).clamp(min=1e-6) / 448.0
        kc[:, :pos] = torch.from_numpy(oat.fp8_encode(_np(k / ks[:, :pos, None]))).to(dev).view(F8)
        vc[:, :pos] = torch.from_numpy(oat.fp8_encode(_np(v / vs[:, :pos, None]))).to(dev).view(F8)
    return qkv, qw, kw, cos, sin, kc, vc, ks, vs


def _attn_run(dev, qkv, qw, kw, cos, sin, kc, vc, ks, vs, pos, parent_np):
    pos_t = torch.tensor([pos], device=dev)
    par = None if parent_np is None else torch.from_numpy(parent_np).to(dev)
    q = attn_prep(qkv, qw, kw, cos, sin, pos_t, kc, vc, A_CFG, ks, vs, parent=par)
    out = attn_decode_fused(q, qkv, kc, vc, pos_t, A_CFG, ks, vs, parent=par)
    torch.cuda.synchronize()
    return q, out


@pytest.mark.parametrize("kind,M,pos", [("random", 32, 1000), ("random", 32, 8192), ("star", 12, 64),
                                        ("chain", 32, 0), ("random", 7, 5)])
def test_attn_tree_matches_oracle(dev, kind, M, pos):
    print(f"attn tree {kind} M={M} pos={pos}", flush=True)
    parent = _tree(kind, M, 200 + M + pos)
    qkv, qw, kw, cos, sin, kc, vc, ks, vs = _attn_inputs(dev, 60 + M, M, pos)
    args = [_np(qkv), _np(qw), _np(kw), _np(cos), _np(sin), pos, parent, _codes(kc), _codes(vc), _np(ks), _np(vs)]
    q, out = _attn_run(dev, qkv, qw, kw, cos, sin, kc, vc, ks, vs, pos, parent)
    rout, rq, rkc, rvc, rks, rvs = oat.attn_tree(*args, HQ, HKV, D, RD, A_CFG.eps)
    gq = _np(q).reshape(M, HQ, D)
    assert np.mean(gq == rq) > 0.99 and np.abs(gq - rq).max() <= np.abs(rq).max() * 2 ** -7
    for got, want in ((_codes(kc), rkc), (_codes(vc), rvc)):
        assert np.array_equal(got[:, :pos], want[:, :pos]) and np.array_equal(got[:, pos + M:], want[:, pos + M:])
        assert np.mean(got[:, pos:pos + M] == want[:, pos:pos + M]) > 0.99
    assert np.allclose(_np(ks), rks, rtol=1e-2) and np.allclose(_np(vs), rvs, rtol=1e-6)
    go = _np(out)
    assert np.isfinite(go).all()
    for t in range(M):
        assert rel(go[t], rout[t]) < 5e-3, (t, rel(go[t], rout[t]))


def test_attn_tree_on_a_chain_equals_the_chain_kernel(dev):
    M, pos = 8, 2000
    parent = _tree("chain", M, 0)
    ins = _attn_inputs(dev, 9, M, pos)
    qkv, qw, kw, cos, sin, kc, vc, ks, vs = ins
    c = [t.clone() for t in (kc, vc, ks, vs)]
    q_c, out_c = _attn_run(dev, qkv, qw, kw, cos, sin, *c, pos, None)
    q_t, out_t = _attn_run(dev, qkv, qw, kw, cos, sin, kc, vc, ks, vs, pos, parent)
    assert torch.equal(q_t, q_c) and torch.equal(out_t, out_c)
    assert torch.equal(kc.view(torch.uint8), c[0].view(torch.uint8)) and torch.equal(ks, c[2])


def test_attn_tree_branch_isolation(dev):
    """Changing one branch's rows changes no output of the other branch, bit for bit."""
    M, pos = 32, 500
    parent = _tree("random", M, 77)
    ins = _attn_inputs(dev, 10, M, pos)
    qkv = ins[0]
    caches = [t.clone() for t in ins[5:]]
    _, out = _attn_run(dev, qkv, *ins[1:5], *caches, pos, parent)
    node = int(np.argmax(oa.tree_depths(parent)))
    on_path = set(og.root_path(parent, node))
    off = [t for t in range(M) if t not in on_path]
    qkv2 = qkv.clone()
    qkv2[off] = torch.randn(len(off), QKV, device=dev).to(torch.bfloat16)
    caches2 = [t.clone() for t in ins[5:]]
    _, out2 = _attn_run(dev, qkv2, *ins[1:5], *caches2, pos, parent)
    for t in sorted(on_path):
        assert torch.equal(out2[t], out[t]), t
