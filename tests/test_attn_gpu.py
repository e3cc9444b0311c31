"""GPU parity of the attention verify step (csrc/attn.hip through tr_attn_prep / tr_attn_decode)
against the numpy oracle (oracle/attn.py) at the config-5 head geometry (24 query heads, 4 kv
heads, head dim 256, rotary 64) over an FP8 cache of up to 8192 live rows, plus the reference's
own property (tokenrush tests/test_fused.py:98-124): an M-query step equals M one-query steps.
Tolerances: q and cache codes equal the oracle's except at rounding ties (>= 99% equal, the
rest within one bf16 / fp8 step); attention outputs within 5e-3 relative Frobenius (bf16 out;
the reference's multi-vs-sequential test allows 2e-2)."""
import numpy as np
import pytest
import torch

from oracle import attn as o
from tokenrush_amd.attn import NSPLIT, AttnConfig, attn_decode_fused, attn_prep, rope_table

pytestmark = pytest.mark.gpu
CFG = AttnConfig()
HQ, HKV, D, RD = CFG.n_heads, CFG.n_kv_heads, CFG.head_dim, CFG.rotary_dim
QKV = HQ * 2 * D + 2 * HKV * D
F8 = torch.float8_e4m3fn


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def _np(t):
    return t.float().cpu().numpy()


def _codes(t):
    return t.view(torch.uint8).cpu().numpy()


def _filled_cache(gen, dev, maxlen, L):
    """A cache whose rows 0..L-1 hold random keys/values written by the prep convention."""
    k = torch.randn(HKV, L, D, device=dev, generator=gen).to(torch.bfloat16).float()
    v = torch.randn(HKV, L, D, device=dev, generator=gen).to(torch.bfloat16).float()
    kc = torch.zeros(HKV, maxlen, D, device=dev, dtype=F8)
    vc = torch.zeros_like(kc)
    ks = torch.ones(HKV, maxlen, device=dev)
    vs = torch.ones_like(ks)
    ks[:, :L] = k.abs().amax(-1).clamp(min=1e-6) / 448.0
    vs[:, :L] = v.abs().amax(-1).clamp(min=1e-6) / 448.0
    kc[:, :L] = torch.from_numpy(o.fp8_encode(_np(k / ks[:, :L, None]))).to(dev).view(F8)
    vc[:, :L] = torch.from_numpy(o.fp8_encode(_np(v / vs[:, :L, None]))).to(dev).view(F8)
    return kc, vc, ks, vs


@pytest.mark.parametrize("M,pos", [(1, 0), (5, 37), (8, 8192)])
def test_attn_prep_matches_oracle(dev, M, pos):
    print(f"attn prep M={M} pos={pos}", flush=True)
    gen = torch.Generator(device=dev)
    gen.manual_seed(20 + M)
    maxlen = pos + M + 8
    qkv = torch.randn(M, QKV, device=dev, generator=gen).to(torch.bfloat16)
    qw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    kw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    cos, sin = rope_table(maxlen, RD, CFG.rope_theta, dev)
    kc = torch.zeros(HKV, maxlen, D, device=dev, dtype=F8)
    vc = torch.zeros_like(kc)
    ks, vs = torch.ones(HKV, maxlen, device=dev), torch.ones(HKV, maxlen, device=dev)
    q = attn_prep(qkv, qw, kw, cos, sin, torch.tensor([pos], device=dev), kc, vc, CFG, ks, vs)
    torch.cuda.synchronize()
    rq, rkc, rvc, rks, rvs = o.attn_prep(_np(qkv), _np(qw), _np(kw), _np(cos), _np(sin), pos,
                                         np.zeros((HKV, maxlen, D), np.uint8), np.zeros((HKV, maxlen, D), np.uint8),
                                         np.ones((HKV, maxlen), np.float32), np.ones((HKV, maxlen), np.float32),
                                         HQ, HKV, D, RD, CFG.eps)
    gq = _np(q).reshape(M, HQ, D)
    assert np.mean(gq == rq) > 0.99 and np.abs(gq - rq).max() <= np.abs(rq).max() * 2 ** -7
    for got, want in ((_codes(kc), rkc), (_codes(vc), rvc)):
        assert np.array_equal(got[:, :pos], want[:, :pos]) and np.array_equal(got[:, pos + M:], want[:, pos + M:])
        g8, w8 = o.fp8_decode(got[:, pos:pos + M]), o.fp8_decode(want[:, pos:pos + M])
        assert np.mean(got[:, pos:pos + M] == want[:, pos:pos + M]) > 0.99
        assert np.abs(g8 - w8).max() <= np.abs(w8).max() * 2 ** -3
    assert np.allclose(_np(ks), rks, rtol=1e-2) and np.allclose(_np(vs), rvs, rtol=1e-6)


@pytest.mark.parametrize("M,pos", [(1, 8192), (5, 1100), (8, 8192), (8, 3)])
def test_attn_decode_matches_oracle(dev, M, pos):
    print(f"attn decode M={M} pos={pos}", flush=True)
    gen = torch.Generator(device=dev)
    gen.manual_seed(30 + M)
    maxlen = pos + M + 16
    kc, vc, ks, vs = _filled_cache(gen, dev, maxlen, pos + M)
    q = (torch.randn(M, HQ * D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qkv = torch.randn(M, QKV, device=dev, generator=gen).to(torch.bfloat16)
    out = attn_decode_fused(q, qkv, kc, vc, torch.tensor([pos], device=dev), CFG, ks, vs)
    torch.cuda.synchronize()
    ref = o.attn_decode(_np(q).reshape(M, HQ, D), _np(qkv), _codes(kc), _codes(vc), _np(ks), _np(vs), pos, HQ, HKV, D,
                        nsplit=NSPLIT)
    got = _np(out)
    assert np.isfinite(got).all()
    for t in range(M):
        assert rel(got[t], ref[t]) < 5e-3, (t, rel(got[t], ref[t]))


def test_attn_multi_query_equals_sequential(dev):
    """tests/test_fused.py:98-124: prep + decode of M tokens at once vs one token at a time."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    M, pos, maxlen = 5, 1100, 1200
    qkv = torch.randn(M, QKV, device=dev, generator=gen).to(torch.bfloat16)
    qw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    kw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    cos, sin = rope_table(maxlen, RD, CFG.rope_theta, dev)
    base = _filled_cache(gen, dev, maxlen, pos)
    caches = [tuple(t.clone() for t in base) for _ in range(2)]
    kc, vc, ks, vs = caches[0]
    q = attn_prep(qkv, qw, kw, cos, sin, torch.tensor([pos], device=dev), kc, vc, CFG, ks, vs)
    y_multi = attn_decode_fused(q, qkv, kc, vc, torch.tensor([pos], device=dev), CFG, ks, vs)
    kc1, vc1, ks1, vs1 = caches[1]
    for t in range(M):
        p = torch.tensor([pos + t], device=dev)
        qt = attn_prep(qkv[t:t + 1], qw, kw, cos, sin, p, kc1, vc1, CFG, ks1, vs1)
        yt = attn_decode_fused(qt, qkv[t:t + 1], kc1, vc1, p, CFG, ks1, vs1)
        torch.cuda.synchronize()
        assert rel(_np(yt[0]), _np(y_multi[t])) < 2e-2, t
    assert torch.equal(kc.view(torch.uint8), kc1.view(torch.uint8)) and torch.equal(ks, ks1)


def test_attn_graph_replay(dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(8)
    M, pos, maxlen = 8, 2000, 2100
    qkv = torch.randn(M, QKV, device=dev, generator=gen).to(torch.bfloat16)
    qw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    kw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    cos, sin = rope_table(maxlen, RD, CFG.rope_theta, dev)
    kc, vc, ks, vs = _filled_cache(gen, dev, maxlen, pos)
    pos_t = torch.tensor([pos], device=dev)

    def step():
        q = attn_prep(qkv, qw, kw, cos, sin, pos_t, kc, vc, CFG, ks, vs)
        return attn_decode_fused(q, qkv, kc, vc, pos_t, CFG, ks, vs)

    y_eager = step().clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_g = step()
    for _ in range(3):
        y_g.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_g, y_eager)


def test_positions_past_the_cache_write_nothing_outside(dev):
    """A device position with pos + M beyond the cache (maxlen rows): the prep writes rows
    pos..maxlen-1 only and leaves every other row of the allocation alone (the next kv head's
    first rows, where an unguarded write of head j's row maxlen would land), and decode reads
    at most maxlen rows."""
    print("attn past the cache", flush=True)
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    M, maxlen = 6, 64
    pos = maxlen - 2                                   # tokens 2..5 fall outside the cache
    qkv = torch.randn(M, QKV, device=dev, generator=gen).to(torch.bfloat16)
    qw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    kw = (torch.randn(D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    cos, sin = rope_table(maxlen, RD, CFG.rope_theta, dev)
    kc, vc, ks, vs = _filled_cache(gen, dev, maxlen, maxlen - 2)
    before = [t.clone() for t in (kc, vc, ks, vs)]
    pos_t = torch.tensor([pos], device=dev)
    q = attn_prep(qkv, qw, kw, cos, sin, pos_t, kc, vc, CFG, ks, vs)
    out = attn_decode_fused(q, qkv, kc, vc, pos_t, CFG, ks, vs)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    for t, t0 in zip((kc, vc), before[:2]):
        assert torch.equal(t[:, :pos].view(torch.uint8), t0[:, :pos].view(torch.uint8))
        assert not torch.equal(t[:, pos:].view(torch.uint8), t0[:, pos:].view(torch.uint8))
    for t, t0 in zip((ks, vs), before[2:]):
        assert torch.equal(t[:, :pos], t0[:, :pos])
    # the two in-cache tokens match a call whose cache is long enough for all six
    big = maxlen + 8
    cos2, sin2 = rope_table(big, RD, CFG.rope_theta, dev)
    kc2 = torch.zeros(HKV, big, D, device=dev, dtype=F8)
    vc2 = torch.zeros_like(kc2)
    ks2, vs2 = torch.ones(HKV, big, device=dev), torch.ones(HKV, big, device=dev)
    attn_prep(qkv, qw, kw, cos2, sin2, pos_t, kc2, vc2, CFG, ks2, vs2)
    torch.cuda.synchronize()
    assert torch.equal(kc[:, pos:].view(torch.uint8), kc2[:, pos:maxlen].view(torch.uint8))
    assert torch.equal(ks[:, pos:], ks2[:, pos:maxlen])
