"""GPU parity of the GDN verify step (csrc/gdn.hip through tr_gdn_step) against the numpy oracle
(oracle/gdn.py) at the config-5 layer shape (16 key heads, 48 value heads, 128 x 128 state per
head, hidden 5120), plus the reference's own properties (tokenrush tests/test_fused.py:49-95):
an M-token step equals M one-token steps, snapshot slots hold the per-token states, and the ring
holds the conv inputs. Tolerances: the ring is bit-exact; states within 1e-4 relative Frobenius;
outputs y within 5e-3 relative Frobenius (bf16 outputs; the reference's own fused-vs-ops test
allows 2e-2)."""
import numpy as np
import pytest
import torch

from oracle import gdn as o
from tokenrush_amd.gdn import GDNConfig, RING, gdn_step_fused

pytestmark = pytest.mark.gpu
CFG = GDNConfig()
H, HV, K, V, HID = CFG.gdn_k_heads, CFG.gdn_v_heads, CFG.gdn_k_dim, CFG.gdn_v_dim, CFG.hidden
C = CFG.conv_dim
NSLOT = 8


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def _layer(gen, dev):
    bf = torch.bfloat16
    return dict(ba_w=(torch.randn(2 * HV, HID, device=dev, generator=gen) * 0.02).to(bf),
                conv_w=(torch.randn(C, 4, device=dev, generator=gen) * 0.3).to(bf),
                A=-torch.exp(torch.randn(HV, device=dev, generator=gen)),
                dt_bias=torch.randn(HV, device=dev, generator=gen),
                norm_w=(1 + 0.5 * torch.randn(V, device=dev, generator=gen)).to(bf))


def _np(t):
    return t.float().cpu().numpy()


def _run_both(dev, seed, M, pos, slot):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    w = _layer(gen, dev)
    qkvz = torch.randn(M, C + HV * V, device=dev, generator=gen).to(torch.bfloat16)
    x = torch.randn(M, HID, device=dev, generator=gen).to(torch.bfloat16)
    ring = torch.randn(C, RING, device=dev, generator=gen).to(torch.bfloat16)
    rec = torch.randn(NSLOT, HV, K, V, device=dev, generator=gen) * 0.1
    ring_np, rec_np = _np(ring), _np(rec)
    slot_t = torch.tensor([slot], device=dev)
    pos_t = torch.tensor([pos], device=dev)
    y = gdn_step_fused(qkvz, x, w["ba_w"], ring, w["conv_w"], w["A"], w["dt_bias"], rec, slot_t, w["norm_w"], pos_t,
                       CFG, 1e-6)
    torch.cuda.synchronize()
    ry, rring, rrec = o.gdn_step(_np(qkvz), _np(x), _np(w["ba_w"]), ring_np, _np(w["conv_w"]), _np(w["A"]),
                                 _np(w["dt_bias"]), rec_np, slot, _np(w["norm_w"]), pos, H, HV, K, V, 1e-6)
    return (_np(y), _np(ring), _np(rec)), (ry, rring, rrec), rec_np


@pytest.mark.parametrize("M,pos,slot", [(1, 0, 0), (2, 2, 1), (5, 14, 3), (8, 37, 7), (8, 1, 5), (3, 1000, 2)])
def test_gdn_step_matches_oracle(dev, M, pos, slot):
    print(f"gdn step M={M} pos={pos} slot={slot}", flush=True)
    (y, ring, rec), (ry, rring, rrec), rec0 = _run_both(dev, 10 + M, M, pos, slot)
    assert np.array_equal(ring, rring), "ring"
    for t in range(M):
        assert rel(rec[t], rrec[t]) < 1e-4, (t, rel(rec[t], rrec[t]))
    assert np.array_equal(rec[M:], rec0[M:]) or M == NSLOT, "slots >= M must be untouched"
    assert np.isfinite(y).all()
    for t in range(M):
        assert rel(y[t], ry[t]) < 5e-3, (t, rel(y[t], ry[t]))


def test_gdn_multi_token_equals_single_steps(dev):
    """tests/test_fused.py:73-95 on the GPU: one M-token step vs M one-token steps."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    w = _layer(gen, dev)
    M, pos = 6, 12
    qkvz = torch.randn(M, C + HV * V, device=dev, generator=gen).to(torch.bfloat16)
    x = torch.randn(M, HID, device=dev, generator=gen).to(torch.bfloat16)
    ring0 = torch.randn(C, RING, device=dev, generator=gen).to(torch.bfloat16)
    rec0 = torch.randn(NSLOT, HV, K, V, device=dev, generator=gen) * 0.1
    ring_m, rec_m = ring0.clone(), rec0.clone()
    y_m = gdn_step_fused(qkvz, x, w["ba_w"], ring_m, w["conv_w"], w["A"], w["dt_bias"], rec_m,
                         torch.tensor([1], device=dev), w["norm_w"], torch.tensor([pos], device=dev), CFG, 1e-6)
    ring_s, rec_s = ring0.clone(), rec0.clone()
    slot = torch.tensor([1], device=dev)
    for t in range(M):
        y_t = gdn_step_fused(qkvz[t:t + 1], x[t:t + 1], w["ba_w"], ring_s, w["conv_w"], w["A"], w["dt_bias"], rec_s,
                             slot, w["norm_w"], torch.tensor([pos + t], device=dev), CFG, 1e-6)
        slot = torch.tensor([0], device=dev)
        torch.cuda.synchronize()
        assert rel(_np(y_t[0]), _np(y_m[t])) < 1e-2, t
        assert rel(_np(rec_s[0]), _np(rec_m[t])) < 1e-3, t
    assert torch.equal(ring_s, ring_m)


def test_gdn_step_graph_replay(dev):
    """The step captured in a hipGraph: every replay (inputs reset between replays, with eager
    work and synchronisation in between) reproduces the eager result bit for bit."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    w = _layer(gen, dev)
    M = 8
    qkvz = torch.randn(M, C + HV * V, device=dev, generator=gen).to(torch.bfloat16)
    x = torch.randn(M, HID, device=dev, generator=gen).to(torch.bfloat16)
    ring0 = torch.randn(C, RING, device=dev, generator=gen).to(torch.bfloat16)
    rec0 = torch.randn(NSLOT, HV, K, V, device=dev, generator=gen) * 0.1
    ring, rec = ring0.clone(), rec0.clone()
    slot_t, pos_t = torch.tensor([2], device=dev), torch.tensor([9], device=dev)
    call = lambda: gdn_step_fused(qkvz, x, w["ba_w"], ring, w["conv_w"], w["A"], w["dt_bias"], rec, slot_t,
                                  w["norm_w"], pos_t, CFG, 1e-6)
    y_eager = call().clone()
    rec_eager, ring_eager = rec.clone(), ring.clone()
    ring.copy_(ring0)
    rec.copy_(rec0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_g = call()
    for _ in range(3):
        ring.copy_(ring0)
        rec.copy_(rec0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_g, y_eager)
        assert torch.equal(rec, rec_eager)
        assert torch.equal(ring, ring_eager)


def test_gdn_step_rejects_bad_shapes(dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    w = _layer(gen, dev)
    M = 9
    qkvz = torch.zeros(M, C + HV * V, device=dev, dtype=torch.bfloat16)
    x = torch.zeros(M, HID, device=dev, dtype=torch.bfloat16)
    ring = torch.zeros(C, RING, device=dev, dtype=torch.bfloat16)
    rec = torch.zeros(16, HV, K, V, device=dev)
    one = torch.zeros(1, dtype=torch.int64, device=dev)
    with pytest.raises(RuntimeError):
        gdn_step_fused(qkvz, x, w["ba_w"], ring, w["conv_w"], w["A"], w["dt_bias"], rec, one, w["norm_w"], one, CFG,
                       1e-6)


def test_workspace_shared_by_calls_of_different_shapes(dev):
    """One zero-filled workspace serves calls with different head counts in any order: the
    arrival counters sit at a fixed place, so a small call's head outputs never land on a larger
    call's counters (the step of the small hybrid, then the full-size head count)."""
    from tokenrush_amd import gdn as gmod
    print("gdn workspace shared across shapes", flush=True)
    small = GDNConfig(512, 2, 4, K, V)
    for cfg, seed in ((small, 1), (CFG, 2), (small, 3), (CFG, 4)):
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        Hs, HVs, hid = cfg.gdn_k_heads, cfg.gdn_v_heads, cfg.hidden
        C = 2 * Hs * K + HVs * V
        M, pos, slot = 8, 21, 0
        qkvz = torch.randn(M, C + HVs * V, device=dev, generator=gen).to(torch.bfloat16)
        x = torch.randn(M, hid, device=dev, generator=gen).to(torch.bfloat16)
        ba = (torch.randn(2 * HVs, hid, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        ring = torch.randn(C, RING, device=dev, generator=gen).to(torch.bfloat16)
        conv = (torch.randn(C, 4, device=dev, generator=gen) * 0.3).to(torch.bfloat16)
        A = -torch.exp(torch.randn(HVs, device=dev, generator=gen))
        dt = torch.randn(HVs, device=dev, generator=gen)
        nw = (torch.randn(V, device=dev, generator=gen) * 0.5 + 1).to(torch.bfloat16)
        rec = torch.randn(8, HVs, K, V, device=dev, generator=gen) * 0.1
        want = o.gdn_step(_np(qkvz), _np(x), _np(ba), _np(ring), _np(conv), _np(A), _np(dt), _np(rec), slot, _np(nw),
                           pos, Hs, HVs, K, V, 1e-6)[0]
        y = gdn_step_fused(qkvz, x, ba, ring, conv, A, dt, rec, torch.tensor([slot], device=dev), nw,
                           torch.tensor([pos], device=dev), cfg, 1e-6)
        torch.cuda.synchronize()
        got = _np(y)
        assert np.isfinite(got).all(), (HVs, seed)
        assert np.linalg.norm(got - want) <= 5e-3 * np.linalg.norm(want), (HVs, seed)
        assert gmod.workspace(M, Hs, HVs, dev).numel() >= _lib_ws(M, Hs, HVs)


def _lib_ws(M, H, HV):
    from tokenrush_amd import _lib
    return int(_lib.lib().tr_gdn_workspace_bytes(M, H, HV))
