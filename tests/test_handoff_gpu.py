"""Cross-workgroup handoffs, repeated back to back.

The GEMM's in-kernel K-slot sum (M > 16), the fused lm_head argmax, the sampled and residual
accepts and the GDN head norm each pass data between workgroups through a last-arriver handoff:
agent-scope stores completed before a relaxed agent-scope counter atomic, agent-scope loads in
the last arriver. A handoff that read a partner's data before it was complete, or a counter left
non-zero, would make some call's output differ from the others'. Each case queues many calls
with no synchronisation between them (so they overlap in the hardware queues as in a step graph)
and requires every output to equal the first bit for bit; the first is also checked against the
path's own reference (the oracle, or the two-launch path) so that agreement is not with a wrong
answer."""
import numpy as np
import pytest
import torch

from oracle import accept as oa
from oracle import int4 as o
from oracle.int4 import f32_to_bf16_bits

pytestmark = pytest.mark.gpu
V_FULL = 248320
F = np.float32


def say(*a):
    print(*a, flush=True)


def _logits(lg):
    return torch.from_numpy(f32_to_bf16_bits(lg).view(np.int16)).to("cuda:0").view(torch.bfloat16)


def _state(M, pos):
    from tokenrush_amd.accept import AcceptState
    st = AcceptState(M, "cuda:0")
    st.pos.fill_(pos)
    return st


def _fields(st):
    return [getattr(st, n).clone() for n in ("pred", "n_accepted", "tok", "pos", "slot", "tokens", "commit")]


def _all_equal(outs, what):
    torch.cuda.synchronize()
    for i, out in enumerate(outs[1:], 1):
        for a, b in zip(out, outs[0]):
            assert torch.equal(a, b), (what, "call", i)


def test_gemm_slot_sum_repeated(dev):
    """M = 32 out mode: two K slots summed by the last-arriving slot workgroup, 40 calls."""
    from tokenrush_amd import gfx950
    say("handoff: gemm slot sum M=32 x40")
    N, K, M = 7168, 5120, 32
    assert gfx950.plan(N, K, M)[0] == 2
    p, s, m = o.make_weights(N, K, seed=21, dtype="fp16")
    B, sp, mp = gfx950.pack(torch.from_numpy(p).to(dev), torch.from_numpy(s).to(torch.float16).to(dev),
                            torch.from_numpy(m).to(torch.float16).to(dev))
    xn = o.make_x(M, K, seed=22)
    x = torch.from_numpy(xn).to(torch.bfloat16).to(dev)
    outs = [[gfx950.mul(x, B, sp, mp)] for _ in range(40)]
    ref = xn.astype(np.float64) @ o.weights_f64(p, s, m).T
    got = outs[0][0].float().cpu().numpy().astype(np.float64)
    assert np.abs(got - ref).max() <= np.abs(ref).max() * 2 ** -7   # the GEMM tests' reference bar
    _all_equal(outs, "gemm slot sum")


def test_lm_head_argmax_repeated(dev):
    """lm_head with the fused greedy argmax and accept (grid-wide last arriver), 30 calls, each
    from a fresh state; the first equals the two-launch path (lm_head, then tr_accept_greedy)."""
    from tokenrush_amd.accept import accept_greedy, lm_head_greedy
    from tokenrush_amd.quant import QLinear
    say("handoff: lm_head argmax x30")
    V, K, M = 65536, 5120, 8
    g = torch.Generator(device=dev).manual_seed(23)
    q = torch.randint(0, 256, (V, K // 2), dtype=torch.uint8, device=dev, generator=g)
    s = (torch.rand(V, K // 128, device=dev, generator=g) * 0.018 + 0.002).to(torch.bfloat16)
    m = (torch.rand(V, K // 128, device=dev, generator=g) * 0.14 - 0.15).to(torch.bfloat16)
    lin = QLinear(q, s, m)
    del q
    h = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    logits = lin(h)
    spec = torch.randint(0, V, (M,), device=dev, generator=g)
    spec[1:4] = logits.float().argmax(-1)[:3]
    st_ref = _state(M, 50)
    accept_greedy(logits, spec, st_ref)
    outs = []
    for _ in range(30):
        st = _state(M, 50)
        lm_head_greedy(lin, h, spec, st)
        outs.append(_fields(st))
    _all_equal([_fields(st_ref)] + outs, "lm_head argmax")


def test_accept_sampled_repeated(dev):
    """Sampled accept (chunk top-64 lists merged by each row's last arriver, then the all-rows
    finish): 30 calls on config-3 logits; the first equals the oracle."""
    from tokenrush_amd.accept import accept_sampled
    from tokenrush_amd.sample import SamplingParams
    say("handoff: sampled accept x30")
    p = SamplingParams(dev)
    p.set(temperature=1.0, top_p=0.95, top_k=64)
    rng = np.random.default_rng(24)
    spec = rng.integers(0, V_FULL, 8).astype(np.int64)
    lg = oa.planted_logits(8, V_FULL, seed=25, drafts_from=spec, prefix=3)
    for i in range(3):
        lg[i, spec[i + 1]] = 60.0
    u = rng.random(8).astype(F)
    x, sd, ud = _logits(lg), torch.from_numpy(spec).to(dev), torch.from_numpy(u).to(dev)
    outs = []
    for _ in range(30):
        st = _state(8, 50)
        accept_sampled(x, sd, p, st, ud)
        outs.append(_fields(st))
    torch.cuda.synchronize()
    assert np.array_equal(outs[0][0].cpu().numpy(), oa.sample(lg, 1.0, 0.95, 64, u))
    _all_equal(outs, "sampled accept")


def test_accept_residual_repeated(dev):
    """Residual accept (phase 2's row handoffs, phase 3's chunk search): 30 calls; the first
    equals the oracle."""
    from tokenrush_amd.accept import accept_residual
    say("handoff: residual accept x30")
    rng = np.random.default_rng(26)
    K = 7
    ql = rng.standard_normal((K, V_FULL)) * 2.0
    e = np.exp(ql - ql.max(-1, keepdims=True))
    q = (e / e.sum(-1, keepdims=True)).astype(F)
    spec = rng.integers(0, V_FULL, K + 1).astype(np.int64)
    lg = oa.planted_logits(K + 1, V_FULL, seed=27, drafts_from=spec, prefix=2)
    u = rng.random(K + 1).astype(F)
    ref = oa.residual_accept(lg, q, spec[1:], u, pos=7)
    x, qd = _logits(lg), torch.from_numpy(q).to(dev)
    sd, ud = torch.from_numpy(spec).to(dev), torch.from_numpy(u).to(dev)
    outs = []
    for _ in range(30):
        st = _state(8, 7)
        accept_residual(x, qd, sd, ud, st)
        outs.append(_fields(st))
    torch.cuda.synchronize()
    assert int(outs[0][1]) == ref["n"] and outs[0][5].cpu().tolist()[:ref["n"] + 1] == ref["tokens"]
    _all_equal(outs, "residual accept")


def test_gdn_head_norm_repeated(dev):
    """GDN step at the config-5 layer shape (each head's last column-block workgroup applies the
    gated norm to the head's outputs): 20 calls from copies of one state; every output and state
    equal."""
    from tokenrush_amd.gdn import GDNConfig, RING, gdn_step_fused
    say("handoff: gdn head norm x20")
    cfg = GDNConfig()
    H, HV, K, V, HID, C = cfg.gdn_k_heads, cfg.gdn_v_heads, cfg.gdn_k_dim, cfg.gdn_v_dim, cfg.hidden, cfg.conv_dim
    g = torch.Generator(device=dev).manual_seed(28)
    bf = torch.bfloat16
    ba = (torch.randn(2 * HV, HID, device=dev, generator=g) * 0.02).to(bf)
    conv = (torch.randn(C, 4, device=dev, generator=g) * 0.3).to(bf)
    A = -torch.exp(torch.randn(HV, device=dev, generator=g))
    dt = torch.randn(HV, device=dev, generator=g)
    nw = (1 + 0.5 * torch.randn(V, device=dev, generator=g)).to(bf)
    M = 8
    qkvz = torch.randn(M, C + HV * V, device=dev, generator=g).to(bf)
    x = torch.randn(M, HID, device=dev, generator=g).to(bf)
    ring0 = torch.randn(C, RING, device=dev, generator=g).to(bf)
    rec0 = torch.randn(8, HV, K, V, device=dev, generator=g) * 0.1
    slot, pos = torch.tensor([3], device=dev), torch.tensor([21], device=dev)
    outs = []
    for _ in range(20):
        ring, rec = ring0.clone(), rec0.clone()
        y = gdn_step_fused(qkvz, x, ba, ring, conv, A, dt, rec, slot, nw, pos, cfg, 1e-6)
        outs.append([y.clone(), ring, rec[:M].clone()])
        del rec
    _all_equal(outs, "gdn head norm")
