"""Pins the GDN-step oracle (oracle/gdn.py): a float64 restatement in the reference's other
formulation (tokenrush/ops.py:150-161), the delta rule's closed forms, a brute-force causal
convolution over the whole history, the M-token == M one-token-steps property
(tokenrush tests/test_fused.py:73-95) and torch's bf16 ops for the gated norm. No GPU."""
import numpy as np
import torch

from oracle import gdn as o
from oracle.int4 import bf16_round

F32 = np.float32
H, HV, K, V, HID, R = 2, 4, 128, 128, 256, 16
C = 2 * H * K + HV * V


def _bf(rng, *shape, std=1.0):
    return bf16_round((rng.standard_normal(shape) * std).astype(F32))


def _layer(rng):
    return dict(ba_w=_bf(rng, 2 * HV, HID, std=0.05), conv_w=_bf(rng, C, 4, std=0.3),
                A=-np.exp(rng.standard_normal(HV)).astype(F32), dt_bias=rng.standard_normal(HV).astype(F32),
                norm_w=bf16_round(_bf(rng, V, std=0.5) + 1))


def _step(rng, w, ring, rec, slot, pos, M):
    qkvz, x = _bf(rng, M, C + HV * V), _bf(rng, M, HID)
    y, ring2, rec2 = o.gdn_step(qkvz, x, w["ba_w"], ring, w["conv_w"], w["A"], w["dt_bias"], rec, slot, w["norm_w"],
                                pos, H, HV, K, V, 1e-6)
    return qkvz, x, y, ring2, rec2


def test_delta_rule_closed_forms():
    rng = np.random.default_rng(0)
    S = rng.standard_normal((HV, K, V)).astype(F32)
    k = rng.standard_normal((HV, K)).astype(F32)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    q, v = rng.standard_normal((HV, K)).astype(F32), rng.standard_normal((HV, V)).astype(F32)
    # beta = 1, g = 0: the state now maps the (unit) key to exactly v
    _, S1 = o.delta_rule(q, k, v, np.zeros(HV, F32), np.ones(HV, F32), S)
    assert np.allclose(np.einsum("hk,hkv->hv", k, S1), v, atol=2e-4)
    # beta = 0: pure decay, and o = q^T S e^g
    g = -rng.random(HV).astype(F32)
    oo, S0 = o.delta_rule(q, k, v, g, np.zeros(HV, F32), S)
    assert np.allclose(S0, S * np.exp(g)[:, None, None], rtol=1e-6)
    assert np.allclose(oo, np.einsum("hk,hkv->hv", q, S0), rtol=1e-5, atol=1e-5)


def _history_conv(hist, w):
    """silu(bf16(causal conv)) over a whole history [T, C] (zeros before position 0)."""
    pad = np.concatenate([np.zeros((3, hist.shape[1]), F32), hist], 0).astype(np.float64)
    y = sum(pad[j:j + hist.shape[0]] * w[:, j].astype(np.float64) for j in range(4))
    yb = bf16_round(y.astype(F32))
    return bf16_round((yb / (1 + np.exp(-yb.astype(np.float64)))).astype(F32))


def test_conv_ring_matches_history_conv():
    rng = np.random.default_rng(1)
    Cs = 64
    w = _bf(rng, Cs, 4, std=0.3)
    ring = np.zeros((Cs, R), F32)
    hist, outs, pos = [], [], 0
    for M in [3, 8, 1, 5, 8, 2, 7, 8, 4, 6]:            # wraps the 16-column ring several times
        rows = _bf(rng, M, Cs)
        out, ring = o.conv_silu(rows, ring, w, pos)
        hist.append(rows)
        outs.append(out)
        pos += M
    ref = _history_conv(np.concatenate(hist, 0), w)
    got = np.concatenate(outs, 0)
    # the conv sum is fp32 in the oracle and fp64 here: they agree except at bf16 rounding ties
    assert np.mean(got == ref) > 0.99
    assert np.abs(got - ref).max() <= np.abs(ref).max() * 2 ** -7


def test_gates_match_float64_dot():
    rng = np.random.default_rng(2)
    x, ba = _bf(rng, 5, HID), _bf(rng, 2 * HV, HID, std=0.05)
    b, a = o.gates(x, ba, HV)
    ref = x.astype(np.float64) @ ba.astype(np.float64).T
    assert np.abs(b - ref[:, :HV]).max() <= np.abs(ref).max() * 2 ** -8
    assert np.abs(a - ref[:, HV:]).max() <= np.abs(ref).max() * 2 ** -8
    assert np.array_equal(b, bf16_round(b)) and np.array_equal(a, bf16_round(a))


def test_gated_rmsnorm_matches_torch_bf16_ops():
    """tokenrush/ops.py:10-19 restated with torch CPU: normalize fp32, cast, bf16 gain, fp32 gate."""
    rng = np.random.default_rng(3)
    ob, w, z = _bf(rng, 6, V), bf16_round(_bf(rng, V, std=0.5) + 1), _bf(rng, 6, V)
    y = o.gated_rmsnorm(ob, w, z, 1e-6)
    xt = torch.from_numpy(ob).bfloat16()
    xf = xt.float()
    hh = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    hh = torch.from_numpy(w).bfloat16() * hh.to(torch.bfloat16)
    ref = (hh * torch.nn.functional.silu(torch.from_numpy(z).float())).to(torch.bfloat16).float().numpy()
    assert np.mean(y == ref) > 0.97
    assert np.abs(y - ref).max() <= np.abs(ref).max() * 2 ** -7


def test_step_matches_float64_formulation():
    """ops.py:150-161 (gdn_step_reference) restated in float64, token by token, on the oracle's
    own conv outputs and bf16 gates (pinned above): states and head outputs agree to fp32 error."""
    rng = np.random.default_rng(4)
    w = _layer(rng)
    rec = (rng.standard_normal((8, HV, K, V)) * 0.1).astype(F32)
    ring = _bf(rng, C, R)
    pos, slot, M = 21, 3, 6
    qkvz, x, y, ring2, rec2 = _step(rng, w, ring, rec, slot, pos, M)
    conv, _ = o.conv_silu(qkvz[:, :C], ring, w["conv_w"], pos)
    b, a = o.gates(x, w["ba_w"], HV)
    S = rec[slot].astype(np.float64)
    QK = H * K
    for t in range(M):
        q = np.repeat(conv[t, :QK].reshape(H, K).astype(np.float64), HV // H, 0)
        k = np.repeat(conv[t, QK:2 * QK].reshape(H, K).astype(np.float64), HV // H, 0)
        v = conv[t, 2 * QK:].reshape(HV, V).astype(np.float64)
        q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) * K ** -0.5
        k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
        beta = bf16_round((1 / (1 + np.exp(-b[t].astype(np.float64)))).astype(F32)).astype(np.float64)
        sp = np.where(a[t] + w["dt_bias"] > 20, a[t] + w["dt_bias"], np.log1p(np.exp(a[t] + w["dt_bias"].astype(np.float64))))
        g = w["A"].astype(np.float64) * sp
        S = S * np.exp(g)[:, None, None]
        delta = (v - np.einsum("hk,hkv->hv", k, S)) * beta[:, None]
        S = S + k[:, :, None] * delta[:, None, :]
        oo = np.einsum("hk,hkv->hv", q, S)
        assert np.linalg.norm(rec2[t] - S) <= 1e-5 * np.linalg.norm(S), t
        yref = o.gated_rmsnorm(oo.astype(F32), w["norm_w"], qkvz[t, C:].reshape(HV, V), 1e-6).reshape(-1)
        assert np.linalg.norm(y[t] - yref) <= 1e-2 * np.linalg.norm(yref), t
    # slots M.. untouched, ring columns pos..pos+M-1 hold this step's conv inputs
    assert np.array_equal(rec2[M:], rec[M:])
    for t in range(M):
        assert np.array_equal(ring2[:, (pos + t) % R], qkvz[t, :C])


def test_multi_token_step_equals_single_steps():
    """tests/test_fused.py:73-95: an M-token step equals M one-token steps (outputs, ring, and the
    snapshot in slot t equals the state after token t)."""
    rng = np.random.default_rng(5)
    w = _layer(rng)
    rec0 = (rng.standard_normal((8, HV, K, V)) * 0.1).astype(F32)
    ring0 = _bf(rng, C, R)
    M, pos, slot = 5, 14, 2                             # the step wraps the ring
    qkvz, x = _bf(rng, M, C + HV * V), _bf(rng, M, HID)
    args = (w["ba_w"], w["conv_w"], w["A"], w["dt_bias"])
    y, ring_m, rec_m = o.gdn_step(qkvz, x, *args[:1], ring0, *args[1:], rec0, slot, w["norm_w"], pos, H, HV, K, V, 1e-6)
    ring, rec, s = ring0, rec0, slot
    for t in range(M):
        yt, ring, rec = o.gdn_step(qkvz[t:t + 1], x[t:t + 1], w["ba_w"], ring, w["conv_w"], w["A"], w["dt_bias"], rec,
                                   s, w["norm_w"], pos + t, H, HV, K, V, 1e-6)
        s = 0
        assert np.array_equal(yt[0], y[t])
        assert np.array_equal(rec[0], rec_m[t])
    assert np.array_equal(ring, ring_m)


def test_tree_step_on_a_chain_is_the_chain_step():
    """A chain tree (parent[t] = t - 1) reduces the tree oracle to gdn_step, bit for bit; the
    commit of the whole path leaves the ring the chain step leaves."""
    rng = np.random.default_rng(7)
    w = _layer(rng)
    rec0 = (rng.standard_normal((8, HV, K, V)) * 0.1).astype(F32)
    ring0 = _bf(rng, C, R)
    M, pos, slot = 6, 21, 3
    qkvz, x = _bf(rng, M, C + HV * V), _bf(rng, M, HID)
    args = (w["ba_w"], ring0, w["conv_w"], w["A"], w["dt_bias"], rec0, slot, w["norm_w"], pos)
    y, ring_c, rec_c = o.gdn_step(qkvz, x, *args, H, HV, K, V, 1e-6)
    parent = np.arange(-1, M - 1, dtype=np.int32)
    yt, rec_t = o.gdn_tree_step(qkvz, x, *args, parent, H, HV, K, V, 1e-6)
    assert np.array_equal(y, yt)
    assert np.array_equal(rec_c[:M], rec_t[:M])
    assert np.array_equal(o.tree_commit(ring0, qkvz[:, :C], list(range(M)), pos), ring_c)


def test_tree_branches_do_not_see_each_other():
    """Two children of the root: each one's output is the two-token chain [root, child], whatever
    the sibling holds."""
    rng = np.random.default_rng(8)
    w = _layer(rng)
    rec0 = (rng.standard_normal((8, HV, K, V)) * 0.1).astype(F32)
    ring0 = _bf(rng, C, R)
    pos, slot = 9, 0
    qkvz, x = _bf(rng, 3, C + HV * V), _bf(rng, 3, HID)
    args = (w["ba_w"], ring0, w["conv_w"], w["A"], w["dt_bias"], rec0, slot, w["norm_w"], pos)
    parent = np.array([-1, 0, 0], np.int32)
    y, rec = o.gdn_tree_step(qkvz, x, *args, parent, H, HV, K, V, 1e-6)
    for child in (1, 2):
        yc, _, rc = o.gdn_step(qkvz[[0, child]], x[[0, child]], *args, H, HV, K, V, 1e-6)
        assert np.array_equal(y[child], yc[1]) and np.array_equal(rec[child], rc[1])
    q2 = qkvz.copy()
    q2[2] = _bf(rng, C + HV * V)
    y2, _ = o.gdn_tree_step(q2, x, *args, parent, H, HV, K, V, 1e-6)
    assert np.array_equal(y2[1], y[1]) and not np.array_equal(y2[2], y[2])
