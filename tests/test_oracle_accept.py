"""Pins the accept oracle (oracle/accept.py): against numpy/torch library routines, brute force
on tiny inputs, the reference's own sampler tests (tests/test_sample.py:24-50 restated as
properties) and the invariants of speculative sampling. No GPU."""
import math

import numpy as np
import pytest
import torch

from oracle import accept as a
from oracle.int4 import bf16_round

F = np.float32


def test_texp_accuracy_and_edges():
    x = np.linspace(-80, 0, 400001, dtype=F)
    y = a.texp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert np.max(np.abs(y - ref) / ref) < 2e-7
    assert a.texp(np.array([0.0], F))[0] == 1.0
    assert a.texp(np.array([-80.5, -1e30, -np.inf], F)).tolist() == [0.0, 0.0, 0.0]
    # monotone on a fine grid (what the inverse-CDF search relies on)
    assert np.all(np.diff(a.texp(np.linspace(-20, 0, 100001, dtype=F))) >= 0)


def test_argmax_first_index_on_ties():
    lg = np.array([[1.0, 3.0, 3.0, -1.0], [0.0, 0.0, 0.0, 0.0]], dtype=F)
    assert a.argmax_rows(lg).tolist() == [1, 0]
    rng = np.random.default_rng(0)
    m = bf16_round(rng.standard_normal((8, 5000)).astype(F) * 2)
    assert np.array_equal(a.argmax_rows(m), torch.from_numpy(m).argmax(-1).numpy())


def test_top64_stable_order_brute_force():
    rng = np.random.default_rng(1)
    row = bf16_round(rng.standard_normal(3000).astype(F) * 2)          # many bf16 ties
    vals, idx = a.top64(row)
    pairs = sorted(((-float(row[i]), i) for i in range(row.shape[0])))[:64]
    assert idx.tolist() == [i for _, i in pairs]
    assert np.array_equal(vals, row[idx])
    assert len(set(row[idx].tolist())) < 64                               # ties were exercised


def test_top64_matches_torch_on_distinct_values():
    rng = np.random.default_rng(2)
    row = rng.permutation(5000).astype(F) / F(100)                        # all distinct
    vals, idx = a.top64(row)
    tv, ti = torch.from_numpy(row).topk(64)
    assert np.array_equal(vals, tv.numpy()) and np.array_equal(idx, ti.numpy())


def test_sample_greedy_is_argmax():
    rng = np.random.default_rng(3)
    lg = bf16_round(rng.standard_normal((4, 1000)).astype(F))
    u = rng.random(4).astype(F)
    assert np.array_equal(a.sample(lg, 0.0, 1.0, 64, u), a.argmax_rows(lg))


def test_sample_probabilities_match_torch_softmax():
    """On a tie-free row the fixed-order fp32 softmax equals torch's to a few ulp."""
    rng = np.random.default_rng(4)
    row = rng.permutation(4000).astype(F) / F(500)
    vals, _ = a.top64(row)
    v = (vals / F(0.7)).astype(F)
    e = a.texp((v - v[0]).astype(F))
    p = e / np.cumsum(e, dtype=F)[-1]
    ref = torch.softmax(torch.from_numpy(vals) / 0.7, 0).numpy()
    assert np.max(np.abs(p - ref)) < 1e-6


def test_sample_masks_and_frequencies():
    """Restates the reference's tests/test_sample.py:24-50 on the oracle."""
    lg = np.zeros((1, 1000), dtype=F)
    lg[0, :8] = [4.0, 3.5, 3.0, 2.0, 1.0, 0.5, 0.0, -1.0]
    n = 20000
    u = np.random.default_rng(5).random(n).astype(F)
    draws = np.array([a.sample(lg, 1.0, 1.0, 3, u[i:i + 1])[0] for i in range(n)])
    assert draws.max() <= 2
    freq = np.bincount(draws, minlength=3) / n
    ref = np.exp([4.0, 3.5, 3.0]) / np.exp([4.0, 3.5, 3.0]).sum()
    assert np.abs(freq - ref).max() < 0.02
    vals, idx = a.top64(lg[0])
    full = np.exp(vals - vals.max()) / np.exp(vals - vals.max()).sum()
    cum = np.cumsum(full)
    kept = set(idx[:int(((cum - full) < 0.7).sum())].tolist())
    draws = {int(a.sample(lg, 1.0, 0.7, 64, u[i:i + 1])[0]) for i in range(2000)}
    assert draws <= kept
    draws = np.array([a.sample(lg, 0.05, 1.0, 64, u[i:i + 1])[0] for i in range(500)])
    assert (draws == 0).mean() > 0.99


def test_sample_inverse_cdf_brute_force():
    """Tiny case computed by hand: three candidates with known masses."""
    lg = np.full((1, 100), -1e4, dtype=F)
    lg[0, [7, 3, 9]] = [0.0, math.log(2.0), math.log(4.0)]               # p = 1/7, 2/7, 4/7
    lg = bf16_round(lg)
    p = np.exp(lg[0, [9, 3, 7]].astype(np.float64))
    cdf = np.cumsum(p / p.sum())
    for uu, want in [(0.0, 9), (cdf[0] - 1e-3, 9), (cdf[0] + 1e-3, 3), (cdf[1] + 1e-3, 7), (0.999, 7)]:
        assert a.sample(lg, 1.0, 1.0, 64, np.array([uu], F))[0] == want


def test_sample_kept_ranks_are_a_prefix():
    """The top-p / top-k kept set is a prefix of the ranks, so the running sums of the kept p
    are the running sums of p up to the last kept rank and constant after it, bit for bit (the
    device kernel takes them from the one pass). Holds because p is sorted descending and
    fl(c + p) >= c: cum - p never decreases, nor does its rounding. Checked with the oracle's own
    arithmetic on rows with long flat tails, heavy ties and tiny masses."""
    rng = np.random.default_rng(11)
    for trial in range(600):
        kind = trial % 4
        if kind == 0:
            row = rng.standard_normal(4096) * 3
        elif kind == 1:
            row = np.round(rng.standard_normal(4096), 1)                  # heavy ties
        elif kind == 2:
            row = np.where(rng.random(4096) < 0.01, 30.0, rng.standard_normal(4096))  # a few dominate
        else:
            row = rng.standard_normal(4096) * 0.01                         # near-uniform, tiny masses
        vals, _ = a.top64(bf16_round(row.astype(F)))
        T = F([0.3, 1.0, 2.5][trial % 3])
        v = (vals / T).astype(F)
        e = a.texp((v - v[0]).astype(F))
        p = (e / np.cumsum(e, dtype=F)[-1]).astype(F)
        cum = np.cumsum(p, dtype=F)
        top_p, top_k = [(0.9, 64), (0.5, 40), (1.0, 7), (0.99, 64), (0.05, 64)][trial % 5]
        keep = ((cum - p).astype(F) < F(top_p)) & (np.arange(a.CANDIDATES) < top_k)
        n = int(keep.sum())
        assert n >= 1 and keep[:n].all() and not keep[n:].any()
        cum2 = np.cumsum(np.where(keep, p, F(0.0)).astype(F), dtype=F)
        assert np.array_equal(cum2.view(np.uint32), np.where(keep, cum, cum[n - 1]).astype(F).view(np.uint32))


def test_verify_chain_planted_prefix():
    rng = np.random.default_rng(6)
    for prefix in range(8):
        spec = rng.integers(0, 1000, 8).astype(np.int64)
        lg = a.planted_logits(8, 1000, seed=prefix, drafts_from=spec, prefix=prefix)
        pred = a.argmax_rows(lg)
        r = a.verify_chain(pred, spec, pos=100)
        expect = prefix
        while expect < 7 and pred[expect] == spec[expect + 1]:      # an accidental extra match
            expect += 1
        assert r["n"] == expect and r["tok"] == pred[expect] and r["pos"] == 100 + expect + 1
        assert r["tokens"][:-1] == spec[1:expect + 1].tolist() and r["commit"] == list(range(100, 101 + expect))


def _rows(M, V, seed, sigma=2.0):
    rng = np.random.default_rng(seed)
    return bf16_round((rng.standard_normal((M, V)) * sigma).astype(F))


def _probs(lg):
    e = np.exp(lg.astype(np.float64) - lg.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(F)


def test_blocked_sum_and_search_brute_force():
    rng = np.random.default_rng(7)
    r = rng.random(3000).astype(F)
    r[rng.random(3000) < 0.3] = 0
    tot = a.blocked_sum(r)
    assert abs(float(tot) - float(r.astype(np.float64).sum())) < 1e-3
    cum = np.cumsum(r.astype(np.float64))
    for t in rng.random(50) * float(tot):
        k = a.blocked_search(r, F(t))
        assert r[k] > 0
        assert cum[k] >= t - 1e-3 and (k == 0 or cum[k - 1] <= t + 1e-3)


def test_softmax_parts_per_chunk_exponentials():
    """e = fl(texp(l - m_c) texp(m_c - M)) against float64 exp(l - max) (relative 1e-6 where it
    is normal), Z against the float64 sum of e (1e-6), over rows whose chunks have very
    different maxima; a one-chunk row is exactly the single-maximum form texp(l - M)."""
    rng = np.random.default_rng(31)
    for V in (1000, 5000, 9000):
        lg = bf16_round((rng.standard_normal(V) * 3).astype(F))
        lg[: min(V, 1024)] -= F(30.0)                                # a chunk far below the maximum
        lg = bf16_round(lg)
        e, Z = a.softmax_parts(lg)
        ref = np.exp(lg.astype(np.float64) - lg.max())
        big = ref > 1e-30
        assert np.all(np.abs(e[big] - ref[big]) <= 1e-6 * ref[big])
        assert np.all(e[~big] < 1e-29)
        assert abs(float(Z) - e.astype(np.float64).sum()) <= 1e-6 * float(Z)
        assert e.argmax() == lg.argmax() and e.max() == F(1.0)
    one = bf16_round((rng.standard_normal(700) * 3).astype(F))
    e1, _ = a.softmax_parts(one)
    assert np.array_equal(e1, a.texp((one - one.max()).astype(F)))


def test_residual_p_equals_q_accepts_all():
    lg = _rows(8, 2048, seed=8)
    parts = [a.softmax_parts(lg[i]) for i in range(7)]
    q = np.stack([(e * a.residual_inv(Z)).astype(F) for e, Z in parts])   # q = the oracle's own p exactly
    drafts = np.random.default_rng(9).integers(0, 2048, 7)
    u = np.random.default_rng(10).random(8).astype(F) * F(0.999)
    r = a.residual_accept(lg, q, drafts, u)
    assert r["n"] == 7


def test_residual_one_hot_draft_accept_rate():
    """q one-hot at d: accepted iff u < p(d), so over many u the rate is p(d)."""
    lg = _rows(2, 1024, seed=11)
    d = 17
    q = np.zeros((1, 1024), F)
    q[0, d] = 1
    e, Z = a.softmax_parts(lg[0])
    pd = float(e[d] / Z)
    us = np.random.default_rng(12).random((4000, 2)).astype(F)
    acc = np.mean([a.residual_accept(lg, q, np.array([d]), us[i])["n"] for i in range(4000)])
    assert abs(acc - pd) < 4 * math.sqrt(pd * (1 - pd) / 4000) + 1e-3


def test_residual_output_distribution_is_target():
    """The first emitted token is distributed as p_0 whatever q is (speculative sampling's
    guarantee): chi-square over 6000 draws on a 1024-token vocabulary with 8 heavy tokens."""
    V = 1024
    rng = np.random.default_rng(13)
    lg = np.full((2, V), -20.0, F)
    lg[:, :8] = rng.standard_normal((2, 8)).astype(F)
    lg = bf16_round(lg)
    qlg = np.full((1, V), -20.0, F)
    qlg[0, :8] = rng.standard_normal(8).astype(F)
    q = _probs(qlg)
    p0 = _probs(lg)[0]
    n = 6000
    counts = np.zeros(V)
    qd = q[0].astype(np.float64)
    qd /= qd.sum()
    for i in range(n):
        dd = np.array([rng.choice(V, p=qd)])
        r = a.residual_accept(lg, q, dd, rng.random(2).astype(F))
        counts[r["tokens"][0]] += 1
    exp = p0[:8] * n
    chi2 = ((counts[:8] - exp) ** 2 / exp).sum()
    assert chi2 < 24.3                                           # chi-square(7) at p = 0.001
    assert counts[8:].sum() <= 2


def test_tree_brute_force_and_chain_equivalence():
    rng = np.random.default_rng(14)
    for trial in range(30):
        n = int(rng.integers(2, 32))
        parent = a.random_tree(n, seed=trial)
        pred = rng.integers(0, 5, n)
        toks = rng.integers(0, 5, n)
        r = a.tree_accept(pred, toks, parent)
        depth = a.tree_depths(parent)
        best_d = 0
        for i in range(1, n):                     # bench/tree_accept.py:91-100, literally
            j, ok = i, True
            while j > 0 and ok:
                ok = toks[j] == pred[parent[j]]
                j = parent[j]
            if ok:
                best_d = max(best_d, int(depth[i]))
        assert r["n"] == best_d
        assert r["commit"][0] == 0 and len(r["commit"]) == best_d + 1
        for k in range(1, len(r["commit"])):
            assert parent[r["commit"][k]] == r["commit"][k - 1]
    chain = np.arange(-1, 7, dtype=np.int32)
    spec = rng.integers(0, 3, 8)
    pred = rng.integers(0, 3, 8)
    t = a.tree_accept(pred, spec, chain, pos=5)
    c = a.verify_chain(pred, spec, pos=5)
    assert (t["n"], t["tok"], t["pos"], t["tokens"]) == (c["n"], c["tok"], c["pos"], c["tokens"])


def test_random_tree_shape():
    parent = a.random_tree(32, seed=0)
    d = a.tree_depths(parent)
    assert parent[0] == -1 and np.all(parent[1:] < np.arange(1, 32)) and d.max() <= 7
    assert np.bincount(parent[1:], minlength=32).max() <= 4
