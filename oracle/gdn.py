"""The M-token gated-delta-rule (GDN) verify step, restated from the reference in numpy.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

bf16 tensors are float32 arrays holding bf16-representable values (oracle.int4.bf16_round).
Arithmetic is float32 in the reference's order of operations; reductions use numpy's order
(the GPU's differs), so comparisons with the HIP kernel are within tolerances, not bitwise.

Functions (reference file:line):
  conv_silu      -- tokenrush/fused.py:98-115 (_conv_ring) and ops.py:99-113 (conv_step): causal
                    conv of kernel 4 over the ring, fp32 products, bf16 round, silu, bf16 round.
  gates          -- fused.py:146-160: b/a = bf16(x . ba_w), fp32 accumulate.
  delta_rule     -- fused.py:179-186: S = S e^g; S += k (beta (v - k^T S))^T; o = q^T S.
  gdn_step       -- fused.py:119-210 (_gdn_step_fused_kernel) with BV == V: conv, gates,
                    L2-normalised q (times K^-1/2) and k, decay exp(g), delta rule, snapshot of
                    the state after every token into slot t, o = q^T S, gated RMSNorm.
  gated_rmsnorm  -- ops.py:10-19 and fused.py:196-204: bf16(o) normalised in fp32, cast, plain
                    gain in bf16, times silu(z) in fp32, cast.
  gdn_tree_step  -- no reference counterpart (the reference verifies chains only; its trees were a
                    host simulation, bench/tree_accept.py:91-100): by definition, node t of a draft
                    tree is gdn_step over its root path (root = node 0 at position pos), so its
                    output and state are that chain's last; the ring is not written.
  tree_commit    -- the ring a gdn_step over the accepted path would leave: columns
                    (pos + d) % R <- the path's conv inputs, d = 0..n (state.py:30-39 ring rule).

Pinning (tests/test_oracle_gdn.py):
  gdn_step       -- (1) a float64 restatement of the single-token update in the reference's
                    other formulation (ops.py:150-161, gdn_step_reference: S = S e^g;
                    delta = (v - k^T S) beta; S += k delta^T; o = q^T S), token by token;
                    (2) the delta rule's closed form: with beta = 1 and g = 0, k^T S_new = v for
                    the unit k; with beta = 0 the state only decays; (3) an M-token step equals M
                    one-token steps (the reference's tests/test_fused.py:73-95 property), state
                    snapshots included.
  conv_silu      -- a brute-force causal convolution over the whole token history (zeros before
                    position 0) after many steps that wrap the ring.
  gates          -- float64 dot products (a library routine) before the bf16 rounding.
  gated_rmsnorm  -- torch CPU restatement of ops.gated_rmsnorm (the reference's dtype order).
  gdn_tree_step  -- built from gdn_step (pinned above) by its definition; a chain tree
  tree_commit       (parent[t] = t - 1) reduces both to one gdn_step, bit for bit.
"""
import numpy as np

from .int4 import bf16_round

F32 = np.float32


def _silu(v):
    v = np.asarray(v, F32)
    return (v / (F32(1) + np.exp(-v))).astype(F32)


def conv_silu(rows, ring, conv_w, pos: int):
    """rows [M, C] (this step's conv inputs), ring [C, R], conv_w [C, 4], all bf16-valued ->
    (out [M, C] bf16-valued, new ring). Column (pos + t) % R holds the input at position pos + t;
    the window of token t is positions pos + t - 3 .. pos + t (fused.py:98-115)."""
    rows = np.asarray(rows, F32)
    ring = np.array(ring, F32, copy=True)
    M, C = rows.shape
    R = ring.shape[1]
    w = np.asarray(conv_w, F32)
    win = np.concatenate([ring[:, [(pos + j - 3) % R for j in range(3)]].T, rows], 0)   # [M + 3, C]
    out = np.empty((M, C), F32)
    for t in range(M):
        y = (win[t] * w[:, 0]).astype(F32)
        y = (y + win[t + 1] * w[:, 1]).astype(F32)
        y = (y + win[t + 2] * w[:, 2]).astype(F32)
        y = (y + win[t + 3] * w[:, 3]).astype(F32)
        out[t] = bf16_round(_silu(bf16_round(y)))
    for t in range(M):
        ring[:, (pos + t) % R] = rows[t]
    return out, ring


def gates(x, ba_w, HV: int):
    """x [M, hidden], ba_w [2 HV, hidden] bf16-valued -> (b, a) [M, HV] bf16-valued."""
    ba = np.asarray(x, F32) @ np.asarray(ba_w, F32).T
    return bf16_round(ba[:, :HV]), bf16_round(ba[:, HV:])


def gated_rmsnorm(o, w, z, eps: float):
    """o [.., V] fp32, w [V] and z [.., V] bf16-valued -> bf16-valued (ops.py:10-19)."""
    ob = bf16_round(np.asarray(o, F32))
    var = (ob * ob).astype(F32).sum(-1, keepdims=True, dtype=F32) / F32(ob.shape[-1])
    n = bf16_round((ob / np.sqrt(var + F32(eps))).astype(F32))
    n = bf16_round((np.asarray(w, F32) * n).astype(F32))
    return bf16_round((n * _silu(z)).astype(F32))


def softplus(v):
    v = np.asarray(v, F32)
    return np.where(v > 20, v, np.log1p(np.exp(np.minimum(v, 20)))).astype(F32)


def delta_rule(q, k, v, g, beta, S):
    """One token of the gated delta rule per value head (fused.py:179-186): q, k [HV, K] (already
    normalised), v [HV, V], g, beta [HV], S [HV, K, V] -> (o [HV, V], new S), fp32."""
    S = (S * np.exp(np.asarray(g, F32))[:, None, None]).astype(F32)
    kv = np.einsum("hk,hkv->hv", k, S).astype(F32)
    dv = (np.asarray(beta, F32)[:, None] * (v - kv)).astype(F32)
    S = (S + k[:, :, None] * dv[:, None, :]).astype(F32)
    return np.einsum("hk,hkv->hv", q, S).astype(F32), S


def gdn_step(qkvz, x, ba_w, ring, conv_w, A, dt_bias, rec, slot: int, norm_w, pos: int, H: int, HV: int,
             K: int, V: int, eps: float):
    """One M-token step (fused.py:119-210). qkvz [M, 2 H K + 2 HV V] (q | k | v | z), x [M, hidden],
    ba_w [2 HV, hidden], ring [C, R], conv_w [C, 4] bf16-valued; A, dt_bias [HV] fp32;
    rec [n_slots, HV, K, V] fp32 with the committed state in slot `slot`.
    Returns (y [M, HV V] bf16-valued, new ring, new rec with slots 0..M-1 = state after token t)."""
    qkvz = np.asarray(qkvz, F32)
    M = qkvz.shape[0]
    QK, VAL = H * K, HV * V
    C = 2 * QK + VAL
    conv, ring = conv_silu(qkvz[:, :C], ring, conv_w, pos)
    b, a = gates(x, ba_w, HV)
    rec = np.array(rec, F32, copy=True)
    S = rec[slot].copy()                                     # [HV, K, V]
    rep = HV // H
    scale = F32(K ** -0.5)
    y = np.empty((M, VAL), F32)
    for t in range(M):
        q = conv[t, :QK].reshape(H, K)
        k = conv[t, QK:2 * QK].reshape(H, K)
        v = conv[t, 2 * QK:].reshape(HV, V)
        q = (q / np.sqrt((q * q).sum(-1, keepdims=True, dtype=F32) + F32(1e-6)) * scale).astype(F32)
        k = (k / np.sqrt((k * k).sum(-1, keepdims=True, dtype=F32) + F32(1e-6))).astype(F32)
        q, k = np.repeat(q, rep, 0), np.repeat(k, rep, 0)   # value head hv uses key head hv // rep
        beta = bf16_round((F32(1) / (F32(1) + np.exp(-b[t]))).astype(F32))
        g = (np.asarray(A, F32) * softplus(a[t] + np.asarray(dt_bias, F32))).astype(F32)
        o, S = delta_rule(q, k, v, g, beta, S)
        rec[t] = S
        z = qkvz[t, C:].reshape(HV, V)
        y[t] = gated_rmsnorm(o, norm_w, z, eps).reshape(-1)
    return y, ring, rec


# ------------------------------------------------------------------ draft trees

def root_path(parent, t: int) -> list:
    """Node indices root..t of a draft tree (parent[t] < t, node 0 the root)."""
    path = [int(t)]
    while path[-1] > 0:
        path.append(int(parent[path[-1]]))
    return path[::-1]


def gdn_tree_step(qkvz, x, ba_w, ring, conv_w, A, dt_bias, rec, slot: int, norm_w, pos: int, parent, H: int, HV: int,
                  K: int, V: int, eps: float):
    """Draft-tree step: node t is gdn_step over its root path. Returns (y [M, HV V], rec with
    slot t = node t's state; the ring is unchanged)."""
    qkvz, x = np.asarray(qkvz, F32), np.asarray(x, F32)
    M = qkvz.shape[0]
    rec0 = np.array(rec, F32, copy=True)
    out_rec = rec0.copy()
    y = np.empty((M, HV * V), F32)
    for t in range(M):
        p = root_path(parent, t)
        yp, _, rp = gdn_step(qkvz[p], x[p], ba_w, ring, conv_w, A, dt_bias, rec0, slot, norm_w, pos, H, HV, K, V, eps)
        y[t] = yp[-1]
        out_rec[t] = rp[len(p) - 1]
    return y, out_rec


def tree_commit(ring, node_in, path, pos: int):
    """ring [C, R] after the accept of `path` (node indices root..best) whose root sat at pos;
    node_in [M, C] the nodes' conv inputs -> the new ring."""
    ring = np.array(ring, F32, copy=True)
    R = ring.shape[1]
    for d, node in enumerate(path):
        ring[:, (pos + d) % R] = np.asarray(node_in, F32)[node]
    return ring
