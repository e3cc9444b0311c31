"""Verify-step acceptance, restated from the reference in numpy -- TEST INFRASTRUCTURE ONLY.

Functions and what they restate:
  argmax_rows        torch argmax over bf16 logits, first index on ties (reference
                     tokenrush/sample.py:37-38; the greedy pick of Engine._verify_step).
  top64              torch topk(logits.float(), 64) (sample.py:36) with an explicit tie rule:
                     descending value, ascending index (torch leaves the tie order unspecified,
                     sample.py:37-38 notes it).
  sample             sample(logits, params, u) (sample.py:30-51), fp32, reductions in a fixed
                     sequential order.
  verify_chain       Engine._verify_step's accept and commit (model.py:293-312).
  softmax_row / blocked_sum / blocked_search / residual_accept
                     stochastic speculative sampling with the residual resample (Leviathan et
                     al. 2023, "Fast Inference from Transformers via Speculative Decoding",
                     Algorithm 1; Chen et al. 2023). The reference has no such code
                     (its sampled verify is sample() + leading-match, model.py:302-308).
  tree_accept        longest accepted root path of a draft tree (reference
                     bench/tree_accept.py:4-7 and :91-100, a host simulation there).

Fixed arithmetic, shared bit-for-bit with the HIP kernels (token-rush_amd/csrc/accept.hip):
  * exp is texp(): Cody-Waite reduction x = n ln2 + r (ln2 split hi/lo), a degree-7 Taylor
    polynomial of e^r in Horner form, then scaling by 2^n through the exponent bits; x < -80
    gives 0. Every operation is one fp32 rounding (no fused multiply-add).
  * Sums over the 64 candidates are sequential in rank order.
  * Sums over a vocabulary row are "blocked": sequential within runs of 16 elements,
    sequential over the 64 runs of each 1024-element chunk, sequential over the 4 chunks of a
    group, sequential over groups (the row is zero-padded to whole groups; adding +0.0 changes
    nothing). The inverse-CDF search descends the same levels.
  * The residual path's exponentials are taken per chunk: with m_c the chunk's maximum and M
    the row's, e = fl(texp(l - m_c) * texp(m_c - M)) (flushed to 0 below the smallest normal),
    and Z sums the chunks as fl(texp(m_c - M) * A_c), A_c the chunk's blocked sum of
    texp(l - m_c). No pass over the row has to wait for the row maximum. p = fl(e * fl(1 / Z)).

Pinning (tests/test_oracle_accept.py): texp against numpy's exp (relative error < 2e-7);
argmax/top64 against numpy argmax/lexsort; sample against brute-force cases, torch's own
topk/softmax on tie-free rows and the frequency tests of the reference's
tests/test_sample.py:24-50; verify_chain against hand-built planted prefixes; residual_accept
against its invariants (p == q accepts everything, a one-hot draft accepts with probability
p(d), the output token is distributed as p: chi-square over many uniforms); tree_accept against
a brute force over all root paths, and chain trees against verify_chain.
"""
import numpy as np

from .int4 import bf16_bits_to_f32

F = np.float32
CANDIDATES = 64
RUN, CHUNK, GROUP = 16, 1024, 4
FLT_MIN = np.finfo(np.float32).tiny            # smallest normal fp32


def _f(bits: int) -> np.float32:
    return np.uint32(bits).view(np.float32)


LOG2E, LN2_HI, LN2_LO = _f(0x3FB8AA3B), _f(0x3F317200), _f(0x35BFBE8E)
# 1/k! for k = 0..7, rounded to fp32
EXP_C = [_f(0x3F800000), _f(0x3F800000), _f(0x3F000000), _f(0x3E2AAAAB), _f(0x3D2AAAAB), _f(0x3C088889),
         _f(0x3AB60B61), _f(0x39500D01)]
TEMP_MIN = _f(0x358637BD)      # 1e-6 (sample.py:41)


def texp(x) -> np.ndarray:
    """e^x for x <= 0 in fp32, the fixed algorithm above (x < -80 -> 0)."""
    x = np.asarray(x, dtype=F)
    small = ~(x >= F(-80.0))                  # also NaN
    x = np.where(small, F(-80.0), x).astype(F)
    t = x * LOG2E
    n = np.rint(t)
    r = x - n * LN2_HI
    r = r - n * LN2_LO
    p = EXP_C[7]
    for k in range(6, -1, -1):
        p = p * r + EXP_C[k]
    ni = np.clip(n, -126, 127).astype(np.int32)
    scale = ((ni + 127) << 23).astype(np.int32).view(F)
    y = (p * scale).astype(F)
    return np.where(small, F(0.0), y).astype(F)


def logits_f32(logits_bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> fp32 values (exact)."""
    return bf16_bits_to_f32(logits_bits)


# ------------------------------------------------------------------ argmax / top-64

def argmax_rows(logits: np.ndarray) -> np.ndarray:
    """[M, V] -> int64 [M]: index of the maximum, first index on ties."""
    return np.argmax(logits, axis=-1).astype(np.int64)


def top64(row: np.ndarray):
    """(values fp32 [64], indices int64 [64]) sorted by value descending, index ascending."""
    order = np.lexsort((np.arange(row.shape[0]), -row.astype(np.float64)))[:CANDIDATES]
    return row[order].astype(F), order.astype(np.int64)


# ------------------------------------------------------------------ sample() (sample.py:30-51)

def sample(logits: np.ndarray, temperature: float, top_p: float, top_k: int, u: np.ndarray) -> np.ndarray:
    """logits fp32 [M, V] (bf16 values), u fp32 [M] -> int64 [M]."""
    M = logits.shape[0]
    out = np.zeros(M, dtype=np.int64)
    T = F(temperature)
    temp = max(T, TEMP_MIN)
    for i in range(M):
        vals, idx = top64(logits[i])
        greedy = idx[0]
        if not T > 0:
            out[i] = greedy
            continue
        v = (vals / temp).astype(F)
        e = texp((v - v[0]).astype(F))
        Z = np.cumsum(e, dtype=F)[-1]
        p = (e / Z).astype(F)
        cum = np.cumsum(p, dtype=F)
        rank = np.arange(CANDIDATES)
        keep = ((cum - p).astype(F) < F(top_p)) & (rank < top_k)
        p2 = np.where(keep, p, F(0.0)).astype(F)
        cum2 = np.cumsum(p2, dtype=F)
        target = F(u[i]) * cum2[-1]
        pick = min(int(np.sum(cum2 < target)), CANDIDATES - 1)
        out[i] = idx[pick]
    return out


# ------------------------------------------------------------------ chain verify (model.py:293-312)

def verify_chain(pred: np.ndarray, spec_toks: np.ndarray, pos: int, slot: int = 0):
    """pred int64 [M] (the target's token per row), spec_toks int64 [M] (committed token then
    K = M - 1 drafts). Returns dict: n (accepted drafts), tok (pred[n], the bonus/correction),
    pos (pos + n + 1), slot (n), tokens ([drafts[:n], tok]), commit (positions pos..pos+n)."""
    M = pred.shape[0]
    match = (pred[:M - 1] == spec_toks[1:M]).astype(np.int64)
    n = int(np.cumprod(match).sum()) if M > 1 else 0
    tok = int(pred[n])
    return {"n": n, "tok": tok, "pos": pos + n + 1, "slot": n,
            "tokens": [int(t) for t in spec_toks[1:n + 1]] + [tok],
            "commit": list(range(pos, pos + n + 1))}


# ------------------------------------------------------------------ blocked reductions

def _padded(row: np.ndarray, fill=0.0) -> np.ndarray:
    V = row.shape[0]
    Vp = -(-V // CHUNK) * CHUNK
    out = np.full(Vp, fill, dtype=F)
    out[:V] = row
    return out


def _run_chunk_sums(x: np.ndarray):
    """x [nchunks, CHUNK] -> (run totals [nchunks, 64], chunk totals [nchunks])."""
    runs = np.cumsum(x.reshape(x.shape[0], CHUNK // RUN, RUN), axis=-1, dtype=F)[..., -1]
    chunks = np.cumsum(runs, axis=-1, dtype=F)[:, -1]
    return runs.astype(F), chunks.astype(F)


def group_parts(chunks: np.ndarray):
    """Chunk totals -> (group totals [ngroups], group prefixes [ngroups + 1]): sequential over
    the 4 chunks of a group (zero chunks pad the last group), then over groups."""
    ng = -(-chunks.shape[0] // GROUP)
    cp = np.zeros(ng * GROUP, F)
    cp[:chunks.shape[0]] = chunks
    groups = np.cumsum(cp.reshape(ng, GROUP), axis=-1, dtype=F)[:, -1].astype(F)
    pref = np.concatenate([[F(0.0)], np.cumsum(groups, dtype=F)]).astype(F)
    return groups, pref


def blocked_parts(row: np.ndarray):
    """(run totals [nchunks, 64], chunk totals [nchunks], group totals, group prefixes)."""
    runs, chunks = _run_chunk_sums(_padded(row).reshape(-1, CHUNK))
    groups, pref = group_parts(chunks)
    return runs, chunks, groups, pref


def blocked_sum(row: np.ndarray) -> np.float32:
    return blocked_parts(row)[3][-1]


def _level(acc, parts, target):
    """One level of the search: the first part whose running sum from acc exceeds target, else
    the last positive part; returns (index, running sum before it)."""
    a = acc
    for i, v in enumerate(parts):
        if F(a + v) > target:
            return i, a
        a = F(a + v)
    i = max(i for i, v in enumerate(parts) if v > 0)
    a = acc
    for v in parts[:i]:
        a = F(a + v)
    return i, a


def blocked_search(row: np.ndarray, target: np.float32) -> int:
    """First index whose blocked running sum exceeds target, found level by level (group, its
    chunks, the chunk's runs, the run's elements); at each level, when rounding leaves no
    crossing, the last positive part."""
    runs, chunks, groups, pref = blocked_parts(row)
    pr = _padded(row)
    nch = chunks.shape[0]
    g, _ = _level(F(0.0), list(groups), target)
    acc = pref[g]
    k, acc = _level(acc, [chunks[c] if c < nch else F(0.0) for c in range(GROUP * g, GROUP * g + GROUP)], target)
    c = GROUP * g + k
    t, acc = _level(acc, list(runs[c]), target)
    base = c * CHUNK + t * RUN
    e, _ = _level(acc, list(pr[base:base + RUN]), target)
    return base + e


def softmax_parts(row: np.ndarray):
    """(e, Z) for one fp32 row with per-chunk exponentials: m_c the chunk maxima, M the row's,
    f_c = texp(m_c - M), e = fl(texp(l - m_c) * f_c) (0 below the smallest normal),
    Z = group-blocked sum over chunks of fl(f_c * A_c), A_c = blocked chunk total of texp(l - m_c)."""
    V = row.shape[0]
    rp = _padded(row, -np.inf).reshape(-1, CHUNK)
    mc = rp.max(axis=1).astype(F)
    M = mc.max()
    a = texp((rp - mc[:, None]).astype(F))
    f = texp((mc - M).astype(F))
    e = (a * f[:, None]).astype(F)
    e = np.where(e < FLT_MIN, F(0.0), e).astype(F).reshape(-1)[:V]
    _, A = _run_chunk_sums(a)
    S = (f * A).astype(F)
    return e, group_parts(S)[1][-1]


# ------------------------------------------------------------------ residual rejection sampling

def residual_inv(Z) -> np.float32:
    """fl(1 / Z): the residual path's probabilities are p = fl(e * fl(1 / Z))."""
    return F(F(1.0) / F(Z))


def residual_accept(logits: np.ndarray, q: np.ndarray, drafts: np.ndarray, u: np.ndarray, pos: int = 0,
                    cache: dict = None):
    """logits fp32 [K+1, V] (target, temperature 1), q fp32 [K, V] (draft probabilities),
    drafts int64 [K], u fp32 [K+1]. Draft i is accepted when u[i] * q[i, d_i] < p[i, d_i]; at the
    first rejection j (or j = K when all pass) one token is drawn with u[K] by inverse CDF from
    max(p[j] - q[j], 0) (from p[K] when j = K). Returns dict like verify_chain plus 'pick'.
    cache: a dict kept by the caller across calls with the same logits and q (many drafts and
    uniforms); it holds each row's p and residual so they are computed once."""
    K = drafts.shape[0]
    cache = {} if cache is None else cache

    def prob(i):
        if ("p", i) not in cache:
            e, Z = softmax_parts(logits[i])
            cache[("p", i)] = (e * residual_inv(Z)).astype(F)
        return cache[("p", i)]

    n = 0
    for i in range(K):
        d = int(drafts[i])
        if F(F(u[i]) * F(q[i, d])) < prob(i)[d]:
            n += 1
        else:
            break
    if ("r", n) not in cache:
        p = prob(n)
        r = np.maximum((p - q[n]).astype(F), F(0.0)).astype(F) if n < K else p
        cache[("r", n)] = (r, blocked_sum(r))
    r, R = cache[("r", n)]
    if R > 0:
        tok = blocked_search(r, F(F(u[K]) * R))
    else:
        tok = int(np.argmax(logits[n]))  # the row's first maximum
    return {"n": n, "tok": tok, "pos": pos + n + 1, "slot": n,
            "tokens": [int(t) for t in drafts[:n]] + [tok], "commit": list(range(pos, pos + n + 1))}


# ------------------------------------------------------------------ tree accept

def tree_depths(parent: np.ndarray) -> np.ndarray:
    d = np.zeros(parent.shape[0], dtype=np.int64)
    for i in range(parent.shape[0]):
        d[i] = 0 if parent[i] < 0 else d[parent[i]] + 1
    return d


def tree_accept(pred: np.ndarray, tokens: np.ndarray, parent: np.ndarray, pos: int = 0):
    """Node 0 is the root (the committed token, parent -1); node i > 0 holds draft tokens[i]
    with parent[i] < i. Row i of the verify batch predicts the token after node i, so node i
    is accepted when tokens[i] == pred[parent[i]] and its parent is accepted. The accepted
    path ends at the deepest accepted node (lowest index among equals); n = its depth, the
    bonus token is pred[best]. commit = node indices root..best (rows to keep, in order),
    their tokens go to positions pos..pos+n. bench/tree_accept.py:91-100 restated: a node is
    accepted when every node on its root path matches."""
    Nn = parent.shape[0]
    depth = tree_depths(parent)
    ok = np.zeros(Nn, dtype=bool)
    ok[0] = True
    for i in range(1, Nn):
        ok[i] = ok[parent[i]] and tokens[i] == pred[parent[i]]
    best = 0
    for i in range(1, Nn):
        if ok[i] and depth[i] > depth[best]:
            best = i
    path = []
    j = best
    while j >= 0:
        path.append(j)
        j = int(parent[j])
    path = path[::-1]
    n = int(depth[best])
    tok = int(pred[best])
    return {"n": n, "tok": tok, "pos": pos + n + 1, "slot": best, "best": best,
            "tokens": [int(tokens[k]) for k in path[1:]] + [tok], "commit": path}


# ------------------------------------------------------------------ synthetic inputs (benchmark configs 3-4)

def planted_logits(M: int, V: int, seed: int, drafts_from: np.ndarray = None, prefix: int = 0, sigma: float = 2.0):
    """bf16-valued logits [M, V] ~ N(0, sigma^2); when drafts_from (int64 [M]) is given, the
    argmax of rows 0..prefix-1 is planted at drafts_from[1..prefix] (strictly above the row)."""
    from .int4 import bf16_round
    rng = np.random.default_rng(seed)
    lg = bf16_round((rng.standard_normal((M, V)) * sigma).astype(F))
    if drafts_from is not None:
        for i in range(prefix):
            lg[i, drafts_from[i + 1]] = bf16_round(np.array([lg[i].max() + 1.0], dtype=F))[0]
    return lg


def random_tree(n: int, seed: int, max_branch: int = 4, max_depth: int = 7) -> np.ndarray:
    """parent int32 [n]: node 0 the root; each later node picks a random earlier node with
    fewer than max_branch children and depth < max_depth."""
    rng = np.random.default_rng(seed)
    parent = np.full(n, -1, dtype=np.int32)
    depth = np.zeros(n, dtype=np.int64)
    kids = np.zeros(n, dtype=np.int64)
    for i in range(1, n):
        cands = [j for j in range(i) if kids[j] < max_branch and depth[j] < max_depth]
        j = int(rng.choice(cands))
        parent[i] = j
        depth[i] = depth[j] + 1
        kids[j] += 1
    return parent


def deep_branch_tree(n: int = 32) -> np.ndarray:
    """parent int32 [n] whose branch nodes sit deep: a chain 0..10, then nodes off depths 8, 9,
    10 and below (node 9, depth 9, has four children; node 12, depth 10, two), and the rest
    hung off the deepest chain. Exercises trees whose branch parents are deeper than a kernel's
    fixed state stack."""
    par = [-1] + list(range(10)) + [9, 9, 10, 12, 12, 14, 11, 15, 9, 13, 20, 17, 8]
    while len(par) < n:
        par.append(len(par) - 1)
    return np.array(par[:n], dtype=np.int32)
