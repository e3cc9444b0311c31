"""On-device accept/commit of the speculative verify step.

Mirrors Engine._verify_step (reference tokenrush/model.py:293-312): after the verify batch's
logits, the target's token per row is compared with the next draft, the accepted prefix is
counted and committed -- n_accepted, tok (the correction or bonus token), pos += n + 1 and the
recurrent-state slot -- all on the device, with no host read, so the step captures in one
graph. Adds the two acceptance rules the reference only simulates or lacks: residual
rejection sampling against draft probabilities (Leviathan et al. 2023) and draft-tree
acceptance (bench/tree_accept.py:91-100), plus the KV-row commit a tree needs.

Every function launches HIP kernels of libtrhip.so (csrc/accept.hip) on the current stream.
"""
import torch

from . import _lib
from .sample import SamplingParams, workspace


class AcceptState:
    """Device outputs of one accept (int64): n_accepted [1], tok [1], slot [1], pred [M] (target
    token per row), tokens [M] (accepted drafts then tok, -1 beyond), commit [M] (chains: the
    positions kept; trees: node indices root..best; -1 beyond). pos [1] is the device position
    (the engine's state.pos_t), advanced in place by n + 1."""

    def __init__(self, M: int, device, pos: torch.Tensor = None):
        z = lambda n: torch.zeros(n, dtype=torch.long, device=device)
        self.M = M
        self.n_accepted, self.tok, self.slot = z(1), z(1), z(1)
        self.pred, self.tokens, self.commit = z(M), z(M), z(M)
        self.pos = z(1) if pos is None else pos

    def outs(self):
        return tuple(_lib.ptr(t) for t in (self.pred, self.n_accepted, self.tok, self.pos, self.slot, self.tokens,
                                           self.commit))


def _prep(logits, st: AcceptState):
    _lib.require_gpu(logits)
    if logits.dtype != torch.bfloat16 or logits.dim() != 2 or not logits.is_contiguous():
        raise RuntimeError("logits must be contiguous bf16 [M, V]")
    M, V = logits.shape
    if st.M < M:
        raise RuntimeError(f"AcceptState holds {st.M} rows, logits have {M}")
    return M, V, workspace(M, V, logits.device)


def accept_greedy(logits: torch.Tensor, spec_toks: torch.Tensor, st: AcceptState) -> AcceptState:
    """Greedy verify (temperature 0): pred = argmax per row (first index on ties),
    n = leading matches of pred[:K] with spec_toks[1:M]; tok = pred[n]; pos += n + 1; slot = n."""
    M, V, ws = _prep(logits, st)
    spec = spec_toks[:M].to(torch.long).contiguous()
    rc = _lib.lib().tr_accept_greedy(_lib.ptr(logits), M, V, _lib.ptr(spec), _lib.ptr(ws), ws.numel(), *st.outs(),
                                     _lib.stream_of(logits))
    _lib.check(rc, "tr_accept_greedy")
    return st


def accept_sampled(logits: torch.Tensor, spec_toks: torch.Tensor, params: SamplingParams, st: AcceptState,
                   u: torch.Tensor = None) -> AcceptState:
    """The reference's verify accept exactly (model.py:302-312): pred = sample(logits, params, u)
    (greedy when params.temperature == 0), then the leading-match commit."""
    M, V, ws = _prep(logits, st)
    if u is None:
        u = torch.rand(M, device=logits.device)
    u = u.to(torch.float32).contiguous()
    spec = spec_toks[:M].to(torch.long).contiguous()
    rc = _lib.lib().tr_accept_sample(_lib.ptr(logits), M, V, _lib.ptr(spec), _lib.ptr(params.temperature),
                                     _lib.ptr(params.top_p), _lib.ptr(params.top_k), _lib.ptr(u), _lib.ptr(ws),
                                     ws.numel(), *st.outs(), _lib.stream_of(logits))
    _lib.check(rc, "tr_accept_sample")
    return st


def accept_residual(logits: torch.Tensor, q: torch.Tensor, spec_toks: torch.Tensor, u: torch.Tensor,
                    st: AcceptState) -> AcceptState:
    """Speculative sampling with residual resample: logits [K+1, V] bf16 (target, temperature 1),
    q [K, V] fp32 draft probabilities of the drafts spec_toks[1:K+1], u [K+1] uniforms. Draft i
    is accepted when u[i] * q[i, d_i] < p[i, d_i]; at the first rejection j (or j = K) one token
    is drawn with u[K] from max(p_j - q_j, 0) (from p_K when every draft passed)."""
    M, V, ws = _prep(logits, st)
    if q.shape != (M - 1, V) or q.dtype != torch.float32 or not q.is_contiguous():
        raise RuntimeError("q must be contiguous fp32 [K, V]")
    spec = spec_toks[:M].to(torch.long).contiguous()
    u = u.to(torch.float32).contiguous()
    o = st.outs()
    rc = _lib.lib().tr_accept_residual(_lib.ptr(logits), M, V, _lib.ptr(q), _lib.ptr(spec), _lib.ptr(u), _lib.ptr(ws),
                                       ws.numel(), *o[1:], _lib.stream_of(logits))
    _lib.check(rc, "tr_accept_residual")
    return st


def accept_tree(logits: torch.Tensor, node_toks: torch.Tensor, parent: torch.Tensor, st: AcceptState) -> AcceptState:
    """Draft-tree verify: node 0 is the root (the committed token), node i > 0 holds draft
    node_toks[i] with parent[i] < i; row i of logits predicts the token after node i. The
    accepted path is the deepest root path whose every node equals its parent row's argmax
    (lowest node index among equals); n = its depth, tok = argmax of its last node's row,
    slot = that node, commit = its node indices."""
    M, V, ws = _prep(logits, st)
    nt = node_toks[:M].to(torch.long).contiguous()
    par = parent[:M].to(torch.int32).contiguous()
    rc = _lib.lib().tr_accept_tree(_lib.ptr(logits), M, V, _lib.ptr(nt), _lib.ptr(par), _lib.ptr(ws), ws.numel(),
                                   *st.outs(), _lib.stream_of(logits))
    _lib.check(rc, "tr_accept_tree")
    return st


def commit_rows(cache: torch.Tensor, st: AcceptState, layout: str, max_n: int = None,
                status: torch.Tensor = None):
    """Tree commit: in every plane of `cache` move the accepted path's rows (written at
    pos_before + node) to consecutive positions pos_before + 1..n. layout names where the
    position axis is: "rows" for [..., max_len, row] (the fp8 KV cache [n_attn, kv_heads,
    max_len, head_dim]), "scalars" for [..., max_len] (its fp32 scales [n_attn, kv_heads,
    max_len]; tokenrush/state.py:19-29). max_n defaults to the st.M - 1 drafts an accept can
    keep. A commit that would reach rows outside the cache, or move more than max_n rows, moves
    nothing and sets status (a device int32 [1], optional) to 1."""
    _lib.require_gpu(cache)
    if not cache.is_contiguous():
        raise RuntimeError("cache must be contiguous")
    if layout == "rows":
        if cache.dim() < 2:
            raise RuntimeError("layout 'rows' needs [..., max_len, row]")
        max_len, row_bytes, lead = cache.shape[-2], cache.shape[-1] * cache.element_size(), cache.shape[:-2]
    elif layout == "scalars":
        max_len, row_bytes, lead = cache.shape[-1], cache.element_size(), cache.shape[:-1]
    else:
        raise RuntimeError(f"layout must be 'rows' or 'scalars', got {layout!r}")
    if row_bytes % 4:
        raise RuntimeError("rows must be a multiple of 4 bytes")
    max_n = st.M - 1 if max_n is None else max_n
    if status is not None and (status.dtype != torch.int32 or not status.is_cuda):
        raise RuntimeError("status must be a device int32 tensor")
    planes = 1
    for d in lead:
        planes *= d
    rc = _lib.lib().tr_commit_rows(_lib.ptr(cache), planes, max_len * row_bytes, row_bytes, _lib.ptr(st.pos),
                                   _lib.ptr(st.n_accepted), _lib.ptr(st.commit), max_n, _lib.ptr(status),
                                   _lib.stream_of(cache))
    _lib.check(rc, "tr_commit_rows")


_lm_ws = {}


def lm_head_greedy(lm_head, hidden: torch.Tensor, spec_toks: torch.Tensor, st: AcceptState,
                   keep_logits: bool = False, out: torch.Tensor = None):
    """logits = lm_head(hidden) and the greedy verify accept in one launch (the GEMM's epilogue
    keeps each row's argmax; the last workgroup finishes the accept exactly as accept_greedy
    does). lm_head: a gfx950 QLinear [V, K]; hidden [M, K] bf16. Returns the logits [M, V] when
    keep_logits (the reference keeps them, model.py:300), else None -- then they are never
    written; out (contiguous bf16 [M, V]) receives them instead of a new tensor. spec_toks None:
    only st.pred is written (argmax per row). Shapes whose plan splits K
    across workgroups (M > 16 at K = 5120) run the product and then the accept kernel."""
    from . import gfx950
    if lm_head.backend != "gfx950" or lm_head.layout != "rows":
        raise RuntimeError("lm_head_greedy needs a gfx950 QLinear in the plain row layout")
    _lib.require_gpu(hidden)
    M, K = hidden.shape
    V = lm_head.shape[0]
    if hidden.dtype != torch.bfloat16 or K != lm_head.shape[1] or st.M < M:
        raise RuntimeError("lm_head_greedy: hidden must be bf16 [M, K] matching the weight")
    need = int(_lib.lib().tr_lm_head_workspace_bytes(V, K, M))
    if out is not None and (out.dtype != torch.bfloat16 or tuple(out.shape) != (M, V) or not out.is_contiguous()):
        raise RuntimeError(f"lm_head_greedy: out must be contiguous bf16 [{M}, {V}]")
    if need == 0:                  # more than one K slot: the product, then the accept kernel
        logits = lm_head(hidden, out=out)
        if spec_toks is None:
            _lib.check(_lib.lib().tr_argmax_rows(_lib.ptr(logits), M, V, _lib.ptr(workspace(M, V, hidden.device)),
                                                 workspace(M, V, hidden.device).numel(), _lib.ptr(st.pred),
                                                 _lib.stream_of(logits)), "tr_argmax_rows")
        else:
            accept_greedy(logits, spec_toks, st)
        return logits if keep_logits else None
    key = hidden.device.index or 0
    ws = _lib.grown_workspace(_lm_ws, key, need, hidden.device)
    logits = (out if out is not None else torch.empty(M, V, dtype=torch.bfloat16, device=hidden.device)) \
        if keep_logits or out is not None else None
    spec = None if spec_toks is None else spec_toks[:M].to(torch.long).contiguous()
    x = hidden.contiguous()
    P = _lib.ptr
    rc = _lib.lib().tr_lm_head_greedy(P(x), P(lm_head.B), P(logits), P(ws), ws.numel(), M, V, K, 128,
                                      gfx950.SCALE_DTYPES[lm_head.s.dtype], P(spec), P(st.pred), P(st.n_accepted),
                                      P(st.tok), P(st.pos), P(st.slot), P(st.tokens), P(st.commit),
                                      _lib.stream_of(x))
    _lib.check(rc, "tr_lm_head_greedy")
    return logits
