"""Full-attention verify step over an FP8 KV cache on gfx950: the reference's tokenrush/fused.py
attn_prep (fused.py:313-325) and attn_decode_fused (fused.py:448-470) over the HIP kernels of
csrc/attn.hip.

attn_prep normalises and ropes the M new tokens' queries and keys and writes their keys and
values into the cache (float8_e4m3fn with one fp32 scale per kv head and position);
attn_decode_fused is flash-decoding over the live rows (query t sees rows <= pos + t) followed by
the split combine and the sigmoid output gate. Both are shape-static in the device position, so
a verify step captures into one hipGraph.
"""
from dataclasses import dataclass

import torch

from . import _lib

NSPLIT = 64        # key-range splits of the flash-decoding kernel: 256 workgroups at 4 kv heads
                   # (the reference uses 32 on a 170-SM part; measured fastest here)
CHAIN_NSPLIT = NSPLIT
SPLIT_SLOTS = 512  # split-kernel workgroups resident at once: 256 CUs, two each (240 registers a lane)


def tree_splits(M: int, cfg) -> int:
    """Key-range splits for a draft tree of M nodes: its G M query rows per kv head run in groups of
    64 (a second grid dimension), so the grid is HKV x splits x groups; the largest count up to
    NSPLIT whose grid fits one pass of SPLIT_SLOTS (42 for 32 nodes at 24 / 4 heads: 21% faster
    per call than 64, which needs a second pass)."""
    groups = -(-(cfg.n_heads // cfg.n_kv_heads) * M // 64)
    return max(1, min(NSPLIT, SPLIT_SLOTS // (cfg.n_kv_heads * groups)))


@dataclass(frozen=True)
class AttnConfig:
    """The ModelConfig fields the step reads (tokenrush/config.py:12-16)."""
    n_heads: int = 24
    n_kv_heads: int = 4
    head_dim: int = 256
    rotary_dim: int = 64
    rope_theta: float = 1e7
    eps: float = 1e-6


def rope_table(max_pos: int, rotary_dim: int, theta: float, device, dtype=torch.bfloat16):
    """cos/sin tables [max_pos, rotary_dim] in the activation dtype (tokenrush/ops.py:25-31)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32, device=device) / rotary_dim))
    pos = torch.arange(max_pos, dtype=torch.float32, device=device)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _check_cache(k_cache, v_cache, k_scale, v_scale, cfg):
    if k_cache.dtype != torch.float8_e4m3fn or v_cache.dtype != torch.float8_e4m3fn:
        raise RuntimeError("attention: the gfx950 path takes a float8_e4m3fn KV cache with fp32 scales")
    if k_scale is None or v_scale is None or k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32:
        raise RuntimeError("attention: fp8 caches need fp32 k_scale and v_scale [HKV, maxlen]")
    HKV, D = cfg.n_kv_heads, cfg.head_dim
    if k_cache.dim() != 3 or k_cache.shape[0] != HKV or k_cache.shape[2] != D or v_cache.shape != k_cache.shape:
        raise RuntimeError("attention: caches must be [HKV, maxlen, D]")
    if tuple(k_scale.shape) != tuple(k_cache.shape[:2]) or tuple(v_scale.shape) != tuple(k_cache.shape[:2]):
        raise RuntimeError("attention: scales must be [HKV, maxlen]")
    for t in (k_cache, v_cache, k_scale, v_scale):
        if not t.is_contiguous():
            raise RuntimeError("attention: caches and scales must be contiguous")


def _parent(parent, M, device):
    if parent is None:
        return None
    if parent.dtype != torch.int32 or not parent.is_cuda or parent.device != device or parent.numel() < M:
        raise RuntimeError("parent must be a device int32 tensor with one entry per node")
    return parent.contiguous()


def attn_prep(qkv, q_norm_w, k_norm_w, cos, sin, pos_t, k_cache, v_cache, cfg, k_scale=None, v_scale=None,
              parent=None):
    """qkv [M, HQ 2D + 2 HKV D] bf16 -> q [M, HQ D] bf16, normed and roped; writes the new keys
    and values into cache rows pos..pos+M-1 (fused.py:313-325). With parent (device int32 [M],
    parent[t] < t, node 0 the root) the M <= 32 rows are the nodes of a draft tree: node t is
    roped at pos + depth(t) and still written to row pos + t."""
    _lib.require_gpu(qkv, q_norm_w, k_norm_w, cos, sin, pos_t, k_cache, v_cache)
    _check_cache(k_cache, v_cache, k_scale, v_scale, cfg)
    if qkv.dtype != torch.bfloat16 or qkv.stride(1) != 1:
        raise RuntimeError("attn_prep: qkv must be bf16 with unit column stride")
    if pos_t.dtype != torch.int64 or cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16:
        raise RuntimeError("attn_prep: int64 pos_t and bf16 cos/sin tables")
    if cos.shape[1] != cfg.rotary_dim or not (cos.is_contiguous() and sin.is_contiguous()):
        raise RuntimeError("attn_prep: cos/sin must be contiguous [max_pos, rotary_dim]")
    M = qkv.shape[0]
    HQ, HKV, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    q = torch.empty(M, HQ * D, device=qkv.device, dtype=torch.bfloat16)
    ld = qkv.stride(0) if M > 1 else qkv.shape[1]
    par = _parent(parent, M, qkv.device)
    P = _lib.ptr
    head = (P(qkv), ld, P(q_norm_w), P(k_norm_w), P(cos), P(sin), cfg.rotary_dim, P(pos_t))
    tail = (P(k_cache), P(v_cache), P(k_scale), P(v_scale), k_cache.shape[1], P(q), M, HQ, HKV, D, float(cfg.eps),
            _lib.stream_of(qkv))
    if par is None:
        _lib.check(_lib.lib().tr_attn_prep(*head, *tail), "tr_attn_prep")
    else:
        _lib.check(_lib.lib().tr_attn_prep_tree(*head, P(par), *tail), "tr_attn_prep_tree")
    return q


_ws = {}


def workspace(M: int, HQ: int, nsplit: int, device):
    need = int(_lib.lib().tr_attn_workspace_bytes(M, HQ, nsplit))
    if need == 0:
        raise RuntimeError(f"attention workspace: unsupported M={M}")
    key = torch.device(device).index or 0
    return _lib.grown_workspace(_ws, key, need, device, zero=False)


def attn_decode_fused(q, qkv, k_cache, v_cache, pos_t, cfg, k_scale=None, v_scale=None, NSPLIT=None,
                      parent=None):
    """q [M, HQ D] (from attn_prep) for the M new tokens at pos.., qkv [M, ..] (for the gates)
    -> gated attention output [M, HQ D] bf16; query t sees cache rows <= pos + t
    (fused.py:448-470). With parent (a draft tree of M <= 32 nodes, as attn_prep), node t sees
    the rows before pos and the rows pos + i of its ancestors and itself. NSPLIT (key-range
    splits) defaults to NSPLIT for a chain and to tree_splits(M, cfg) for a tree."""
    _lib.require_gpu(q, qkv, k_cache, v_cache, pos_t)
    _check_cache(k_cache, v_cache, k_scale, v_scale, cfg)
    if q.dtype != torch.bfloat16 or not q.is_contiguous() or qkv.dtype != torch.bfloat16 or qkv.stride(1) != 1:
        raise RuntimeError("attn_decode_fused: bf16 q (contiguous) and qkv")
    M = q.shape[0]
    HQ, HKV, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    out = torch.empty(M, HQ * D, device=q.device, dtype=torch.bfloat16)
    if NSPLIT is None:
        NSPLIT = CHAIN_NSPLIT if parent is None else tree_splits(M, cfg)
    ws = workspace(M, HQ, NSPLIT, q.device)
    ld = qkv.stride(0) if M > 1 else qkv.shape[1]
    par = _parent(parent, M, q.device)
    P = _lib.ptr
    head = (P(q), P(qkv), ld, P(k_cache), P(v_cache), P(k_scale), P(v_scale), k_cache.shape[1], P(pos_t))
    tail = (P(out), P(ws), ws.numel(), M, HQ, HKV, D, NSPLIT, _lib.stream_of(q))
    if par is None:
        _lib.check(_lib.lib().tr_attn_decode(*head, *tail), "tr_attn_decode")
    else:
        _lib.check(_lib.lib().tr_attn_decode_tree(*head, P(par), *tail), "tr_attn_decode_tree")
    return out
