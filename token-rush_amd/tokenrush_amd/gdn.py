"""The M-token gated-delta-rule (GDN) verify step on gfx950: the reference's
tokenrush/fused.py gdn_step_fused (fused.py:213-236) over the HIP kernel of csrc/gdn.hip.

One launch per layer and step: causal conv over the ring (which it updates), b/a gates, the
recurrence with the state after token t written to snapshot slot t (so the accept commits a
prefix by naming its slot, tokenrush/state.py:30-39), and the gated RMSNorm that feeds the
output projection.
"""
from dataclasses import dataclass

import torch

from . import _lib

RING = 16          # conv ring columns (tokenrush/state.py:10): must exceed the longest step by 3
MAX_TOKENS = 8     # tokens per chain step (the reference kernel's MP, fused.py:150)
MAX_NODES = 32     # nodes per draft-tree step


@dataclass(frozen=True)
class GDNConfig:
    """The ModelConfig fields the step reads (tokenrush/config.py:17-21, 58-68)."""
    hidden: int = 5120
    gdn_k_heads: int = 16
    gdn_v_heads: int = 48
    gdn_k_dim: int = 128
    gdn_v_dim: int = 128

    @property
    def gdn_qk_dim(self):
        return self.gdn_k_heads * self.gdn_k_dim

    @property
    def gdn_val_dim(self):
        return self.gdn_v_heads * self.gdn_v_dim

    @property
    def conv_dim(self):
        return 2 * self.gdn_qk_dim + self.gdn_val_dim


_ws = {}


def workspace(M: int, H: int, HV: int, device):
    """Per-device workspace (arrival counters, head outputs for the gated norm, conv outputs and
    gates of the step), zero-filled once: every call leaves its counters at zero."""
    need = int(_lib.lib().tr_gdn_workspace_bytes(M, H, HV))
    if need == 0:
        raise RuntimeError(f"gdn workspace: unsupported M={M}, H={H} or HV={HV}")
    key = torch.device(device).index or 0
    return _lib.grown_workspace(_ws, key, need, device)


def gdn_step_fused(qkvz, x, ba_w, ring, conv_w, A, dt_bias, rec, slot, norm_w, pos_t, cfg, eps, parent=None,
                   node_in=None):
    """M-token GDN step (M = qkvz.shape[0] <= 8), as the reference's gdn_step_fused
    (fused.py:213): qkvz [M, 2 qk + 2 val] bf16 (rows may be strided), x [M, hidden] bf16, ba_w
    [2 HV, hidden] bf16, ring [conv_dim, R] bf16 (updated), conv_w [conv_dim, 4] bf16, A and dt_bias
    [HV] fp32, rec [n_slots, HV, K, V] fp32 (a strided per-layer view is fine) with the committed
    state in slot *slot, norm_w [V] bf16, pos_t [1] int64 -> y [M, val] bf16. Writes rec slots
    0..M-1.

    With parent (device int32 [M], parent[t] < t) and node_in ([M, conv_dim] bf16) the M <= 32 rows
    are the nodes of a draft tree: node t continues from its parent's state (the root from slot
    *slot), its conv window is its root path's, the ring is left alone and the nodes' conv inputs
    go to node_in for tree_commit."""
    _lib.require_gpu(qkvz, x, ba_w, ring, conv_w, A, dt_bias, rec, slot, norm_w, pos_t)
    M = qkvz.shape[0]
    H, HV, K, V = cfg.gdn_k_heads, cfg.gdn_v_heads, cfg.gdn_k_dim, cfg.gdn_v_dim
    if rec.shape[0] < M:
        raise RuntimeError("not enough recurrent-state slots for this many tokens")
    bf = torch.bfloat16
    if any(t.dtype != bf for t in (qkvz, x, ba_w, ring, conv_w, norm_w)) or rec.dtype != torch.float32 \
            or A.dtype != torch.float32 or dt_bias.dtype != torch.float32:
        raise RuntimeError("gdn_step_fused: bf16 activations/weights/ring, fp32 A, dt_bias and rec")
    if slot.dtype != torch.int64 or pos_t.dtype != torch.int64:
        raise RuntimeError("gdn_step_fused: slot and pos_t must be int64 device scalars")
    if qkvz.stride(1) != 1:
        qkvz = qkvz.contiguous()
    if not (x.is_contiguous() and ba_w.is_contiguous() and ring.is_contiguous() and conv_w.is_contiguous()):
        raise RuntimeError("gdn_step_fused: x, ba_w, ring and conv_w must be contiguous")
    if tuple(rec.shape[1:]) != (HV, K, V) or rec.stride()[1:] != (K * V, V, 1):
        raise RuntimeError("gdn_step_fused: rec must be [n_slots, HV, K, V] with contiguous [HV, K, V] slots")
    y = torch.empty(M, HV * V, device=qkvz.device, dtype=bf)
    ws = workspace(M, H, HV, qkvz.device)
    ld = qkvz.stride(0) if M > 1 else qkvz.shape[1]
    P = _lib.ptr
    head = (P(qkvz), ld, P(x), P(ba_w), P(ring), P(conv_w), P(A), P(dt_bias), P(rec), rec.stride(0), P(slot),
            P(norm_w), P(pos_t))
    tail = (P(y), P(ws), ws.numel(), M, H, HV, K, V, cfg.hidden, ring.shape[1], float(eps), _lib.stream_of(qkvz))
    if parent is None:
        _lib.check(_lib.lib().tr_gdn_step(*head, *tail), "tr_gdn_step")
        return y
    if parent.dtype != torch.int32 or parent.device != qkvz.device or parent.numel() < M:
        raise RuntimeError("gdn_step_fused: parent must be a device int32 tensor with one entry per node")
    if node_in is None or node_in.dtype != bf or not node_in.is_contiguous() or node_in.device != qkvz.device \
            or node_in.shape[0] < M or node_in.shape[-1] != cfg.conv_dim:
        raise RuntimeError("gdn_step_fused: tree steps need node_in [>= M, conv_dim] bf16, contiguous")
    _lib.check(_lib.lib().tr_gdn_tree_step(*head, P(parent.contiguous()), P(node_in), *tail), "tr_gdn_tree_step")
    return y


def tree_commit(ring, node_in, st, status=None):
    """After a draft-tree accept: write the accepted path's conv inputs into the rings, columns
    (pos_before + d) % R for d = 0..n, as a chain step over the path would have. ring
    [layers, conv_dim, R] (or one layer [conv_dim, R]) bf16, node_in [layers, M, conv_dim] (or
    [M, conv_dim]) bf16 as the tree steps wrote it, st the AcceptState of the tree accept (pos
    already advanced, n_accepted, commit = path nodes). A path outside the nodes sets status
    (device int32 [1], optional) to 1 and commits nothing."""
    _lib.require_gpu(ring, node_in)
    if ring.dim() == 2:
        ring, node_in = ring.unsqueeze(0), node_in.unsqueeze(0)
    if ring.dtype != torch.bfloat16 or node_in.dtype != torch.bfloat16 or not ring.is_contiguous() \
            or not node_in.is_contiguous() or ring.shape[0] != node_in.shape[0] or ring.shape[1] != node_in.shape[2]:
        raise RuntimeError("tree_commit: ring [layers, C, R] and node_in [layers, M, C], bf16 and contiguous")
    if status is not None and (status.dtype != torch.int32 or status.device != ring.device):
        raise RuntimeError("status must be a device int32 tensor")
    L, C, R = ring.shape
    M = node_in.shape[1]
    rc = _lib.lib().tr_gdn_tree_commit(_lib.ptr(ring), C * R, _lib.ptr(node_in), M * C, L, C, R, M, _lib.ptr(st.pos),
                                       _lib.ptr(st.n_accepted), _lib.ptr(st.commit), _lib.ptr(status),
                                       _lib.stream_of(ring))
    _lib.check(rc, "tr_gdn_tree_commit")
