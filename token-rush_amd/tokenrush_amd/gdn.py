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
MAX_TOKENS = 8     # tokens per step (the reference kernel's MP, fused.py:150)


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


def gdn_step_fused(qkvz, x, ba_w, ring, conv_w, A, dt_bias, rec, slot, norm_w, pos_t, cfg, eps):
    """M-token GDN step (M = qkvz.shape[0] <= 8), as the reference's gdn_step_fused
    (fused.py:213): qkvz [M, 2 qk + 2 val] bf16 (rows may be strided), x [M, hidden] bf16, ba_w
    [2 HV, hidden] bf16, ring [conv_dim, R] bf16 (updated), conv_w [conv_dim, 4] bf16, A and dt_bias
    [HV] fp32, rec [n_slots, HV, K, V] fp32 (a strided per-layer view is fine) with the committed
    state in slot *slot, norm_w [V] bf16, pos_t [1] int64 -> y [M, val] bf16. Writes rec slots
    0..M-1."""
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
    rc = _lib.lib().tr_gdn_step(
        _lib.ptr(qkvz), ld, _lib.ptr(x), _lib.ptr(ba_w), _lib.ptr(ring), _lib.ptr(conv_w), _lib.ptr(A),
        _lib.ptr(dt_bias), _lib.ptr(rec), rec.stride(0), _lib.ptr(slot), _lib.ptr(norm_w), _lib.ptr(pos_t),
        _lib.ptr(y), _lib.ptr(ws), ws.numel(), M, H, HV, K, V, cfg.hidden, ring.shape[1], float(eps),
        _lib.stream_of(qkvz))
    _lib.check(rc, "tr_gdn_step")
    return y
