"""Sampling inside the verify graph: the reference's tokenrush/sample.py API (sample.py:12-51)
over the gfx950 kernels.

As in the reference, everything is shape-static and branch-free on the host: the candidate
set is the top 64 of each row, temperature / top_p / top_k are device tensors read at replay
time, greedy (temperature 0) is chosen on the device, and u (one uniform per row) is drawn on
the device when not given, so a captured graph advances torch's generator per replay.

One launch (tr_sample) computes the per-row top-64 (ties: lower index first), the masked
softmax and the inverse-CDF pick in fixed-order fp32 arithmetic.
"""
import torch

from . import _lib

CANDIDATES = 64


class SamplingParams:
    """Device-resident parameters; change them between replays with .set() (sample.py:15-28)."""

    def __init__(self, device):
        self.temperature = torch.zeros(1, device=device, dtype=torch.float32)   # 0 -> greedy
        self.top_p = torch.ones(1, device=device, dtype=torch.float32)
        self.top_k = torch.full((1,), CANDIDATES, device=device, dtype=torch.long)

    def set(self, temperature=0.0, top_p=1.0, top_k=CANDIDATES):
        assert 1 <= top_k <= CANDIDATES
        self.temperature.fill_(temperature)
        self.top_p.fill_(top_p)
        self.top_k.fill_(top_k)


_ws = {}


def workspace(M: int, V: int, device):
    """The per-device accept workspace, grown to fit M rows of V logits (zero-filled: its
    counters read zero between calls, which every call restores). Grow before graph capture."""
    key = torch.device(device).index or 0
    need = int(_lib.lib().tr_accept_workspace_bytes(M, V))
    if need == 0:
        raise RuntimeError(f"accept shape (M={M}, V={V}) not supported: need 1 <= M <= 32, 64 <= V <= 262144")
    return _lib.grown_workspace(_ws, key, need, device)


def _check_logits(logits):
    _lib.require_gpu(logits)
    if logits.dtype != torch.bfloat16 or logits.dim() != 2 or not logits.is_contiguous():
        raise RuntimeError("logits must be contiguous bf16 [M, V]")


def sample(logits: torch.Tensor, params: SamplingParams, u: torch.Tensor = None) -> torch.Tensor:
    """logits [M, V] bf16 -> tokens [M] (long), one independent draw per row.
    u: uniform [M] in [0, 1), drawn on the device if None."""
    _check_logits(logits)
    M, V = logits.shape
    if u is None:
        u = torch.rand(M, device=logits.device)
    u = u.to(torch.float32).contiguous()
    out = torch.empty(M, dtype=torch.long, device=logits.device)
    ws = workspace(M, V, logits.device)
    rc = _lib.lib().tr_sample(_lib.ptr(logits), M, V, _lib.ptr(params.temperature), _lib.ptr(params.top_p),
                              _lib.ptr(params.top_k), _lib.ptr(u), _lib.ptr(ws), ws.numel(), _lib.ptr(out),
                              _lib.stream_of(logits))
    _lib.check(rc, "tr_sample")
    return out
