"""Row kernels around the verify GEMMs: the reference's tokenrush/fused.py add_rmsnorm and
silu_mul (fused.py:23-87) over the gfx950 kernels of csrc/fused.hip.

add_rmsnorm is the consumer of QLinear.partials: it takes the [S, T, N] fp32 split-K slots
directly, sums them in slot order, rounds to bf16, adds the residual and normalizes -- so
hidden-sized projections never write a bf16 output of their own.
"""
import torch

from . import _lib

H_NONE, H_BF16, H_PARTIALS = 0, 1, 2


def add_rmsnorm(x: torch.Tensor, h, weight: torch.Tensor, eps: float, plain: bool = False, out: torch.Tensor = None):
    """x [T, N] bf16; h None, [T, N] bf16 or [S, T, N] fp32 partials -> (x + h as bf16,
    rmsnorm(x + h)); with h None -> (x, rmsnorm(x)). plain: weight * x gain instead of
    (1 + weight) (fused.py:50-60). out (contiguous bf16 [T, N]) receives the norm."""
    _lib.require_gpu(x, weight)
    if x.dtype != torch.bfloat16 or x.dim() != 2 or weight.dtype != torch.bfloat16:
        raise RuntimeError("add_rmsnorm: x must be bf16 [T, N] and weight bf16 [N]")
    T, N = x.shape
    x = x.contiguous()
    if out is not None and (out.dtype != torch.bfloat16 or out.shape != x.shape or not out.is_contiguous()):
        raise RuntimeError("add_rmsnorm: out must be contiguous bf16 [T, N]")
    y = torch.empty_like(x) if out is None else out
    if h is None:
        mode, S, hp, xo = H_NONE, 1, None, x
    elif h.dim() == 2:
        if h.dtype != torch.bfloat16 or h.shape != x.shape:
            raise RuntimeError("add_rmsnorm: h must be bf16 [T, N] or fp32 [S, T, N]")
        mode, S, hp, xo = H_BF16, 1, h.contiguous(), torch.empty_like(x)
    else:
        if h.dtype != torch.float32 or h.shape[1:] != x.shape:
            raise RuntimeError("add_rmsnorm: partials must be fp32 [S, T, N]")
        mode, S, hp, xo = H_PARTIALS, h.shape[0], h.contiguous(), torch.empty_like(x)
    rc = _lib.lib().tr_add_rmsnorm(_lib.ptr(x), _lib.ptr(hp), mode, S, _lib.ptr(weight.contiguous()),
                                   _lib.ptr(xo) if mode != H_NONE else None, _lib.ptr(y), T, N, float(eps), int(plain),
                                   _lib.stream_of(x))
    _lib.check(rc, "tr_add_rmsnorm")
    return xo, y


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """gate_up [T, 2F] bf16 (rows may be strided, e.g. a column slice) -> silu(gate) * up
    [T, F] bf16, one launch (fused.py:77-87)."""
    _lib.require_gpu(gate_up)
    if gate_up.dtype != torch.bfloat16 or gate_up.dim() != 2 or gate_up.shape[1] % 2:
        raise RuntimeError("silu_mul: gate_up must be bf16 [T, 2F]")
    if gate_up.stride(1) != 1:
        gate_up = gate_up.contiguous()
    T, F2 = gate_up.shape
    y = torch.empty(T, F2 // 2, dtype=torch.bfloat16, device=gate_up.device)
    _lib.check(_lib.lib().tr_silu_mul(_lib.ptr(gate_up), gate_up.stride(0) if T > 1 else F2, _lib.ptr(y), T, F2 // 2,
                                      _lib.stream_of(gate_up)), "tr_silu_mul")
    return y


def embed_rows(table: torch.Tensor, ids: torch.Tensor, out: torch.Tensor = None, status: torch.Tensor = None):
    """table [V, H] bf16, ids int64 [T] on the device -> table[ids] [T, H] bf16, one launch
    (the reference's x = embed[tokens], model.py:215). An id outside [0, V) gives a zero row and
    sets status (int32 [1], optional) to 1."""
    _lib.require_gpu(table, ids)
    if table.dtype != torch.bfloat16 or table.dim() != 2 or ids.dtype != torch.int64 or ids.dim() != 1:
        raise RuntimeError("embed_rows: table must be bf16 [V, H] and ids int64 [T]")
    V, H = table.shape
    T = ids.shape[0]
    if out is None:
        out = torch.empty(T, H, dtype=torch.bfloat16, device=table.device)
    if out.dtype != torch.bfloat16 or tuple(out.shape) != (T, H) or not out.is_contiguous():
        raise RuntimeError("embed_rows: out must be contiguous bf16 [T, H]")
    if status is not None and (status.dtype != torch.int32 or not status.is_cuda):
        raise RuntimeError("embed_rows: status must be a device int32 tensor")
    _lib.check(_lib.lib().tr_embed_rows(_lib.ptr(table.contiguous()), _lib.ptr(ids.contiguous()), _lib.ptr(out), T, H,
                                        V, _lib.ptr(status), _lib.stream_of(table)), "tr_embed_rows")
    return out
