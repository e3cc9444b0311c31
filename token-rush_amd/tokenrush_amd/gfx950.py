"""Strip-layout int4 GEMM for M <= 32 rows on MI355X (gfx950).

This module plays the role of the reference's tokenrush/marlin.py (marlin.py:1-168): it
converts the engine's packing to the kernel's weight layout and back, and launches the
kernel. The kernel itself (csrc/int4_gemm.hip) is our own design, not Marlin:

* weight layout: codes [N/16, K/128, 64, 16] uint8 -- one 1 KiB tile per (16-row strip,
  group of 128), in the order one wave's 16-byte loads consume it; scale and min stay in the
  engine's [N, K/128] layout;
* every M in 1..32 runs the same MFMA instructions (rows beyond M are zero lanes), so each
  output row is bit-identical for every M, as Marlin's is (reference test_marlin.py:42-52);
* no locks and no reduce buffer: split-K happens inside a workgroup and is reduced through
  LDS in a fixed order; mul_partial writes fp32 slots [S, M, N] whose sum is the product.

API (same names and argument meaning as marlin.py): ext, available, pack, unpack,
workspaces, mul, partial_slots, mul_partial.
"""
import ctypes

import torch

from . import _lib

GROUP = 128
MAX_ROWS = 32        # the kernel's row limit (two 16-row MFMA tiles)
SCALE_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def ext():
    """The loaded C-ABI library (raises if it is not built)."""
    return _lib.lib()


def available() -> bool:
    """True when the library loads. Nothing falls back when it does not: callers raise."""
    try:
        ext()
        return True
    except Exception as e:  # not built, wrong arch
        print(f"gfx950 library unavailable: {str(e)[:200]}")
        return False


def _check_shape(N: int, K: int):
    if N % 16 or K % GROUP:
        raise RuntimeError(f"problem shape (n={N}, k={K}) not supported: need n % 16 == 0, k % {GROUP} == 0")


def pack(qweight: torch.Tensor, scale: torch.Tensor, mn: torch.Tensor):
    """Engine packing (uint8 [N, K/2], bf16/fp16 [N, K/128] x2) -> strip layout
    (uint8 [N/16, K/128, 64, 16], scale, mn). The counterpart of marlin.pack (marlin.py:73-96)."""
    _lib.require_gpu(qweight, scale, mn)
    N, K = qweight.shape[0], qweight.shape[1] * 2
    _check_shape(N, K)
    assert qweight.dtype == torch.uint8 and scale.shape == mn.shape == (N, K // GROUP), (scale.shape, N, K)
    q = qweight.contiguous()
    B = torch.empty(N // 16, K // GROUP, 64, 16, dtype=torch.uint8, device=q.device)
    _lib.check(ext().tr_pack_int4(_lib.ptr(q), _lib.ptr(B), N, K, _lib.stream_of(q)), "tr_pack_int4")
    return B, scale.contiguous(), mn.contiguous()


def unpack(B: torch.Tensor, s: torch.Tensor, m: torch.Tensor):
    """Inverse of pack -> (qweight uint8 [N, K/2], scale, mn) (marlin.unpack, marlin.py:99-118)."""
    _lib.require_gpu(B, s, m)
    N, K = B.shape[0] * 16, B.shape[1] * GROUP
    q = torch.empty(N, K // 2, dtype=torch.uint8, device=B.device)
    _lib.check(ext().tr_unpack_int4(_lib.ptr(B), _lib.ptr(q), N, K, _lib.stream_of(B)), "tr_unpack_int4")
    return q, s.contiguous(), m.contiguous()


def workspaces(N: int, device):
    """Kept for API parity with marlin.workspaces (marlin.py:121-135): this kernel needs no
    lock array and no reduce buffer, so there is nothing to size before graph capture."""
    return None, None


def plan(N: int, K: int):
    """(T, W, S): strips per workgroup, waves per workgroup, K slots. Depends on (N, K) only."""
    T, W, S = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _lib.check(ext().tr_gemm_plan(N, K, ctypes.byref(T), ctypes.byref(W), ctypes.byref(S)), "tr_gemm_plan")
    return T.value, W.value, S.value


def _launch(x, B, s, m, y, partial, n_slots, thread_t, thread_w):
    M, K = x.shape
    N = B.shape[0] * 16
    if x.dtype != torch.bfloat16 or s.dtype not in SCALE_DTYPES or m.dtype != s.dtype:
        raise RuntimeError("dtypes: x must be bf16, scale/min bf16 or fp16")
    if not (x.is_contiguous() and B.is_contiguous() and s.is_contiguous() and m.is_contiguous()):
        raise RuntimeError("inputs must be contiguous")
    if M > MAX_ROWS or K != B.shape[1] * GROUP:
        raise RuntimeError(f"problem shape (m={M}, n={N}, k={K}) not supported: need m <= {MAX_ROWS}")
    _lib.require_gpu(x, B, s, m, y)
    st = _lib.stream_of(x)
    out, part = (None, y) if partial else (y, None)
    if thread_t == -1 and thread_w == -1:
        rc = ext().tr_int4_gemm(_lib.ptr(x), _lib.ptr(B), _lib.ptr(s), _lib.ptr(m), _lib.ptr(out), _lib.ptr(part),
                                M, N, K, GROUP, SCALE_DTYPES[s.dtype], n_slots, st)
    else:
        T0, W0, _ = plan(N, K)
        T = T0 if thread_t == -1 else thread_t
        W = W0 if thread_w == -1 else thread_w
        rc = ext().tr_int4_gemm_ex(_lib.ptr(x), _lib.ptr(B), _lib.ptr(s), _lib.ptr(m), _lib.ptr(out), _lib.ptr(part),
                                   M, N, K, GROUP, SCALE_DTYPES[s.dtype], n_slots, T, W, st)
    _lib.check(rc, f"tr_int4_gemm (m={M}, n={N}, k={K})")


def mul(x: torch.Tensor, B: torch.Tensor, s: torch.Tensor, m: torch.Tensor, thread_t=-1, thread_w=-1):
    """x [M, K] bf16 (M <= 32) -> [M, N] bf16 (marlin.mul, marlin.py:138-145)."""
    M = x.shape[0]
    y = torch.empty(M, B.shape[0] * 16, dtype=torch.bfloat16, device=x.device)
    _launch(x, B, s, m, y, False, 0, thread_t, thread_w)
    return y


_slots = {}


def partial_slots(N: int, K: int) -> int:
    """fp32 slots mul_partial writes for an N x K weight (marlin.partial_slots, marlin.py:151-155)."""
    key = (N, K)
    if key not in _slots:
        S = ext().tr_partial_slots(N, K, 1)
        if S < 1:
            raise RuntimeError(f"problem shape (n={N}, k={K}) not supported")
        _slots[key] = S
    return _slots[key]


def mul_partial(x: torch.Tensor, B: torch.Tensor, s: torch.Tensor, m: torch.Tensor, n_slots: int = None,
                thread_t=-1, thread_w=-1):
    """x [M, K] bf16 (M <= 32) -> fp32 partials [S, M, N] whose sum over S is the product
    (marlin.mul_partial, marlin.py:158-168). Every slot is written."""
    M, K = x.shape
    N = B.shape[0] * 16
    S = partial_slots(N, K) if n_slots is None else n_slots
    y = torch.empty(S, M, N, dtype=torch.float32, device=x.device)
    _launch(x, B, s, m, y, True, S, thread_t, thread_w)
    return y


def dequantize(qweight: torch.Tensor, scale: torch.Tensor, mn: torch.Tensor) -> torch.Tensor:
    """Engine packing -> dense weight [N, K], w = round(round(q * s) + m) in the scale dtype
    (bf16 for the engine format: quant.dequantize_int4, quant.py:47-53)."""
    _lib.require_gpu(qweight, scale, mn)
    N, K = qweight.shape[0], qweight.shape[1] * 2
    if scale.dtype not in SCALE_DTYPES or mn.dtype != scale.dtype:
        raise RuntimeError("scale/min must be bf16 or fp16")
    q, s, m = qweight.contiguous(), scale.contiguous(), mn.contiguous()
    out = torch.empty(N, K, dtype=scale.dtype, device=q.device)
    _lib.check(ext().tr_dequant_int4(_lib.ptr(q), _lib.ptr(s), _lib.ptr(m), _lib.ptr(out), N, K, K // s.shape[1],
                                     SCALE_DTYPES[s.dtype], _lib.stream_of(q)), "tr_dequant_int4")
    return out
