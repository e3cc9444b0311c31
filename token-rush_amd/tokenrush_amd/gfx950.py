"""Strip-layout int4 GEMM for M <= 32 rows on MI355X (gfx950).

This module plays the role of the reference's tokenrush/marlin.py (marlin.py:1-168): it
converts the engine's packing to the kernel's weight layout and back, sizes the workspace
before graph capture, and launches the kernel. The kernel (csrc/int4_gemm.hip) is our own
design, not Marlin:

* weight layout ("quad layout"): uint8 [N/16, Gp/4, 4352], Gp = K/128 rounded up to a multiple
  of 4 (padding groups are zeros). One quad per (16-row strip, four groups of 128): 4 x 1 KiB of
  codes in the order one wave's 16-byte loads consume them, then the 16 rows' (scale, min)
  pairs for the four groups (16 bytes per row). A strip is one contiguous stream of whole
  128-byte lines;
* every M in 1..16 runs the same instructions (rows beyond M are padding lanes), so each
  output row is bit-identical for every M, as Marlin's is (reference test_marlin.py:42-52);
  the same holds within M = 17..32;
* no locks: split-K inside a workgroup is reduced through LDS in a fixed order; split-K
  across workgroups (K = 17408, or M > 16) writes fp32 slots, which mul_partial returns as
  [S, M, N] and mul reduces in the last-arriving workgroup through the workspace.

API (same names and argument meaning as marlin.py): ext, available, pack, unpack,
workspaces, mul, partial_slots, mul_partial; ext() also answers the extension module's own
mul / partial_slots (marlin_bf16.cpp:14-57).
"""
import ctypes

import torch

from . import _lib

GROUP = 128
QUAD = 4352          # bytes of one (16-row strip, 4 groups) quad
SM_OFF = 4096        # offset of the quad's scale/min words
MAX_ROWS = 32        # two 16-row MFMA tiles
SCALE_DTYPES = {torch.bfloat16: 0, torch.float16: 1}
WS_COUNTER_BYTES = 4096 * 128   # the workspace's counter region (one counter per 128-byte line)


class _Ext:
    """The loaded library as the reference's compiled extension module (marlin.ext(), the torch
    binding of marlin_bf16.cpp:14-57): mul(A, B, C, s, m, workspace, red, thread_k, thread_n, sms)
    and partial_slots(n, k, thread_k, thread_n, sms), with the binding's argument meaning -- C bf16
    [m, n] is the product, C fp32 [slots, m, n] the split-K partials -- and RuntimeError where the
    binding's TORCH_CHECKs fail. thread_k / thread_n / sms are accepted and ignored (this kernel
    plans its own tiling); red is accepted and unused (the workspace holds everything). Every other
    attribute is the C ABI's entry point of that name (tr_*)."""

    def __init__(self, lib):
        self._lib = lib

    def __getattr__(self, name):
        return getattr(self._lib, name)

    def mul(self, A, B, C, s, m, workspace, red=None, thread_k=-1, thread_n=-1, sms=-1):
        del m, red, thread_k, thread_n, sms
        M, K = A.shape
        N = B.shape[0] * 16
        if C.dtype == torch.float32:
            if C.dim() != 3 or tuple(C.shape[1:]) != (M, N):
                raise RuntimeError("partial buffer must be [slots, m, n]")
            _launch(A, B, s, C, True, C.shape[0])
        elif C.dtype == torch.bfloat16:
            if tuple(C.shape) != (M, N) or not C.is_contiguous():
                raise RuntimeError("C must be bf16 [m, n] (or an fp32 [slots, m, n] partial buffer)")
            if workspace is not None and workspace.numel() < workspace_bytes(N, K, M):
                raise RuntimeError("workspace too small")
            _launch(A, B, s, C, False, 0)
        else:
            raise RuntimeError("C must be bf16 (or an fp32 [slots, m, n] partial buffer)")

    def partial_slots(self, n, k, thread_k=-1, thread_n=-1, sms=-1):
        del thread_k, thread_n, sms
        return partial_slots(n, k)


_ext = None


def ext():
    """The loaded C-ABI library (raises if it is not built), as the reference's extension module."""
    global _ext
    if _ext is None:
        _ext = _Ext(_lib.lib())
    return _ext


def available() -> bool:
    """True when the library loads. Nothing falls back when it does not: callers raise."""
    try:
        ext()
        return True
    except Exception as e:  # not built, wrong arch
        print(f"gfx950 library unavailable: {str(e)[:200]}")
        return False


def padded_groups(K: int) -> int:
    """K/128 rounded up to whole quads of four groups."""
    return -(-(K // GROUP) // 4) * 4


def _check_shape(N: int, K: int):
    if N % 16 or K % GROUP or N <= 0 or K <= 0 or int(ext().tr_packed_bytes(N, K)) == 0:
        raise RuntimeError(f"problem shape (n={N}, k={K}) not supported: need n % 16 == 0, k % {GROUP} == 0 "
                           f"and a packed size below 2 GiB")


def _sm_views(B: torch.Tensor, dtype):
    """(scale, min) as strided views [N/16, Gp/4, 16 rows, 4 groups] into the quads of B."""
    sm = B[..., SM_OFF:].view(dtype).unflatten(-1, (16, 4, 2))
    return sm[..., 0], sm[..., 1]


def pack(qweight: torch.Tensor, scale: torch.Tensor, mn: torch.Tensor, pairs: bool = False):
    """Engine packing (uint8 [N, K/2], bf16/fp16 [N, K/128] x2) -> (B, s, m): B is the quad
    layout uint8 [N/16, Gp/4, 4352] holding codes, scale and min; s and m are views into B
    (they carry the scale dtype). The counterpart of marlin.pack (marlin.py:73-96).
    pairs: the weight is [gate; up] (N % 32 == 0); strip s holds gate rows 8s.. and up rows
    N/2 + 8s.., the layout mul_silu needs."""
    _lib.require_gpu(qweight, scale, mn)
    N, K = qweight.shape[0], qweight.shape[1] * 2
    _check_shape(N, K)
    if qweight.dtype != torch.uint8 or scale.shape != (N, K // GROUP) or mn.shape != scale.shape:
        raise RuntimeError(f"expected uint8 [N, K/2] and [N, K/{GROUP}] scale/min, got {scale.shape}")
    if scale.dtype not in SCALE_DTYPES or mn.dtype != scale.dtype:
        raise RuntimeError("scale/min must both be bf16 or fp16")
    q, s, m = qweight.contiguous(), scale.contiguous(), mn.contiguous()
    if pairs and N % 32:
        raise RuntimeError(f"pair layout needs n % 32 == 0, got n={N}")
    B = torch.empty(N // 16, padded_groups(K) // 4, QUAD, dtype=torch.uint8, device=q.device)
    fn = ext().tr_pack_int4_pairs if pairs else ext().tr_pack_int4
    _lib.check(fn(_lib.ptr(q), _lib.ptr(s), _lib.ptr(m), _lib.ptr(B), N, K, _lib.stream_of(q)), "tr_pack_int4")
    return (B,) + _sm_views(B, scale.dtype)


def unpack(B: torch.Tensor, s: torch.Tensor, m: torch.Tensor, K: int = None, pairs: bool = False):
    """Inverse of pack -> (qweight uint8 [N, K/2], scale [N, K/128], mn [N, K/128])
    (marlin.unpack, marlin.py:99-118). s only supplies the scale dtype. K defaults to the
    padded width; pass the true K when K/128 is not a multiple of 4."""
    _lib.require_gpu(B)
    N = B.shape[0] * 16
    K = B.shape[1] * 4 * GROUP if K is None else K
    if padded_groups(K) != B.shape[1] * 4:
        raise RuntimeError(f"K = {K} does not match the packed weight ({B.shape[1]} quads per strip)")
    q = torch.empty(N, K // 2, dtype=torch.uint8, device=B.device)
    sc = torch.empty(N, K // GROUP, dtype=s.dtype, device=B.device)
    mn = torch.empty_like(sc)
    fn = ext().tr_unpack_int4_pairs if pairs else ext().tr_unpack_int4
    _lib.check(fn(_lib.ptr(B), _lib.ptr(q), _lib.ptr(sc), _lib.ptr(mn), N, K, _lib.stream_of(B)), "tr_unpack_int4")
    return q, sc, mn


_ws = {}


def workspace_bytes(N: int, K: int, M: int = MAX_ROWS) -> int:
    return int(ext().tr_gemm_workspace_bytes(N, K, M))


def workspaces(N: int, device, K: int = None, M: int = MAX_ROWS, min_bytes: int = 0):
    """The per-device workspace of mul(), grown to fit an N x K weight at up to M rows
    (marlin.workspaces, marlin.py:121-135: grow before graph capture; QLinear does so at
    construction). Zero-filled: its counters must read zero between calls, which every call
    restores. Calls that overlap on one device (different streams) would share it."""
    key = torch.device(device).index or 0
    need = min_bytes
    if K is not None:
        need = max([need] + [workspace_bytes(N, K, mm) for mm in {1, min(M, 16), M}])
    ws = _lib.grown_workspace(_ws, key, need, device)
    return ws, ws.numel()


def plan(N: int, K: int, M: int = 1):
    """(S, W, R): K slots, waves per workgroup, strips per workgroup. Depends on M only
    through M > 16."""
    S, W, R = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _lib.check(ext().tr_gemm_plan(N, K, M, ctypes.byref(S), ctypes.byref(W), ctypes.byref(R)), "tr_gemm_plan")
    return S.value, W.value, R.value


def _launch(x, B, s, y, partial, n_slots, strips_per_wg=-1, slots=0):
    M, K = x.shape
    N = B.shape[0] * 16
    if x.dtype != torch.bfloat16 or s.dtype not in SCALE_DTYPES:
        raise RuntimeError("dtypes: x must be bf16, scale/min bf16 or fp16")
    if not (x.is_contiguous() and B.is_contiguous()):
        raise RuntimeError("inputs must be contiguous")
    if M > MAX_ROWS or K % GROUP or padded_groups(K) != B.shape[1] * 4 or B.shape[2] != QUAD:
        raise RuntimeError(f"problem shape (m={M}, n={N}, k={K}) not supported: need m <= {MAX_ROWS}")
    _lib.require_gpu(x, B, y)
    ws, nbytes = None, 0
    need = workspace_bytes(N, K, M) if slots == 0 else (WS_COUNTER_BYTES + 4 * slots * M * N if slots > 1 else 0)
    if not partial and need > 0:
        ws, nbytes = workspaces(N, x.device, K, M, min_bytes=need)
        if nbytes < need:
            raise RuntimeError("workspace too small: call workspaces(N, device, K) before graph capture")
    out, part = (None, y) if partial else (y, None)
    args = (_lib.ptr(x), _lib.ptr(B), _lib.ptr(out), _lib.ptr(part), _lib.ptr(ws), nbytes, M, N, K, GROUP,
            SCALE_DTYPES[s.dtype], n_slots)
    st = _lib.stream_of(x)
    if strips_per_wg == -1 and slots == 0:
        rc = ext().tr_int4_gemm(*args, st)
    else:
        if not partial:
            args = args[:-1] + (slots,)
        rc = ext().tr_int4_gemm_ex(*args, strips_per_wg, st)
    _lib.check(rc, f"tr_int4_gemm (m={M}, n={N}, k={K})")


def mul(x: torch.Tensor, B: torch.Tensor, s: torch.Tensor, m: torch.Tensor = None, thread_k=-1, thread_n=-1, sms=-1,
        *, strips_per_wg=-1, slots=0, out: torch.Tensor = None):
    """x [M, K] bf16 (M <= 32) -> [M, N] bf16 (marlin.mul, marlin.py:138-145).
    s (from pack) supplies the scale dtype; m is accepted for call compatibility. thread_k,
    thread_n and sms sit where marlin.mul has them and are ignored (this kernel picks its own
    tiling). strips_per_wg / slots (keyword-only) override the tiling (-1 / 0 = default); out, a
    contiguous bf16 [M, N] tensor, receives the product instead of a new one."""
    del thread_k, thread_n, sms
    shape = (x.shape[0], B.shape[0] * 16)
    if out is not None and (out.dtype != torch.bfloat16 or tuple(out.shape) != shape or not out.is_contiguous()):
        raise RuntimeError(f"mul: out must be contiguous bf16 {list(shape)}")
    y = torch.empty(*shape, dtype=torch.bfloat16, device=x.device) if out is None else out
    _launch(x, B, s, y, False, 0, strips_per_wg, slots)
    return y


def unpair(y: torch.Tensor) -> torch.Tensor:
    """Columns of a pair-layout product [..., N] (strip s: gate 8s..8s+7, up N/2 + 8s..) back to
    the engine order [gate | up]."""
    lead, N = y.shape[:-1], y.shape[-1]
    return y.view(*lead, N // 16, 2, 8).transpose(-3, -2).reshape(*lead, N)


def mul_silu(x: torch.Tensor, B: torch.Tensor, s: torch.Tensor):
    """x [M, K] bf16 (M <= 32), B a pair-layout [gate; up] weight -> silu(x . gate^T) * (x . up^T)
    as bf16 [M, N/2] in one launch: the gate/up GEMM with the activation of
    tokenrush/fused.py:67-87 in its epilogue (each product rounded to bf16 first)."""
    M, K = x.shape
    N = B.shape[0] * 16
    if x.dtype != torch.bfloat16 or s.dtype not in SCALE_DTYPES or not (x.is_contiguous() and B.is_contiguous()):
        raise RuntimeError("mul_silu: x must be contiguous bf16, scale/min bf16 or fp16")
    if M > MAX_ROWS or K % GROUP or padded_groups(K) != B.shape[1] * 4 or B.shape[2] != QUAD or N % 32:
        raise RuntimeError(f"problem shape (m={M}, n={N}, k={K}) not supported")
    _lib.require_gpu(x, B)
    y = torch.empty(M, N // 2, dtype=torch.bfloat16, device=x.device)
    need = workspace_bytes(N, K, M)
    ws, nbytes = (None, 0) if need == 0 else workspaces(N, x.device, K, M, min_bytes=need)
    rc = ext().tr_int4_gemm_silu(_lib.ptr(x), _lib.ptr(B), _lib.ptr(y), _lib.ptr(ws), nbytes, M, N, K, GROUP,
                                 SCALE_DTYPES[s.dtype], _lib.stream_of(x))
    _lib.check(rc, f"tr_int4_gemm_silu (m={M}, n={N}, k={K})")
    return y


_slots = {}


def partial_slots(N: int, K: int, M: int = 1) -> int:
    """fp32 slots mul_partial writes for an N x K weight at M rows
    (marlin.partial_slots, marlin.py:151-155)."""
    key = (N, K, 0 if M <= 8 else (1 if M <= 16 else 2))  # the plan depends on M through these ranges
    if key not in _slots:
        S = ext().tr_partial_slots(N, K, M)
        if S < 1:
            raise RuntimeError(f"problem shape (n={N}, k={K}) not supported")
        _slots[key] = S
    return _slots[key]


def mul_partial(x: torch.Tensor, B: torch.Tensor, s: torch.Tensor, m: torch.Tensor = None, n_slots: int = None,
                strips_per_wg=-1):
    """x [M, K] bf16 (M <= 32) -> fp32 partials [S, M, N] whose sum over S is the product
    (marlin.mul_partial, marlin.py:158-168). Every slot is written."""
    M, K = x.shape
    N = B.shape[0] * 16
    S = partial_slots(N, K, M) if n_slots is None else n_slots
    y = torch.empty(S, M, N, dtype=torch.float32, device=x.device)
    _launch(x, B, s, y, True, S, strips_per_wg)
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
