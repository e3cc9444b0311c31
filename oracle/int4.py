"""int4 g128 (scale + min) weights and the GEMM, restated from the reference in numpy.

bf16/fp16 tensors are held as float32 arrays whose values are exactly representable in
that format; *_bits helpers convert to and from the 16-bit patterns.

Pinning:
  f32_to_bf16_bits / bf16_round  -- known-answer values (tests/test_oracle_int4.py) and torch's
                                    own bf16 cast on CPU (a library routine, not the reference).
  unpack_int4, pack_engine       -- closed form; round trip; hand-built bytes.
  dequantize_int4                -- hand-computed two-rounding cases; torch CPU bf16 in-place
                                    mul/add (the very ops quant.py:47-53 runs).
  quantize_int4                  -- RTN bound |w - deq| <= s/2 + bf16 rounding; exact round trip
                                    on weights built from codes.
  gemm_exact / gemm_dequant      -- brute-force triple loop on tiny shapes; fp64 matmul.
  gemm_fold                      -- equals gemm_exact within fp32 error (algebraic identity).
  torch_dequant_linear           -- equals gemm_dequant within bf16 output rounding plus a bf16
                                    matmul's accumulation error (the same dequantized weights).
  pack_quads                     -- our own layout (not the reference's): its definition is
                                    checked by a per-element brute force and by unpack_quads.
"""
import numpy as np

GROUP = 128


# ------------------------------------------------------------------ 16-bit float helpers

def f32_to_bf16_bits(a) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(a) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def f16_round(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(a, dtype: str) -> np.ndarray:
    return bf16_round(a) if dtype == "bf16" else f16_round(a)


def to_bits(a, dtype: str) -> np.ndarray:
    return f32_to_bf16_bits(a) if dtype == "bf16" else np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def from_bits(b, dtype: str) -> np.ndarray:
    return bf16_bits_to_f32(b) if dtype == "bf16" else np.asarray(b, np.uint16).view(np.float16).astype(np.float32)


# ------------------------------------------------------------------ packing

def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """uint8 [N, K/2] -> codes uint8 [N, K]; element 2j is the low nibble of byte j
    (reference tokenrush/quant.py:39-44)."""
    lo = packed & 0xF
    hi = packed >> 4
    return np.stack([lo, hi], axis=-1).reshape(packed.shape[0], -1)


def pack_engine(codes: np.ndarray) -> np.ndarray:
    """codes uint8 [N, K] (0..15) -> uint8 [N, K/2] (reference tokenrush/quant.py:34-35)."""
    c = codes.reshape(codes.shape[0], -1, 2).astype(np.uint8)
    return (c[..., 0] | (c[..., 1] << 4)).astype(np.uint8)


# nibble p of a strip-layout word holds element NIBBLE_K[p] of its 8-element run
NIBBLE_K = np.array([0, 2, 4, 6, 1, 3, 5, 7])


QUAD = 4352          # bytes per (16-row strip, 4 groups) quad
SM_OFF = 4096        # offset of the quad's (scale, min) words


def padded_groups(K: int) -> int:
    """K/128 rounded up to whole quads of four groups."""
    return -(-(K // GROUP) // 4) * 4


def pack_quads(packed: np.ndarray, scale: np.ndarray, mn: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """Engine packing + scale/min -> the gfx950 quad layout uint8 [N/16, Gp/4, 4352] (the layout
    token-rush_amd/csrc/int4_gemm.hip documents; it has no counterpart in the reference, whose
    load-time repack is Marlin's, marlin.py:73-96). Groups are padded with zeros to Gp, a
    multiple of 4. Per (strip, quad): four 1024-byte blocks of codes in lane order (lane
    16 c + n, word j holds k = 32 j + 8 c .. + 7 of row n, code k0 + 2p in nibble p and
    k0 + 2p + 1 in nibble p + 4), then
    16 rows x 4 groups of (scale bits | min bits << 16)."""
    codes = unpack_int4(packed).astype(np.uint32)
    N, K = codes.shape
    S, G, Gp = N // 16, K // GROUP, padded_groups(K)
    c = np.zeros((N, Gp * GROUP), dtype=np.uint32)
    c[:, :K] = codes
    a = c.reshape(S, 16, Gp, 4, 4, 8)                    # strip, n, g, j, c, kk: k = 32 j + 8 c + kk
    a = a.transpose(0, 2, 4, 1, 3, 5).reshape(S, Gp, 64, 4, 8)   # lane = 16 c + n, word j
    words = np.zeros((S, Gp, 64, 4), dtype=np.uint32)
    for p in range(8):
        words |= a[..., NIBBLE_K[p]] << np.uint32(4 * p)
    sm = np.zeros((N, Gp), dtype=np.uint32)
    sm[:, :G] = to_bits(scale, dtype).astype(np.uint32) | (to_bits(mn, dtype).astype(np.uint32) << np.uint32(16))
    sm = sm.reshape(S, 16, Gp // 4, 4).transpose(0, 2, 1, 3).reshape(S, Gp // 4, 64)   # [S, q, row, t]
    out = np.concatenate([words.reshape(S, Gp // 4, 1024), sm], axis=-1)
    return np.ascontiguousarray(out).view(np.uint8).reshape(S, Gp // 4, QUAD)


def unpack_quads(quads: np.ndarray, K: int, dtype: str = "bf16"):
    """Inverse of pack_quads (padding dropped) -> (engine packing uint8 [N, K/2], scale, mn)."""
    S, nq = quads.shape[:2]
    Gp, G = nq * 4, K // GROUP
    words = np.ascontiguousarray(quads).view(np.uint32).reshape(S, nq, QUAD // 4)
    w = words[..., :1024].reshape(S, Gp, 64, 4)
    a = np.zeros((S, Gp, 64, 4, 8), dtype=np.uint32)
    for p in range(8):
        a[..., NIBBLE_K[p]] = (w >> np.uint32(4 * p)) & 0xF
    a = a.reshape(S, Gp, 4, 16, 4, 8).transpose(0, 3, 1, 4, 2, 5).reshape(S * 16, Gp * GROUP)[:, :K]
    sm = words[..., 1024:].reshape(S, nq, 16, 4).transpose(0, 2, 1, 3).reshape(S * 16, Gp)[:, :G]
    scale = from_bits((sm & 0xFFFF).astype(np.uint16), dtype)
    mn = from_bits((sm >> 16).astype(np.uint16), dtype)
    return pack_engine(a.astype(np.uint8)), scale, mn


# ------------------------------------------------------------------ quantize / dequantize

def quantize_int4(w: np.ndarray, group: int = GROUP):
    """bf16-valued [N, K] -> (packed uint8 [N, K/2], scale, mn) (bf16-valued float32).
    Reference tokenrush/quant.py:20-36: per-group min/max, scale = (max-min)/15 (0 -> 1), both
    rounded to bf16 first, codes = clamp(round((w - mn)/scale), 0, 15)."""
    N, K = w.shape
    wf = w.astype(np.float32).reshape(N, K // group, group)
    mn = wf.min(-1)
    scale = (wf.max(-1) - mn) / np.float32(15.0)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    scale, mn = bf16_round(scale), bf16_round(mn)
    q = np.clip(np.rint((wf - mn[..., None]) / scale[..., None]), 0, 15).astype(np.uint8)
    return pack_engine(q.reshape(N, K)), scale, mn


def dequantize_int4(packed: np.ndarray, scale: np.ndarray, mn: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """-> [N, K] float32 holding round(round(q * s) + m) in `dtype` (reference
    tokenrush/quant.py:47-53: in-place bf16 mul_ then add_, each computed in fp32 and rounded).
    For fp16 parameters the same two roundings happen in fp16."""
    codes = unpack_int4(packed).astype(np.float32)
    N, K = codes.shape
    G = scale.shape[1]
    c = codes.reshape(N, G, K // G)
    t = round_to(c * scale.astype(np.float32)[..., None], dtype)
    return round_to(t + mn.astype(np.float32)[..., None], dtype).reshape(N, K)


# ------------------------------------------------------------------ the GEMM

def weights_f64(packed, scale, mn) -> np.ndarray:
    """The exact dense weight q * s + m in float64 (no intermediate rounding)."""
    codes = unpack_int4(packed).astype(np.float64)
    N, K = codes.shape
    G = scale.shape[1]
    w = codes.reshape(N, G, K // G) * scale.astype(np.float64)[..., None] + mn.astype(np.float64)[..., None]
    return w.reshape(N, K)


def gemm_exact(x, packed, scale, mn) -> np.ndarray:
    """y = x . (q s + m)^T in float64: the mathematical product the kernels approximate."""
    return x.astype(np.float64) @ weights_f64(packed, scale, mn).T


def gemm_dequant(x, packed, scale, mn, dtype: str = "bf16") -> np.ndarray:
    """The reference's torch path: x.float() @ dequantize_int4(q, s, m).float().t()
    (tokenrush/quant.py:373-374; the `ref` of tests/test_marlin.py:33), in float64."""
    return x.astype(np.float64) @ dequantize_int4(packed, scale, mn, dtype).astype(np.float64).T


def gemm_fold(x, packed, scale, mn) -> np.ndarray:
    """The per-(row, group) fold s * sum(q x) + m * sum(x) in fp32 (reference
    tokenrush/quant.py:113-119, the Triton GEMV's inner step), accumulated over groups in order."""
    codes = unpack_int4(packed).astype(np.float32)
    N, K = codes.shape
    G = scale.shape[1]
    xf = x.astype(np.float32)
    M = xf.shape[0]
    acc = np.zeros((M, N), dtype=np.float32)
    for g in range(G):
        sl = slice(g * (K // G), (g + 1) * (K // G))
        qx = (xf[:, sl] @ codes[:, sl].T).astype(np.float32)          # [M, N]
        xs = xf[:, sl].sum(-1, dtype=np.float32)[:, None]              # [M, 1]
        acc = acc + scale[:, g][None, :].astype(np.float32) * qx + mn[:, g][None, :].astype(np.float32) * xs
    return acc


# ------------------------------------------------------------------ synthetic inputs (benchmark configs)

def make_weights(N: int, K: int, seed: int, dtype: str = "fp16"):
    """Codes uniform in 0..15 (engine packing), scale ~U(0.002, 0.02), min ~U(-0.15, -0.01),
    rounded to `dtype` (benchmark configs 1-2)."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    scale = round_to(rng.uniform(0.002, 0.02, size=(N, K // GROUP)).astype(np.float32), dtype)
    mn = round_to(rng.uniform(-0.15, -0.01, size=(N, K // GROUP)).astype(np.float32), dtype)
    return pack_engine(codes), scale, mn


def make_x(M: int, K: int, seed: int) -> np.ndarray:
    """bf16-valued activations ~N(0, 1)."""
    rng = np.random.default_rng(seed)
    return bf16_round(rng.standard_normal((M, K)).astype(np.float32))


def torch_dequant_linear(x, packed, scale, mn):
    """The reference's `dequant` backend as torch runs it on the CPU: unpack, one bf16 (or fp16)
    temporary multiplied and added in place, then F.linear in that dtype (tokenrush/quant.py:39-53,
    quant.py:373-374). Arguments are torch CPU tensors: x [M, K] bf16, packed uint8 [N, K/2],
    scale / mn [N, K/128] in the parameter dtype. Returns [M, N] in x's dtype. Used as the CPU
    baseline's timed body and checked against gemm_dequant."""
    import torch
    import torch.nn.functional as F
    N, G = scale.shape
    w = torch.stack([packed & 0xF, packed >> 4], dim=-1).view(N, -1).to(scale.dtype).view(N, G, -1)
    w.mul_(scale[..., None]).add_(mn[..., None])
    return F.linear(x, w.view(N, -1).to(x.dtype))
