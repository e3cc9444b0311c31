"""Full-attention verify step over an FP8 KV cache, restated from the reference in numpy.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

bf16 tensors are float32 arrays holding bf16-representable values (oracle.int4.bf16_round); fp8
codes are uint8 arrays (float8_e4m3fn bit patterns).

Functions (reference file:line):
  fp8_encode / fp8_decode  -- torch's float8_e4m3fn cast (fused.py:300-312 and kv_write_prefill,
                              fused.py:336-347): round to nearest even, largest finite 448.
  attn_prep                -- fused.py:247-325 (_attn_prep_kernel): q/k RMSNorm with (1 + w) gain,
                              partial rope with bf16 rounding of every product and sum, k and v
                              written as fp8 with one scale per (kv head, position) = amax / 448.
  attn_decode              -- fused.py:355-470 (_attn_split_kernel + _attn_reduce_kernel): keys
                              in blocks of 32 split over `nsplit` ranges, online softmax per split
                              (running max per block, l summed before the value scale, P rounded to
                              bf16 after the scale), splits combined by their maxima, bf16(o) times
                              bf16(sigmoid(gate)).
  attn_tree                -- no reference counterpart (the reference verifies chains only): by
                              definition node t of a draft tree attends as the last query of a chain
                              over its root path (rows pos .. pos + depth), prepped at those
                              positions; its key and value rows land at row pos + t.

Pinning (tests/test_oracle_attn.py):
  fp8_encode / fp8_decode  -- torch CPU float8_e4m3fn casts (a library routine): all 256 codes and
                              a sweep of values including ties and the subnormal range.
  attn_prep                -- the reference's eager ops restated with torch CPU bf16 tensors
                              (tokenrush/ops.py:16-20 rmsnorm, :40-48 apply_rope).
  attn_decode              -- a float64 softmax attention over the dequantised cache (the causal
                              rule written directly); independence of the split count; causality
                              (keys past pos + t do not change query t).
  attn_tree                -- built from attn_prep / attn_decode by its definition; a chain tree
                              reduces it to them.
"""
import numpy as np

from .int4 import bf16_round

F32 = np.float32
FP8_MAX = 448.0
BLOCK = 32


# ------------------------------------------------------------------ fp8 e4m3fn

def fp8_decode(codes) -> np.ndarray:
    """uint8 float8_e4m3fn codes -> float32 (NaN codes 0x7F / 0xFF -> NaN)."""
    c = np.asarray(codes, np.uint8).astype(np.int64)
    e, m, s = (c >> 3) & 0xF, c & 7, np.where(c & 0x80, -1.0, 1.0)
    mag = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8.0) * 2.0 ** (e - 7))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return (s * mag).astype(F32)


def fp8_encode(x) -> np.ndarray:
    """float32 -> float8_e4m3fn codes, round to nearest even; |x| beyond 448 saturates to 448
    (the path's writers keep |x| <= 448 up to rounding)."""
    x = np.asarray(x, F32)
    a = np.abs(x).astype(np.float64)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.int64)
    # subnormals: steps of 2^-9 (8 steps reach 2^-6, the smallest normal, whose code is 8)
    sub = np.rint(a * 512.0).astype(np.int64)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -6))).astype(np.int64)
    q = a / 2.0 ** e * 8.0                                  # 8 .. 16
    mq = np.rint(q).astype(np.int64)                        # numpy rounds half to even
    e = np.where(mq == 16, e + 1, e)
    mq = np.where(mq == 16, 8, mq)
    norm = ((e + 7) << 3) | (mq - 8)
    norm = np.where((e + 7 > 15) | (norm > 0x7E), 0x7E, norm)
    code = np.where(a < 2.0 ** -6, sub, norm)
    return (sign | code).astype(np.uint8)


# ------------------------------------------------------------------ prep

def _rmsnorm_1pw(x, w, eps):
    x = np.asarray(x, F32)
    var = (x * x).astype(F32).sum(-1, keepdims=True, dtype=F32) / F32(x.shape[-1])
    inv = (F32(1) / np.sqrt(var + F32(eps))).astype(F32)
    return bf16_round((x * inv * (F32(1) + np.asarray(w, F32))).astype(F32))


def _rope(xn, c, s, RD):
    h = RD // 2
    x1, x2 = xn[..., :h], xn[..., h:RD]
    o1 = bf16_round(bf16_round(x1 * c) + bf16_round(-x2 * s))
    o2 = bf16_round(bf16_round(x2 * c) + bf16_round(x1 * s))
    out = xn.copy()
    out[..., :h], out[..., h:RD] = o1, o2
    return out


def attn_prep(qkv, q_norm_w, k_norm_w, cos, sin, pos: int, k_cache, v_cache, k_scale, v_scale, HQ: int, HKV: int,
              D: int, RD: int, eps: float):
    """qkv [M, HQ 2D + 2 HKV D] bf16-valued; cos/sin [max_pos, RD] bf16-valued; caches uint8
    [HKV, maxlen, D] and scales [HKV, maxlen] fp32 (copied, rows pos..pos+M-1 written) ->
    (q [M, HQ, D] bf16-valued, k_cache, v_cache, k_scale, v_scale)."""
    qkv = np.asarray(qkv, F32)
    M = qkv.shape[0]
    k_cache, v_cache = np.array(k_cache, np.uint8, copy=True), np.array(v_cache, np.uint8, copy=True)
    k_scale, v_scale = np.array(k_scale, F32, copy=True), np.array(v_scale, F32, copy=True)
    q = np.empty((M, HQ, D), F32)
    h = RD // 2
    for t in range(M):
        p = pos + t
        c, s = np.asarray(cos, F32)[p, :h], np.asarray(sin, F32)[p, :h]
        qh = qkv[t, :HQ * 2 * D].reshape(HQ, 2 * D)[:, :D]
        q[t] = _rope(_rmsnorm_1pw(qh, q_norm_w, eps), c, s, RD)
        kh = qkv[t, HQ * 2 * D:HQ * 2 * D + HKV * D].reshape(HKV, D)
        kr = _rope(_rmsnorm_1pw(kh, k_norm_w, eps), c, s, RD)
        vh = qkv[t, HQ * 2 * D + HKV * D:HQ * 2 * D + 2 * HKV * D].reshape(HKV, D)
        for src, cache, scale in ((kr, k_cache, k_scale), (vh, v_cache, v_scale)):
            sc = (np.maximum(np.abs(src).max(-1), F32(1e-6)) / F32(FP8_MAX)).astype(F32)
            cache[:, p] = fp8_encode((src / sc[:, None]).astype(F32))
            scale[:, p] = sc
    return q, k_cache, v_cache, k_scale, v_scale


# ------------------------------------------------------------------ decode

def attn_decode(q, qkv, k_cache, v_cache, k_scale, v_scale, pos: int, HQ: int, HKV: int, D: int, nsplit: int = 32):
    """q [M, HQ, D] bf16-valued, qkv [M, ..] (gates), fp8 caches [HKV, maxlen, D] + scales ->
    out [M, HQ D] bf16-valued. Query t sees cache rows <= pos + t (fused.py:355-470)."""
    q = np.asarray(q, F32)
    M = q.shape[0]
    G = HQ // HKV
    L = pos + M
    nblk = -(-L // BLOCK)
    per = -(-nblk // nsplit)
    scale = F32(D ** -0.5)
    out = np.empty((M, HQ * D), F32)
    for j in range(HKV):
        kd = bf16_round((fp8_decode(k_cache[j, :L]) * np.asarray(k_scale, F32)[j, :L, None]).astype(F32))
        vd = fp8_decode(v_cache[j, :L])                       # exact in bf16
        vs = np.asarray(v_scale, F32)[j, :L]
        qj = q[:, j * G:(j + 1) * G].reshape(M * G, D)         # rows: t * G + g
        lim = pos + np.repeat(np.arange(M), G)
        ms, ls, accs = [], [], []
        for s in range(nsplit):
            m_i = np.full(M * G, -np.inf, F32)
            l_i = np.zeros(M * G, F32)
            acc = np.zeros((M * G, D), F32)
            for blk in range(s * per, min(s * per + per, nblk)):
                kid = np.arange(blk * BLOCK, min(blk * BLOCK + BLOCK, L))
                sc = (qj @ kd[kid].T).astype(F32) * scale
                sc = np.where(kid[None, :] <= lim[:, None], sc, -np.inf).astype(F32)
                m_new = np.maximum(m_i, sc.max(1))
                m_safe = np.where(m_new == -np.inf, F32(0), m_new)
                alpha = np.exp(m_i - m_safe).astype(F32)
                p = np.exp(sc - m_safe[:, None]).astype(F32)
                l_i = (l_i * alpha + p.sum(1, dtype=F32)).astype(F32)
                pb = bf16_round((p * vs[kid][None, :]).astype(F32))
                acc = (acc * alpha[:, None] + pb @ vd[kid]).astype(F32)
                m_i = m_new
            ms.append(m_i)
            ls.append(l_i)
            accs.append(acc)
        m, l, acc = np.stack(ms, 1), np.stack(ls, 1), np.stack(accs, 1)   # [rows, S], [rows, S, D]
        mmax = m.max(1)
        w = np.where(m == -np.inf, F32(0), np.exp(m - mmax[:, None])).astype(F32)
        lt = (w * l).sum(1, dtype=F32)
        o = bf16_round(((acc * w[:, :, None]).sum(1, dtype=F32) / lt[:, None]).astype(F32))
        for t in range(M):
            for g in range(G):
                hq = j * G + g
                gate = np.asarray(qkv, F32)[t, hq * 2 * D + D:hq * 2 * D + 2 * D]
                gs = bf16_round((F32(1) / (F32(1) + np.exp(-gate))).astype(F32))
                out[t, hq * D:(hq + 1) * D] = bf16_round((o[t * G + g] * gs).astype(F32))
    return out


def attn_tree(qkv, q_norm_w, k_norm_w, cos, sin, pos: int, parent, k_cache, v_cache, k_scale, v_scale, HQ: int,
              HKV: int, D: int, RD: int, eps: float, nsplit: int = 32):
    """Draft-tree prep + decode: node t is the last query of a chain over its root path. Returns
    (out [M, HQ D], q [M, HQ, D], k_cache, v_cache, k_scale, v_scale) with node t's key and value
    at row pos + t (roped at pos + depth(t))."""
    from .gdn import root_path
    qkv = np.asarray(qkv, F32)
    M = qkv.shape[0]
    kc, vc = np.array(k_cache, np.uint8, copy=True), np.array(v_cache, np.uint8, copy=True)
    ks, vs = np.array(k_scale, F32, copy=True), np.array(v_scale, F32, copy=True)
    out = np.empty((M, HQ * D), F32)
    q = np.empty((M, HQ, D), F32)
    for t in range(M):
        p = root_path(parent, t)
        d = len(p) - 1
        qp, kp, vp, ksp, vsp = attn_prep(qkv[p], q_norm_w, k_norm_w, cos, sin, pos, k_cache, v_cache, k_scale, v_scale,
                                         HQ, HKV, D, RD, eps)
        out[t] = attn_decode(qp, qkv[p], kp, vp, ksp, vsp, pos, HQ, HKV, D, nsplit)[-1]
        q[t] = qp[-1]
        kc[:, pos + t], vc[:, pos + t] = kp[:, pos + d], vp[:, pos + d]
        ks[:, pos + t], vs[:, pos + t] = ksp[:, pos + d], vsp[:, pos + d]
    return out, q, kc, vc, ks, vs
