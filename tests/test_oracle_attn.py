"""Pins the attention oracle (oracle/attn.py): torch's float8_e4m3fn casts, the reference's eager
rmsnorm + rope restated with torch CPU bf16 ops (tokenrush/ops.py:16-20, :33-48), a float64
softmax attention written directly from the causal rule, split-count independence and causality.
No GPU."""
import numpy as np
import torch

from oracle import attn as o
from oracle.int4 import bf16_round

F32 = np.float32
HQ, HKV, D, RD = 6, 2, 256, 64


def _bf(rng, *shape, std=1.0):
    return bf16_round((rng.standard_normal(shape) * std).astype(F32))


def test_fp8_codec_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    dec = o.fp8_decode(codes)
    finite = np.isfinite(ref)
    assert np.array_equal(np.isnan(dec), ~finite)
    assert np.array_equal(dec[finite], ref[finite])
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(20000) * 50, rng.standard_normal(20000) * 0.01,
                           rng.uniform(-448, 448, 20000), o.fp8_decode(codes[np.isfinite(ref)]),
                           # exact midpoints between neighbouring codes (ties to even)
                           (ref[finite][1:120] + ref[finite][2:121]) / 2, [0.0, -0.0, 2 ** -10, 2 ** -9 * 1.5]])
    vals = vals.astype(F32)
    want = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(o.fp8_encode(vals), want)


def _torch_prep(qkv, qw, kw, cos, sin, pos, eps):
    """tokenrush/ops.py rmsnorm (fp32 normalize, (1 + w) gain, cast) then apply_rope in bf16."""
    t = torch.from_numpy(qkv).bfloat16()
    M = t.shape[0]
    q = t[:, :HQ * 2 * D].view(M, HQ, 2 * D)[..., :D]
    k = t[:, HQ * 2 * D:HQ * 2 * D + HKV * D].view(M, HKV, D)

    def rms(x, w):
        xf = x.float()
        out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        return (out * (1.0 + torch.from_numpy(w).float())).to(torch.bfloat16)

    def rope(x, c, s):
        xr, xp = x[..., :RD], x[..., RD:]
        rot = torch.cat([-xr[..., RD // 2:], xr[..., :RD // 2]], -1)
        return torch.cat([xr * c + rot * s, xp], -1)

    c = torch.from_numpy(cos[pos:pos + M]).bfloat16()[:, None, :]
    s = torch.from_numpy(sin[pos:pos + M]).bfloat16()[:, None, :]
    return rope(rms(q, qw), c, s).float().numpy(), rope(rms(k, kw), c, s).float().numpy()


def test_prep_matches_torch_ops():
    rng = np.random.default_rng(1)
    M, pos, maxlen = 5, 40, 64
    qkv = _bf(rng, M, HQ * 2 * D + 2 * HKV * D)
    qw, kw = _bf(rng, D, std=0.5), _bf(rng, D, std=0.5)
    ang = np.arange(maxlen)[:, None] * (1e7 ** -(np.arange(0, RD, 2) / RD))[None, :]
    emb = np.concatenate([ang, ang], 1)
    cos, sin = bf16_round(np.cos(emb).astype(F32)), bf16_round(np.sin(emb).astype(F32))
    kc = np.zeros((HKV, maxlen, D), np.uint8)
    ks = np.ones((HKV, maxlen), F32)
    q, kc2, vc2, ks2, vs2 = o.attn_prep(qkv, qw, kw, cos, sin, pos, kc, kc, ks, ks, HQ, HKV, D, RD, 1e-6)
    tq, tk = _torch_prep(qkv, qw, kw, cos, sin, pos, 1e-6)
    # rsqrt vs 1/sqrt: equal except where a product lands on a bf16 rounding tie
    assert np.mean(q == tq) > 0.99 and np.abs(q - tq).max() <= np.abs(tq).max() * 2 ** -7
    kdq = o.fp8_decode(kc2[:, pos:pos + M]) * ks2[:, pos:pos + M, None]          # [HKV, M, D]
    assert np.abs(kdq.transpose(1, 0, 2) - tk).max() <= np.abs(tk).max() * 2 ** -3
    v = qkv[:, HQ * 2 * D + HKV * D:].reshape(M, HKV, D)
    vdq = o.fp8_decode(vc2[:, pos:pos + M]) * vs2[:, pos:pos + M, None]
    assert np.abs(vdq.transpose(1, 0, 2) - v).max() <= np.abs(v).max() * 2 ** -3
    assert np.array_equal(kc2[:, :pos], kc[:, :pos]) and np.array_equal(kc2[:, pos + M:], kc[:, pos + M:])


def _cache(rng, maxlen, L):
    kc = np.zeros((HKV, maxlen, D), np.uint8)
    vc = np.zeros((HKV, maxlen, D), np.uint8)
    k, v = _bf(rng, HKV, L, D), _bf(rng, HKV, L, D)
    ks = (np.abs(k).max(-1) / 448).astype(F32)
    vs = (np.abs(v).max(-1) / 448).astype(F32)
    kc[:, :L] = o.fp8_encode(k / ks[..., None])
    vc[:, :L] = o.fp8_encode(v / vs[..., None])
    kso = np.ones((HKV, maxlen), F32)
    vso = np.ones((HKV, maxlen), F32)
    kso[:, :L], vso[:, :L] = ks, vs
    return kc, vc, kso, vso


def _float64_attention(q, qkv, kc, vc, ks, vs, pos):
    M = q.shape[0]
    G = HQ // HKV
    out = np.empty((M, HQ * D))
    for t in range(M):
        L = pos + t + 1
        for hq in range(HQ):
            j = hq // G
            kd = bf16_round((o.fp8_decode(kc[j, :L]) * ks[j, :L, None]).astype(F32)).astype(np.float64)
            vd = o.fp8_decode(vc[j, :L]).astype(np.float64) * vs[j, :L, None]
            sc = kd @ q[t, hq].astype(np.float64) / np.sqrt(D)
            p = np.exp(sc - sc.max())
            oo = (p @ vd) / p.sum()
            gate = qkv[t, hq * 2 * D + D:hq * 2 * D + 2 * D].astype(np.float64)
            out[t, hq * D:(hq + 1) * D] = oo / (1 + np.exp(-gate))
    return out


def test_decode_matches_float64_attention_and_is_causal():
    rng = np.random.default_rng(2)
    M, pos, maxlen = 4, 300, 400
    q = _bf(rng, M, HQ, D, std=0.5)
    qkv = _bf(rng, M, HQ * 2 * D + 2 * HKV * D)
    kc, vc, ks, vs = _cache(rng, maxlen, pos + M)
    out = o.attn_decode(q, qkv, kc, vc, ks, vs, pos, HQ, HKV, D, nsplit=4)
    ref = _float64_attention(q, qkv, kc, vc, ks, vs, pos)
    assert np.linalg.norm(out - ref) <= 1e-2 * np.linalg.norm(ref)
    # causality: rows past pos + t never reach query t
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, pos + 1:] = 0x38
    vc2[:, pos + 1:] = 0x48
    out2 = o.attn_decode(q, qkv, kc2, vc2, ks, vs, pos, HQ, HKV, D, nsplit=4)
    assert np.array_equal(out2[0], out[0])
    assert not np.array_equal(out2[1], out[1])


def test_decode_split_count_independent():
    rng = np.random.default_rng(3)
    M, pos, maxlen = 3, 500, 512
    q = _bf(rng, M, HQ, D, std=0.5)
    qkv = _bf(rng, M, HQ * 2 * D + 2 * HKV * D)
    kc, vc, ks, vs = _cache(rng, maxlen, pos + M)
    a = o.attn_decode(q, qkv, kc, vc, ks, vs, pos, HQ, HKV, D, nsplit=1)
    b = o.attn_decode(q, qkv, kc, vc, ks, vs, pos, HQ, HKV, D, nsplit=32)
    assert np.linalg.norm(a - b) <= 1e-2 * np.linalg.norm(a)


def _rope_tab(maxlen):
    ang = np.arange(maxlen)[:, None] * (1e7 ** -(np.arange(0, RD, 2) / RD))[None, :]
    emb = np.concatenate([ang, ang], 1)
    return bf16_round(np.cos(emb).astype(F32)), bf16_round(np.sin(emb).astype(F32))


def test_tree_on_a_chain_is_the_chain_step():
    """A chain tree reduces the tree oracle to attn_prep + attn_decode: bit for bit with one
    split (masked keys add exact zeros, so the longer key range changes nothing)."""
    rng = np.random.default_rng(11)
    M, pos, maxlen = 5, 90, 128
    qkv = _bf(rng, M, HQ * 2 * D + 2 * HKV * D)
    qw, kw = _bf(rng, D, std=0.5), _bf(rng, D, std=0.5)
    cos, sin = _rope_tab(maxlen)
    kc, vc, ks, vs = _cache(rng, maxlen, pos)
    q, kc2, vc2, ks2, vs2 = o.attn_prep(qkv, qw, kw, cos, sin, pos, kc, vc, ks, vs, HQ, HKV, D, RD, 1e-6)
    out = o.attn_decode(q, qkv, kc2, vc2, ks2, vs2, pos, HQ, HKV, D, nsplit=1)
    parent = np.arange(-1, M - 1, dtype=np.int32)
    ot, qt, kct, vct, kst, vst = o.attn_tree(qkv, qw, kw, cos, sin, pos, parent, kc, vc, ks, vs, HQ, HKV, D, RD, 1e-6,
                                             nsplit=1)
    assert np.array_equal(out, ot) and np.array_equal(q, qt)
    assert np.array_equal(kc2, kct) and np.array_equal(vc2, vct) and np.array_equal(ks2, kst)


def test_tree_rows_and_masks():
    """Node t's key row sits at pos + t, roped at pos + depth(t); its output does not depend on
    nodes off its root path."""
    rng = np.random.default_rng(12)
    pos, maxlen = 70, 128
    parent = np.array([-1, 0, 0, 1, 2, 3], np.int32)   # two branches: 0-1-3-5 and 0-2-4
    M = parent.shape[0]
    qkv = _bf(rng, M, HQ * 2 * D + 2 * HKV * D)
    qw, kw = _bf(rng, D, std=0.5), _bf(rng, D, std=0.5)
    cos, sin = _rope_tab(maxlen)
    kc, vc, ks, vs = _cache(rng, maxlen, pos)
    out, q, kct, vct, kst, vst = o.attn_tree(qkv, qw, kw, cos, sin, pos, parent, kc, vc, ks, vs, HQ, HKV, D, RD, 1e-6)
    # node 4 (depth 2): its key equals a prep of its row at position pos + 2
    _, k1, _, s1, _ = o.attn_prep(qkv[4:5], qw, kw, cos, sin, pos + 2, kc, vc, ks, vs, HQ, HKV, D, RD, 1e-6)
    assert np.array_equal(kct[:, pos + 4], k1[:, pos + 2]) and np.array_equal(kst[:, pos + 4], s1[:, pos + 2])
    q2 = qkv.copy()
    q2[[2, 4]] = _bf(rng, 2, HQ * 2 * D + 2 * HKV * D)         # the other branch
    out2 = o.attn_tree(q2, qw, kw, cos, sin, pos, parent, kc, vc, ks, vs, HQ, HKV, D, RD, 1e-6)[0]
    for t in (0, 1, 3, 5):
        assert np.array_equal(out2[t], out[t])
    assert not np.array_equal(out2[4], out[4])
