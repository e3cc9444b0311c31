"""Pins the numpy oracle for the int4 weights and GEMM (oracle/int4.py) against known
answers, torch's own CPU bf16/fp16 arithmetic (the ops the reference's dequantize runs),
brute force on tiny inputs, and algebraic identities. No GPU."""
import numpy as np
import pytest
import torch

from oracle import int4 as o


def test_bf16_rounding_known_answers():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -2.5, 0.0, 65504.0, 3e38],
                    dtype=np.float32)
    bits = o.f32_to_bf16_bits(vals)
    # 1+2^-8 is a tie -> even (0x3F80); 1+3*2^-8 is a tie -> even (0x3F82); just above a tie rounds up
    assert bits.tolist() == [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0xC020, 0x0000, 0x4780, 0x7F62]


def test_bf16_rounding_matches_torch_cast():
    rng = np.random.default_rng(0)
    a = (rng.standard_normal(100000) * 10 ** rng.uniform(-6, 6, 100000)).astype(np.float32)
    ref = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(o.f32_to_bf16_bits(a), ref)


def test_unpack_known_bytes():
    packed = np.array([[0x21, 0xF0, 0x7A]], dtype=np.uint8)
    assert o.unpack_int4(packed).tolist() == [[1, 2, 0, 15, 10, 7]]
    assert np.array_equal(o.pack_engine(o.unpack_int4(packed)), packed)


def test_dequant_two_roundings_hand_case():
    # q = 15, s = bf16(0.0123) -> q*s rounds to bf16, then + m rounds again
    s = o.bf16_round(np.float32(0.0123)).reshape(1, 1)
    m = o.bf16_round(np.float32(-0.1)).reshape(1, 1)
    packed = np.full((1, 64), 0xFF, dtype=np.uint8)
    w = o.dequantize_int4(packed, s, m)
    t = o.bf16_round(np.float32(15) * s[0, 0])
    assert w[0, 0] == o.bf16_round(t + m[0, 0])
    # single rounding would differ here: the two-rounding result is what the reference computes
    assert np.all(w == w[0, 0])


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_dequant_matches_torch_inplace_ops(dtype):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    p, s, m = o.make_weights(64, 512, seed=3, dtype=dtype)
    codes = torch.from_numpy(o.unpack_int4(p).astype(np.int64))
    w = codes.to(tdt).view(64, 4, 128)
    w.mul_(torch.from_numpy(s).to(tdt)[..., None]).add_(torch.from_numpy(m).to(tdt)[..., None])
    assert np.array_equal(w.float().view(64, 512).numpy(), o.dequantize_int4(p, s, m, dtype))


def test_quantize_roundtrip_and_bound():
    rng = np.random.default_rng(1)
    w = o.bf16_round(rng.standard_normal((32, 256)).astype(np.float32) * 0.02)
    p, s, m = o.quantize_int4(w)
    deq = o.dequantize_int4(p, s, m)
    err = np.abs(deq - w).reshape(32, 2, 128)
    assert np.all(err <= s[..., None] / 2 + np.abs(w).reshape(32, 2, 128).max() * 2 ** -7 + 1e-6)
    # the codes chosen are the nearest: no other code is closer to w
    codes = o.unpack_int4(p).astype(np.float32).reshape(32, 2, 128)
    wg = w.reshape(32, 2, 128)
    for d in (-1, 1):
        alt = np.clip(codes + d, 0, 15) * s[..., None] + m[..., None]
        assert np.all(np.abs(alt - wg) >= np.abs(codes * s[..., None] + m[..., None] - wg) - 1e-7)


def test_quantize_matches_torch_restatement():
    """quant.py:20-36 run as torch CPU ops (what tests/test_marlin.py:10-14 uses to build weights)."""
    from tokenrush_amd.quant import quantize_int4 as q_torch
    rng = np.random.default_rng(2)
    w = o.bf16_round(rng.standard_normal((16, 384)).astype(np.float32) * 0.02)
    pt, st, mt = q_torch(torch.from_numpy(w).to(torch.bfloat16))
    p, s, m = o.quantize_int4(w)
    assert np.array_equal(pt.numpy(), p)
    assert np.array_equal(st.float().numpy(), s) and np.array_equal(mt.float().numpy(), m)


def test_gemm_exact_brute_force():
    p, s, m = o.make_weights(16, 256, seed=4, dtype="bf16")
    x = o.make_x(2, 256, seed=5)
    codes = o.unpack_int4(p)
    y = np.zeros((2, 16))
    for i in range(2):
        for n in range(16):
            y[i, n] = sum(float(x[i, k]) * (int(codes[n, k]) * float(s[n, k // 128]) + float(m[n, k // 128]))
                          for k in range(256))
    assert np.allclose(o.gemm_exact(x, p, s, m), y, rtol=1e-12, atol=1e-12)


def test_gemm_fold_equals_exact():
    p, s, m = o.make_weights(64, 1024, seed=6)
    x = o.make_x(4, 1024, seed=7)
    ref = o.gemm_exact(x, p, s, m)
    assert np.abs(o.gemm_fold(x, p, s, m) - ref).max() <= np.abs(ref).max() * 1e-5


def test_gemm_dequant_is_within_reference_tolerance():
    p, s, m = o.make_weights(64, 1024, seed=8, dtype="bf16")
    x = o.make_x(4, 1024, seed=9)
    ref = o.gemm_exact(x, p, s, m)
    assert np.abs(o.gemm_dequant(x, p, s, m) - ref).max() <= np.abs(ref).max() * 2 ** -7


def test_pack_quads_per_element():
    """The quad layout, element by element, from its definition: code (n, k) sits in quad
    (n // 16, g // 4) with g = k // 128, block t = g % 4 at byte 1024 t, lane 16 c + n % 16 with
    c = (k % 32) // 8, word j = (k % 128) // 32, nibble p with NIBBLE_K[p] == k % 8; row n's
    (scale, min) bits of group g at byte 4096 + 16 (n % 16) + 4 t. K = 640 has 5 groups, so the
    second quad holds 3 zero padding groups."""
    p, s, m = o.make_weights(32, 640, seed=10, dtype="fp16")
    codes = o.unpack_int4(p)
    st = o.pack_quads(p, s, m, "fp16")
    assert st.shape == (2, 2, 4352)
    words = st.view(np.uint32).reshape(2, 2, 1088)
    inv = {int(k): pp for pp, k in enumerate(o.NIBBLE_K)}
    for n in range(32):
        for k in range(640):
            g, c, j = k // 128, (k % 32) // 8, (k % 128) // 32
            w = int(words[n // 16, g // 4, 256 * (g % 4) + 4 * (16 * c + n % 16) + j])
            assert (w >> (4 * inv[k % 8])) & 0xF == codes[n, k]
        for g in range(5):
            sm = int(words[n // 16, g // 4, 1024 + 4 * (n % 16) + g % 4])
            assert sm & 0xFFFF == int(o.to_bits(s[n, g], "fp16")) and sm >> 16 == int(o.to_bits(m[n, g], "fp16"))
    assert not words[:, 1, 256:1024].any()                                      # padding codes
    assert not words[:, 1, 1024:].reshape(2, 16, 4)[:, :, 1:].any()             # padding scale/min
    p2, s2, m2 = o.unpack_quads(st, 640, "fp16")
    assert np.array_equal(p2, p) and np.array_equal(s2, s) and np.array_equal(m2, m)


def test_torch_dequant_linear_matches_numpy_path():
    import torch
    p, s, m = o.make_weights(256, 1024, seed=77, dtype="bf16")
    x = o.make_x(4, 1024, seed=78)
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16)
    y = o.torch_dequant_linear(bf(x), torch.from_numpy(p), bf(s), bf(m)).float().numpy()
    ref = o.gemm_dequant(x, p, s, m, "bf16")
    assert np.abs(y - ref).max() <= np.abs(ref).max() * 2 ** -7
    assert np.linalg.norm(y - ref) <= 1e-2 * np.linalg.norm(ref)
