"""Parity of the gfx950 int4 verify GEMM with the CPU oracle (oracle/int4.py), called through
the C-ABI (tokenrush_amd.gfx950 -> libtrhip.so). Mirrors the reference's tests/test_marlin.py:
the same shapes and M values, its tolerance (max-abs <= max|ref| * 2^-7, test_marlin.py:35-36),
rows independent of M (:42-52), graph replay == eager (:55-72), partials sum to the product
(:75-87); plus a tight bound, the fp16 benchmark format and M up to 32."""
import numpy as np
import pytest
import torch

from oracle import int4 as o

pytestmark = pytest.mark.gpu

TDT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def say(*a):
    print(*a, flush=True)


def dev_weights(p, s, m, dtype):
    d = torch.device("cuda:0")
    return (torch.from_numpy(p).to(d), torch.from_numpy(s).to(TDT[dtype]).to(d),
            torch.from_numpy(m).to(TDT[dtype]).to(d))


def dev_x(x):
    return torch.from_numpy(x).to(torch.bfloat16).to("cuda:0")


def check_close(y: torch.Tensor, ref: np.ndarray, what=""):
    y = y.float().cpu().numpy().astype(np.float64)
    err = np.abs(y - ref)
    amax = np.abs(ref).max()
    assert err.max() <= amax * 2 ** -7, (what, err.max(), amax)                      # reference bar
    assert np.linalg.norm(y - ref) <= 1e-2 * np.linalg.norm(ref), what
    # tight: bf16 output rounding (2^-9 relative) plus fp32 accumulation noise
    assert np.all(err <= np.abs(ref) * 2 ** -8 + amax * 2 ** -14), (what, (err - np.abs(ref) * 2 ** -8).max())


@pytest.mark.parametrize("N,K", [(5120, 6144), (256, 5120), (1280, 5120), (5120, 17408), (256, 384), (512, 2176)])
def test_pack_matches_oracle(dev, N, K):
    from tokenrush_amd import gfx950
    say(f"pack N={N} K={K}")
    p, s, m = o.make_weights(N, K, seed=0, dtype="bf16")
    q, sd, md = dev_weights(p, s, m, "bf16")
    B, sp, mp = gfx950.pack(q, sd, md)
    torch.cuda.synchronize()
    assert B.shape == (N // 16, o.padded_groups(K) // 4, 4352)
    assert np.array_equal(B.cpu().numpy(), o.pack_quads(p, s, m, "bf16"))
    assert torch.equal(sp[:, :, :, :].reshape(N // 16, -1, 16, 4).permute(0, 2, 1, 3).reshape(N, -1)[:, :K // 128], sd)
    q2, s2, m2 = gfx950.unpack(B, sp, mp, K)
    assert torch.equal(q, q2) and torch.equal(sd, s2) and torch.equal(md, m2)


@pytest.mark.parametrize("N,K", [(5120, 6144), (256, 5120), (1280, 5120), (14336, 5120), (5120, 17408),
                                 (256, 384), (1280, 2176), (512, 128)])
@pytest.mark.parametrize("M", [1, 3, 8, 9, 13, 16])
def test_mul_matches_oracle(dev, N, K, M):
    from tokenrush_amd import gfx950
    say(f"mul N={N} K={K} M={M}")
    p, s, m = o.make_weights(N, K, seed=1, dtype="bf16")
    x = o.make_x(M, K, seed=2)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "bf16"))
    y = gfx950.mul(dev_x(x), B, sp, mp)
    torch.cuda.synchronize()
    check_close(y, o.gemm_exact(x, p, s, m), f"N={N} K={K} M={M}")


@pytest.mark.parametrize("M", [17, 24, 32])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_mul_two_row_tiles(dev, M, dtype):
    from tokenrush_amd import gfx950
    say(f"mul M={M} {dtype}")
    p, s, m = o.make_weights(1280, 5120, seed=3, dtype=dtype)
    x = o.make_x(M, 5120, seed=4)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, dtype))
    y = gfx950.mul(dev_x(x), B, sp, mp)
    torch.cuda.synchronize()
    check_close(y, o.gemm_exact(x, p, s, m), f"M={M}")


@pytest.mark.parametrize("R", [1, 2, 3, 7, 32])
@pytest.mark.parametrize("M", [8, 24])
def test_strips_per_workgroup_agree(dev, R, M):
    """Every strips-per-workgroup choice gives the same bits (the reduction order per strip
    does not depend on it)."""
    from tokenrush_amd import gfx950
    say(f"strips per wg R={R} M={M}")
    p, s, m = o.make_weights(512, 17408, seed=5, dtype="fp16")
    x = o.make_x(M, 17408, seed=6)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "fp16"))
    y = gfx950.mul(dev_x(x), B, sp, mp, strips_per_wg=R)
    torch.cuda.synchronize()
    check_close(y, o.gemm_exact(x, p, s, m), f"R={R}")
    assert torch.equal(y, gfx950.mul(dev_x(x), B, sp, mp))
    if R == 1 and M == 8:
        # marlin.mul's positional thread_k, thread_n, sms (marlin.py:138) are accepted and ignored
        assert torch.equal(gfx950.mul(dev_x(x), B, sp, mp, 64, 256, 16), y)


@pytest.mark.parametrize("slots", [2, 3, 5, 12])
@pytest.mark.parametrize("M", [8, 24])
def test_slot_counts_in_kernel_sum(dev, slots, M):
    """Out mode with K slots summed in the kernel by the last-arriving slot: every slot count
    (odd ones included, which leave the last load step of the slot sum half used) matches the
    oracle."""
    from tokenrush_amd import gfx950
    say(f"slots={slots} M={M}")
    N, K = 1024, 6144
    p, s, m = o.make_weights(N, K, seed=7, dtype="fp16")
    x = o.make_x(M, K, seed=8)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "fp16"))
    y = gfx950.mul(dev_x(x), B, sp, mp, slots=slots)
    torch.cuda.synchronize()
    check_close(y, o.gemm_exact(x, p, s, m), f"slots={slots}")


def test_rows_independent_of_m(dev):
    """Row i of an M-row call is bit-identical whatever M is (reference test_marlin.py:42-52)."""
    from tokenrush_amd import gfx950
    say("rows independent of M")
    p, s, m = o.make_weights(5120, 17408, seed=7, dtype="bf16")
    x = dev_x(o.make_x(32, 17408, seed=8))
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "bf16"))
    y16 = gfx950.mul(x[:16].contiguous(), B, sp, mp)
    y32 = gfx950.mul(x, B, sp, mp)
    for M in (1, 3, 8):
        assert torch.equal(gfx950.mul(x[:M].contiguous(), B, sp, mp), y16[:M]), M
    for M in (17, 24):
        assert torch.equal(gfx950.mul(x[:M].contiguous(), B, sp, mp), y32[:M]), M


@pytest.mark.parametrize("N,K", [(512, 128), (16, 384), (1280, 2176), (48, 5120)])
@pytest.mark.parametrize("M", [17, 25, 31])
def test_two_row_tiles_small_and_odd_k(dev, N, K, M):
    """Above 16 rows the activations are staged in two 16-row passes through an LDS area shared
    with the reduction ring: one group (K = 128, padded to a quad), an odd group count
    (K = 2176), one strip (N = 16) and rows past M in both tiles, against float64."""
    from tokenrush_amd import gfx950
    say(f"two tiles small N={N} K={K} M={M}")
    p, s, m = o.make_weights(N, K, seed=40 + M, dtype="bf16")
    x = o.make_x(M, K, seed=41 + M)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "bf16"))
    check_close(gfx950.mul(dev_x(x), B, sp, mp), x.astype(np.float64) @ o.weights_f64(p, s, m).T, f"N={N} K={K} M={M}")


def test_repeat_is_deterministic(dev):
    from tokenrush_amd import gfx950
    say("determinism")
    p, s, m = o.make_weights(7168, 5120, seed=9, dtype="fp16")
    x = dev_x(o.make_x(8, 5120, seed=10))
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "fp16"))
    y0 = gfx950.mul(x, B, sp, mp)
    for _ in range(5):
        assert torch.equal(gfx950.mul(x, B, sp, mp), y0)


def test_graph_replay_matches_eager(dev):
    """Reference test_marlin.py:55-72, replayed several times with eager work in between."""
    from tokenrush_amd import gfx950
    say("graph replay")
    p, s, m = o.make_weights(1280, 5120, seed=11, dtype="bf16")
    x = dev_x(o.make_x(4, 5120, seed=12))
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "bf16"))
    y = gfx950.mul(x, B, sp, mp)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        out = gfx950.mul(x, B, sp, mp)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out.copy_(gfx950.mul(x, B, sp, mp))
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y), i
        _ = gfx950.mul(x, B, sp, mp)        # eager work between replays


@pytest.mark.parametrize("N,K", [(5120, 6144), (5120, 17408), (256, 5120)])
@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("slots", [None, 3])
def test_partials_sum_to_product(dev, N, K, M, slots):
    """Reference test_marlin.py:75-87: every slot written, the sum is the product."""
    from tokenrush_amd import gfx950
    say(f"partials N={N} K={K} M={M} slots={slots}")
    p, s, m = o.make_weights(N, K, seed=13, dtype="bf16")
    x = o.make_x(M, K, seed=14)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "bf16"))
    xd = dev_x(x)
    y = gfx950.mul(xd, B, sp, mp)
    part = gfx950.mul_partial(xd, B, sp, mp, n_slots=slots)
    assert part.shape[1:] == (M, N) and part.shape[0] == (slots or gfx950.partial_slots(N, K))
    ref = o.gemm_exact(x, p, s, m)
    tot = part.sum(0).double().cpu().numpy()
    assert np.abs(tot - ref).max() <= np.abs(ref).max() * 2 ** -7
    assert (part.sum(0).to(torch.bfloat16).float() - y.float()).abs().max().item() <= np.abs(ref).max() * 2 ** -7
    part2 = torch.full_like(part, float("nan"))
    part2.copy_(gfx950.mul_partial(xd, B, sp, mp, n_slots=slots))
    assert torch.equal(part, part2)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_dequant_bit_exact(dev, dtype):
    from tokenrush_amd import gfx950
    say(f"dequant {dtype}")
    p, s, m = o.make_weights(256, 5120, seed=15, dtype=dtype)
    w = gfx950.dequantize(*dev_weights(p, s, m, dtype))
    assert np.array_equal(w.float().cpu().numpy(), o.dequantize_int4(p, s, m, dtype))


def test_config1_full_size(dev):
    """benchmark config 1: M=1, 5120 x 5120, fp16 scale/min."""
    from tokenrush_amd import gfx950
    say("config1")
    p, s, m = o.make_weights(5120, 5120, seed=101, dtype="fp16")
    x = o.make_x(1, 5120, seed=102)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "fp16"))
    check_close(gfx950.mul(dev_x(x), B, sp, mp), o.gemm_exact(x, p, s, m), "config1")


@pytest.mark.parametrize("N,K", [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408)])
def test_config2_layer_set_m8(dev, N, K):
    """benchmark config 2: one layer's projection set at M=8, fp16 scale/min, full size."""
    from tokenrush_amd import gfx950
    say(f"config2 N={N} K={K}")
    p, s, m = o.make_weights(N, K, seed=200 + N % 97, dtype="fp16")
    x = o.make_x(8, K, seed=201)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "fp16"))
    check_close(gfx950.mul(dev_x(x), B, sp, mp), o.gemm_exact(x, p, s, m), f"config2 {N}x{K}")


def test_qlinear_api(dev):
    """The reference QLinear surface: __call__, partials, nibbles, rows, cat, dequantize,
    nbytes, shape, and the T > MAX_ROWS prefill path."""
    from tokenrush_amd.quant import QLinear
    say("qlinear api")
    p, s, m = o.make_weights(512, 1024, seed=16, dtype="bf16")
    qd, sd, md = dev_weights(p, s, m, "bf16")
    lin = QLinear(qd, sd, md, split_k=4)
    assert lin.shape == (512, 1024) and lin.backend == "gfx950" and lin.group == 128
    assert lin.nbytes == 512 // 16 * 2 * 4352
    x = o.make_x(8, 1024, seed=17)
    ref = o.gemm_exact(x, p, s, m)
    check_close(lin(dev_x(x)), ref, "call")
    part = lin.partials(dev_x(x))
    assert part.dtype == torch.float32 and part.shape[1:] == (8, 512)
    q2, s2, m2 = lin.nibbles()
    assert torch.equal(q2, qd) and torch.equal(s2, sd) and torch.equal(m2, md)
    ids = torch.tensor([5, 17, 300, 511, 0, 1, 2, 3, 4, 6, 7, 8, 9, 10, 11, 12], device="cuda")
    sub = lin.rows(ids)
    check_close(sub(dev_x(x)), ref[:, ids.cpu().numpy()], "rows")
    both = QLinear.cat([lin, sub])
    assert both.shape == (528, 1024)
    assert torch.equal(lin.dequantize().float().cpu(), torch.from_numpy(o.dequantize_int4(p, s, m)))
    xl = o.make_x(40, 1024, seed=18)                  # T > 32: dequant + matmul (prefill path)
    y = lin(dev_x(xl)).float().cpu().numpy()
    r = o.gemm_dequant(xl, p, s, m)
    assert np.abs(y - r).max() <= np.abs(r).max() * 2 ** -7


@pytest.mark.parametrize("N,K", [(2048, 5120), (34816, 5120), (1024, 17408), (512, 384)])
@pytest.mark.parametrize("M", [1, 8, 24])
def test_gate_up_pair_layout_and_fused_silu(dev, N, K, M):
    """Pair layout: byte-exact against the oracle's quad layout of the row-permuted weight, a
    round trip through unpack, the plain product unchanged after unpair, and the fused silu
    epilogue bit-identical to the product followed by the activation kernel (incl. K split
    across workgroups, K = 17408)."""
    from tokenrush_amd import gfx950
    from tokenrush_amd.fused import silu_mul
    say(f"pairs N={N} K={K} M={M}")
    p, s, m = o.make_weights(N, K, seed=21, dtype="bf16")
    qd, sd, md = dev_weights(p, s, m, "bf16")
    Bp, sp, mp = gfx950.pack(qd, sd, md, pairs=True)
    F = N // 2
    perm = np.array([(8 * (r // 16) + r % 16) if r % 16 < 8 else F + 8 * (r // 16) + r % 16 - 8 for r in range(N)])
    if M == 1:
        assert np.array_equal(Bp.cpu().numpy(), o.pack_quads(p[perm], s[perm], m[perm], "bf16"))
        q2, s2, m2 = gfx950.unpack(Bp, sp, mp, K, pairs=True)
        assert torch.equal(q2, qd) and torch.equal(s2, sd) and torch.equal(m2, md)
    B, sb, _ = gfx950.pack(qd, sd, md)
    x = dev_x(o.make_x(M, K, seed=22))
    y = gfx950.mul(x, B, sb)
    assert torch.equal(gfx950.unpair(gfx950.mul(x, Bp, sp)), y)
    assert torch.equal(gfx950.mul_silu(x, Bp, sp), silu_mul(y))


def test_qlinear_gate_up_layout(dev):
    from tokenrush_amd.fused import silu_mul
    from tokenrush_amd.quant import QLinear
    p, s, m = o.make_weights(1024, 1024, seed=23, dtype="bf16")
    qd, sd, md = dev_weights(p, s, m, "bf16")
    plain, gu = QLinear(qd, sd, md), QLinear(qd, sd, md, layout="gate_up")
    x = dev_x(o.make_x(8, 1024, seed=24))
    assert torch.equal(gu(x), plain(x))
    assert torch.equal(gu.silu_mul(x), silu_mul(plain(x)))
    q2, s2, m2 = gu.nibbles()
    assert torch.equal(q2, qd) and torch.equal(s2, sd) and torch.equal(m2, md)
    check_close(gu(x), o.gemm_exact(o.make_x(8, 1024, seed=24), p, s, m), "gate_up layout")


_C2 = {}


def _config2_case(N, K):
    """Config-2 weights (fp16 scale/min) on the device and their float64 dense form, cached per
    shape so the M sweep builds each only once."""
    from tokenrush_amd import gfx950
    if (N, K) not in _C2:
        _C2.clear()
        p, s, m = o.make_weights(N, K, seed=300 + N % 89, dtype="fp16")
        B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "fp16"))
        _C2[(N, K)] = (B, sp, mp, o.weights_f64(p, s, m))
    return _C2[(N, K)]


@pytest.mark.parametrize("N,K", [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408)])
@pytest.mark.parametrize("M", [2, 4, 12, 24, 32])
def test_config2_shapes_m_sweep(dev, N, K, M):
    """The bench's M sweep (config 2 at M = 2, 4), a 12-row call (the one-tile kernel's second
    staging pass) and config 4's M = 32 verify GEMM (with M = 24 between the row-tile boundaries)
    on every config-2 shape against float64."""
    from tokenrush_amd import gfx950
    say(f"config2 sweep N={N} K={K} M={M}")
    B, sp, mp, W = _config2_case(N, K)
    x = o.make_x(M, K, seed=400 + M)
    check_close(gfx950.mul(dev_x(x), B, sp, mp), x.astype(np.float64) @ W.T, f"{N}x{K} M={M}")


@pytest.mark.parametrize("N,K", [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408)])
@pytest.mark.parametrize("M", [17, 32])
def test_config2_partials_two_row_tiles(dev, N, K, M):
    """Partial mode above 16 rows (config 4 runs the o and down projections this way at M = 32):
    every slot written, the slot sum matches float64 to the GEMM bar, and equals mul()'s output
    after the bf16 rounding up to summation order."""
    from tokenrush_amd import gfx950
    say(f"config2 partials N={N} K={K} M={M}")
    B, sp, mp, W = _config2_case(N, K)
    x = o.make_x(M, K, seed=500 + M)
    xd = dev_x(x)
    part = torch.full((gfx950.partial_slots(N, K, M), M, N), float("nan"), device="cuda:0")
    part.copy_(gfx950.mul_partial(xd, B, sp, mp))
    assert part.shape[0] == gfx950.partial_slots(N, K, M) and not torch.isnan(part).any()
    ref = x.astype(np.float64) @ W.T
    check_close(part.sum(0), ref, f"partials {N}x{K} M={M}")
    y = gfx950.mul(xd, B, sp, mp).float()
    assert (part.sum(0) - y).abs().max().item() <= np.abs(ref).max() * 2 ** -8


def test_ext_mul_binding_semantics(dev):
    """ext().mul(A, B, C, s, m, workspace, red) as the reference's torch binding calls it
    (marlin_bf16.cpp:14-44): C bf16 -> the product, C fp32 [slots, m, n] -> the partials; the same
    bits as gfx950.mul / mul_partial."""
    from tokenrush_amd import gfx950
    say("ext().mul binding")
    p, s, m = o.make_weights(5120, 17408, seed=31, dtype="bf16")
    x = o.make_x(8, 17408, seed=32)
    B, sp, mp = gfx950.pack(*dev_weights(p, s, m, "bf16"))
    xd = dev_x(x)
    ws, _ = gfx950.workspaces(5120, dev, 17408, 8)
    C = torch.empty(8, 5120, dtype=torch.bfloat16, device=dev)
    gfx950.ext().mul(xd, B, C, sp, mp, ws, None, -1, -1, -1)
    S = gfx950.ext().partial_slots(5120, 17408)
    P = torch.empty(S, 8, 5120, dtype=torch.float32, device=dev)
    gfx950.ext().mul(xd, B, P, sp, mp, ws, None)
    torch.cuda.synchronize()
    assert torch.equal(C, gfx950.mul(xd, B, sp, mp))
    assert torch.equal(P, gfx950.mul_partial(xd, B, sp, mp))
    with pytest.raises(RuntimeError):
        gfx950.ext().mul(xd, B, torch.empty(8, 5120, dtype=torch.float16, device=dev), sp, mp, ws, None)
