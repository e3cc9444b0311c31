"""Parity of the gfx950 row kernels (csrc/fused.hip) with the oracle (oracle/fused.py), through
the C-ABI. The residual output of add_rmsnorm is bit-exact; the normalized output is within one
bf16 ulp of a float64-mean restatement (its fp32 reduction order differs); silu_mul within one
bf16 ulp. Mirrors tests/test_fused.py:230-262 of the reference (partials == pre-summed bf16)."""
import numpy as np
import pytest
import torch

from oracle import fused as f
from oracle.int4 import bf16_round

pytestmark = pytest.mark.gpu
F32 = np.float32


def _bf(rng, *shape, std=1.0):
    return bf16_round((rng.standard_normal(shape) * std).astype(F32))


def _dev(a, dt=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dt).to("cuda:0")


def _ulp_close(got, ref, ulps=1):
    """|got - ref| <= ulps bf16 ulps of ref (elementwise)."""
    got = got.float().cpu().numpy()
    e = np.floor(np.log2(np.maximum(np.abs(ref), 1e-30)))
    assert np.all(np.abs(got - ref) <= ulps * 2.0 ** (e - 7) + 1e-30), np.abs(got - ref).max()


@pytest.mark.parametrize("T,N,S", [(1, 5120, 1), (8, 5120, 3), (8, 5120, 1), (32, 5120, 4), (5, 1000, 2), (3, 8192, 6), (2, 8, 8)])
def test_add_rmsnorm_partials(dev, T, N, S):
    from tokenrush_amd.fused import add_rmsnorm
    print(f"add_rmsnorm T={T} N={N} S={S}", flush=True)
    rng = np.random.default_rng(T * 100 + S)
    x, w = _bf(rng, T, N), _bf(rng, N, std=0.2)
    parts = (rng.standard_normal((S, T, N)) * 0.3).astype(F32)
    xo_r, y_r = f.add_rmsnorm(x, parts, w, 1e-6)
    xo, y = add_rmsnorm(_dev(x), _dev(parts, torch.float32), _dev(w), 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(xo.float().cpu().numpy(), xo_r)
    _ulp_close(y, y_r)


def test_add_rmsnorm_modes_and_presum(dev):
    from tokenrush_amd.fused import add_rmsnorm
    rng = np.random.default_rng(7)
    x, w = _bf(rng, 8, 5120), _bf(rng, 5120, std=0.2)
    parts = (rng.standard_normal((3, 8, 5120)) * 0.3).astype(F32)
    pre = bf16_round(((parts[0] + parts[1]).astype(F32) + parts[2]).astype(F32))
    xo1, y1 = add_rmsnorm(_dev(x), _dev(parts, torch.float32), _dev(w), 1e-6)
    xo2, y2 = add_rmsnorm(_dev(x), _dev(pre), _dev(w), 1e-6)
    assert torch.equal(xo1, xo2) and torch.equal(y1, y2)               # reference test_fused.py:243-245
    xo3, y3 = add_rmsnorm(_dev(x), None, _dev(w), 1e-6)
    _, y_r = f.add_rmsnorm(x, None, w, 1e-6)
    assert torch.equal(xo3, _dev(x))
    _ulp_close(y3, y_r)
    _, yp = add_rmsnorm(_dev(x), _dev(pre), _dev(w), 1e-6, plain=True)
    _, yp_r = f.add_rmsnorm(x, pre, w, 1e-6, plain=True)
    _ulp_close(yp, yp_r, ulps=2)


@pytest.mark.parametrize("T,F", [(1, 17408), (8, 17408), (32, 1000), (3, 8)])
def test_silu_mul(dev, T, F):
    from tokenrush_amd.fused import silu_mul
    rng = np.random.default_rng(F + T)
    gu = _bf(rng, T, 2 * F, std=3.0)
    _ulp_close(silu_mul(_dev(gu)), f.silu_mul(gu))


def test_silu_mul_strided_slice(dev):
    """A column slice of a wider row (the stand-in mixers read qkvz[:, :2F])."""
    from tokenrush_amd.fused import silu_mul
    rng = np.random.default_rng(11)
    wide = _bf(rng, 8, 16384, std=2.0)
    got = silu_mul(_dev(wide)[:, :12288])
    _ulp_close(got, f.silu_mul(wide[:, :12288]))


@pytest.mark.parametrize("T,H", [(8, 5120), (1, 1000), (32, 64)])
def test_embed_rows(dev, T, H):
    """tr_embed_rows equals the table's rows at the ids bit for bit (model.py:215); an id outside
    the vocabulary gives a zero row and raises the status word."""
    from tokenrush_amd.fused import embed_rows
    print(f"embed_rows T={T} H={H}", flush=True)
    rng = np.random.default_rng(T + H)
    V = 3001
    table = _bf(rng, V, H)
    ids = rng.integers(0, V, T).astype(np.int64)
    ids[0] = V - 1
    status = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    got = embed_rows(_dev(table), torch.from_numpy(ids).to("cuda:0"), status=status)
    torch.cuda.synchronize()
    assert np.array_equal(got.float().cpu().numpy(), table[ids]) and int(status) == 0
    bad = ids.copy()
    bad[-1] = V
    got = embed_rows(_dev(table), torch.from_numpy(bad).to("cuda:0"), status=status)
    torch.cuda.synchronize()
    assert int(status) == 1
    assert np.array_equal(got.float().cpu().numpy()[:-1], table[ids[:-1]])
    assert not got[-1].float().abs().sum().item()
