"""Pins the row-op oracle (oracle/fused.py) against the reference's eager chain restated with
torch CPU ops, closed forms, and the reference's own partials property. No GPU."""
import numpy as np
import torch

from oracle import fused as f
from oracle.int4 import bf16_round

F32 = np.float32


def _bf(rng, *shape, std=1.0):
    return bf16_round((rng.standard_normal(shape) * std).astype(F32))


def _torch_rmsnorm(x, w, eps):
    """tokenrush/ops.py:16-20 restated: fp32 normalize, (1 + w) gain, cast to x's dtype."""
    xf = x.float()
    out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (out * (1.0 + w.float())).to(x.dtype)


def test_add_rmsnorm_matches_torch_chain():
    rng = np.random.default_rng(0)
    x, h, w = _bf(rng, 8, 5120), _bf(rng, 8, 5120, std=0.5), _bf(rng, 5120, std=0.1)
    xo, y = f.add_rmsnorm(x, h, w, 1e-6)
    tx = torch.from_numpy(x).bfloat16() + torch.from_numpy(h).bfloat16()      # bf16 + bf16 -> bf16
    assert np.array_equal(xo, tx.float().numpy())
    ty = _torch_rmsnorm(tx, torch.from_numpy(w).bfloat16(), 1e-6).float().numpy()
    assert np.abs(y - ty).max() <= np.abs(ty).max() * 2 ** -7
    assert np.mean(y == ty) > 0.95


def test_add_rmsnorm_partials_equal_presummed_bf16():
    """tests/test_fused.py:230-245: S fp32 partials give bit-for-bit the result of their
    pre-summed bf16 value."""
    rng = np.random.default_rng(1)
    x, w = _bf(rng, 4, 5120), _bf(rng, 5120, std=0.5)
    parts = (rng.standard_normal((3, 4, 5120)) * 0.3).astype(F32)
    pre = bf16_round(((parts[0] + parts[1]).astype(F32) + parts[2]).astype(F32))
    xo1, y1 = f.add_rmsnorm(x, parts, w, 1e-6)
    xo2, y2 = f.add_rmsnorm(x, pre, w, 1e-6)
    assert np.array_equal(xo1, xo2) and np.array_equal(y1, y2)


def test_add_rmsnorm_constant_row_closed_form():
    """A constant row c normalizes to c / sqrt(c^2 + eps), times the gain."""
    x = np.full((1, 256), 3.0, F32)
    w = bf16_round(np.linspace(-0.5, 0.5, 256).astype(F32))
    xo, y = f.add_rmsnorm(x, None, w, 1e-6)
    assert np.array_equal(xo, x)
    assert np.allclose(y[0], bf16_round((3.0 / np.sqrt(9.0 + 1e-6) * (1.0 + w)).astype(F32)), rtol=0, atol=0)


def test_add_rmsnorm_plain_gain():
    rng = np.random.default_rng(2)
    x, w = _bf(rng, 2, 1024), _bf(rng, 1024)
    _, y = f.add_rmsnorm(x, None, w, 1e-6, plain=True)
    tx = torch.from_numpy(x)
    n = (tx * torch.rsqrt(tx.pow(2).mean(-1, keepdim=True) + 1e-6)).bfloat16()
    ref = (torch.from_numpy(w).bfloat16() * n).float().numpy()          # Qwen3RMSNorm: weight * cast(x)
    assert np.abs(y - ref).max() <= np.abs(ref).max() * 2 ** -7


def test_silu_mul_matches_torch_and_closed_forms():
    rng = np.random.default_rng(3)
    gu = _bf(rng, 8, 2 * 1024, std=3.0)
    y = f.silu_mul(gu)
    t = torch.from_numpy(gu)
    ref = (torch.nn.functional.silu(t[:, :1024]) * t[:, 1024:]).bfloat16().float().numpy()
    assert np.abs(y - ref).max() <= np.abs(ref).max() * 2 ** -8
    z = np.zeros((1, 4), F32)
    z[0, 2:] = [5.0, 2.0]
    assert f.silu_mul(z)[0, 0] == 0.0
    big = np.array([[40.0, 3.0]], F32)
    assert f.silu_mul(big)[0, 0] == bf16_round(np.array([120.0], F32))[0]
