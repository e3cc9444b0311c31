"""Row ops around the verify GEMMs, restated from the reference in numpy: the split-K partial
consumer add_rmsnorm and the MLP activation silu_mul. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

bf16 tensors are float32 arrays holding bf16-representable values (oracle.int4.bf16_round).

Pinning (tests/test_oracle_fused.py):
  add_rmsnorm  -- the reference's eager chain (tokenrush/ops.py:16-20 rmsnorm after x + h),
                  restated with torch CPU ops; closed form on constant rows; the reference's
                  own property that S fp32 partials give bit-for-bit the result of their
                  pre-summed bf16 value (tests/test_fused.py:230-245); plain-gain variant
                  against torch's bf16 cast.
  silu_mul     -- torch.nn.functional.silu(g) * u in fp32 (a library routine); closed forms
                  silu(0) = 0, silu(g) -> g for large g.
"""
import numpy as np

from .int4 import bf16_round

F32 = np.float32


def add_rmsnorm(x, h, weight, eps: float, plain: bool = False):
    """x [T, N] bf16-valued; h None, [T, N] bf16-valued or [S, T, N] fp32 partials; weight [N]
    bf16-valued -> (xo, y) as tokenrush/fused.py:23-60: partials summed in slot order in fp32 and
    rounded to bf16, x' = bf16(x + h) (x' = x when h is None), y = x' * rsqrt(mean(x'^2) + eps) times
    (1 + w), or bf16(w * bf16(x' * rsqrt(...))) when plain; y rounded to bf16. The mean is taken
    in float64 (the GPU's order differs; y is compared within a bf16 ulp)."""
    x = np.asarray(x, F32)
    if h is None:
        xo = x
    else:
        h = np.asarray(h, F32)
        if h.ndim == 3:
            acc = h[0].copy()
            for s in range(1, h.shape[0]):
                acc = (acc + h[s]).astype(F32)
            h = bf16_round(acc)
        xo = bf16_round((x + h).astype(F32))
    xd = xo.astype(np.float64)
    r = 1.0 / np.sqrt((xd * xd).mean(-1, keepdims=True) + eps)
    w = np.asarray(weight, np.float64)
    if plain:
        y = bf16_round((w * bf16_round((xd * r).astype(F32)).astype(np.float64)).astype(F32))
    else:
        y = bf16_round((xd * r * (1.0 + w)).astype(F32))
    return xo, y


def silu_mul(gate_up):
    """gate_up [T, 2F] bf16-valued -> bf16(silu(gate) * up) [T, F] (tokenrush/fused.py:67-87), fp64."""
    gu = np.asarray(gate_up, np.float64)
    F = gu.shape[-1] // 2
    g, u = gu[..., :F], gu[..., F:]
    return bf16_round((g / (1.0 + np.exp(-g)) * u).astype(F32))
