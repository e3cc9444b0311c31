"""Weight-only int4 linear layer, group 128, asymmetric (w = q * s + m): the reference's
tokenrush/quant.py API (QLinear and helpers) over the gfx950 kernels.

Packing (unchanged from the reference, quant.py:9-10): element 2j sits in the low nibble of
byte j, element 2j+1 in the high nibble, along the input dimension: uint8 [N, K/2]. Scale
and min are [N, K/128], bf16 in the engine (fp16 is accepted for the benchmark format).

Backends:
  gfx950   the strip-layout MFMA kernel (gfx950.py), M <= 32 rows in one launch, the default.
  dequant  dequantize (HIP kernel) then torch matmul at every T: the reference's own
           correctness path (quant.py:56-74, quant.py:373-374).
The reference's marlin/triton/tinygemm backends are CUDA/Triton and have no place here; a
QLinear built with one of those names gets the gfx950 kernel.
"""
import torch
import torch.nn.functional as F

from . import gfx950

GROUP = 128
BACKENDS = ("gfx950", "dequant")
DEFAULT_BACKEND = "gfx950"
MAX_ROWS = gfx950.MAX_ROWS        # beyond this T the prefill path (dequant + matmul) runs
_ALIASES = {"marlin": "gfx950", "triton": "gfx950", "tinygemm": "gfx950"}


def quantize_int4(w: torch.Tensor, group: int = GROUP):
    """bf16 [out, in] -> (qweight uint8 [out, in/2], scale bf16 [out, in/group], mn bf16 [out, in/group]).
    Round-to-nearest with the group parameters rounded to bf16 before the codes are chosen
    (reference quant.py:20-36). Offline tooling: plain torch ops on w's device."""
    out, inp = w.shape
    assert inp % group == 0 and inp % 2 == 0
    wf = w.float().view(out, inp // group, group)
    mn = wf.amin(-1)
    scale = (wf.amax(-1) - mn) / 15.0
    scale = torch.where(scale == 0, torch.ones_like(scale), scale).to(torch.bfloat16)
    mn = mn.to(torch.bfloat16)
    q = ((wf - mn.float()[..., None]) / scale.float()[..., None]).round().clamp_(0, 15).to(torch.uint8)
    q = q.view(out, inp // 2, 2)
    return (q[..., 0] | (q[..., 1] << 4)).contiguous(), scale.contiguous(), mn.contiguous()


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """uint8 [out, in/2] -> uint8 codes [out, in] (reference quant.py:39-44)."""
    return torch.stack([packed & 0xF, packed >> 4], dim=-1).view(packed.shape[0], -1)


def dequantize_int4(packed, scale, mn) -> torch.Tensor:
    """-> [out, in] in the scale dtype: round(round(q * s) + m), the reference's two bf16
    roundings (quant.py:47-53), computed by the HIP dequant kernel."""
    return gfx950.dequantize(packed, scale, mn)


class QLinear:
    """int4 group-wise weight (reference quant.py:282-391): same constructor, same methods.

    split_k > 1 marks a matrix whose consumer sums fp32 partials (the reference sets it on
    the hidden-sized outputs, weights.py:163-174); partials(x) then returns [S, T, N] with
    S = gfx950.partial_slots(N, K), whose sum over S is the product."""

    def __init__(self, qweight, scale, mn, backend=DEFAULT_BACKEND, split_k: int = 1, layout: str = "rows"):
        backend = _ALIASES.get(backend, backend)
        assert backend in BACKENDS, backend
        assert layout in ("rows", "gate_up"), layout
        self.shape_ = (qweight.shape[0], qweight.shape[1] * 2)
        self.group = self.shape_[1] // scale.shape[1]
        self.backend = backend
        self.split_k = split_k
        # "gate_up": the weight is [gate; up] and silu_mul(x) fuses the activation (gfx950 only)
        self.layout = layout if backend == "gfx950" else "rows"
        if backend == "gfx950":
            if self.group != GROUP:
                raise RuntimeError(f"gfx950 backend needs group {GROUP}, got {self.group}")
            self.B, self.s, self.m = gfx950.pack(qweight, scale, mn, pairs=self.layout == "gate_up")
            gfx950.workspaces(self.shape_[0], qweight.device, self.shape_[1])   # sized before any graph capture
            self.qweight = self.scale = self.mn = None
        else:
            self.qweight, self.scale, self.mn = qweight, scale, mn

    @staticmethod
    def cat(parts, backend=DEFAULT_BACKEND):
        """Concatenate along the output dimension (rows are independent in this packing)."""
        nib = [p.nibbles() for p in parts]
        return QLinear(torch.cat([n[0] for n in nib]), torch.cat([n[1] for n in nib]),
                       torch.cat([n[2] for n in nib]), backend)

    @property
    def shape(self):
        return self.shape_

    @property
    def nbytes(self):
        ts = (self.B,) if self.backend == "gfx950" else (self.qweight, self.scale, self.mn)
        return sum(t.numel() * t.element_size() for t in ts)

    def nibbles(self):
        """(qweight, scale, mn) in the engine's packing (unpacked from the strip layout if needed)."""
        if self.backend == "gfx950":
            return gfx950.unpack(self.B, self.s, self.m, self.shape_[1], pairs=self.layout == "gate_up")
        return self.qweight, self.scale, self.mn

    def rows(self, ids: torch.Tensor):
        """A QLinear over the output rows `ids` (the truncated draft vocabulary)."""
        return QLinear(*(t.index_select(0, ids) for t in self.nibbles()), backend=self.backend, split_k=self.split_k)

    def dequantize(self) -> torch.Tensor:
        return dequantize_int4(*self.nibbles())

    def __call__(self, x: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
        """x [T, K] -> [T, N]; out (bf16 [T, N], contiguous) receives the product when given."""
        T = x.shape[0]
        if self.backend == "dequant" or T > MAX_ROWS:
            y = F.linear(x, self.dequantize().to(x.dtype))
        elif self.layout == "gate_up":
            y = gfx950.unpair(gfx950.mul(x.contiguous(), self.B, self.s))
        else:
            return gfx950.mul(x.contiguous(), self.B, self.s, out=out)
        return y if out is None else out.copy_(y)

    def silu_mul(self, x: torch.Tensor) -> torch.Tensor:
        """silu(gate) * up of this [gate; up] weight's product, [T, N/2] bf16: one fused launch
        for a "gate_up" layout, else the product followed by the activation kernel
        (tokenrush/model.py:156-160 with fused.py:67-87)."""
        if self.layout == "gate_up" and x.shape[0] <= MAX_ROWS:
            return gfx950.mul_silu(x.contiguous(), self.B, self.s)
        from .fused import silu_mul
        return silu_mul(self(x))

    def partials(self, x: torch.Tensor) -> torch.Tensor:
        """x [T, K] -> [S, T, N] fp32 whose sum over S is the product (S == 1 unless split-K)."""
        T = x.shape[0]
        if self.backend == "gfx950" and self.split_k > 1 and T <= MAX_ROWS:
            return gfx950.mul_partial(x.contiguous(), self.B, self.s)
        return self(x).float()[None]
