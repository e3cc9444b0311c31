"""One speculative verify step of the 64-layer hybrid model, random-init,
capturable as a single hipGraph.

The layer body follows Engine._body (reference tokenrush/model.py:211-260) with the verify-path
pieces of this package:

    per layer li:
      x, n = add_rmsnorm(x, h, ln1)          h: the previous layer's down partials [S, M, hidden]
      GDN layer (li % 4 != 3):  u = in_qkvz(n)   [M, 16384]   (model.py:76, marlin.mul)
      attention (li % 4 == 3):  u = qkv(n)       [M, 14336]   (model.py:121)
      y = mixer(u)                            [M, 6144]   STAND-IN (see below)
      h = out.partials(y)                     [S, M, hidden] fp32 (model.py:85, split-K partials)
      x, n = add_rmsnorm(x, h, ln2)
      a = silu_mul(gate_up(n))                [M, 17408]  (model.py:156-160), one fused launch
      h = down.partials(a)                    [S, M, hidden] fp32
    _, n = add_rmsnorm(x, h, final_norm); logits = lm_head(n)   [M, 248320]
    greedy accept: n_accepted, tok, pos += n + 1, slot = n (model.py:302-312), in the lm_head
    GEMM's epilogue (one launch)

Stand-ins: the GDN recurrence (fused.py:119-237) and attention (fused.py:247-470) are not part of
this build; each mixer is replaced by silu(u[:, :6144]) * u[:, 6144:12288], one launch that reads
the projection output and writes the [M, 6144] input of the output projection. Every GEMM, the
partial consumers, lm_head and the accept are the real kernels. The embedding gather is replaced
by the step's input buffer x0.
"""
from dataclasses import dataclass

import torch

from . import gfx950
from .accept import AcceptState, lm_head_greedy
from .fused import add_rmsnorm, silu_mul
from .quant import QLinear


@dataclass
class StepConfig:
    n_layers: int = 64
    hidden: int = 5120
    mlp: int = 17408
    gdn_in: int = 16384        # in_qkvz output
    attn_qkv: int = 14336      # q, k, v (+ gate) output
    mixer_out: int = 6144      # input of the output projection
    vocab: int = 248320
    eps: float = 1e-6
    attn_every: int = 4        # layer li is full attention when li % attn_every == attn_every - 1

    def is_attention(self, li: int) -> bool:
        return li % self.attn_every == self.attn_every - 1


SMALL = StepConfig(n_layers=4, hidden=512, mlp=1024, gdn_in=2048, attn_qkv=1792, mixer_out=768, vocab=4096)


def _random_linear(N, K, gen, device, split_k=1, scale_dtype=torch.bfloat16, layout="rows"):
    """Codes uniform in 0..15, scale ~U(0.002, 0.02), min ~U(-0.15, -0.01)."""
    q = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=device, generator=gen)
    s = (torch.rand(N, K // 128, device=device, generator=gen) * 0.018 + 0.002).to(scale_dtype)
    m = (torch.rand(N, K // 128, device=device, generator=gen) * 0.14 - 0.15).to(scale_dtype)
    lin = QLinear(q, s, m, split_k=split_k, layout=layout)
    del q, s, m
    return lin


class Layer:
    def __init__(self, cfg: StepConfig, li: int, gen, device):
        H = cfg.hidden
        self.attention = cfg.is_attention(li)
        n_in = cfg.attn_qkv if self.attention else cfg.gdn_in
        self.proj = _random_linear(n_in, H, gen, device)
        self.out = _random_linear(H, cfg.mixer_out, gen, device, split_k=4)      # weights.py:163-174
        self.gate_up = _random_linear(2 * cfg.mlp, H, gen, device, layout="gate_up")   # silu fused in its epilogue
        self.down = _random_linear(H, cfg.mlp, gen, device, split_k=4)
        self.ln1 = (torch.randn(H, device=device, generator=gen) * 0.1).to(torch.bfloat16)
        self.ln2 = (torch.randn(H, device=device, generator=gen) * 0.1).to(torch.bfloat16)


class VerifyModel:
    """Random-init weights of the config-5 hybrid (int4 g128, bf16 scale/min) and the verify step.
    Weights are packed once at construction (QLinear packs them into the quad layout)."""

    def __init__(self, cfg: StepConfig = StepConfig(), device="cuda:0", seed: int = 0):
        self.cfg = cfg
        self.device = torch.device(device)
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        self.layers = [Layer(cfg, li, gen, self.device) for li in range(cfg.n_layers)]
        self.final_norm = (torch.randn(cfg.hidden, device=self.device, generator=gen) * 0.1).to(torch.bfloat16)
        self.lm_head = _random_linear(cfg.vocab, cfg.hidden, gen, self.device)

    def nbytes(self) -> int:
        n = self.lm_head.nbytes
        for L in self.layers:
            n += L.proj.nbytes + L.out.nbytes + L.gate_up.nbytes + L.down.nbytes
        return n

    def mixer(self, u: torch.Tensor) -> torch.Tensor:
        """Stand-in for the GDN / attention mixer: [M, n_in] -> [M, mixer_out]."""
        F = self.cfg.mixer_out
        return silu_mul(u[:, :2 * F])

    def hidden(self, x0: torch.Tensor) -> torch.Tensor:
        """x0 [M, hidden] bf16 -> post-final-norm hidden [M, hidden] bf16 (model.py:252-254)."""
        cfg = self.cfg
        x, h = x0, None
        for L in self.layers:
            x, n = add_rmsnorm(x, h, L.ln1, cfg.eps)
            y = self.mixer(L.proj(n))
            h = L.out.partials(y)
            x, n = add_rmsnorm(x, h, L.ln2, cfg.eps)
            h = L.down.partials(L.gate_up.silu_mul(n))
        _, n = add_rmsnorm(x, h, self.final_norm, cfg.eps)
        return n

    def body(self, x0: torch.Tensor) -> torch.Tensor:
        """x0 [M, hidden] bf16 -> logits [M, vocab] bf16."""
        return self.lm_head(self.hidden(x0))

    def step(self, x0: torch.Tensor, spec_toks: torch.Tensor, st: AcceptState) -> torch.Tensor:
        """Body + lm_head with the greedy accept/commit in its epilogue (one launch). Returns the
        logits, kept as the reference keeps them (model.py:300; graph-owned under capture)."""
        return lm_head_greedy(self.lm_head, self.hidden(x0), spec_toks, st, keep_logits=True)


def prepare(model: VerifyModel, M: int):
    """Allocate every workspace a step at M rows uses (before graph capture)."""
    cfg = model.cfg
    for L in model.layers:
        for lin in (L.proj, L.gate_up):
            gfx950.workspaces(lin.shape[0], model.device, lin.shape[1], M)
    gfx950.workspaces(cfg.vocab, model.device, cfg.hidden, M)
