"""One speculative verify step of the 64-layer hybrid model (benchmark config 5), random-init,
capturable as a single hipGraph.

The layer body follows Engine._body (reference tokenrush/model.py:211-260) with the verify-path
kernels of this package:

    per layer li:
      x, n = add_rmsnorm(x, h, ln1)          h: the previous layer's down partials [S, M, hidden]
      GDN layer (li % 4 != 3) (model.py:76-80, fused path):
        u = in_qkvz(n)                        [M, 16384]  q | k | v | z
        y = gdn_step_fused(u, n, ...)         [M, 6144]   conv ring, gates, delta rule with
                                                          snapshot slots, gated norm (one launch)
        h = out.partials(y)                   [S, M, hidden] fp32 split-K partials
      attention layer (li % 4 == 3) (model.py:115-121, fused path):
        u = qkv(n)                            [M, 14336]  q | gate per head, k, v
        q = attn_prep(u, ...)                 q/k norm + rope, k/v into the FP8 cache
        y = attn_decode_fused(q, u, ...)      [M, 6144]   flash-decoding + output gate
        h = o.partials(y)
      x, n = add_rmsnorm(x, h, ln2)
      a = silu_mul(gate_up(n))                [M, 17408]  (model.py:156-160), one fused launch
      h = down.partials(a)
    _, n = add_rmsnorm(x, h, final_norm); logits = lm_head(n)   [M, 248320]
    greedy accept: n_accepted, tok, pos += n + 1, slot = n (model.py:302-312), in the lm_head
    GEMM's epilogue (one launch)

A draft-tree step (step_tree, benchmark config 4: up to 32 nodes) runs the same body with the
tree mixers (ancestor-masked attention, per-node GDN states), then the tree accept and its commit:
the accepted path's KV rows and scales move to consecutive positions, the conv rings take the
path's inputs, and the slot names the deepest accepted node, whose state snapshot the next step
continues from.

The decode state (tokenrush/state.py:14-43) lives on the device: the position and the committed
recurrent-state slot (read by the mixers, written by the accept), the conv rings and the fp32
recurrent state in 8 snapshot slots per GDN layer, and the FP8 KV cache with per-(head, position)
scales per attention layer, preloaded with `live` random tokens. `verify(spec_toks, ...)` is the
reference's _verify_step (model.py:293-312) whole: the embedding gather of the verify tokens, the
body, the lm_head and the accept, keeping spec_logits[:M] and spec_hidden[:M] (the post-final-norm
rows the draft head reads next, model.py:300-301). `step(x0, ...)` starts from given input rows.
"""
from dataclasses import dataclass

import torch

from . import gfx950
from .accept import AcceptState, accept_residual, accept_sampled, accept_tree, commit_rows, lm_head_greedy
from .attn import AttnConfig, attn_decode_fused, attn_prep, rope_table
from .attn import NSPLIT as ATTN_NSPLIT
from .attn import workspace as attn_workspace
from .fused import add_rmsnorm, embed_rows
from .gdn import RING, GDNConfig, gdn_step_fused, tree_commit
from .gdn import workspace as gdn_workspace
from .quant import QLinear
from .sample import SamplingParams
from .sample import workspace as accept_workspace

MAX_M = 8          # verify rows per step (1 committed + 7 drafts); also the snapshot slots


@dataclass
class StepConfig:
    n_layers: int = 64
    hidden: int = 5120
    mlp: int = 17408
    vocab: int = 248320
    eps: float = 1e-6
    attn_every: int = 4        # layer li is full attention when li % attn_every == attn_every - 1
    # GDN geometry (tokenrush/config.py:17-21)
    gdn_k_heads: int = 16
    gdn_v_heads: int = 48
    gdn_k_dim: int = 128
    gdn_v_dim: int = 128
    # attention geometry (config.py:12-16)
    n_heads: int = 24
    n_kv_heads: int = 4
    head_dim: int = 256
    rotary_dim: int = 64
    rope_theta: float = 1e7
    live: int = 8192           # tokens already in the KV cache when the step runs
    headroom: int = 1024       # cache rows past `live` for the steps that follow
    layer_types: tuple = None  # a checkpoint's 'linear_attention' / 'full_attention' per layer
    tree_nodes: int = 0        # > 0: room for draft-tree steps of up to this many nodes (<= 32)

    def is_attention(self, li: int) -> bool:
        if self.layer_types is not None:
            return self.layer_types[li] == "full_attention"
        return li % self.attn_every == self.attn_every - 1

    @property
    def gdn(self) -> GDNConfig:
        return GDNConfig(self.hidden, self.gdn_k_heads, self.gdn_v_heads, self.gdn_k_dim, self.gdn_v_dim)

    @property
    def attn(self) -> AttnConfig:
        return AttnConfig(self.n_heads, self.n_kv_heads, self.head_dim, self.rotary_dim, self.rope_theta, self.eps)

    @property
    def gdn_in(self) -> int:       # in_qkvz output: conv channels + z
        return self.gdn.conv_dim + self.gdn.gdn_val_dim

    @property
    def attn_qkv(self) -> int:     # q | gate per head, k, v
        return self.n_heads * 2 * self.head_dim + 2 * self.n_kv_heads * self.head_dim

    @property
    def gdn_out(self) -> int:
        return self.gdn.gdn_val_dim

    @property
    def attn_out(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def maxlen(self) -> int:
        return self.live + self.headroom

    @property
    def n_slots(self) -> int:      # recurrent-state snapshots: one per verify row or tree node
        return max(MAX_M, self.tree_nodes)


SMALL = StepConfig(n_layers=4, hidden=512, mlp=1024, vocab=4096, gdn_k_heads=2, gdn_v_heads=4, n_heads=2,
                   n_kv_heads=1, live=300, headroom=64)


def _random_linear(N, K, gen, device, split_k=1, scale_dtype=torch.bfloat16, layout="rows"):
    """Codes uniform in 0..15, scale ~U(0.002, 0.02), min ~U(-0.15, -0.01) (benchmark configs)."""
    q = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=device, generator=gen)
    s = (torch.rand(N, K // 128, device=device, generator=gen) * 0.018 + 0.002).to(scale_dtype)
    m = (torch.rand(N, K // 128, device=device, generator=gen) * 0.14 - 0.15).to(scale_dtype)
    lin = QLinear(q, s, m, split_k=split_k, layout=layout)
    del q, s, m
    return lin


def _bf16(shape, std, gen, device, mean=0.0):
    return (torch.randn(*shape, device=device, generator=gen) * std + mean).to(torch.bfloat16)


class Layer:
    """One layer's weights: proj (in_qkvz or qkv), out (out_proj / o_proj), the mixer's small
    tensors, gate_up (pair layout, silu fused), down, ln1 / ln2. `split` holds the output sizes of
    the matrices joined in proj (conv channels | z, or q | k | v)."""

    def __init__(self, cfg: StepConfig, li: int, gen, device):
        H = cfg.hidden
        self.attention = cfg.is_attention(li)
        self.split = ((cfg.n_heads * 2 * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim) if self.attention
                      else (cfg.gdn.conv_dim,))
        if self.attention:
            self.proj = _random_linear(cfg.attn_qkv, H, gen, device)
            self.out = _random_linear(H, cfg.attn_out, gen, device, split_k=4)       # weights.py:163-174
            self.q_norm_w = _bf16((cfg.head_dim,), 0.5, gen, device)
            self.k_norm_w = _bf16((cfg.head_dim,), 0.5, gen, device)
        else:
            g = cfg.gdn
            self.proj = _random_linear(cfg.gdn_in, H, gen, device)
            self.out = _random_linear(H, cfg.gdn_out, gen, device, split_k=4)
            self.in_ba = _bf16((2 * g.gdn_v_heads, H), 0.02, gen, device)
            self.conv_w = _bf16((g.conv_dim, 4), 0.3, gen, device)
            self.A_log = torch.randn(g.gdn_v_heads, device=device, generator=gen)
            self.A = -torch.exp(self.A_log)
            self.dt_bias = torch.randn(g.gdn_v_heads, device=device, generator=gen)
            self.norm_w = _bf16((g.gdn_v_dim,), 0.5, gen, device, mean=1.0)
        self.gate_up = _random_linear(2 * cfg.mlp, H, gen, device, layout="gate_up")   # silu fused in its epilogue
        self.down = _random_linear(H, cfg.mlp, gen, device, split_k=4)
        self.ln1 = _bf16((H,), 0.1, gen, device)
        self.ln2 = _bf16((H,), 0.1, gen, device)

    @classmethod
    def from_tensors(cls, cfg: StepConfig, li: int, tensors: dict, device):
        """A layer from a packed checkpoint's tensors (weights.py:185-203)."""
        from .checkpoint import SPLIT_K, linear
        L = cls.__new__(cls)
        dev = lambda n, dt=None: tensors[n].to(device=device, dtype=dt or tensors[n].dtype).contiguous()
        p = f"layers.{li}."
        L.attention = cfg.is_attention(li)
        if L.attention:
            m = p + "self_attn."
            L.split = (cfg.n_heads * 2 * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim)
            L.proj = linear(tensors, [m + "q_proj.weight", m + "k_proj.weight", m + "v_proj.weight"], device)
            L.out = linear(tensors, m + "o_proj.weight", device, split_k=SPLIT_K)
            L.q_norm_w, L.k_norm_w = dev(m + "q_norm.weight"), dev(m + "k_norm.weight")
        else:
            m = p + "linear_attn."
            L.split = (cfg.gdn.conv_dim,)
            L.proj = linear(tensors, [m + "in_proj_qkv.weight", m + "in_proj_z.weight"], device)
            L.out = linear(tensors, m + "out_proj.weight", device, split_k=SPLIT_K)
            L.in_ba = torch.cat([dev(m + "in_proj_b.weight"), dev(m + "in_proj_a.weight")])
            L.conv_w = dev(m + "conv1d.weight").reshape(cfg.gdn.conv_dim, -1).contiguous()
            L.A_log = dev(m + "A_log", torch.float32)
            L.A = -torch.exp(L.A_log)
            L.dt_bias = dev(m + "dt_bias", torch.float32)
            L.norm_w = dev(m + "norm.weight")
        L.gate_up = linear(tensors, [p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"], device, layout="gate_up")
        L.down = linear(tensors, p + "mlp.down_proj.weight", device, split_k=SPLIT_K)
        L.ln1, L.ln2 = dev(p + "input_layernorm.weight"), dev(p + "post_attention_layernorm.weight")
        return L

    def weight_bytes(self) -> int:
        n = self.proj.nbytes + self.out.nbytes + self.gate_up.nbytes + self.down.nbytes
        if not self.attention:
            n += (self.in_ba.numel() + self.conv_w.numel() + self.norm_w.numel()) * 2 + self.A.numel() * 8
        return n


class StepState:
    """Decode state of the step (tokenrush/state.py:14-43) for the GDN and attention layers:
    position and committed slot, conv rings, recurrent state in cfg.n_slots snapshot slots, FP8
    KV cache with per-(head, position) scales; rows 0..live-1 of the cache hold random tokens.
    With cfg.tree_nodes, node_in [n_gdn, tree_nodes, conv_dim] keeps a tree step's conv inputs
    for the ring commit."""

    def __init__(self, cfg: StepConfig, n_gdn: int, n_attn: int, gen, device):
        g = cfg.gdn
        self.pos = torch.full((1,), cfg.live, dtype=torch.int64, device=device)
        self.slot = torch.zeros(1, dtype=torch.int64, device=device)
        self.ring = _bf16((n_gdn, g.conv_dim, RING), 1.0, gen, device)
        self.rec = torch.randn(cfg.n_slots, n_gdn, g.gdn_v_heads, g.gdn_k_dim, g.gdn_v_dim, device=device,
                               generator=gen) * 0.05
        self.node_in = (torch.zeros(n_gdn, cfg.tree_nodes, g.conv_dim, dtype=torch.bfloat16, device=device)
                        if cfg.tree_nodes else None)
        HKV, D, L = cfg.n_kv_heads, cfg.head_dim, cfg.maxlen
        self.k = torch.zeros(n_attn, HKV, L, D, dtype=torch.float8_e4m3fn, device=device)
        self.v = torch.zeros_like(self.k)
        self.k_scale = torch.full((n_attn, HKV, L), 0.01, device=device)
        self.v_scale = torch.full((n_attn, HKV, L), 0.01, device=device)
        for a in range(n_attn):
            self.k[a, :, :cfg.live] = (torch.randn(HKV, cfg.live, D, device=device, generator=gen) * 64).to(
                torch.float8_e4m3fn)
            self.v[a, :, :cfg.live] = (torch.randn(HKV, cfg.live, D, device=device, generator=gen) * 64).to(
                torch.float8_e4m3fn)
        self.cos, self.sin = rope_table(L, cfg.rotary_dim, cfg.rope_theta, device)

    def tensors(self):
        return [self.pos, self.slot, self.ring, self.rec, self.k, self.v, self.k_scale, self.v_scale]

    def snapshot(self):
        return [t.clone() for t in self.tensors()]

    def restore(self, snap):
        for t, s in zip(self.tensors(), snap):
            t.copy_(s)

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors()[2:])


class VerifyModel:
    """Random-init weights and decode state of the config-5 hybrid (int4 g128 projections,
    bf16 scale/min) and the verify step. Weights are packed once at construction."""

    def __init__(self, cfg: StepConfig = StepConfig(), device="cuda:0", seed: int = 0, tensors: dict = None):
        self.cfg = cfg
        self.device = torch.device(device)
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        if tensors is None:
            self.layers = [Layer(cfg, li, gen, self.device) for li in range(cfg.n_layers)]
            self.final_norm = _bf16((cfg.hidden,), 0.1, gen, self.device)
            self.lm_head = _random_linear(cfg.vocab, cfg.hidden, gen, self.device)
            # the step takes its input rows x0 directly; the table is kept so that a saved
            # checkpoint holds every tensor the reference's loader reads
            self.embed = _bf16((cfg.vocab, cfg.hidden), 0.02, gen, self.device)
        else:
            from .checkpoint import linear
            self.layers = [Layer.from_tensors(cfg, li, tensors, self.device) for li in range(cfg.n_layers)]
            self.final_norm = tensors["norm.weight"].to(self.device)
            self.lm_head = linear(tensors, "lm_head.weight", self.device)
            self.embed = tensors["embed_tokens.weight"].to(self.device)
        self.gdn_index, self.attn_index = {}, {}
        for li, L in enumerate(self.layers):
            d = self.attn_index if L.attention else self.gdn_index
            d[li] = len(d)
        self.state = StepState(cfg, len(self.gdn_index), len(self.attn_index), gen, self.device)
        # the verify step's consumer buffers (model.py:300-301): rows 0..M-1 hold the last step's
        # logits and post-final-norm hidden; spec_x holds its embedded input rows
        R = cfg.n_slots
        self.spec_x = torch.zeros(R, cfg.hidden, dtype=torch.bfloat16, device=self.device)
        self.spec_hidden = torch.zeros(R, cfg.hidden, dtype=torch.bfloat16, device=self.device)
        self.spec_logits = torch.zeros(R, cfg.vocab, dtype=torch.bfloat16, device=self.device)
        self.embed_status = torch.zeros(1, dtype=torch.int32, device=self.device)

    def nbytes(self) -> int:
        return self.lm_head.nbytes + sum(L.weight_bytes() for L in self.layers)

    def mixer(self, li: int, L: Layer, n: torch.Tensor, pos_t, slot_t, parent=None) -> torch.Tensor:
        """The layer's token mixer: [M, hidden] normed input -> [M, mixer out] (model.py:76-121);
        with parent, the rows are the nodes of a draft tree."""
        cfg, st = self.cfg, self.state
        u = L.proj(n)
        if L.attention:
            a = self.attn_index[li]
            q = attn_prep(u, L.q_norm_w, L.k_norm_w, st.cos, st.sin, pos_t, st.k[a], st.v[a], cfg.attn,
                          st.k_scale[a], st.v_scale[a], parent=parent)
            return attn_decode_fused(q, u, st.k[a], st.v[a], pos_t, cfg.attn, st.k_scale[a], st.v_scale[a],
                                     parent=parent)
        g = self.gdn_index[li]
        node_in = None if parent is None else st.node_in[g]
        return gdn_step_fused(u, n, L.in_ba, st.ring[g], L.conv_w, L.A, L.dt_bias, st.rec[:, g], slot_t, L.norm_w,
                              pos_t, cfg.gdn, cfg.eps, parent=parent, node_in=node_in)

    def hidden(self, x0: torch.Tensor, pos_t=None, slot_t=None, parent=None, out=None) -> torch.Tensor:
        """x0 [M, hidden] bf16 -> post-final-norm hidden [M, hidden] bf16 (model.py:252-254),
        written into out when given."""
        cfg = self.cfg
        pos_t = self.state.pos if pos_t is None else pos_t
        slot_t = self.state.slot if slot_t is None else slot_t
        if parent is not None and (not cfg.tree_nodes or x0.shape[0] > cfg.tree_nodes):
            raise RuntimeError(f"a {x0.shape[0]}-node tree step needs StepConfig(tree_nodes >= {x0.shape[0]})")
        x, h = x0, None
        for li, L in enumerate(self.layers):
            x, n = add_rmsnorm(x, h, L.ln1, cfg.eps)
            h = L.out.partials(self.mixer(li, L, n, pos_t, slot_t, parent))
            x, n = add_rmsnorm(x, h, L.ln2, cfg.eps)
            h = L.down.partials(L.gate_up.silu_mul(n))
        _, n = add_rmsnorm(x, h, self.final_norm, cfg.eps, out=out)
        return n

    @classmethod
    def from_checkpoint(cls, path: str, device="cuda:0", seed: int = 0, **cfg_overrides):
        """Weights from a packed checkpoint directory (weights.py:238-254 load_packed); the decode
        state (rings, recurrent slots, KV cache) is random-initialised from `seed`."""
        from .checkpoint import is_packed, read_config, read_tensors
        if not is_packed(path):
            raise RuntimeError(f"{path} is not a packed checkpoint (no tokenrush.json)")
        return cls(read_config(path, **cfg_overrides), device=device, seed=seed, tensors=read_tensors(path))

    def save_checkpoint(self, dst: str, meta: dict = None):
        """Write the weights in the packed checkpoint format (weights.py:60-102): every tensor the
        reference's build_weights reads (weights.py:185-211), checked before anything is written."""
        from .checkpoint import model_items, required_names, write_packed
        items = model_items(self)
        missing = required_names(self.cfg) - {n for n, _ in items}
        if missing:
            raise RuntimeError(f"checkpoint would miss {sorted(missing)[:4]}")
        return write_packed(dst, items, self.cfg, meta=meta)

    def body(self, x0: torch.Tensor) -> torch.Tensor:
        """x0 [M, hidden] bf16 -> logits [M, vocab] bf16, at the state's position and slot."""
        return self.lm_head(self.hidden(x0))

    def step(self, x0: torch.Tensor, spec_toks: torch.Tensor, st: AcceptState, params: SamplingParams = None,
             u: torch.Tensor = None, q: torch.Tensor = None) -> torch.Tensor:
        """Body at st.pos / st.slot, the lm_head and the accept/commit, which advances st.pos by
        n + 1 and sets st.slot = n (model.py:293-312). Returns the logits [M, vocab]: a view of
        spec_logits[:M], which keeps them as the reference does (model.py:300), beside
        spec_hidden[:M] (model.py:301); the next step overwrites both. The accept rule:
          greedy    (params None, q None): in the lm_head GEMM's epilogue, one launch;
          sampled   (params given): pred = sample(logits, params, u) with the device-side
                    SamplingParams and uniforms u [M] (drawn on the device when None, as
                    sample.py:47-48 does), then the leading-match commit (model.py:306-312);
          residual  (q given, fp32 [M - 1, vocab] draft probabilities, u [M]): rejection
                    sampling with the residual resample."""
        M = x0.shape[0]
        if M > self.spec_hidden.shape[0]:
            raise RuntimeError(f"step: {M} rows, room for {self.spec_hidden.shape[0]}")
        n = self.hidden(x0, st.pos, st.slot, out=self.spec_hidden[:M])
        if params is None and q is None:
            return lm_head_greedy(self.lm_head, n, spec_toks, st, keep_logits=True, out=self.spec_logits[:M])
        logits = self.lm_head(n, out=self.spec_logits[:M])
        if q is not None:
            if u is None:
                u = torch.rand(logits.shape[0], device=logits.device)
            accept_residual(logits, q, spec_toks, u, st)
        else:
            accept_sampled(logits, spec_toks, params, st, u)
        return logits


    def verify(self, spec_toks: torch.Tensor, st: AcceptState, params: SamplingParams = None,
               u: torch.Tensor = None, q: torch.Tensor = None) -> torch.Tensor:
        """The reference's _verify_step (model.py:293-312) from token ids: spec_toks int64 [M] on
        the device (the committed token, then M - 1 drafts) are embedded on the device
        (model.py:215) into spec_x, then step() runs; spec_logits[:M] and spec_hidden[:M] keep the
        logits and the post-final-norm rows. Capturable as one hipGraph. An id outside the
        vocabulary embeds as a zero row and sets embed_status to 1."""
        M = spec_toks.shape[0]
        if M > self.spec_x.shape[0]:
            raise RuntimeError(f"verify: {M} rows, room for {self.spec_x.shape[0]}")
        x0 = embed_rows(self.embed, spec_toks, out=self.spec_x[:M], status=self.embed_status)
        return self.step(x0, spec_toks, st, params=params, u=u, q=q)

    def step_tree(self, x0: torch.Tensor, node_toks: torch.Tensor, parent: torch.Tensor,
                  st: AcceptState) -> torch.Tensor:
        """Draft-tree verify (benchmark config 4): x0 [M, hidden] the nodes' input rows, node_toks
        [M] int64 (node 0 the committed token), parent [M] int32 device (parent[t] < t). The body
        runs the tree mixers at st.pos / st.slot; the lm_head's logits [M, vocab] feed the tree
        accept (the deepest root path whose every node equals its parent row's argmax), which
        advances st.pos by n + 1 and sets st.slot to that path's last node; then the commit moves
        the path's KV rows and scales to positions pos..pos+n and writes its conv inputs into the
        rings. Returns the logits."""
        S = self.state
        logits = self.lm_head(self.hidden(x0, st.pos, st.slot, parent))
        accept_tree(logits, node_toks, parent, st)
        for cache, layout in ((S.k, "rows"), (S.v, "rows"), (S.k_scale, "scalars"), (S.v_scale, "scalars")):
            commit_rows(cache, st, layout, max_n=x0.shape[0] - 1)
        tree_commit(S.ring, S.node_in, st)
        return logits


def prepare(model: VerifyModel, M: int):
    """Allocate every workspace a step at M rows uses (before graph capture)."""
    cfg = model.cfg
    for L in model.layers:
        for lin in (L.proj, L.gate_up):
            gfx950.workspaces(lin.shape[0], model.device, lin.shape[1], M)
    gfx950.workspaces(cfg.vocab, model.device, cfg.hidden, M)
    gdn_workspace(M, cfg.gdn_k_heads, cfg.gdn_v_heads, model.device)
    accept_workspace(M, cfg.vocab, model.device)
    attn_workspace(M, cfg.n_heads, ATTN_NSPLIT, model.device)
