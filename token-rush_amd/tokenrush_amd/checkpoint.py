"""The reference's packed int4 checkpoint on disk, read into (and written from) the verify step's
weights.

Format (tokenrush/weights.py:60-102 write_packed, :238-254 load_packed, config.py:30-52):
  <dir>/config.json              the HF text config (hidden_size, num_hidden_layers, layer_types,
                                 linear_* GDN geometry, head_dim, rope_parameters, ...)
  <dir>/tokenrush.json           {"format": "int4", "group": 128, "quantized": [names], ...}
  <dir>/model-NNNNN.safetensors  every tensor by name; a quantized matrix `name` is stored as the
                                 triple name.qweight (uint8 [N, K/2], element 2j in the low
                                 nibble), name.scale and name.mn (bf16 [N, K/128])
Names follow weights.py:185-211: layers.{i}.linear_attn.{in_proj_qkv, in_proj_z, in_proj_b,
in_proj_a, conv1d, A_log, dt_bias, norm, out_proj}, layers.{i}.self_attn.{q_proj, k_proj, v_proj,
o_proj, q_norm, k_norm}, layers.{i}.mlp.{gate_proj, up_proj, down_proj},
layers.{i}.{input_layernorm, post_attention_layernorm}, norm.weight, lm_head.weight,
embed_tokens.weight.

Files are read with safetensors (no pickle); matrices that are concatenated along the output
dimension (q|k|v, in_proj_qkv|in_proj_z, gate|up) are joined in the engine packing before the
gfx950 packing, as weights.py:166-174 does.
"""
import glob
import json
import os

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from .quant import GROUP, QLinear

PACK_META = "tokenrush.json"
SPLIT_K = 4   # out_proj / o_proj / down_proj: their consumer sums split-K partials (weights.py:163)


def is_packed(path: str) -> bool:
    return os.path.exists(os.path.join(path, PACK_META))


# ------------------------------------------------------------------ config.json <-> StepConfig

def read_config(path: str, **overrides):
    """config.json (HF text config, optionally under "text_config") -> StepConfig, with the
    fields config.py:32-52 reads; overrides set the step's own fields (live, headroom)."""
    from .step import StepConfig
    c = json.load(open(os.path.join(path, "config.json")))
    t = c.get("text_config", c)
    rp = t.get("rope_parameters", {})
    prf = rp.get("partial_rotary_factor", t.get("partial_rotary_factor", 1.0))
    if t.get("linear_conv_kernel_dim", 4) != 4:
        raise RuntimeError("the GDN kernels take a conv kernel of 4")
    cfg = StepConfig(n_layers=t["num_hidden_layers"], hidden=t["hidden_size"], mlp=t["intermediate_size"],
                     vocab=t["vocab_size"], eps=t["rms_norm_eps"], gdn_k_heads=t["linear_num_key_heads"],
                     gdn_v_heads=t["linear_num_value_heads"], gdn_k_dim=t["linear_key_head_dim"],
                     gdn_v_dim=t["linear_value_head_dim"], n_heads=t["num_attention_heads"],
                     n_kv_heads=t["num_key_value_heads"], head_dim=t["head_dim"],
                     rotary_dim=int(t["head_dim"] * prf), rope_theta=rp.get("rope_theta", t.get("rope_theta")),
                     layer_types=tuple(t["layer_types"]), **overrides)
    return cfg


def config_json(cfg) -> dict:
    """StepConfig -> the config.json fields read_config (and config.py) reads."""
    return {"hidden_size": cfg.hidden, "num_hidden_layers": cfg.n_layers,
            "layer_types": [("full_attention" if cfg.is_attention(li) else "linear_attention")
                            for li in range(cfg.n_layers)],
            "vocab_size": cfg.vocab, "intermediate_size": cfg.mlp, "num_attention_heads": cfg.n_heads,
            "num_key_value_heads": cfg.n_kv_heads, "head_dim": cfg.head_dim,
            "rope_parameters": {"rope_theta": cfg.rope_theta, "partial_rotary_factor": cfg.rotary_dim / cfg.head_dim},
            "linear_num_key_heads": cfg.gdn_k_heads, "linear_num_value_heads": cfg.gdn_v_heads,
            "linear_key_head_dim": cfg.gdn_k_dim, "linear_value_head_dim": cfg.gdn_v_dim,
            "linear_conv_kernel_dim": 4, "rms_norm_eps": cfg.eps, "max_position_embeddings": cfg.maxlen}


# ------------------------------------------------------------------ tensors

MTP_PREFIX = "mtp."   # the draft head's tensors: loaded only on request (weights.py:238-254)


def read_tensors(path: str, device="cpu", with_mtp: bool = False) -> dict:
    """Every tensor of the packed checkpoint's shards, by name (weights.py:238-254); the mtp.*
    draft-head tensors are skipped unless with_mtp, as load_packed skips them."""
    shards = sorted(glob.glob(os.path.join(path, "model-*.safetensors")))
    if not shards:
        raise RuntimeError(f"{path}: no model-*.safetensors shards")
    out = {}
    for shard in shards:
        with safe_open(shard, framework="pt", device=str(device)) as f:
            for name in f.keys():
                if with_mtp or not name.startswith(MTP_PREFIX):
                    out[name] = f.get_tensor(name)
    return out


def _stored(name: str, v):
    """The tensors one item is stored as, (key, CPU tensor): a plain tensor under its name, a
    quantized matrix (qweight, scale, mn) as name.qweight, name.scale and name.mn."""
    pairs = zip((name + ".qweight", name + ".scale", name + ".mn"), v) if isinstance(v, tuple) else [(name, v)]
    return [(k, t.detach().cpu().contiguous()) for k, t in pairs]


def _shard_plan(sizes, shard_bytes: int):
    """Indices of `sizes` grouped into consecutive shards: a shard is closed at the first whole
    matrix (all of its stored tensors) that brings it to shard_bytes or more."""
    groups, cur, acc = [], [], 0
    for i, n in enumerate(sizes):
        cur.append(i)
        acc += n
        if acc >= shard_bytes:
            groups.append(cur)
            cur, acc = [], 0
    return groups + ([cur] if cur else [])


def write_packed(dst: str, items, cfg=None, group: int = GROUP, meta: dict = None, shard_bytes: int = 4 << 30):
    """Write the packed checkpoint format: the tensors in model-NNNNN.safetensors shards of about
    shard_bytes each (a matrix's triple never straddles two shards), tokenrush.json with the
    format, group, quantized names, shard count and stored bytes (weights.py:60-102), and
    config.json from cfg when given."""
    os.makedirs(dst, exist_ok=True)
    units = [(_stored(name, v), isinstance(v, tuple), name) for name, v in items]
    sizes = [sum(t.numel() * t.element_size() for _, t in ents) for ents, _, _ in units]
    plan = _shard_plan(sizes, shard_bytes)
    for si, idx in enumerate(plan):
        save_file({k: t for i in idx for k, t in units[i][0]}, os.path.join(dst, f"model-{si:05d}.safetensors"))
    info = dict(format="int4", group=group, quantized=[name for _, q, name in units if q], shards=len(plan),
                packed_bytes=sum(sizes))
    info.update(meta or {})
    with open(os.path.join(dst, PACK_META), "w") as f:
        json.dump(info, f, indent=1)
    if cfg is not None:
        with open(os.path.join(dst, "config.json"), "w") as f:
            json.dump(config_json(cfg), f, indent=1)
    return info


def linear(tensors: dict, names, device, split_k: int = 1, layout: str = "rows") -> QLinear:
    """One QLinear from one or more quantized matrices joined along the output dimension
    (weights.py:166-174): the engine-packed triples are concatenated row-wise, then packed once."""
    names = [names] if isinstance(names, str) else list(names)
    for n in names:
        if n + ".qweight" not in tensors:
            raise RuntimeError(f"{n}: not a quantized matrix in this checkpoint")
    q, s, m = (torch.cat([tensors[n + suf] for n in names]).to(device) for suf in (".qweight", ".scale", ".mn"))
    return QLinear(q, s, m, split_k=split_k, layout=layout)


def layer_items(L, li: int):
    """(name, tensor or triple) of one step Layer, in the checkpoint's names (the inverse of
    step.Layer.from_tensors)."""
    p = f"layers.{li}."
    out = [(p + "input_layernorm.weight", L.ln1), (p + "post_attention_layernorm.weight", L.ln2)]
    if L.attention:
        m = p + "self_attn."
        q, s, mn = L.proj.nibbles()
        nq, nk = L.split[0], L.split[1]
        for name, a, b in ((m + "q_proj.weight", 0, nq), (m + "k_proj.weight", nq, nq + nk),
                           (m + "v_proj.weight", nq + nk, q.shape[0])):
            out.append((name, (q[a:b], s[a:b], mn[a:b])))
        out += [(m + "o_proj.weight", L.out.nibbles()), (m + "q_norm.weight", L.q_norm_w),
                (m + "k_norm.weight", L.k_norm_w)]
    else:
        m = p + "linear_attn."
        q, s, mn = L.proj.nibbles()
        c = L.split[0]
        out += [(m + "in_proj_qkv.weight", (q[:c], s[:c], mn[:c])), (m + "in_proj_z.weight", (q[c:], s[c:], mn[c:]))]
        hv = L.A.numel()
        out += [(m + "in_proj_b.weight", L.in_ba[:hv]), (m + "in_proj_a.weight", L.in_ba[hv:]),
                (m + "conv1d.weight", L.conv_w.unsqueeze(1)), (m + "A_log", L.A_log),
                (m + "dt_bias", L.dt_bias), (m + "norm.weight", L.norm_w), (m + "out_proj.weight", L.out.nibbles())]
    q, s, mn = L.gate_up.nibbles()
    F = q.shape[0] // 2
    out += [(p + "mlp.gate_proj.weight", (q[:F], s[:F], mn[:F])), (p + "mlp.up_proj.weight", (q[F:], s[F:], mn[F:])),
            (p + "mlp.down_proj.weight", L.down.nibbles())]
    return out


def model_items(model):
    """(name, tensor or triple) of a whole step.VerifyModel: its layers, the final norm, the
    lm_head and the embedding table."""
    items = [it for li, L in enumerate(model.layers) for it in layer_items(L, li)]
    return items + [("norm.weight", model.final_norm), ("lm_head.weight", model.lm_head.nibbles()),
                    ("embed_tokens.weight", model.embed)]


def required_names(cfg) -> set:
    """Every name the reference's loader reads for a model of this config (build_layer and
    build_weights, weights.py:180-211): per layer its mixer's tensors, the MLP and the two norms,
    then embed_tokens, norm and lm_head."""
    names = {"embed_tokens.weight", "norm.weight", "lm_head.weight"}
    for li in range(cfg.n_layers):
        p = f"layers.{li}."
        names |= {p + "input_layernorm.weight", p + "post_attention_layernorm.weight",
                  p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", p + "mlp.down_proj.weight"}
        if cfg.is_attention(li):
            names |= {p + "self_attn." + n for n in ("q_proj.weight", "k_proj.weight", "v_proj.weight",
                                                     "o_proj.weight", "q_norm.weight", "k_norm.weight")}
        else:
            names |= {p + "linear_attn." + n for n in ("in_proj_qkv.weight", "in_proj_z.weight", "in_proj_b.weight",
                                                       "in_proj_a.weight", "conv1d.weight", "A_log", "dt_bias",
                                                       "norm.weight", "out_proj.weight")}
    return names
