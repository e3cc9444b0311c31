"""The packed checkpoint format (tokenrush/weights.py:60-102, :238-254; config.py:30-52) on the CPU:
shards + tokenrush.json written and read back by name with safetensors, config.json <-> StepConfig.
The GPU round trip (a model saved, loaded and stepping bit-identically) is in test_step_gpu.py."""
import json

import pytest
import torch

from tokenrush_amd import checkpoint as ck
from tokenrush_amd.step import SMALL, StepConfig


def test_write_read_round_trip(tmp_path):
    g = torch.Generator().manual_seed(0)
    q = torch.randint(0, 256, (32, 64), dtype=torch.uint8, generator=g)
    s = torch.rand(32, 1, generator=g).to(torch.bfloat16)
    m = -torch.rand(32, 1, generator=g).to(torch.bfloat16)
    w = torch.randn(128, generator=g).to(torch.bfloat16)
    info = ck.write_packed(str(tmp_path), [("layers.0.mlp.down_proj.weight", (q, s, m)), ("norm.weight", w)],
                           shard_bytes=1)
    assert info["quantized"] == ["layers.0.mlp.down_proj.weight"] and info["group"] == 128 and info["shards"] == 2
    assert ck.is_packed(str(tmp_path))
    assert json.load(open(tmp_path / ck.PACK_META))["format"] == "int4"
    t = ck.read_tensors(str(tmp_path))
    assert set(t) == {"layers.0.mlp.down_proj.weight.qweight", "layers.0.mlp.down_proj.weight.scale",
                      "layers.0.mlp.down_proj.weight.mn", "norm.weight"}
    assert torch.equal(t["layers.0.mlp.down_proj.weight.qweight"], q)
    assert torch.equal(t["layers.0.mlp.down_proj.weight.scale"], s) and torch.equal(t["norm.weight"], w)


@pytest.mark.parametrize("cfg", [SMALL, StepConfig()])
def test_config_round_trip(tmp_path, cfg):
    json.dump(ck.config_json(cfg), open(tmp_path / "config.json", "w"))
    got = ck.read_config(str(tmp_path), live=cfg.live, headroom=cfg.headroom)
    for f in ("n_layers", "hidden", "mlp", "vocab", "eps", "gdn_k_heads", "gdn_v_heads", "gdn_k_dim", "gdn_v_dim",
              "n_heads", "n_kv_heads", "head_dim", "rotary_dim", "rope_theta", "live", "headroom"):
        assert getattr(got, f) == getattr(cfg, f), f
    assert [got.is_attention(i) for i in range(cfg.n_layers)] == [cfg.is_attention(i) for i in range(cfg.n_layers)]


def test_hf_text_config_nesting(tmp_path):
    """config.py reads the text config under "text_config" when present, partial rotary from
    rope_parameters."""
    c = ck.config_json(SMALL)
    json.dump({"text_config": c, "architectures": ["x"]}, open(tmp_path / "config.json", "w"))
    assert ck.read_config(str(tmp_path)).rotary_dim == SMALL.rotary_dim


def test_missing_shards_and_matrix(tmp_path):
    with pytest.raises(RuntimeError):
        ck.read_tensors(str(tmp_path))
    with pytest.raises(RuntimeError):
        ck.linear({}, "lm_head.weight", "cpu")


class _FakeLinear:
    """CPU stand-in for a QLinear: nibbles() returns an engine-packed triple of the given shape."""

    def __init__(self, N, K):
        self.t = (torch.zeros(N, K // 2, dtype=torch.uint8), torch.ones(N, K // 128, dtype=torch.bfloat16),
                  torch.zeros(N, K // 128, dtype=torch.bfloat16))

    def nibbles(self):
        return self.t


def _fake_model(cfg):
    """An object with the attributes checkpoint.model_items reads, on the CPU."""
    from types import SimpleNamespace as NS
    H, z = cfg.hidden, lambda *s: torch.zeros(*s, dtype=torch.bfloat16)
    layers = []
    for li in range(cfg.n_layers):
        L = NS(attention=cfg.is_attention(li), ln1=z(H), ln2=z(H), gate_up=_FakeLinear(2 * cfg.mlp, H),
               down=_FakeLinear(H, cfg.mlp))
        if L.attention:
            L.split = (cfg.n_heads * 2 * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim)
            L.proj, L.out = _FakeLinear(cfg.attn_qkv, H), _FakeLinear(H, cfg.attn_out)
            L.q_norm_w, L.k_norm_w = z(cfg.head_dim), z(cfg.head_dim)
        else:
            g = cfg.gdn
            L.split = (g.conv_dim,)
            L.proj, L.out = _FakeLinear(cfg.gdn_in, H), _FakeLinear(H, cfg.gdn_out)
            L.in_ba, L.conv_w, L.norm_w = z(2 * g.gdn_v_heads, H), z(g.conv_dim, 4), z(g.gdn_v_dim)
            L.A_log, L.A, L.dt_bias = (torch.zeros(g.gdn_v_heads) for _ in range(3))
        layers.append(L)
    return NS(layers=layers, final_norm=z(H), lm_head=_FakeLinear(cfg.vocab, H), embed=z(cfg.vocab, H), cfg=cfg)


def test_saved_names_cover_the_reference_loader(tmp_path):
    """A saved model holds every name the reference's build_weights reads (weights.py:180-211),
    embed_tokens.weight included, and nothing outside that set; the quantized matrices are
    exactly the projections and the lm_head."""
    m = _fake_model(SMALL)
    items = ck.model_items(m)
    names = [n for n, _ in items]
    assert set(names) == ck.required_names(SMALL) and len(names) == len(set(names))
    info = ck.write_packed(str(tmp_path), items, SMALL, shard_bytes=1 << 20)
    assert set(info["quantized"]) == {n for n in names if "_proj" in n and not n.endswith(("_a.weight", "_b.weight"))} | {"lm_head.weight"}
    t = ck.read_tensors(str(tmp_path))
    stored = {n[:-len(suf)] for n in t for suf in (".qweight",) if n.endswith(suf)} | {
        n for n in t if not n.endswith((".qweight", ".scale", ".mn"))}
    assert stored == ck.required_names(SMALL)
    assert t["layers.0.linear_attn.conv1d.weight"].shape == (SMALL.gdn.conv_dim, 1, 4)   # the HF conv1d shape


def test_shards_keep_triples_together_and_skip_mtp(tmp_path):
    """Every shard holds whole matrices (qweight, scale and mn of one name together); mtp.*
    tensors are read only on request, as load_packed does (weights.py:238-254)."""
    from safetensors import safe_open
    q = _FakeLinear(64, 256).nibbles()
    items = [(f"layers.{i}.mlp.down_proj.weight", tuple(t.clone() for t in q)) for i in range(5)] + [("mtp.fc.weight", torch.ones(4))]
    info = ck.write_packed(str(tmp_path), items, shard_bytes=10000)
    assert info["shards"] == 3 and info["packed_bytes"] == 5 * (64 * 128 + 2 * 64 * 2 * 2) + 16
    for f in sorted(tmp_path.glob("model-*.safetensors")):
        keys = set(safe_open(str(f), framework="pt").keys())
        for k in keys:
            base = k.rsplit(".", 1)[0]
            if k.endswith(".qweight"):
                assert {base + ".scale", base + ".mn"} <= keys
    assert "mtp.fc.weight" not in ck.read_tensors(str(tmp_path))
    assert "mtp.fc.weight" in ck.read_tensors(str(tmp_path), with_mtp=True)
