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
