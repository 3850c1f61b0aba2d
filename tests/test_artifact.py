"""CPU tier: the artifact reader against artifacts written in the reference's layout (the shards by
the `safetensors` library itself): verbatim tensors, index/manifest resolution, config fields, and
the reference reader's errors (src/quanta/qwen35/artifact.py:38-123,187-203)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from quanta_amd.artifact import LM_PREFIX, QuantaArtifact
from tests._artifact import ArtifactBuilder, moe_config_json, u32


def _block(rng, E=4, H=128, I=64, Is=64):
    p = LM_PREFIX + "layers.0.mlp."
    b = ArtifactBuilder()
    t = {}
    t["gate"] = torch.randn(E, H, generator=rng).to(torch.bfloat16)
    t["sgate"] = torch.randn(1, H, generator=rng).to(torch.bfloat16)
    b.add_dense(p + "gate.weight", t["gate"])
    b.add_dense(p + "shared_expert_gate.weight", t["sgate"])
    for proj, shp in (("gate_proj", (Is, H)), ("up_proj", (Is, H)), ("down_proj", (H, Is))):
        t[proj] = torch.randn(*shp, generator=rng).to(torch.bfloat16)
        b.add_dense(p + f"shared_expert.{proj}.weight", t[proj])
    for key, (rows, K) in (("experts.gate_up_proj", (2 * I, H)), ("experts.down_proj", (H, I))):
        words = torch.randint(0, 2**31, (E, rows, K // 8), generator=rng, dtype=torch.int64)
        t[key] = (u32(words.numpy().astype(np.uint32)),
                  torch.rand(E, rows, K // 64, generator=rng).to(torch.bfloat16),
                  torch.randn(E, rows, K // 64, generator=rng).to(torch.bfloat16))
        b.add_quantized(p + key, *t[key], bits=4, group_size=64)
    return b, t


def test_reader_returns_tensors_verbatim(tmp_path):
    rng = torch.Generator().manual_seed(0)
    b, t = _block(rng)
    art = QuantaArtifact(b.write(tmp_path / "a", moe_config_json(128, 4, 2, 64, 64), n_shards=3))
    p = LM_PREFIX + "layers.0.mlp."
    assert len(set(art.weight_map.values())) == 3
    assert torch.equal(art.get(p + "gate.weight"), t["gate"])
    assert torch.equal(art.read(p + "shared_expert.down_proj.weight", "cpu"), t["down_proj"])
    for key in ("experts.gate_up_proj", "experts.down_proj"):
        tr = art.packed_triplet(p + key, "cpu")
        assert tr["bits"] == 4 and tr["group_size"] == 64
        assert tr["packed"].dtype == torch.int32
        assert torch.equal(tr["packed"], t[key][0].view(torch.int32))
        assert torch.equal(tr["scale"], t[key][1]) and torch.equal(tr["bias"], t[key][2])


def test_reader_maps_without_copying(tmp_path):
    rng = torch.Generator().manual_seed(1)
    b, _ = _block(rng)
    art = QuantaArtifact(b.write(tmp_path / "a", moe_config_json(128, 4, 2, 64, 64), n_shards=1))
    name = LM_PREFIX + "layers.0.mlp.experts.gate_up_proj.weight_packed"
    x = art.get(name)
    shard = art._shards[art.weight_map[name]]
    lo = shard.mm.ctypes.data
    assert lo <= x.data_ptr() < lo + shard.mm.size   # a view of the mapping, no host copy


def test_moe_packed_and_config(tmp_path):
    rng = torch.Generator().manual_seed(2)
    b, t = _block(rng)
    art = QuantaArtifact(b.write(tmp_path / "a", moe_config_json(128, 4, 2, 64, 64, norm=False)))
    p = art.moe_packed(0, "cpu")
    assert set(p) == {"gate", "experts_gate_up", "experts_down", "shared_gate_proj",
                      "shared_up_proj", "shared_down_proj", "shared_expert_gate"}
    assert torch.equal(p["shared_expert_gate"], t["sgate"])
    cfg = art.moe_config()
    assert (cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate_size,
            cfg.shared_expert_intermediate_size, cfg.norm_topk_prob) == (128, 4, 2, 64, 64, False)
    assert (cfg.scoring_func, cfg.n_group, cfg.topk_group, cfg.routed_scaling_factor) == \
        ("softmax", 1, 1, 1.0)


def test_moe_config_router_fields(tmp_path):
    """scoring_func (src/quanta/qwen35/config.py:361) and the DeepSeek/GLM router fields are read
    from config.json; a scoring function the block does not run is refused."""
    rng = torch.Generator().manual_seed(4)
    b, _ = _block(rng)
    cj = moe_config_json(128, 4, 2, 64, 64)
    cj["text_config"].update(scoring_func="sigmoid", n_group=2, topk_group=1,
                             routed_scaling_factor=2.5)
    cfg = QuantaArtifact(b.write(tmp_path / "a", cj)).moe_config()
    assert (cfg.scoring_func, cfg.n_group, cfg.topk_group, cfg.routed_scaling_factor) == \
        ("sigmoid", 2, 1, 2.5)
    cj["text_config"]["scoring_func"] = "argmax"
    with pytest.raises(ValueError, match="scoring_func"):
        QuantaArtifact(b.write(tmp_path / "b", cj)).moe_config()


def test_manifest_resolution_rule(tmp_path):
    """The four cases of the manifest rule: a dense record at the key wins over an affine_packed
    stem, an affine_packed stem resolves the .weight key, another format at either place is a
    ValueError, and no record is a KeyError."""
    rng = torch.Generator().manual_seed(5)
    b, _ = _block(rng)
    p = LM_PREFIX + "layers.0.mlp."
    # both a dense record at "twin.weight" and an affine_packed one at "twin": dense wins
    b.add_dense(p + "twin.weight", torch.ones(2, 64).to(torch.bfloat16))
    b.add_quantized(p + "twin", u32(np.zeros((2, 8), np.uint32)), torch.ones(2, 1).to(torch.bfloat16),
                    torch.zeros(2, 1).to(torch.bfloat16), bits=4, group_size=64)
    b.manifest[p + "weird.weight"] = {"format": "fp3"}
    b.tensors[p + "weird.weight"] = torch.zeros(2)
    art = QuantaArtifact(b.write(tmp_path / "a", moe_config_json(128, 4, 2, 64, 64)))
    assert art._meta(p + "twin.weight") == (p + "twin.weight", {"format": "dense", "dtype": "bfloat16"})
    base, meta = art._meta(p + "experts.down_proj.weight")
    assert base == p + "experts.down_proj" and meta["format"] == "affine_packed"
    assert art._meta(p + "experts.down_proj")[0] == p + "experts.down_proj"
    with pytest.raises(ValueError, match="fp3"):
        art._meta(p + "weird.weight")
    with pytest.raises(KeyError):
        art._meta(p + "absent.weight")
    assert art.has(p + "twin") and art.has(p + "weird.weight") and not art.has(p + "absent.weight")
    art.release()
    assert not art._shards


def test_reader_errors_follow_the_reference(tmp_path):
    rng = torch.Generator().manual_seed(3)
    b, _ = _block(rng)
    p = LM_PREFIX + "layers.0.mlp."
    b.manifest[p + "odd"] = {"format": "int5_magic"}
    b.tensors[p + "odd.weight_packed"] = torch.zeros(4, dtype=torch.int32)
    d = b.write(tmp_path / "a", moe_config_json(128, 4, 2, 64, 64))
    art = QuantaArtifact(d)
    assert art.has(p + "experts.down_proj.weight") and not art.has(p + "nope.weight")
    with pytest.raises(KeyError):
        art.read(p + "nope.weight", "cpu")
    with pytest.raises(KeyError):
        art.get(p + "nope")
    with pytest.raises(ValueError, match="unknown manifest format"):
        art.read(p + "odd.weight", "cpu")
    with pytest.raises(ValueError, match="not an affine_packed weight"):
        art.packed_triplet(p + "gate.weight", "cpu")
    man = json.loads((d / "manifest.json").read_text())
    man["format"] = "mlx"
    (d / "manifest.json").write_text(json.dumps(man))
    with pytest.raises(ValueError, match="not a quanta artifact"):
        QuantaArtifact(d)
