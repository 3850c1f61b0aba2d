"""Test helper: write a quanta artifact directory in the reference's layout.

The layout follows the reference's ArtifactWriter (src/quanta/bake/artifact.py:44-85): tensors in
safetensors shards (written here by the `safetensors` library itself), `model.safetensors.index.json`
{"weight_map"}, `manifest.json` {"format": "quanta", "tensors"}, `config.json`. An affine_packed
weight `key` is stored as key.weight_packed / .weight_scale / .weight_bias
(ArtifactWriter.add_quantized); a dense one verbatim under its key (ArtifactWriter.add_dense).
MoE key names follow src/quanta/qwen35/bake.py:143-155 under LM_PREFIX (loader.py:49).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch
from safetensors.torch import save_file

LM_PREFIX = "model.language_model."


def bf16_from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def u32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).view(torch.uint32)


class ArtifactBuilder:
    def __init__(self) -> None:
        self.tensors: dict[str, torch.Tensor] = {}
        self.manifest: dict[str, dict] = {}

    def add_dense(self, name: str, t: torch.Tensor) -> None:
        self.tensors[name] = t.contiguous()
        self.manifest[name] = {"format": "dense", "dtype": str(t.dtype).split(".")[-1]}

    def add_quantized(self, key: str, packed: torch.Tensor, scale: torch.Tensor,
                      bias: torch.Tensor, bits: int, group_size: int) -> None:
        self.tensors[key + ".weight_packed"] = packed.contiguous()
        self.tensors[key + ".weight_scale"] = scale.contiguous()
        self.tensors[key + ".weight_bias"] = bias.contiguous()
        self.manifest[key] = {"format": "affine_packed", "bits": bits, "group_size": group_size}

    def write(self, d: Path, config: dict, n_shards: int = 2, fmt: str = "quanta") -> Path:
        d.mkdir(parents=True, exist_ok=True)
        names = sorted(self.tensors)
        weight_map = {}
        for s in range(n_shards):
            part = names[s::n_shards]
            if not part:
                continue
            fn = f"model-{s:05d}-of-{n_shards:05d}.safetensors"
            save_file({n: self.tensors[n] for n in part}, str(d / fn))
            weight_map.update({n: fn for n in part})
        (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
        (d / "manifest.json").write_text(json.dumps({"format": fmt, "tensors": self.manifest}))
        (d / "config.json").write_text(json.dumps(config))
        return d


def moe_config_json(H, E, k, I, Is, norm=True) -> dict:
    """A source-style config.json with the decoder fields nested under text_config."""
    return {"model_type": "qwen3_5_moe",
            "text_config": {"hidden_size": H, "num_experts": E, "num_experts_per_tok": k,
                            "moe_intermediate_size": I, "shared_expert_intermediate_size": Is,
                            "norm_topk_prob": norm}}
