"""Reader of the MoE blocks of a quanta artifact (the reference's baked model format) into the
tensors quanta_amd takes, so real bakes feed the kernels.

Format (written by the reference's ArtifactWriter, src/quanta/bake/artifact.py:44-85; read by
Qwen35Artifact, src/quanta/qwen35/artifact.py:35-229):
  * `model.safetensors.index.json`: {"weight_map": {tensor name: shard file name}};
  * `manifest.json`: {"format": "quanta", "tensors": {key: entry}} with entry
    {"format": "affine_packed", "bits", "group_size"} for a quantized weight stored at
    `key.weight_packed` (uint32 codes, LSB-first, [.., out, in*bits/32]) plus `key.weight_scale`
    and `key.weight_bias` ([.., out, in/group_size]), or {"format": "dense", "dtype"} for a tensor
    stored verbatim under `key`;
  * `config.json`: the source model config, decoder fields under `text_config`
    (src/quanta/qwen35/config.py:258-364);
  * the shards: safetensors files.
MoE keys of layer i (src/quanta/qwen35/loader.py:49,74; src/quanta/qwen35/bake.py:143-155):
`model.language_model.layers.{i}.mlp.` + `gate.weight` (dense), `shared_expert_gate.weight`
(dense), `shared_expert.{gate,up,down}_proj` (int8 g64 affine, or dense),
`experts.gate_up_proj` / `experts.down_proj` (int4 g64 affine, pre-stacked [E, out, in]).

Shards are memory-mapped: a tensor is a view of the mapping (no host copy) until it is copied to
the device. Resolution and errors follow Qwen35Artifact: an unknown manifest format raises
ValueError, a missing key KeyError, a non-quanta directory ValueError. Quantized weights that the
block reads as bf16 (the shared expert) are dequantized on the GPU by `qmoe_dequant` (int4 or int8,
group 64); the routed expert stacks stay packed.
"""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import torch

from quanta_amd import ops
from quanta_amd.moe import MoEConfig, Qwen35MoEModule

LM_PREFIX = "model.language_model."                       # src/quanta/qwen35/loader.py:49
SHARED_EXPERT_PROJS = ("gate_proj", "up_proj", "down_proj")   # src/quanta/qwen35/loader.py:74
_WEIGHT_SUFFIX = ".weight"

# safetensors dtype -> (numpy storage dtype, torch view dtype or None)
_ST_DTYPES = {
    "BF16": (np.uint16, torch.bfloat16),
    "F16": (np.float16, None),
    "F32": (np.float32, None),
    "F64": (np.float64, None),
    "U8": (np.uint8, None),
    "I8": (np.int8, None),
    "I16": (np.int16, None),
    "U16": (np.uint16, torch.uint16),
    "I32": (np.int32, None),
    "U32": (np.uint32, torch.uint32),
    "I64": (np.int64, None),
    "BOOL": (np.bool_, None),
}


class _Shard:
    """One safetensors file, mapped: 8-byte little-endian header length, JSON header
    {name: {dtype, shape, data_offsets}}, then the data section."""

    def __init__(self, path: Path) -> None:
        with open(path, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            header = json.loads(f.read(n))
        self.path = path
        self.meta = {k: v for k, v in header.items() if k != "__metadata__"}
        self.base = 8 + n
        # copy-on-write mapping: torch needs a writable array, nothing is written back
        self.mm = np.memmap(path, dtype=np.uint8, mode="c")

    def tensor(self, name: str) -> torch.Tensor:
        m = self.meta[name]
        if m["dtype"] not in _ST_DTYPES:
            raise ValueError(f"{self.path.name}: {name}: unsupported safetensors dtype {m['dtype']}")
        npdt, tdt = _ST_DTYPES[m["dtype"]]
        b, e = m["data_offsets"]
        raw = self.mm[self.base + b:self.base + e]
        if (self.base + b) % np.dtype(npdt).itemsize:
            raw = np.array(raw)   # unaligned in the file: one host copy
        arr = raw.view(npdt).reshape(m["shape"])
        t = torch.from_numpy(arr)
        return t.view(tdt) if tdt is not None else t


class _Manifest:
    """What an artifact directory declares, indexed once when it is opened.

    The writer (src/quanta/bake/artifact.py:51-77) stores a dense tensor verbatim under its own
    key and records {"format": "dense"} at that key; it stores a quantized weight as three tensors
    `<stem>.weight_packed/_scale/_bias` and records {"format": "affine_packed", bits,
    group_size} at the stem, the weight's key without its ".weight" suffix. A reader therefore
    resolves a weight key by this rule (the one Qwen35Artifact applies,
    src/quanta/qwen35/artifact.py:77-94):
      1. a dense record at the key itself wins;
      2. else an affine_packed record at the stem;
      3. a record at either place in any other format is an error (ValueError): decoding it at a
         guessed width would be silently wrong;
      4. no record at all is a missing weight (KeyError).
    """

    def __init__(self, root: Path) -> None:
        index = json.loads((root / "model.safetensors.index.json").read_text())
        self.shard_of: dict[str, str] = dict(index["weight_map"])
        doc = json.loads((root / "manifest.json").read_text())
        if doc.get("format") != "quanta":
            raise ValueError(f"{root}: manifest.json declares format={doc.get('format')!r}, so this is not a quanta artifact")
        self.entries: dict[str, dict] = doc["tensors"]
        self.dense = {k for k, e in self.entries.items() if e.get("format") == "dense"}
        self.packed = {k: (int(e["bits"]), int(e["group_size"]))
                       for k, e in self.entries.items() if e.get("format") == "affine_packed"}

    @staticmethod
    def stem(key: str) -> str:
        return key[:-len(_WEIGHT_SUFFIX)] if key.endswith(_WEIGHT_SUFFIX) else key

    def resolve(self, key: str) -> tuple[str, str]:
        """A weight key -> (stored key, "dense" | "affine_packed"), by the rule above."""
        if key in self.dense:
            return key, "dense"
        stem = self.stem(key)
        if stem in self.packed:
            return stem, "affine_packed"
        for where in (key, stem):
            if where in self.entries:
                raise ValueError(f"{where}: unknown manifest format "
                                 f"{self.entries[where].get('format')!r} (a reader decodes dense "
                                 "and affine_packed records only)")
        raise KeyError(f"{key}: the manifest records neither a dense tensor at this key nor an "
                       f"affine_packed weight at {stem!r}")


class QuantaArtifact:
    """Lazy reader over a quanta artifact directory: the manifest indexed at open time, each
    shard mapped on first use (the reference's reader: src/quanta/qwen35/artifact.py:38-123)."""

    def __init__(self, art_dir: str | Path) -> None:
        self.dir = Path(art_dir)
        self._man = _Manifest(self.dir)
        cfg_file = self.dir / "config.json"
        self.config: dict = json.loads(cfg_file.read_text()) if cfg_file.exists() else {}
        self._open: dict[str, _Shard] = {}

    @property
    def weight_map(self) -> dict[str, str]:
        """Stored tensor name -> shard file (the index's weight_map)."""
        return self._man.shard_of

    @property
    def manifest(self) -> dict[str, dict]:
        """Manifest records by key."""
        return self._man.entries

    @property
    def _shards(self) -> dict[str, _Shard]:
        return self._open

    # --- tensors --------------------------------------------------------------------------
    def get(self, name: str) -> torch.Tensor:
        """The stored tensor `name` (exact key) as a host view of its mapped shard."""
        fn = self._man.shard_of.get(name)
        if fn is None:
            raise KeyError(f"{name}: no such tensor in the artifact index")
        if fn not in self._open:
            self._open[fn] = _Shard(self.dir / fn)
        return self._open[fn].tensor(name)

    def has(self, key: str) -> bool:
        """Whether a weight key is stored verbatim or resolves to an affine_packed weight."""
        return key in self._man.shard_of or self._man.stem(key) in self._man.packed

    def release(self) -> None:
        """Unmap every shard; tensors already copied elsewhere are unaffected."""
        self._open = {}

    def _meta(self, key: str) -> tuple[str, dict]:
        """(stored key, manifest record) of a weight key; see _Manifest.resolve."""
        where, _ = self._man.resolve(key)
        return where, self._man.entries[where]

    def read(self, key: str, device: torch.device | str) -> torch.Tensor:
        """A bf16 weight on `device` for a logical key: a dense tensor cast to bf16, or an
        affine_packed one dequantized on the GPU (src/quanta/qwen35/artifact.py:96-123)."""
        base, meta = self._meta(key)
        if meta["format"] == "dense":
            return self.get(base).to(device).to(torch.bfloat16)
        tr = self.packed_triplet(base, device)
        if tr["group_size"] != 64 or tr["bits"] not in (4, 8):
            raise ValueError(f"{base}: dequant of bits={tr['bits']} group_size={tr['group_size']} "
                             "is not supported (int4 or int8, group 64)")
        return ops.dequant(tr["packed"], tr["scale"], tr["bias"], bits=tr["bits"],
                           group_size=tr["group_size"])

    def packed_triplet(self, base: str, device: torch.device | str) -> dict:
        """The packed affine triplet {packed, scale, bias, group_size, bits} of `base`, verbatim,
        on `device`; the decode width comes from the manifest
        (src/quanta/qwen35/artifact.py:187-203). Not an affine_packed weight: ValueError."""
        meta = self.manifest.get(base)
        if meta is None or meta.get("format") != "affine_packed":
            raise ValueError(f"{base}: not an affine_packed weight (format="
                             f"{None if meta is None else meta.get('format')!r})")
        packed = self.get(base + ".weight_packed")
        if packed.dtype == torch.uint32:
            packed = packed.view(torch.int32)
        return {"packed": packed.to(device),
                "scale": self.get(base + ".weight_scale").to(device),
                "bias": self.get(base + ".weight_bias").to(device),
                "group_size": int(meta["group_size"]),
                "bits": int(meta["bits"])}

    # --- the MoE block --------------------------------------------------------------------
    def moe_packed(self, i: int, device: torch.device | str, *, prefix: str = LM_PREFIX,
                   shared: str = "bf16") -> dict:
        """The parameter dict of layer i's MoE block for `qwen35_moe`: the routed experts as packed
        triplets, the router gate, the shared expert and its gate in bf16
        (src/quanta/qwen35/artifact.py:205-229). A block without a shared expert omits its keys.
        shared="int8": a shared expert the bake stored as int8 (bake.py:150-151) is handed over
        as its packed triplets, which the block reads at half the bytes with the same outputs
        (a dense one is still read as bf16)."""
        if shared not in ("bf16", "int8"):
            raise ValueError("moe_packed: shared must be 'bf16' or 'int8'")
        p = f"{prefix}layers.{i}.mlp."
        out: dict[str, object] = {
            "gate": self.read(p + "gate.weight", device),
            "experts_gate_up": self.packed_triplet(p + "experts.gate_up_proj", device),
            "experts_down": self.packed_triplet(p + "experts.down_proj", device),
        }
        # a sigmoid router's selection bias, where the bake stores one (the HF key of the
        # DeepSeek/GLM gates, src/quanta/loader.py:50)
        if self.has(p + "gate.e_score_correction_bias"):
            out["e_score_correction_bias"] = self.get(p + "gate.e_score_correction_bias").to(
                device).to(torch.float32)
        if self.has(p + "shared_expert.gate_proj.weight"):
            for proj in SHARED_EXPERT_PROJS:
                base = p + f"shared_expert.{proj}"
                meta = self.manifest.get(base)
                if (shared == "int8" and meta is not None and meta.get("format") == "affine_packed"
                        and int(meta.get("bits", 0)) == 8):
                    out[f"shared_{proj}"] = self.packed_triplet(base, device)
                else:
                    out[f"shared_{proj}"] = self.read(base + ".weight", device)
            if self.has(p + "shared_expert_gate.weight"):
                out["shared_expert_gate"] = self.read(p + "shared_expert_gate.weight", device)
        return out

    def moe_config(self) -> MoEConfig:
        """The MoE fields of the artifact's config.json (`text_config` when nested), with the
        reference's defaults (src/quanta/qwen35/config.py:340-364): the router's scoring_func
        (:361, softmax unless stated) and, where present, the DeepSeek/GLM router fields n_group,
        topk_group and routed_scaling_factor (src/quanta/glm/config.py:65-69)."""
        tc = self.config.get("text_config", self.config)
        scoring = str(tc.get("scoring_func", "softmax"))
        if scoring not in ("softmax", "sigmoid"):
            raise ValueError(f"config.json: scoring_func {scoring!r} is not a Qwen3.5 router "
                             "(softmax | sigmoid)")
        return MoEConfig(
            hidden_size=int(tc["hidden_size"]),
            num_experts=int(tc["num_experts"]),
            num_experts_per_tok=int(tc["num_experts_per_tok"]),
            moe_intermediate_size=int(tc["moe_intermediate_size"]),
            shared_expert_intermediate_size=int(tc.get("shared_expert_intermediate_size", 0)),
            scoring_func=scoring,
            n_group=int(tc.get("n_group", 1) or 1),
            topk_group=int(tc.get("topk_group", 1) or 1),
            routed_scaling_factor=float(tc.get("routed_scaling_factor", 1.0) or 1.0),
            norm_topk_prob=bool(tc.get("norm_topk_prob", True)),
            norm_eps=float(tc.get("rms_norm_eps", 1e-6)),
            hidden_act=str(tc.get("hidden_act", "silu")),
            swiglu_alpha=float(tc.get("swiglu_alpha", 1.702)),
            swiglu_limit=float(tc.get("swiglu_limit", 0.0) or 0.0),
        )

    def post_attention_norm(self, i: int, device: torch.device | str, *,
                            prefix: str = LM_PREFIX) -> torch.Tensor:
        """Layer i's post_attention_layernorm weight in its resident form, source + 1 in bf16, as
        the reference wires it into nn.RMSNorm (key: src/quanta/qwen35/loader.py:136-142; the +1:
        src/quanta/qwen35/runtime.py:57-63,121): the `norm_weight` of `qwen35_moe_residual`."""
        w = self.read(f"{prefix}layers.{i}.post_attention_layernorm.weight", device)
        return (w.to(torch.bfloat16) + 1.0).to(torch.bfloat16)

    def moe_module(self, i: int, device: torch.device | str, *,
                   prefix: str = LM_PREFIX) -> Qwen35MoEModule:
        """A Qwen35MoEModule holding layer i's MoE block, as the reference loader builds it
        (src/quanta/qwen35/loader.py:178-188)."""
        p = self.moe_packed(i, device, prefix=prefix)
        m = Qwen35MoEModule(self.moe_config(), device=device)
        with torch.no_grad():
            m.gate.copy_(p["gate"])
            for proj in SHARED_EXPERT_PROJS:
                if f"shared_{proj}" in p:
                    getattr(m, f"shared_{proj}").copy_(p[f"shared_{proj}"])
            if "shared_expert_gate" in p:
                m.shared_expert_gate.copy_(p["shared_expert_gate"])
            else:   # an ungated shared expert
                m.shared_expert_gate = None
        if "e_score_correction_bias" in p:
            m.e_score_correction_bias = p["e_score_correction_bias"]
        m.set_experts_packed(p["experts_gate_up"], p["experts_down"])
        return m
