"""Write the golden fixtures under tests/golden/ from this build's oracle.

    python tests/golden/make_golden.py

The reference commits no golden vectors for the MoE path and its MLX implementation cannot run
here (MLX absent, Python 3.13 required), so these vectors come from the CPU oracle (oracle/),
which tests/test_oracle.py pins against exact arithmetic, brute force and transformers' modules.
Each fixture holds the inputs (bf16 as uint16 bit patterns, packed int4 as uint32 words) and the
oracle's expected outputs for one block configuration:

  c0.npz      BASELINE config 0 at full size (H512/E16/top-2 softmax/I256, fp32 router, N=8)
  c1mini.npz  config-1 routing style (softmax top-k, sigmoid-gated shared expert), small dims
  c3mini.npz  config-3 routing style (sigmoid + correction bias, 8 groups keep 4, x2.5 scaling,
              ungated shared expert), small dims
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import moe as om  # noqa: E402
from oracle import quant as oq  # noqa: E402
from quanta_amd import synth  # noqa: E402

OUT = Path(__file__).resolve().parent

CASES = {
    "c0": (synth.spec("c0"), 8),
    "c1mini": (synth.scaled_spec("c1", hidden_size=256, num_experts=16, num_experts_per_tok=4,
                                 moe_intermediate_size=128, shared_expert_intermediate_size=128), 16),
    "c3mini": (synth.scaled_spec("c3", hidden_size=256, num_experts=16, num_experts_per_tok=4,
                                 moe_intermediate_size=128, shared_expert_intermediate_size=128,
                                 n_group=8, topk_group=4), 12),
}


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().astype(np.uint16)


def _words(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().numpy().view(np.uint32)


def oracle_params(arrs: dict) -> dict:
    """Fixture arrays -> the oracle's parameter dict (float64 values for bf16 data)."""
    f = lambda k: oq.bf16_bits_to_f32(arrs[k]).astype(np.float64)
    p = {"gate": arrs["gate_f32"].astype(np.float64) if "gate_f32" in arrs else f("gate"),
         "gu_packed": arrs["gu_packed"], "gu_scale": arrs["gu_scale"], "gu_bias": arrs["gu_bias"],
         "dn_packed": arrs["dn_packed"], "dn_scale": arrs["dn_scale"], "dn_bias": arrs["dn_bias"]}
    for k in ("shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
        if k in arrs:
            p[k] = f(k)
    if "e_score_correction_bias" in arrs:
        p["e_score_correction_bias"] = arrs["e_score_correction_bias"].astype(np.float64)
    return p


def make(name: str) -> dict:
    spec, n = CASES[name]
    c = spec.cfg
    p = synth.make_layer(spec, device="cpu", seed=4242 + sum(map(ord, name)), layer=0)
    x = synth.make_inputs(spec, n, device="cpu", seed=17)
    arrs: dict[str, np.ndarray] = {"x": _bits16(x)}
    if p["gate"].dtype == torch.float32:
        arrs["gate_f32"] = p["gate"].numpy()
    else:
        arrs["gate"] = _bits16(p["gate"])
    for pre, key in (("gu", "experts_gate_up"), ("dn", "experts_down")):
        arrs[f"{pre}_packed"] = _words(p[key]["packed"])
        arrs[f"{pre}_scale"] = _bits16(p[key]["scale"])
        arrs[f"{pre}_bias"] = _bits16(p[key]["bias"])
    for k in ("shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
        if k in p:
            arrs[k] = _bits16(p[k])
    if "e_score_correction_bias" in p:
        arrs["e_score_correction_bias"] = p["e_score_correction_bias"].numpy()
    arrs["dims"] = np.array([c.hidden_size, c.num_experts, c.num_experts_per_tok,
                             c.moe_intermediate_size, c.shared_expert_intermediate_size, c.n_group,
                             c.topk_group, int(c.norm_topk_prob), int(c.scoring_func == "sigmoid")],
                            np.int64)
    arrs["routed_scale"] = np.array([c.routed_scaling_factor], np.float64)

    op = oracle_params(arrs)
    xf = oq.bf16_bits_to_f32(arrs["x"]).astype(np.float64)
    y, it = om.moe_forward(xf, op, k=c.num_experts_per_tok, inter=c.moe_intermediate_size,
                           scoring=c.scoring_func, norm_topk=c.norm_topk_prob, n_group=c.n_group,
                           topk_group=c.topk_group, scale=c.routed_scaling_factor)
    counts, offsets, order, inv = om.permute(it["idx"], c.num_experts)
    arrs.update(
        y=oq.f32_to_bf16_bits(y.astype(np.float32)), y_exact=it["y_exact"],
        idx=it["idx"], w=it["w"], margin=om.route_margin(it["choice"], c.num_experts_per_tok),
        counts=counts, offsets=offsets, order=order, inv=inv,
        h=oq.f32_to_bf16_bits(it["h"].astype(np.float32)),
        deq_gu_e0=oq.dequant_bf16_bits(arrs["gu_packed"][0], arrs["gu_scale"][0], arrs["gu_bias"][0],
                                       c.hidden_size),
    )
    return arrs


def main() -> None:
    torch.manual_seed(0)
    for name in CASES:
        arrs = make(name)
        path = OUT / f"{name}.npz"
        np.savez_compressed(path, **arrs)
        print(f"wrote {path} ({path.stat().st_size / 1024:.0f} KiB)")


if __name__ == "__main__":
    main()
