"""Seeded synthetic MoE layers and inputs for the BASELINE configurations (any torch device).

Config ids follow BASELINE.json `configs`:
  c0  H512  / E16  / top-2 softmax / I256, no shared expert, fp32 router      (N = 8)
  c1  H2048 / E256 / top-8 softmax / I512, shared I512 with sigmoid gate      (N = 1, 8, 32, 64)
  c2  H4096 / E512 / top-10 softmax / I1024, shared I1024 with sigmoid gate   (N = 1, 8, 32, 128)
  c3  H7168 / E256 / sigmoid + correction bias, 8 groups keep 4, top-8, x2.5, ungated shared
      I2048, expert I2048                                                      (N = 1, 16, 64)
  c4  the c2 shape at a 4096-token prefill with Zipf(1.1) expert popularity  (N = 4096)
Weights: router N(0, 0.02) (fp32 for c0, bf16 otherwise, as the artifact stores it); experts
bf16 N(0, 0.02) quantized RTN affine int4 g64 (quanta_amd.quant.quantize_affine); shared expert
bf16 N(0, 0.02); c3 correction bias N(0, 0.01) fp32. Inputs x ~ N(0, 1) in bf16.

c4 popularity: a seeded permutation assigns every expert a popularity rank r_e, and router
column 0 carries the logit bias beta_e = -1.1 * tau * log(r_e) while x[:, 0] is held at 1.0, so
logit_e = beta_e + (noise of std sqrt(H-1)*0.02). tau = 0.8 was calibrated offline so that the
realised top-10 histogram over 4096 tokens has a log-log slope of about -1.1 across ranks 2..64
(hottest experts take thousands of tokens, the median a handful, some none).

Generation is chunked over experts so even c2 (3.4 GiB of packed experts) stays within a few GiB
of temporaries. All randomness comes from one torch.Generator seeded per (config, layer).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from quanta_amd.moe import MoEConfig
from quanta_amd.quant import quantize_affine

ZIPF_TAU = 0.8
ZIPF_S = 1.1


@dataclass(frozen=True)
class SynthSpec:
    cfg: MoEConfig
    batches: tuple
    router_fp32: bool
    shared_gated: bool
    bias_std: float
    zipf: bool


SPECS = {
    "c0": SynthSpec(MoEConfig(512, 16, 2, 256, 0), (8,), True, False, 0.0, False),
    "c1": SynthSpec(MoEConfig(2048, 256, 8, 512, 512), (1, 8, 32, 64), False, True, 0.0, False),
    "c2": SynthSpec(MoEConfig(4096, 512, 10, 1024, 1024), (1, 8, 32, 128), False, True, 0.0, False),
    "c3": SynthSpec(MoEConfig(7168, 256, 8, 2048, 2048, scoring_func="sigmoid", norm_topk_prob=True,
                              n_group=8, topk_group=4, routed_scaling_factor=2.5),
                    (1, 16, 64), False, False, 0.01, False),
    "c4": SynthSpec(MoEConfig(4096, 512, 10, 1024, 1024), (4096,), False, True, 0.0, True),
}


def spec(name: str) -> SynthSpec:
    return SPECS[name]


def scaled_spec(name: str, **dims) -> SynthSpec:
    """A spec with some MoEConfig fields replaced (same routing style), for reduced-size tests."""
    s = SPECS[name]
    c = s.cfg
    fields = {f: getattr(c, f) for f in c.__dataclass_fields__}
    fields.update(dims)
    return SynthSpec(MoEConfig(**fields), s.batches, s.router_fp32, s.shared_gated, s.bias_std,
                     s.zipf)


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _normal(shape, std, g, device, dtype=torch.float32):
    return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(dtype)


def _quantized_stack(E, rows, K, g, device, chunk_elems=1 << 28, bits=4, group_size=64):
    """Stack of E experts [rows, K] ~ N(0, 0.02) bf16, RTN int`bits` -> packed triplet dict."""
    packed = torch.empty(E, rows, K * bits // 32, dtype=torch.int32, device=device)
    scale = torch.empty(E, rows, K // group_size, dtype=torch.bfloat16, device=device)
    bias = torch.empty_like(scale)
    per = max(1, chunk_elems // (rows * K))
    for e0 in range(0, E, per):
        e1 = min(E, e0 + per)
        w = _normal((e1 - e0, rows, K), 0.02, g, device, torch.bfloat16)
        q, s, b = quantize_affine(w, bits, group_size, scale_dtype=torch.bfloat16)
        packed[e0:e1], scale[e0:e1], bias[e0:e1] = q, s, b
        del w, q, s, b
    return {"packed": packed, "scale": scale, "bias": bias, "group_size": group_size, "bits": bits}


def make_mixed_experts(name: str, *, device="cuda", seed: int = 0, choices=(3, 4),
                       group_size: int = 128) -> dict:
    """Routed experts of widths drawn per expert from `choices`, one draw for gate and up
    together and one for down (Kimi's per-projection bake, src/quanta/modeling/quantized.py:
    40-51, whose canonical split is gate/up int3 + down int4), as the reference's
    (stacks, pbits, pslot): one stack per (projection, width), experts in id order."""
    c = SPECS[name].cfg
    E, H, I = c.num_experts, c.hidden_size, c.moe_intermediate_size
    g = _gen(device, seed * 1009 + 7)
    rng = np.random.default_rng(seed)
    stacks, pbits, pslot = {}, {}, {}
    pb_gu = rng.choice(np.asarray(choices), E)
    for proj in ("gate", "up", "down"):
        rows, K = (I, H) if proj != "down" else (H, I)
        pb = pb_gu if proj != "down" else rng.choice(np.asarray(choices), E)
        ps = np.zeros(E, np.int64)
        stacks[proj] = {}
        for b in sorted(set(pb.tolist())):
            ids = np.flatnonzero(pb == b)
            ps[ids] = np.arange(ids.size)
            stacks[proj][b] = _quantized_stack(ids.size, rows, K, g, device, bits=b, group_size=group_size)
        pbits[proj], pslot[proj] = pb, ps
    return {"stacks": stacks, "pbits": pbits, "pslot": pslot, "group_size": group_size}


def mixed_expert_bytes(mixed: dict, cfg) -> float:
    """Mean bytes per expert of a mixed-width layer (codes + a bf16 scale and bias per group)."""
    H, I, gs = cfg.hidden_size, cfg.moe_intermediate_size, mixed["group_size"]
    tot = sum(I * H * (np.asarray(mixed["pbits"][proj]) * gs + 32) / (8 * gs)
              for proj in ("gate", "up", "down"))
    return float(np.mean(tot))


def zipf_logit_bias(E: int, g: torch.Generator, device) -> torch.Tensor:
    perm = torch.randperm(E, generator=g, device=device)
    rank = torch.empty(E, dtype=torch.float32, device=device)
    rank[perm] = torch.arange(1, E + 1, dtype=torch.float32, device=device)
    return -ZIPF_S * ZIPF_TAU * torch.log(rank)


def zipf_router(gate: torch.Tensor, seed: int = 4) -> torch.Tensor:
    """A copy of a router weight [E, H] whose column 0 carries the c4 Zipf popularity bias (used
    with inputs whose channel 0 is 1.0), turning a c2 layer into the c4 prefill workload without
    regenerating its experts."""
    g = _gen(gate.device, (1000 + seed) * 1009 + 7)
    out = gate.clone()
    out[:, 0] = zipf_logit_bias(gate.shape[0], g, gate.device).to(gate.dtype)
    return out


def make_layer(name: str | SynthSpec, *, device="cuda", seed: int | None = None,
               layer: int = 0, bits: int = 4, down_bits: int | None = None,
               group_size: int = 64, shared_bits: int = 16) -> dict:
    """Parameter dict with the reference keys (src/quanta/qwen35/moe.py:159-161); routed experts as
    packed triplets in the reference's native layout (gate_up int`bits`, down int`down_bits`,
    default the same width). shared_bits 8: the shared expert as the bake stores it, int8 g64
    triplets of the same bf16 draws (src/quanta/qwen35/bake.py:106-110, 150-151)."""
    s = SPECS[name] if isinstance(name, str) else name
    c = s.cfg
    cid = int(name[1]) if isinstance(name, str) else 9
    g = _gen(device, (1000 + cid if seed is None else seed) * 1009 + layer)
    H, E, I, Is = c.hidden_size, c.num_experts, c.moe_intermediate_size, c.shared_expert_intermediate_size
    p: dict = {}
    gate = _normal((E, H), 0.02, g, device)
    if s.zipf:
        gate[:, 0] = zipf_logit_bias(E, g, device)
    p["gate"] = gate if s.router_fp32 else gate.to(torch.bfloat16)
    p["experts_gate_up"] = _quantized_stack(E, 2 * I, H, g, device, bits=bits, group_size=group_size)
    p["experts_down"] = _quantized_stack(E, H, I, g, device, group_size=group_size,
                                         bits=bits if down_bits is None else down_bits)
    if Is > 0:
        p["shared_gate_proj"] = _normal((Is, H), 0.02, g, device, torch.bfloat16)
        p["shared_up_proj"] = _normal((Is, H), 0.02, g, device, torch.bfloat16)
        p["shared_down_proj"] = _normal((H, Is), 0.02, g, device, torch.bfloat16)
        if shared_bits == 8:
            for key in ("shared_gate_proj", "shared_up_proj", "shared_down_proj"):
                pk, sc, bi = quantize_affine(p[key], 8, group_size=64)
                p[key] = {"packed": pk, "scale": sc, "bias": bi, "group_size": 64, "bits": 8}
        elif shared_bits != 16:
            raise ValueError("shared_bits: 16 (bf16) or 8 (int8 g64, as baked)")
        if s.shared_gated:
            p["shared_expert_gate"] = _normal((1, H), 0.02, g, device, torch.bfloat16)
    if s.bias_std > 0:
        p["e_score_correction_bias"] = _normal((E,), s.bias_std, g, device)
    return p


def make_inputs(name: str | SynthSpec, N: int, *, device="cuda", seed: int = 0) -> torch.Tensor:
    """x [N, H] bf16 ~ N(0, 1); for the Zipf config channel 0 is held at 1.0."""
    s = SPECS[name] if isinstance(name, str) else name
    g = _gen(device, 7919 + seed)
    x = torch.randn(N, s.cfg.hidden_size, generator=g, device=device, dtype=torch.float32)
    if s.zipf:
        x[:, 0] = 1.0
    return x.to(torch.bfloat16)


def algorithmic_bytes(cfg, distinct_experts: int, N: int, router_bytes_per_elem: int = 2,
                      bits: int = 4, down_bits: int | None = None, group_size: int = 64,
                      shared_bits: int = 16) -> int:
    """Bytes a layer call must move at minimum: U*B_e + S + R + A with
    B_e = 2*I*H*(bits/8 + 4/g) + I*H*(down_bits/8 + 4/g) (codes + a bf16 scale and bias per group
    of g: 0.5625 B per weight for int4 g64, 0.8125 for int6 g64, 0.40625 for int3 g128),
    S = 3*Is*H*2 (bf16) or 3*Is*H*(1 + 4/64) (int8 g64), R = E*H*elem, A = 4*N*H (bf16 in and
    out)."""
    H, E, I = cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size
    Is = cfg.shared_expert_intermediate_size
    db = bits if down_bits is None else down_bits
    be = (2 * I * H * (bits * group_size + 32) + I * H * (db * group_size + 32)) // (8 * group_size)
    sh = 3 * Is * H * 2 if shared_bits == 16 else 3 * Is * H * (8 * 64 + 32) // (8 * 64)
    return distinct_experts * be + sh + E * H * router_bytes_per_elem + 4 * N * H


def algorithmic_flops(cfg, N: int, k: int | None = None) -> int:
    """2*N*(k*3*I*H + 3*Is*H + E*H)."""
    H, E, I = cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size
    Is = cfg.shared_expert_intermediate_size
    k = cfg.num_experts_per_tok if k is None else k
    return 2 * N * (k * 3 * I * H + 3 * Is * H + E * H)


def expected_distinct(E: int, k: int, N: int) -> float:
    """E[U] under uniform routing: E * (1 - (1 - k/E)^N)."""
    return E * (1.0 - math.pow(1.0 - k / E, N))
