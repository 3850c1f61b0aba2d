"""CPU tier: the timed CPU baseline (oracle/torch_cpu.py, bench.py's `cpu_baseline`) computes the
same block as the oracle, so the baseline's tokens/s are those of a verified computation.

Checked on the golden fixtures (c0: fp32 router, no shared expert; c1mini: softmax with a gated
shared expert; c3mini: sigmoid + correction bias, groups, x2.5, ungated shared expert) and at
k = 1: routing ids equal the oracle's, the output within the BASELINE gates of the oracle's
float64 result (the port computes in float32 and rounds to bf16).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq
from oracle import torch_cpu
from quanta_amd.moe import MoEConfig
from tests._util import assert_close
from tests.golden.make_golden import oracle_params

GOLDEN = Path(__file__).resolve().parent / "golden"


def _bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _torch_params(a):
    p = {"gate": torch.from_numpy(a["gate_f32"]) if "gate_f32" in a else _bf16(a["gate"])}
    for pre, key in (("gu", "experts_gate_up"), ("dn", "experts_down")):
        p[key] = {"packed": torch.from_numpy(a[f"{pre}_packed"].view(np.int32)),
                  "scale": _bf16(a[f"{pre}_scale"]), "bias": _bf16(a[f"{pre}_bias"])}
    for k in ("shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
        if k in a:
            p[k] = _bf16(a[k])
    if "e_score_correction_bias" in a:
        p["e_score_correction_bias"] = torch.from_numpy(a["e_score_correction_bias"])
    return p


@pytest.mark.parametrize("name", ["c0", "c1mini", "c3mini"])
@pytest.mark.parametrize("k1", [False, True])
def test_torch_cpu_port_matches_oracle(name, k1):
    a = dict(np.load(GOLDEN / f"{name}.npz"))
    H, E, k, I, Is, ng, tg, norm, sig = a["dims"].tolist()
    scale = float(a["routed_scale"][0])
    cfg = MoEConfig(H, E, k, I, Is, scoring_func="sigmoid" if sig else "softmax",
                    norm_topk_prob=bool(norm), n_group=ng, topk_group=tg,
                    routed_scaling_factor=scale)
    kk = 1 if k1 else k
    xf = oq.bf16_bits_to_f32(a["x"]).astype(np.float64)
    op = oracle_params(a)
    moegate = bool(sig) and "e_score_correction_bias" in a
    _, it = om.moe_forward(xf, op, k=kk, inter=I, scoring=cfg.scoring_func, norm_topk=bool(norm),
                           n_group=ng, topk_group=tg, scale=scale, norm_single=not moegate)
    p = _torch_params(a)
    y = torch_cpu.moe_forward(_bf16(a["x"]), p, cfg, k=kk)
    bias = p.get("e_score_correction_bias")
    idx, w = torch_cpu.route(_bf16(a["x"]), p["gate"], cfg, kk, bias)
    ok = om.route_margin(it["choice"], kk) > 1e-5
    assert all(set(r) == set(o) for r, o, m in zip(idx.tolist(), it["idx"].tolist(), ok) if m)
    assert_close(y.float().numpy().astype(np.float64), it["y_exact"], f"torch_cpu {name} k={kk}")


def test_torch_cpu_port_int8_shared_matches_oracle():
    """The CPU port with the bake's int8 shared expert (c1mini fixture's shared weights
    quantized): load_shared gives the bf16 dequant the oracle's shared_weight makes, and the
    block stays within the gates of the oracle run on the same triplets."""
    a = dict(np.load(GOLDEN / "c1mini.npz"))
    H, E, k, I, Is, ng, tg, norm, sig = a["dims"].tolist()
    cfg = MoEConfig(H, E, k, I, Is, norm_topk_prob=bool(norm))
    op = oracle_params(a)
    p = _torch_params(a)
    for key in ("shared_gate_proj", "shared_up_proj", "shared_down_proj"):
        w = oq.bf16_bits_to_f32(a[key]).astype(np.float32)
        words, sb, bb, _ = oq.quantize_rtn(w, bits=8, group_size=64)
        op[key] = {"packed": words, "scale": sb, "bias": bb, "group_size": 64, "bits": 8}
        p[key] = {"packed": torch.from_numpy(words.view(np.int32)), "scale": _bf16(sb),
                  "bias": _bf16(bb), "group_size": 64, "bits": 8}
        got = torch_cpu.load_shared(p)[key].float().numpy().astype(np.float64)
        assert np.array_equal(got, om.shared_weight(op[key]))
    xf = oq.bf16_bits_to_f32(a["x"]).astype(np.float64)
    _, it = om.moe_forward(xf, op, k=k, inter=I)
    y = torch_cpu.moe_forward(_bf16(a["x"]), p, cfg)
    assert_close(y.float().numpy().astype(np.float64), it["y_exact"], "torch_cpu c1mini int8 shared")
