"""GPU tier: the block at the reference's own dtypes and group sizes (qmoe_forward_general).

The reference's block takes whatever float dtype was baked: its packed-expert parity gate runs
float32 activations, float32 scale/bias and int4 group 32 at hidden 32
(parity/qwen35_forward_test.py:213-271), its sparse-vs-dense gate float32 dense stacks at
moe_intermediate 16 (parity/qwen35_forward_test.py:192-209). qwen35_moe dispatches such inputs to
qmoe_forward_general. Each case compares the GPU output with the oracle's restatement of the
reference's dtype flow (oracle.moe.moe_forward_general) and repeats the reference's own gates
between paths (packed == dequantized dense == run-every-expert, module == function).

Tolerances: float32 outputs within 1e-5 of the oracle, scaled by max(1, max|y|) (the GPU sums in
float32 in another order; the reference's own float32 gates allow 1e-4 between paths, which the
path-to-path checks assert as written); bf16 outputs within the bf16 gates of the fast path
(max-abs 2e-2, rel-L2 5e-3, tests/_util.assert_close).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq
from quanta_amd import moe as qm
from quanta_amd.moe import MoEConfig, Qwen35MoEModule, qwen35_moe
from tests._util import assert_close

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
REF_GATE = 1e-4


def _f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def _t(a, dev, dtype=torch.float32) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=np.float32))).to(dev).to(dtype)


def _layer(seed, *, E=8, H=32, I=64, Is=64, bits=4, gs=32, sb="f32", shared="f32", gated=True,
           wscale=0.1):
    """(oracle params, torch params on the GPU-less host) of a packed layer: float32 weights
    quantized with float32 scales (sb="f32", mx.quantize of float32 arrays) or bf16 scales."""
    rng = np.random.default_rng(seed)
    gu_w = (rng.standard_normal((E, 2 * I, H)) * wscale).astype(np.float32)
    dn_w = (rng.standard_normal((E, H, I)) * wscale).astype(np.float32)
    if sb == "f32":
        gq, dq = oq.quantize_rtn_f32(gu_w, bits, gs), oq.quantize_rtn_f32(dn_w, bits, gs)
        conv = _f32
    else:
        gq, dq = oq.quantize_rtn(gu_w, bits, gs), oq.quantize_rtn(dn_w, bits, gs)
        conv = lambda b: oq.bf16_bits_to_f32(b).astype(np.float64)
    rnd = _f32 if shared == "f32" else oq.round_bf16
    o = dict(gate=_f32(rng.standard_normal((E, H))),
             gu_packed=gq[0], gu_scale=conv(gq[1]), gu_bias=conv(gq[2]),
             dn_packed=dq[0], dn_scale=conv(dq[1]), dn_bias=conv(dq[2]),
             bits=bits, group_size=gs, sb_dtype=sb)
    if Is:
        o.update(shared_gate_proj=rnd(rng.standard_normal((Is, H)) * 0.1),
                 shared_up_proj=rnd(rng.standard_normal((Is, H)) * 0.1),
                 shared_down_proj=rnd(rng.standard_normal((H, Is)) * 0.1), shared_dtype=shared)
        if gated:
            o["shared_expert_gate"] = _f32(rng.standard_normal((1, H)))
    return o


def _torch_params(o: dict, dev) -> dict:
    sdt = torch.float32 if o.get("sb_dtype", "f32") == "f32" else torch.bfloat16
    p = {"gate": _t(o["gate"], dev)}
    if "gu_packed" in o:
        for pre, key in (("gu", "experts_gate_up"), ("dn", "experts_down")):
            p[key] = {"packed": torch.from_numpy(o[f"{pre}_packed"].view(np.int32)).to(dev),
                      "scale": _t(o[f"{pre}_scale"], dev, sdt), "bias": _t(o[f"{pre}_bias"], dev, sdt),
                      "group_size": o["group_size"], "bits": o["bits"]}
    else:
        edt = torch.float32 if o["expert_dtype"] == "f32" else torch.bfloat16
        p["experts_gate_up"] = _t(o["gu_dense"], dev, edt)
        p["experts_down"] = _t(o["dn_dense"], dev, edt)
    if "shared_gate_proj" in o:
        shd = torch.float32 if o["shared_dtype"] == "f32" else torch.bfloat16
        for k in ("shared_gate_proj", "shared_up_proj", "shared_down_proj"):
            p[k] = _t(o[k], dev, shd)
        if "shared_expert_gate" in o:
            p["shared_expert_gate"] = _t(o["shared_expert_gate"], dev)
    if "e_score_correction_bias" in o:
        p["e_score_correction_bias"] = _t(o["e_score_correction_bias"], dev)
    return p


def _dense_of(o: dict, H: int, I: int) -> dict:
    """The layer with its packed stacks dequantized to float32 (mx.dequantize of float32 scales)."""
    q = {k: v for k, v in o.items()
         if not k.startswith(("gu_", "dn_")) and k not in ("bits", "group_size", "sb_dtype")}
    q["gu_dense"] = _f32(oq.dequant_float(o["gu_packed"], o["gu_scale"], o["gu_bias"], H,
                                          bits=o["bits"], group_size=o["group_size"]))
    q["dn_dense"] = _f32(oq.dequant_float(o["dn_packed"], o["dn_scale"], o["dn_bias"], I,
                                          bits=o["bits"], group_size=o["group_size"]))
    q["expert_dtype"] = "f32"
    return q


def _cfg(H, E, k, I, Is, **kw):
    return MoEConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=I,
                     shared_expert_intermediate_size=Is, **kw)


def _check_f32(got: torch.Tensor, x: np.ndarray, o: dict, cfg, what: str, **kw):
    """float32 GPU output vs the oracle, rows at a router near-tie excluded (and counted)."""
    k, I = cfg.num_experts_per_tok, cfg.moe_intermediate_size
    want, inter = om.moe_forward_general(x, o, k=k, inter=I, x_dtype="f32",
                                         scoring=cfg.scoring_func, **kw)
    # a row whose k-th and (k+1)-th choice values lie within float32 evaluation error of each
    # other (relative: a peaked softmax leaves both tiny) may pick the other expert on the GPU
    srt = -np.sort(-inter["choice"], axis=1)
    ties = np.zeros(len(srt), dtype=bool)
    if k < srt.shape[1]:
        ties = (srt[:, k - 1] - srt[:, k]) <= 1e-5 * np.abs(srt[:, k - 1])
    g = got.detach().float().cpu().numpy().reshape(want.shape).astype(np.float64)
    keep = ~ties
    assert keep.sum() >= max(1, int(0.9 * len(keep))), f"{what}: too many near-tie rows"
    d = np.max(np.abs(g[keep] - want[keep]))
    scale = max(1.0, float(np.max(np.abs(want[keep]))))
    print(f"[parity] {what}: f32 max_abs={d:.3e} (scaled {d / scale:.3e}) ties={int(ties.sum())}",
          flush=True)
    assert np.all(np.isfinite(g)), what
    assert d <= F32_TOL * scale, f"{what}: max_abs {d:.3e} > {F32_TOL * scale:.3e}"
    return want


def test_reference_packed_parity_config(gpu):
    """parity/qwen35_forward_test.py:213-271 on the GPU: float32 x [1, 9, 32], int4 group-32
    experts with float32 scale/bias, float32 router and shared expert. The packed path matches
    the oracle; packed == dequantized dense == run-every-expert within the reference's 1e-4;
    Qwen35MoEModule.set_experts_packed reproduces the function-level result."""
    E, H, I, Is, k = 8, 32, 64, 64, 3
    cfg = _cfg(H, E, k, I, Is)
    o = _layer(3, E=E, H=H, I=I, Is=Is)
    q = _dense_of(o, H, I)
    x = _f32(np.random.default_rng(4).standard_normal((9, H)))
    xt = _t(x, gpu)[None]
    p_pack, p_dense = _torch_params(o, gpu), _torch_params(q, gpu)
    assert qm.needs_general(xt, p_pack, cfg)
    y_pack = qwen35_moe(xt, p_pack, cfg, sparse=True)
    y_bf = qwen35_moe(xt, p_dense, cfg, sparse=True)
    y_dense = qwen35_moe(xt, p_dense, cfg, sparse=False)
    assert y_pack.dtype == torch.float32 and y_pack.shape == (1, 9, H)
    _check_f32(y_pack, x, o, cfg, "packed g32 f32")
    _check_f32(y_bf, x, q, cfg, "dense f32")
    _check_f32(y_dense, x, q, cfg, "run-every-expert f32", dense_all=True)
    assert (y_pack - y_bf).abs().max().item() < REF_GATE
    assert (y_bf - y_dense).abs().max().item() < REF_GATE
    mod = Qwen35MoEModule(cfg, device=gpu, dtype=torch.float32)
    mod.gate.copy_(p_pack["gate"])
    for kk in ("shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
        getattr(mod, kk).copy_(p_pack[kk])
    mod.set_experts_packed(p_pack["experts_gate_up"], p_pack["experts_down"])
    y_mod = mod(xt, sparse=True)
    assert torch.equal(y_mod, y_pack)


def test_reference_sparse_equals_dense_f32(gpu):
    """parity/qwen35_forward_test.py:192-209 on the GPU: float32 dense stacks at the tiny
    config's moe_intermediate 16; sparse == dense within 1e-4, both matching the oracle."""
    E, H, I, Is, k = 8, 32, 16, 16, 3
    cfg = _cfg(H, E, k, I, Is)
    rng = np.random.default_rng(3)
    o = dict(gate=_f32(rng.standard_normal((E, H))),
             gu_dense=_f32(rng.standard_normal((E, 2 * I, H)) * 0.1),
             dn_dense=_f32(rng.standard_normal((E, H, I)) * 0.1), expert_dtype="f32",
             shared_gate_proj=_f32(rng.standard_normal((Is, H)) * 0.1),
             shared_up_proj=_f32(rng.standard_normal((Is, H)) * 0.1),
             shared_down_proj=_f32(rng.standard_normal((H, Is)) * 0.1), shared_dtype="f32",
             shared_expert_gate=_f32(rng.standard_normal((1, H))))
    x = _f32(rng.standard_normal((9, H)))
    p = _torch_params(o, gpu)
    xt = _t(x, gpu)[None]
    ys = qwen35_moe(xt, p, cfg, sparse=True)
    yd = qwen35_moe(xt, p, cfg, sparse=False)
    _check_f32(ys, x, o, cfg, "sparse f32 I=16")
    _check_f32(yd, x, o, cfg, "dense f32 I=16", dense_all=True)
    assert (ys - yd).abs().max().item() < REF_GATE


@pytest.mark.parametrize("bits, gs, H, I", [(2, 32, 64, 64), (3, 32, 96, 64), (5, 32, 64, 128),
                                           (6, 64, 128, 64), (8, 128, 128, 128), (4, 128, 256, 128)])
def test_widths_and_groups_f32(gpu, bits, gs, H, I):
    """Code widths 2..8 (the LSB-first bitstream crosses word boundaries for 3, 5, 6) and groups
    of 32/64/128, float32 throughout, against the oracle."""
    E, Is, k = 6, 32, 2
    cfg = _cfg(H, E, k, I, Is)
    o = _layer(10 + bits, E=E, H=H, I=I, Is=Is, bits=bits, gs=gs)
    x = _f32(np.random.default_rng(bits).standard_normal((13, H)))
    y = qwen35_moe(_t(x, gpu)[None], _torch_params(o, gpu), cfg)
    _check_f32(y, x, o, cfg, f"int{bits} g{gs} H={H} I={I}")


def test_f32_activations_over_bf16_scales(gpu):
    """float32 x over bf16-scaled int4 g64 codes (a bf16 bake run with float32 activations): the
    experts compute in float32 (the promotion of the two dtypes), x is not rounded to bf16, and
    the output is float32."""
    E, H, I, Is, k = 8, 128, 128, 128, 2
    cfg = _cfg(H, E, k, I, Is)
    o = _layer(21, E=E, H=H, I=I, Is=Is, bits=4, gs=64, sb="bf16", shared="bf16", wscale=0.05)
    x = _f32(np.random.default_rng(22).standard_normal((11, H)))
    p = _torch_params(o, gpu)
    y = qwen35_moe(_t(x, gpu)[None], p, cfg)
    assert y.dtype == torch.float32
    _check_f32(y, x, o, cfg, "f32 x, bf16 g64 scales")


@pytest.mark.parametrize("H, I, gs", [(128, 128, 32), (96, 64, 32)])
def test_bf16_group32_and_odd_dims(gpu, H, I, gs):
    """bf16 activations and scales at group 32 or at a hidden size the tiled kernels do not take:
    the general path against the bf16 oracle (moe_forward) within the bf16 gates."""
    E, Is, k = 8, 64, 3
    cfg = _cfg(H, E, k, I, Is)
    o = _layer(30 + H, E=E, H=H, I=I, Is=Is, bits=4, gs=gs, sb="bf16", shared="bf16", wscale=0.05)
    o["gate"] = oq.round_bf16(o["gate"] * 0.1)
    o["shared_expert_gate"] = oq.round_bf16(o["shared_expert_gate"] * 0.1)
    p = _torch_params(o, gpu)
    p["gate"] = p["gate"].to(torch.bfloat16)
    p["shared_expert_gate"] = p["shared_expert_gate"].to(torch.bfloat16)
    x = oq.round_bf16(np.random.default_rng(31).standard_normal((17, H)))
    xt = _t(x, gpu, torch.bfloat16)[None]
    assert qm.needs_general(xt, p, cfg)
    y = qwen35_moe(xt, p, cfg)
    assert y.dtype == torch.bfloat16
    o16 = dict(gate=o["gate"], gu_packed=o["gu_packed"], dn_packed=o["dn_packed"],
               gu_scale=oq.f32_to_bf16_bits(o["gu_scale"]), gu_bias=oq.f32_to_bf16_bits(o["gu_bias"]),
               dn_scale=oq.f32_to_bf16_bits(o["dn_scale"]), dn_bias=oq.f32_to_bf16_bits(o["dn_bias"]),
               shared_gate_proj=o["shared_gate_proj"], shared_up_proj=o["shared_up_proj"],
               shared_down_proj=o["shared_down_proj"], shared_expert_gate=o["shared_expert_gate"])
    _, inter = om.moe_forward(x, o16, k=k, inter=I, group_size=gs)
    got = y.float().cpu().numpy().reshape(17, H).astype(np.float64)
    assert_close(got, inter["y_exact"], f"bf16 g{gs} H={H} I={I}")


def test_sigmoid_bias_routing_f32(gpu):
    """The DeepSeek/GLM router fields on the general path: sigmoid scores, selection by score +
    e_score_correction_bias, bias-free weights renormalised and scaled."""
    E, H, I, Is, k = 16, 64, 64, 0, 4
    cfg = _cfg(H, E, k, I, Is, scoring_func="sigmoid", routed_scaling_factor=2.5)
    o = _layer(40, E=E, H=H, I=I, Is=0)
    o["e_score_correction_bias"] = _f32(np.random.default_rng(41).standard_normal(E) * 0.1)
    x = _f32(np.random.default_rng(42).standard_normal((10, H)))
    y = qwen35_moe(_t(x, gpu)[None], _torch_params(o, gpu), cfg)
    _check_f32(y, x, o, cfg, "sigmoid + bias", norm_topk=True, scale=2.5, norm_single=False)


def test_chunking_and_batch_invariance(gpu):
    """Every output value is one wavefront's fixed-order sum: token chunks and batch size do not
    change a token's result, bit for bit, and repeated calls are identical."""
    E, H, I, Is, k = 8, 32, 64, 64, 3
    cfg = _cfg(H, E, k, I, Is)
    o = _layer(3, E=E, H=H, I=I, Is=Is)
    p = _torch_params(o, gpu)
    x = _t(np.random.default_rng(5).standard_normal((1, 40, H)), gpu)
    whole = qwen35_moe(x, p, cfg)
    assert torch.equal(qwen35_moe(x, p, cfg, token_chunk=7), whole)
    assert torch.equal(qwen35_moe(x, p, cfg), whole)
    for t in (0, 17, 39):
        assert torch.equal(qwen35_moe(x[:, t:t + 1], p, cfg)[0, 0], whole[0, t])


def test_general_errors(gpu):
    """Fail-loud: the tiled resident form cannot serve float32 activations, an unsupported width
    is refused, and the dense oracle still refuses packed experts."""
    E, H, I, Is, k = 8, 128, 128, 128, 2
    cfg = _cfg(H, E, k, I, Is)
    o = _layer(50, E=E, H=H, I=I, Is=Is, bits=4, gs=64, sb="bf16", shared="bf16")
    p = _torch_params(o, gpu)
    x32 = torch.zeros(1, 2, H, device=gpu)
    tiled = dict(p, experts_gate_up=qm.tile_experts_packed(p["experts_gate_up"]),
                 experts_down=qm.tile_experts_packed(p["experts_down"]))
    with pytest.raises(TypeError, match="native packed triplet"):
        qwen35_moe(x32, tiled, cfg)
    bad = dict(p, experts_gate_up=dict(p["experts_gate_up"], bits=7))
    with pytest.raises(ValueError):
        qwen35_moe(x32, bad, cfg)
    with pytest.raises(ValueError, match="dense oracle"):
        qwen35_moe(x32, p, cfg, sparse=False)
