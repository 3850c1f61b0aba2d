"""CPU tier: the reference-dtype block (qmoe_forward_general) -- its oracle pinned by checks that
do not share its code, and the host-side choice between it and the tiled fast path.

The oracle restates the reference's dtype flow (src/quanta/qwen35/moe.py:36-56, 66-124,
145-151, 154-202) for float32 or bf16 data. It is pinned by:
  - equality with the bf16 oracle (moe_forward) where the flows coincide (bf16 data, bf16 scales),
    which is itself pinned against transformers' Qwen3.5-MoE block and brute force;
  - transformers' own (third-party) Qwen3.5-MoE sparse block in float64 on the dequantized
    float32 stacks, at the reference's own float32 parity configuration
    (parity/qwen35_forward_test.py:213-271: hidden 32, 8 experts, top 3, int4 group 32);
  - the run-every-expert form equal to the sparse form (the reference's sparse == dense gate,
    parity/qwen35_forward_test.py:192-209);
  - pure-Python loops over bits, groups and slots on tiny inputs;
  - rounding invariants: every materialised intermediate is representable in the dtype the
    reference materialises it in, and float32 data keeps values bf16 would not.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq


def _f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def _f32_layer(rng, E=8, H=32, I=64, Is=64, bits=4, gs=32, gated=True):
    """The reference's float32 packed-expert layer: float32 weights quantized with float32 scales
    (mx.quantize of float32 arrays), float32 router and shared expert."""
    gu_w = (rng.standard_normal((E, 2 * I, H)) * 0.1).astype(np.float32)
    dn_w = (rng.standard_normal((E, H, I)) * 0.1).astype(np.float32)
    gq = oq.quantize_rtn_f32(gu_w, bits, gs)
    dq = oq.quantize_rtn_f32(dn_w, bits, gs)
    p = dict(gate=_f32(rng.standard_normal((E, H))),
             gu_packed=gq[0], gu_scale=_f32(gq[1]), gu_bias=_f32(gq[2]),
             dn_packed=dq[0], dn_scale=_f32(dq[1]), dn_bias=_f32(dq[2]),
             bits=bits, group_size=gs, sb_dtype="f32")
    if Is:
        p.update(shared_gate_proj=_f32(rng.standard_normal((Is, H)) * 0.1),
                 shared_up_proj=_f32(rng.standard_normal((Is, H)) * 0.1),
                 shared_down_proj=_f32(rng.standard_normal((H, Is)) * 0.1), shared_dtype="f32")
        if gated:
            p["shared_expert_gate"] = _f32(rng.standard_normal((1, H)))
    return p


def _dense_of(p: dict, H: int, I: int) -> dict:
    """The same layer with the packed stacks dequantized to float32 (mx.dequantize of float32
    scales gives float32 weights): the reference's p_bf16 dict of its packed parity gate."""
    q = {k: v for k, v in p.items() if not k.startswith(("gu_", "dn_")) and k not in ("bits", "group_size", "sb_dtype")}
    q["gu_dense"] = _f32(oq.dequant_float(p["gu_packed"], p["gu_scale"], p["gu_bias"], H,
                                          bits=p["bits"], group_size=p["group_size"]))
    q["dn_dense"] = _f32(oq.dequant_float(p["dn_packed"], p["dn_scale"], p["dn_bias"], I,
                                          bits=p["bits"], group_size=p["group_size"]))
    q["expert_dtype"] = "f32"
    return q


# ----------------------------------------------------------------------------- oracle pins


@pytest.mark.parametrize("gs", [64, 32])
def test_general_bf16_flow_equals_bf16_oracle(gs):
    """bf16 data with bf16 scales: the general flow is the bf16 flow of moe_forward, value for
    value (same materialisation points)."""
    rng = np.random.default_rng(41)
    E, H, I, Is, k = 6, 128, 64, 64, 3
    gu_w = (rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float32)
    dn_w = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    gq, dq = oq.quantize_rtn(gu_w, 4, gs), oq.quantize_rtn(dn_w, 4, gs)
    bf = lambda a: oq.round_bf16(a)
    shared = dict(shared_gate_proj=bf(rng.standard_normal((Is, H)) * 0.05),
                  shared_up_proj=bf(rng.standard_normal((Is, H)) * 0.05),
                  shared_down_proj=bf(rng.standard_normal((H, Is)) * 0.05),
                  shared_expert_gate=bf(rng.standard_normal((1, H)) * 0.1))
    gate = bf(rng.standard_normal((E, H)) * 0.1)
    p16 = dict(gate=gate, gu_packed=gq[0], gu_scale=gq[1], gu_bias=gq[2], dn_packed=dq[0],
               dn_scale=dq[1], dn_bias=dq[2], **shared)
    pg = dict(gate=gate, gu_packed=gq[0], gu_scale=oq.bf16_bits_to_f32(gq[1]).astype(np.float64),
              gu_bias=oq.bf16_bits_to_f32(gq[2]).astype(np.float64), dn_packed=dq[0],
              dn_scale=oq.bf16_bits_to_f32(dq[1]).astype(np.float64),
              dn_bias=oq.bf16_bits_to_f32(dq[2]).astype(np.float64), bits=4, group_size=gs,
              sb_dtype="bf16", shared_dtype="bf16", **shared)
    x = bf(rng.standard_normal((7, H)))
    want, wi = om.moe_forward(x, p16, k=k, inter=I, group_size=gs)
    got, gi = om.moe_forward_general(x, pg, k=k, inter=I, x_dtype="bf16")
    assert gi["routed_dtype"] == "bf16"
    for key in ("idx", "gu", "h", "d"):
        np.testing.assert_array_equal(gi[key], wi[key], err_msg=key)
    np.testing.assert_allclose(gi["y_exact"], wi["y_exact"], rtol=1e-13, atol=1e-15)
    np.testing.assert_array_equal(got, want)


def _hf_block(p: dict, H: int, E: int, k: int, I: int, Is: int):
    pytest.importorskip("transformers")
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeSparseMoeBlock

    cfg = Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k,
                               moe_intermediate_size=I, shared_expert_intermediate_size=Is)
    blk = Qwen3_5MoeSparseMoeBlock(cfg).double()
    with torch.no_grad():
        blk.gate.weight.copy_(torch.from_numpy(p["gate"]))
        blk.experts.gate_up_proj.copy_(torch.from_numpy(p["gu_dense"]))
        blk.experts.down_proj.copy_(torch.from_numpy(p["dn_dense"]))
        blk.shared_expert.gate_proj.weight.copy_(torch.from_numpy(p["shared_gate_proj"]))
        blk.shared_expert.up_proj.weight.copy_(torch.from_numpy(p["shared_up_proj"]))
        blk.shared_expert.down_proj.weight.copy_(torch.from_numpy(p["shared_down_proj"]))
        blk.shared_expert_gate.weight.copy_(torch.from_numpy(p["shared_expert_gate"]))
    return blk


def test_general_f32_reference_parity_config_matches_transformers():
    """The reference's float32 packed-expert parity configuration: the oracle's packed flow, its
    dense flow on the dequantized stacks, and its run-every-expert form agree within the
    reference's own 1e-4 gate, and all three match transformers' float64 Qwen3.5-MoE block on
    the same dequantized weights to float32 accuracy."""
    rng = np.random.default_rng(3)
    E, H, I, Is, k = 8, 32, 64, 64, 3
    p = _f32_layer(rng, E=E, H=H, I=I, Is=Is)
    q = _dense_of(p, H, I)
    x = _f32(rng.standard_normal((9, H)))
    y_pack, gi = om.moe_forward_general(x, p, k=k, inter=I)
    y_dense, _ = om.moe_forward_general(x, q, k=k, inter=I)
    y_all, _ = om.moe_forward_general(x, q, k=k, inter=I, dense_all=True)
    assert gi["routed_dtype"] == "f32"
    assert np.max(np.abs(y_pack - y_dense)) < 1e-4
    assert np.max(np.abs(y_dense - y_all)) < 1e-4
    blk = _hf_block(q, H, E, k, I, Is)
    with torch.no_grad():
        y_hf = blk(torch.from_numpy(x)[None])[0].numpy()
    scale = max(1.0, float(np.max(np.abs(y_hf))))
    for y in (y_pack, y_dense, y_all):
        assert np.max(np.abs(y - y_hf)) < 2e-5 * scale


@pytest.mark.parametrize("bits, gs", [(3, 32), (2, 32), (5, 32), (8, 64), (6, 128)])
def test_general_brute_force_loops(bits, gs):
    """Pure-Python loops (codes read bit by bit from the packed words, group index k // gs,
    slot-by-slot combine) equal the oracle's unrounded sum to float32 accuracy."""
    rng = np.random.default_rng(50 + bits)
    E, H, I, Is, k, N = 3, 128, 128, 32, 2, 2
    p = _f32_layer(rng, E=E, H=H, I=I, Is=Is, bits=bits, gs=gs)
    x = _f32(rng.standard_normal((N, H)))
    y, gi = om.moe_forward_general(x, p, k=k, inter=I)

    def code(words, e, o, kk):
        v = 0
        for b in range(bits):
            pos = kk * bits + b
            v |= ((int(words[e, o, pos // 32]) >> (pos % 32)) & 1) << b
        return v

    def wval(proj, e, o, kk):
        g = kk // gs
        return float(p[f"{proj}_scale"][e, o, g]) * code(p[f"{proj}_packed"], e, o, kk) + \
            float(p[f"{proj}_bias"][e, o, g])

    silu = lambda v: v / (1.0 + np.exp(-v))
    for t in range(N):
        idx, w = gi["idx"][t], gi["w"][t]
        routed = np.zeros(H)
        for s in range(k):
            e = int(idx[s])
            gu = [sum(float(x[t, kk]) * wval("gu", e, o, kk) for kk in range(H)) for o in range(2 * I)]
            h = [silu(gu[i]) * gu[I + i] for i in range(I)]
            for o in range(H):
                routed[o] += w[s] * sum(h[i] * wval("dn", e, o, i) for i in range(I))
        g = x[t] @ p["shared_gate_proj"].T
        u = x[t] @ p["shared_up_proj"].T
        sh = (silu(g) * u) @ p["shared_down_proj"].T
        sg = 1.0 / (1.0 + np.exp(-(x[t] @ p["shared_expert_gate"].reshape(-1))))
        want = routed + sh * sg
        assert np.max(np.abs(gi["y_exact"][t] - want)) < 1e-5 * max(1.0, np.max(np.abs(want)))


def test_general_rounding_points():
    """x float32 over bf16-scaled codes computes in float32 (x is not rounded: the promotion of
    the two dtypes); x float32 over bf16 dense stacks computes in bf16 (x cast to the stack's
    dtype, src/quanta/qwen35/moe.py:77); every intermediate is representable where it is
    materialised, and the output is cast to x's dtype."""
    rng = np.random.default_rng(60)
    E, H, I, k = 4, 64, 64, 2
    gu_w = (rng.standard_normal((E, 2 * I, H)) * 0.1).astype(np.float32)
    dn_w = (rng.standard_normal((E, H, I)) * 0.1).astype(np.float32)
    gq, dq = oq.quantize_rtn(gu_w, 4, 32), oq.quantize_rtn(dn_w, 4, 32)
    f = lambda b: oq.bf16_bits_to_f32(b).astype(np.float64)
    gate = _f32(rng.standard_normal((E, H)))
    p = dict(gate=gate, gu_packed=gq[0], gu_scale=f(gq[1]), gu_bias=f(gq[2]), dn_packed=dq[0],
             dn_scale=f(dq[1]), dn_bias=f(dq[2]), bits=4, group_size=32, sb_dtype="bf16")
    x = _f32(rng.standard_normal((5, H)))
    y, gi = om.moe_forward_general(x, p, k=k, inter=I, x_dtype="f32")
    assert gi["routed_dtype"] == "f32"
    for key in ("gu", "h", "d"):
        assert np.array_equal(_f32(gi[key]), gi[key])
    assert not np.array_equal(oq.round_bf16(gi["gu"]), gi["gu"])
    assert np.array_equal(_f32(y), y)
    q = dict(gate=gate, gu_dense=oq.round_bf16(gu_w), dn_dense=oq.round_bf16(dn_w), expert_dtype="bf16")
    y2, g2 = om.moe_forward_general(x, q, k=k, inter=I, x_dtype="f32")
    assert g2["routed_dtype"] == "bf16"
    for key in ("gu", "h", "d"):
        assert np.array_equal(oq.round_bf16(g2[key]), g2[key])
    # x rounded to bf16 first: the same routed products as bf16 x
    xb = oq.round_bf16(x)
    _, g3 = om.moe_forward_general(xb, q, k=k, inter=I, x_dtype="bf16")
    same = np.all(g2["idx"] == g3["idx"], axis=1)
    assert same.any()
    rows = np.repeat(same, k)
    assert np.array_equal(g2["gu"][rows], g3["gu"][rows])


def test_quantize_rtn_f32_error_bound():
    """The float32 test quantizer reconstructs each weight within half a step (plus float32
    rounding), with codes in range, and dequant_float reads its words back."""
    rng = np.random.default_rng(61)
    w = (rng.standard_normal((3, 16, 64)) * 0.2).astype(np.float32)
    for bits in (2, 3, 4, 5, 6, 8):
        packed, s, b, q = oq.quantize_rtn_f32(w, bits, 32)
        assert q.max() < (1 << bits)
        deq = oq.dequant_float(packed, s, b, 64, bits=bits, group_size=32)
        step = np.repeat(s.astype(np.float64), 32, axis=-1)
        assert np.all(np.abs(deq - w) <= 0.5 * step + 1e-6)
        # dequant_float of bf16-valued scales equals dequant_exact of their bits
        sb, bb = oq.f32_to_bf16_bits(s), oq.f32_to_bf16_bits(b)
        np.testing.assert_array_equal(
            oq.dequant_float(packed, oq.bf16_bits_to_f32(sb), oq.bf16_bits_to_f32(bb), 64, bits=bits,
                             group_size=32),
            oq.dequant_exact(packed, sb, bb, 64, bits=bits, group_size=32))


# ----------------------------------------------------------------------------- host dispatch


def _cfg(H=32, I=64, Is=64):
    from quanta_amd.moe import MoEConfig
    return MoEConfig(hidden_size=H, num_experts=8, num_experts_per_tok=3, moe_intermediate_size=I,
                     shared_expert_intermediate_size=Is)


def _params(H, I, Is, *, x_dtype=torch.bfloat16, packed=None, dense_dtype=torch.bfloat16,
            sh_dtype=torch.bfloat16):
    E = 8
    p = {"gate": torch.zeros(E, H, dtype=torch.bfloat16)}
    if packed is None:
        p["experts_gate_up"] = torch.zeros(E, 2 * I, H, dtype=dense_dtype)
        p["experts_down"] = torch.zeros(E, H, I, dtype=dense_dtype)
    else:
        bits, gs, sdt = packed
        mk = lambda rows, K: {"packed": torch.zeros(E, rows, K * bits // 32, dtype=torch.int32),
                              "scale": torch.zeros(E, rows, K // gs, dtype=sdt),
                              "bias": torch.zeros(E, rows, K // gs, dtype=sdt),
                              "group_size": gs, "bits": bits}
        p["experts_gate_up"], p["experts_down"] = mk(2 * I, H), mk(H, I)
    p["shared_gate_proj"] = torch.zeros(Is, H, dtype=sh_dtype)
    p["shared_up_proj"] = torch.zeros(Is, H, dtype=sh_dtype)
    p["shared_down_proj"] = torch.zeros(H, Is, dtype=sh_dtype)
    p["shared_expert_gate"] = torch.zeros(1, H, dtype=torch.bfloat16)
    return p, torch.zeros(1, 2, H, dtype=x_dtype)


@pytest.mark.parametrize("case, want", [
    (dict(H=256, I=128, Is=128, packed=(4, 64, torch.bfloat16)), False),
    (dict(H=256, I=128, Is=128, packed=(6, 128, torch.bfloat16)), False),
    (dict(H=256, I=128, Is=128), False),
    (dict(H=256, I=128, Is=128, packed=(4, 32, torch.bfloat16)), True),
    (dict(H=256, I=128, Is=128, packed=(4, 64, torch.float32)), True),
    (dict(H=256, I=128, Is=128, packed=(8, 64, torch.bfloat16)), True),
    (dict(H=256, I=128, Is=128, packed=(4, 64, torch.bfloat16), x_dtype=torch.float32), True),
    (dict(H=256, I=128, Is=128, dense_dtype=torch.float32), True),
    (dict(H=256, I=128, Is=128, sh_dtype=torch.float32), True),
    (dict(H=32, I=64, Is=64, packed=(4, 32, torch.float32), x_dtype=torch.float32), True),
    (dict(H=96, I=128, Is=128, packed=(4, 32, torch.bfloat16)), True),
    (dict(H=256, I=64, Is=128), True),
])
def test_needs_general_routes_formats(case, want):
    """The tiled kernels take bf16 activations over bf16-scaled int3/int4/int6 g64/g128 codes or
    bf16 stacks at multiples of 128; anything else goes to the reference-dtype path."""
    from quanta_amd.moe import needs_general
    H, I, Is = case.pop("H"), case.pop("I"), case.pop("Is")
    p, x = _params(H, I, Is, **case)
    assert needs_general(x, p, _cfg(H, I, Is)) is want


def test_qwen35_moe_refuses_other_activation_dtypes():
    from quanta_amd.moe import qwen35_moe
    p, _ = _params(256, 128, 128)
    with pytest.raises(TypeError, match="bf16 or float32"):
        qwen35_moe(torch.zeros(1, 2, 256, dtype=torch.float16), p, _cfg(256, 128, 128))
