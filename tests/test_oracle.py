"""CPU tier: pin the oracle (oracle/) against independent checks, and the product's host-side
format code (quanta_amd.quant) against the oracle.

No reference golden vectors exist for this path (the reference's MoE gates regenerate their data
from mx.random and need a live MLX, which is absent), so every oracle function is pinned here by
something that does not share its code: exact rational arithmetic, brute force on tiny inputs,
bit-level known answers, torch/scipy library routines, invariants, special cases that reduce to a
dense product, and transformers' own (third-party) DeepSeek-V3 and Qwen3.5-MoE modules.
"""

from __future__ import annotations

import itertools
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq

# ----------------------------------------------------------------------------------- bf16


def _rne_bf16_fraction(v: Fraction) -> Fraction:
    """Round an exact rational to the nearest bf16 value (ties to even), normal range only."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** (e - 7)
    q, r = divmod(a, ulp)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return sign * q * ulp


def _rne_f32_fraction(v: Fraction) -> Fraction:
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(a, ulp)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return sign * q * ulp


def test_bf16_known_answers():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.0, 0.0, np.inf, np.nan], np.float32)
    bits = oq.f32_to_bf16_bits(vals)
    assert bits[0] == 0x3F80
    assert bits[1] == 0x3F80          # halfway, ties to even (down)
    assert bits[2] == 0x3F82          # halfway, ties to even (up)
    assert bits[3] == 0xC000
    assert bits[4] == 0x0000
    assert bits[5] == 0x7F80
    assert bits[6] == 0x7FC0


def test_bf16_matches_torch_rne():
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(100_000) * 10.0 ** rng.integers(-6, 6, 100_000)).astype(np.float32)
    ours = oq.f32_to_bf16_bits(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
    assert np.array_equal(ours, ref)


# ----------------------------------------------------------------------------------- pack / unpack


def test_pack_int4_known_answer():
    codes = np.array([[0, 1, 2, 3, 4, 5, 6, 7, 15, 15, 15, 15, 15, 15, 15, 15]], np.uint32)
    w = oq.pack_affine(codes, 4)
    assert w.tolist() == [[0x76543210, 0xFFFFFFFF]]


def _brute_pack(codes, bits):
    out = []
    for row in codes:
        stream = []
        for c in row:
            stream += [(int(c) >> b) & 1 for b in range(bits)]
        out.append([sum(stream[32 * w + j] << j for j in range(32)) for w in range(len(stream) // 32)])
    return np.array(out, dtype=np.uint64).astype(np.uint32)


@pytest.mark.parametrize("bits", [2, 3, 4, 6, 8])
def test_pack_unpack_brute_force_and_roundtrip(bits):
    rng = np.random.default_rng(bits)
    n_in = 64 if bits in (2, 4, 8) else 96
    codes = rng.integers(0, 1 << bits, size=(5, n_in)).astype(np.uint32)
    packed = oq.pack_affine(codes, bits)
    assert np.array_equal(packed, _brute_pack(codes, bits))
    assert np.array_equal(oq.unpack_affine(packed, n_in, bits), codes)


def test_unpack_int4_fast_equals_general():
    rng = np.random.default_rng(3)
    words = rng.integers(0, 2 ** 32, size=(7, 3, 16), dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(oq.unpack_int4_fast(words, 128), oq.unpack_affine(words, 128, 4))


@pytest.mark.parametrize("bits", [2, 3, 4, 6, 8])
def test_product_pack_matches_oracle(bits):
    from quanta_amd import quant as q

    rng = np.random.default_rng(10 + bits)
    n_in = 128 if bits in (2, 4, 8) else 96
    codes = rng.integers(0, 1 << bits, size=(3, 4, n_in)).astype(np.uint32)
    ours = q.pack_affine(torch.from_numpy(codes.astype(np.int64)), bits).numpy().view(np.uint32)
    assert np.array_equal(ours, oq.pack_affine(codes, bits))
    back = q.unpack_affine(torch.from_numpy(ours.view(np.int32)), n_in, bits).numpy()
    assert np.array_equal(back.astype(np.uint32), codes)


# ----------------------------------------------------------------------------------- quantize / dequant


def test_quantizer_error_bound_and_product_equality():
    from quanta_amd import quant as q

    rng = np.random.default_rng(4)
    w = (rng.standard_normal((6, 256)) * 0.02).astype(np.float32)
    packed, s_bits, b_bits, codes = oq.quantize_rtn(w, 4, 64)
    assert codes.max() <= 15
    deq = oq.dequant_exact(packed, s_bits, b_bits, 256)
    wb = oq.bf16_bits_to_f32(oq.f32_to_bf16_bits(w)).astype(np.float64)
    s = np.repeat(oq.bf16_bits_to_f32(s_bits).astype(np.float64), 64, axis=-1)
    # RTN: within half a step (plus the bf16 rounding of scale/bias, which can push the
    # top code's reconstruction one bf16 step of the bias away)
    assert np.all(np.abs(deq - wb) <= 0.5 * s * (1 + 2 ** -6) + np.abs(wb) * 2 ** -7 + 1e-12)
    qp, qs, qb = q.quantize_affine(torch.from_numpy(w), 4, 64, scale_dtype=torch.bfloat16)
    assert np.array_equal(qp.numpy().view(np.uint32), packed)
    assert np.array_equal(qs.view(torch.int16).numpy().astype(np.uint16), s_bits)
    assert np.array_equal(qb.view(torch.int16).numpy().astype(np.uint16), b_bits)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_exact_rational(bits):
    """bf16(fp32(s)*q + fp32(b)) checked with exact rationals (independent of numpy rounding)."""
    rng = np.random.default_rng(5 + bits)
    w = (rng.standard_normal((3, 128)) * 0.05).astype(np.float32)
    packed, s_bits, b_bits, codes = oq.quantize_rtn(w, bits, 64)
    got = oq.dequant_bf16_bits(packed, s_bits, b_bits, 128, bits=bits)
    sf = oq.bf16_bits_to_f32(s_bits)
    bf = oq.bf16_bits_to_f32(b_bits)
    for r, c in itertools.product(range(3), range(128)):
        g = c // 64
        exact = Fraction(float(sf[r, g])) * int(codes[r, c]) + Fraction(float(bf[r, g]))
        want = _rne_bf16_fraction(_rne_f32_fraction(exact))
        assert Fraction(float(oq.bf16_bits_to_f32(got[r, c]))) == want, (r, c)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_special_codes(bits):
    top = (1 << bits) - 1
    s_bits = oq.f32_to_bf16_bits(np.full((1, 1), 0.0625, np.float32))
    b_bits = oq.f32_to_bf16_bits(np.full((1, 1), -0.5, np.float32))
    codes = np.array([[0] * 32 + [top] * 32], np.uint32)
    words = oq.pack_affine(codes, bits)
    vals = oq.bf16_bits_to_f32(oq.dequant_bf16_bits(words, s_bits, b_bits, 64, bits=bits))
    assert np.all(vals[0, :32] == -0.5) and np.all(vals[0, 32:] == top * 0.0625 - 0.5)


# ----------------------------------------------------------------------------------- routing


def _brute_route(x, wr, k, scoring, bias=None, n_group=1, topk_group=1, norm=True, scale=1.0,
                 norm_single=True):
    out_idx, out_w = [], []
    for t in range(x.shape[0]):
        logit = [float(np.dot(x[t].astype(np.float64), wr[e].astype(np.float64)))
                 for e in range(wr.shape[0])]
        if scoring == "softmax":
            m = max(logit)
            ex = [np.exp(v - m) for v in logit]
            sc = [v / sum(ex) for v in ex]
        else:
            sc = [1 / (1 + np.exp(-v)) for v in logit]
        ch = [sc[e] + (bias[e] if bias is not None else 0.0) for e in range(len(sc))]
        allowed = set(range(len(sc)))
        if n_group > 1:
            gs = len(sc) // n_group
            gscore = [sum(sorted(ch[g * gs:(g + 1) * gs])[-2:]) for g in range(n_group)]
            keep = sorted(range(n_group), key=lambda g: (-gscore[g], g))[:topk_group]
            allowed = {e for e in range(len(sc)) if e // gs in keep}
        sel = sorted(allowed, key=lambda e: (-ch[e], e))[:k]
        w = [sc[e] for e in sel]
        if norm and (len(sel) > 1 or norm_single):
            tot = sum(w) + 1e-20
            w = [v / tot for v in w]
        out_idx.append(sel)
        out_w.append([v * scale for v in w])
    return np.array(out_idx), np.array(out_w)


@pytest.mark.parametrize("case", [
    dict(scoring="softmax"),
    dict(scoring="sigmoid"),
    dict(scoring="sigmoid", bias=True, n_group=4, topk_group=2, scale=2.5),
    dict(scoring="sigmoid", bias=True, norm=False),
    # k = 1: qwen35_route divides the single weight by itself, a MoEGate keeps the score
    dict(scoring="softmax", k=1),
    dict(scoring="sigmoid", bias=True, scale=2.5, k=1, norm_single=False),
    dict(scoring="sigmoid", bias=True, scale=2.5, k=1, norm_single=True),
])
def test_route_brute_force(case):
    rng = np.random.default_rng(6)
    E, H, N = 16, 24, 9
    k = case.get("k", 3)
    x = rng.standard_normal((N, H))
    wr = rng.standard_normal((E, H)) * 0.3
    bias = rng.standard_normal(E) * 0.1 if case.get("bias") else None
    kw = dict(scoring=case["scoring"], bias=bias, n_group=case.get("n_group", 1),
              topk_group=case.get("topk_group", 1), norm=case.get("norm", True),
              scale=case.get("scale", 1.0), norm_single=case.get("norm_single", True))
    bi, bw = _brute_route(x, wr, k, **kw)
    idx, w, *_ = om.route(x, wr, k=k, scoring=kw["scoring"], norm_topk=kw["norm"], bias=bias,
                          n_group=kw["n_group"], topk_group=kw["topk_group"], scale=kw["scale"],
                          norm_single=kw["norm_single"])
    assert np.array_equal(idx, bi)
    assert np.allclose(w, bw, rtol=1e-12, atol=0)
    if k == 1 and kw["norm"]:
        # closed forms: a renormalised single weight is 1 (times the scale); a kept score is
        # sigmoid(x . wr[e]) times the scale
        if kw["norm_single"]:
            assert np.allclose(w, kw["scale"], rtol=1e-12)
        else:
            want = kw["scale"] / (1 + np.exp(-np.einsum("nh,nh->n", x, wr[idx[:, 0]])))
            assert np.allclose(w[:, 0], want, rtol=1e-12)


def test_route_softmax_matches_torch_topk():
    from scipy.special import softmax

    rng = np.random.default_rng(7)
    x = rng.standard_normal((64, 128))
    wr = rng.standard_normal((64, 128)) * 0.02
    idx, w, logits, scores, _ = om.route(x, wr, k=8, scoring="softmax")
    assert np.allclose(scores, softmax(x @ wr.T, axis=-1), rtol=1e-12)
    tv, ti = torch.topk(torch.from_numpy(scores), 8, dim=-1)
    assert all(set(a) == set(b) for a, b in zip(idx.tolist(), ti.numpy().tolist()))
    assert np.allclose(w, (tv / tv.sum(-1, keepdim=True)).numpy(), rtol=1e-12)


def test_group_route_matches_transformers_deepseek_v3():
    tf = pytest.importorskip("transformers")
    from transformers.models.deepseek_v3.configuration_deepseek_v3 import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter

    E, H, N, k = 32, 48, 40, 4
    cfg = DeepseekV3Config(hidden_size=H, n_routed_experts=E, num_experts_per_tok=k, n_group=8,
                           topk_group=3, norm_topk_prob=True, routed_scaling_factor=2.5)
    router = DeepseekV3TopkRouter(cfg).double()
    rng = np.random.default_rng(8)
    wr = rng.standard_normal((E, H)) * 0.2
    bias = rng.standard_normal(E) * 0.05
    with torch.no_grad():
        router.weight.copy_(torch.from_numpy(wr))
        router.e_score_correction_bias.copy_(torch.from_numpy(bias))
    x = rng.standard_normal((N, H))
    with torch.no_grad():
        out = router(torch.from_numpy(x))
    tw, ti = out[1].numpy(), out[2].numpy()
    idx, w, *_ = om.route(x, wr, k=k, scoring="sigmoid", bias=bias, n_group=8, topk_group=3,
                          scale=2.5)
    for t in range(N):
        assert set(idx[t]) == set(ti[t])
        d_ours = dict(zip(idx[t], w[t]))
        for e, v in zip(ti[t], tw[t]):   # transformers' router evaluates in float32
            assert abs(d_ours[e] - v) < 1e-6 * max(1.0, abs(v))


# ----------------------------------------------------------------------------------- permute


def test_permute_brute_force_and_invariants():
    rng = np.random.default_rng(9)
    N, k, E = 37, 5, 13
    idx = np.stack([rng.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    counts, offsets, order, inv = om.permute(idx, E)
    exp = idx.reshape(-1)
    brute = sorted(range(N * k), key=lambda m: (exp[m], m))
    assert order.tolist() == brute
    assert offsets[-1] == N * k and np.array_equal(np.diff(offsets), counts)
    assert np.array_equal(inv[order], np.arange(N * k))
    assert np.array_equal(counts, np.bincount(exp, minlength=E))


# ----------------------------------------------------------------------------------- expert math


def _tiny_layer(rng, E=6, H=128, I=64, Is=64, gated=True):
    gu_w = (rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float32)
    dn_w = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    gq = oq.quantize_rtn(gu_w, 4, 64)
    dq = oq.quantize_rtn(dn_w, 4, 64)
    bf = lambda a: oq.bf16_bits_to_f32(oq.f32_to_bf16_bits(a)).astype(np.float64)
    p = dict(gate=bf(rng.standard_normal((E, H)) * 0.1),
             gu_packed=gq[0], gu_scale=gq[1], gu_bias=gq[2],
             dn_packed=dq[0], dn_scale=dq[1], dn_bias=dq[2])
    if Is:
        p.update(shared_gate_proj=bf(rng.standard_normal((Is, H)) * 0.05),
                 shared_up_proj=bf(rng.standard_normal((Is, H)) * 0.05),
                 shared_down_proj=bf(rng.standard_normal((H, Is)) * 0.05))
        if gated:
            p["shared_expert_gate"] = bf(rng.standard_normal((1, H)) * 0.1)
    return p


def test_gather_qmm_matches_explicit_loop():
    rng = np.random.default_rng(11)
    p = _tiny_layer(rng, E=3, H=128, I=64)
    x = oq.round_bf16(rng.standard_normal((5, 128)))
    ex = np.array([2, 0, 1, 2, 0])
    got = om.gather_qmm(x, ex, p["gu_packed"], p["gu_scale"], p["gu_bias"], 128, round_out=False)
    codes = oq.unpack_affine(p["gu_packed"], 128, 4)
    s = oq.bf16_bits_to_f32(p["gu_scale"])
    b = oq.bf16_bits_to_f32(p["gu_bias"])
    for m in range(5):
        for o in range(0, 128, 17):
            acc = 0.0
            for kk in range(128):
                acc += float(x[m, kk]) * (float(s[ex[m], o, kk // 64]) * int(codes[ex[m], o, kk])
                                          + float(b[ex[m], o, kk // 64]))
            assert abs(got[m, o] - acc) < 1e-9


def test_sparse_equals_dense_when_k_equals_E():
    """k = E: the sparse gather path equals the run-every-expert oracle (special case that reduces
    to dense per-expert products, src/quanta/qwen35/moe.py:127-142)."""
    rng = np.random.default_rng(12)
    E, H, I = 4, 128, 64
    p = _tiny_layer(rng, E=E, H=H, I=I, Is=0)
    x = oq.round_bf16(rng.standard_normal((6, H)))
    idx, w, *_ = om.route(x, p["gate"], k=E)
    gu_d = oq.dequant_exact(p["gu_packed"], p["gu_scale"], p["gu_bias"], H)
    dn_d = oq.dequant_exact(p["dn_packed"], p["dn_scale"], p["dn_bias"], I)
    dense = om.moe_dense_reference(x, idx, w, gu_d, dn_d, I)
    exp = idx.reshape(-1)
    tok = np.repeat(np.arange(6), E)
    gu = om.gather_qmm(x[tok], exp, p["gu_packed"], p["gu_scale"], p["gu_bias"], H, round_out=False)
    hh = gu[:, :I] / (1 + np.exp(-gu[:, :I])) * gu[:, I:]
    d = om.gather_qmm(hh, exp, p["dn_packed"], p["dn_scale"], p["dn_bias"], I, round_out=False)
    assert np.allclose(om.combine(d, w), dense, rtol=1e-10, atol=1e-12)


def test_block_matches_transformers_qwen35_moe():
    """The oracle's routing + expert + gated-shared structure equals transformers' independent
    Qwen3.5-MoE sparse block (float64, dequantized weights). The oracle's bf16 materialisation
    points are disabled by comparing its unrounded dense reference path plus shared expert."""
    pytest.importorskip("transformers")
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeSparseMoeBlock

    rng = np.random.default_rng(13)
    E, H, I, Is, k, N = 8, 128, 64, 64, 3, 7
    p = _tiny_layer(rng, E=E, H=H, I=I, Is=Is)
    cfg = Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k,
                               moe_intermediate_size=I, shared_expert_intermediate_size=Is)
    blk = Qwen3_5MoeSparseMoeBlock(cfg).double()
    gu_d = oq.dequant_exact(p["gu_packed"], p["gu_scale"], p["gu_bias"], H)
    dn_d = oq.dequant_exact(p["dn_packed"], p["dn_scale"], p["dn_bias"], I)
    with torch.no_grad():
        blk.gate.weight.copy_(torch.from_numpy(p["gate"]))
        blk.experts.gate_up_proj.copy_(torch.from_numpy(gu_d))
        blk.experts.down_proj.copy_(torch.from_numpy(dn_d))
        blk.shared_expert.gate_proj.weight.copy_(torch.from_numpy(p["shared_gate_proj"]))
        blk.shared_expert.up_proj.weight.copy_(torch.from_numpy(p["shared_up_proj"]))
        blk.shared_expert.down_proj.weight.copy_(torch.from_numpy(p["shared_down_proj"]))
        blk.shared_expert_gate.weight.copy_(torch.from_numpy(p["shared_expert_gate"]))
    x = oq.round_bf16(rng.standard_normal((N, H)))
    with torch.no_grad():
        y_hf = blk(torch.from_numpy(x)[None])[0].numpy()
    idx, w, *_ = om.route(x, p["gate"], k=k)
    routed = om.moe_dense_reference(x, idx, w, gu_d, dn_d, I)
    g = x @ p["shared_gate_proj"].T
    u = x @ p["shared_up_proj"].T
    sh = ((g / (1 + np.exp(-g))) * u) @ p["shared_down_proj"].T
    sg = 1 / (1 + np.exp(-(x @ p["shared_expert_gate"].reshape(-1))))
    y = routed + sh * sg[:, None]
    # transformers' router evaluates its softmax in float32; everything else is float64
    assert np.allclose(y, y_hf, rtol=1e-6, atol=1e-7)
    with torch.no_grad():
        _, _, hf_idx = blk.gate(torch.from_numpy(x))
    assert all(set(a) == set(b) for a, b in zip(idx.tolist(), hf_idx.numpy().tolist()))
    # and the bf16-materialising oracle stays within bf16 distance of the exact block
    y_bf, _ = om.moe_forward(x, p, k=k, inter=I)
    assert np.max(np.abs(y_bf - y)) < 2e-2 * max(1.0, np.max(np.abs(y)))


def test_route_margin_flags_ties():
    choice = np.array([[3.0, 1.0, 1.0, 0.5], [4.0, 3.0, 2.0, 1.0]])
    m = om.route_margin(choice, 2)
    assert m[0] == 0.0 and m[1] == 1.0


# ----------------------------------------------------------------------------- layer norm
def test_rmsnorm_matches_torch_rms_norm():
    """oracle rmsnorm == torch.nn.functional.rms_norm (float64), i.e. x * rsqrt(mean(x^2) + eps)
    * w over the last dim; a dropped eps, a sum in place of the mean or the weight applied twice
    all fail here."""
    rng = np.random.default_rng(11)
    for H, eps in ((64, 1e-6), (4096, 1e-6), (96, 0.5)):
        x = oq.round_bf16(rng.standard_normal((7, H)) * 3.0)
        w = oq.round_bf16(1.0 + 0.1 * rng.standard_normal(H))
        want = torch.nn.functional.rms_norm(torch.from_numpy(x), (H,), weight=torch.from_numpy(w),
                                            eps=eps).numpy()
        np.testing.assert_allclose(om.rmsnorm(x, w, eps), want, rtol=1e-12, atol=1e-12)


def test_rmsnorm_closed_forms():
    """A constant row c gives w * c / sqrt(c^2 + eps); with eps = 0 the norm is invariant under
    positive scaling of the row and every normalised row has mean square 1 (w = 1)."""
    c, eps = -2.5, 1e-2
    w = np.array([1.0, 0.5, 2.0, -1.0])
    got = om.rmsnorm(np.full((1, 4), c), w, eps)
    np.testing.assert_allclose(got, w[None] * c / np.sqrt(c * c + eps), rtol=1e-15)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 33))
    ones = np.ones(33)
    np.testing.assert_allclose(om.rmsnorm(7.25 * x, ones, 0.0), om.rmsnorm(x, ones, 0.0), rtol=1e-13)
    np.testing.assert_allclose(np.mean(om.rmsnorm(x, ones, 0.0) ** 2, axis=-1), 1.0, rtol=1e-13)


def test_residual_add_rounds_once():
    """bf16 + bf16 rounds once to bf16: exact sums stay, a tie rounds to even."""
    a = np.array([1.0, 1.0, 256.0])
    b = np.array([2.0, 2.0 ** -8, 1.0])     # 1 + 2^-8: tie between 1 and 1+2^-7 -> 1 (even)
    np.testing.assert_array_equal(om.residual_add(a, b), [3.0, 1.0, 256.0])


# ----------------------------------------------------------------------------- gated activations
def test_swigluoai_matches_transformers_gpt_oss():
    """glu("swigluoai") == transformers GptOssExperts._apply_gate (float64), which the reference's
    swigluoai is written against (src/quanta/minimax/model_m3.py:112-128). GPT-OSS interleaves
    gate/up columns; the reference (and this build) splits halves, so the input is interleaved
    for transformers and the halves compared."""
    from types import SimpleNamespace

    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts

    rng = np.random.default_rng(21)
    g = oq.round_bf16(rng.standard_normal((6, 40)) * 6.0)
    u = oq.round_bf16(rng.standard_normal((6, 40)) * 6.0)
    inter = np.empty((6, 80))
    inter[:, ::2], inter[:, 1::2] = g, u
    want = GptOssExperts._apply_gate(SimpleNamespace(alpha=1.702, limit=7.0),
                                     torch.from_numpy(inter)).numpy()
    np.testing.assert_allclose(om.glu(g, u, "swigluoai", 1.702, 7.0), want, rtol=1e-12, atol=1e-12)
    assert np.any(g > 7.0) and np.any(np.abs(u) > 7.0)       # the clamps are exercised


def test_clamped_silu_known_answers():
    """The DeepSeek-V4 clamp (src/quanta/dsv4/moe.py:74-77): the gate is clamped from above only,
    the up branch both ways; limit 0 is the plain silu(g) * u."""
    g = np.array([10.0, -10.0, 3.0])
    u = np.array([10.0, -10.0, 0.5])
    L = 7.0
    silu = lambda v: v / (1.0 + np.exp(-v))
    np.testing.assert_allclose(om.glu(g, u, "silu", limit=L),
                               [silu(7.0) * 7.0, silu(-10.0) * -7.0, silu(3.0) * 0.5], rtol=1e-15)
    np.testing.assert_allclose(om.glu(g, u, "silu", limit=0.0), silu(g) * u, rtol=1e-15)
    np.testing.assert_allclose(om.glu(g, u, "swigluoai", 1.0, 0.0), silu(g) * (u + 1.0), rtol=1e-15)


def test_dequant_group128_explicit_loop():
    """group_size 128 (Kimi's stacks, src/quanta/modeling/quantized.py:29-34): one (scale, bias)
    per 128 codes, checked element by element."""
    rng = np.random.default_rng(8)
    rows, K = 3, 256
    codes = rng.integers(0, 16, size=(rows, K))
    words = oq.pack_affine(codes, 4)
    sb = oq.f32_to_bf16_bits(rng.standard_normal((rows, K // 128)).astype(np.float32) * 0.1)
    bb = oq.f32_to_bf16_bits(rng.standard_normal((rows, K // 128)).astype(np.float32))
    got = oq.dequant_exact(words, sb, bb, K, group_size=128)
    s, b = oq.bf16_bits_to_f32(sb).astype(np.float64), oq.bf16_bits_to_f32(bb).astype(np.float64)
    for r in range(rows):
        for k in range(K):
            assert got[r, k] == s[r, k // 128] * codes[r, k] + b[r, k // 128]


def test_dequant_int6_explicit_loop():
    """int6 codes (MiniMax M3's expert format, src/quanta/minimax/model_m3.py:414-450) packed as the
    LSB-first bitstream (src/quanta/bake/quant.py:48-63; pack_affine is pinned bit by bit above),
    dequantized element by element for groups of 64 and 128."""
    rng = np.random.default_rng(6)
    rows, K = 2, 256
    codes = rng.integers(0, 64, size=(rows, K))
    words = oq.pack_affine(codes, 6)
    assert words.shape == (rows, K * 6 // 32)
    for gs in (64, 128):
        sb = oq.f32_to_bf16_bits(rng.standard_normal((rows, K // gs)).astype(np.float32) * 0.1)
        bb = oq.f32_to_bf16_bits(rng.standard_normal((rows, K // gs)).astype(np.float32))
        got = oq.dequant_exact(words, sb, bb, K, bits=6, group_size=gs)
        s, b = oq.bf16_bits_to_f32(sb).astype(np.float64), oq.bf16_bits_to_f32(bb).astype(np.float64)
        for r in range(rows):
            for k in range(K):
                assert got[r, k] == s[r, k // gs] * codes[r, k] + b[r, k // gs]


def test_dequant_int3_explicit_loop():
    """int3 codes (Kimi's gate/up width, src/quanta/modeling/quantized.py:4-7) packed as the
    LSB-first bitstream (codes straddle word boundaries: code 10 holds bits 30..32), dequantized
    element by element for groups of 64 and 128."""
    rng = np.random.default_rng(3)
    rows, K = 2, 256
    codes = rng.integers(0, 8, size=(rows, K))
    words = oq.pack_affine(codes, 3)
    assert words.shape == (rows, K * 3 // 32)
    # code 10 of row 0: bits 30, 31 of word 0 and bit 0 of word 1
    c10 = ((int(words[0, 0]) >> 30) & 3) | ((int(words[0, 1]) & 1) << 2)
    assert c10 == codes[0, 10]
    for gs in (64, 128):
        sb = oq.f32_to_bf16_bits(rng.standard_normal((rows, K // gs)).astype(np.float32) * 0.1)
        bb = oq.f32_to_bf16_bits(rng.standard_normal((rows, K // gs)).astype(np.float32))
        got = oq.dequant_exact(words, sb, bb, K, bits=3, group_size=gs)
        s, b = oq.bf16_bits_to_f32(sb).astype(np.float64), oq.bf16_bits_to_f32(bb).astype(np.float64)
        for r in range(rows):
            for k in range(K):
                assert got[r, k] == s[r, k // gs] * codes[r, k] + b[r, k // gs]


# ----------------------------------------------------------------------------------- AWQ scales


def test_awq_divide_is_fp32_division_rounded_to_bf16():
    """awq_divide (float64 quotient -> fp32 -> bf16) against numpy's IEEE float32 division then
    the bf16 rounding, over every finite bf16 numerator and a spread of positive bf16 scales."""
    num = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    num = num[np.isfinite(oq.bf16_bits_to_f32(num))]
    rng = np.random.default_rng(0)
    den = oq.f32_to_bf16_bits((2.0 ** rng.uniform(-6, 6, 96)).astype(np.float32))
    x = oq.bf16_bits_to_f32(num)[:, None].astype(np.float32)
    s = oq.bf16_bits_to_f32(den)[None, :].astype(np.float32)
    with np.errstate(over="ignore", under="ignore"):
        want = oq.bf16_bits_to_f32(oq.f32_to_bf16_bits(x / s))
        got = om.awq_divide(x.astype(np.float64), s.astype(np.float64))
    assert np.array_equal(got.astype(np.float32), want, equal_nan=True)


def _awq_case(seed, E=4, H=128, I=128):
    rng = np.random.default_rng(seed)
    gu_w = rng.standard_normal((E, 2 * I, H)) * 0.05
    dn_w = rng.standard_normal((E, H, I)) * 0.05
    p = {}
    for pre, w in (("gu", gu_w), ("dn", dn_w)):
        packed, sb, bb, _ = oq.quantize_rtn(w, 4, 64)
        p[f"{pre}_packed"], p[f"{pre}_scale"], p[f"{pre}_bias"] = packed, sb, bb
    x = oq.round_bf16(rng.standard_normal((6, H)))
    exp = rng.integers(0, E, 6)
    return p, x, exp, rng


def test_awq_rows_reduce_to_the_plain_path_with_unit_scales():
    p, x, exp, _ = _awq_case(1)
    E, I, H = 4, 128, 128
    q = dict(p, gu_awq=np.ones((E, 2, H)), dn_awq=np.ones((E, I)))
    gu, h = om.awq_expert_rows(x, exp, q, I, H, act="silu", limit=7.0)
    gu_plain = om.gather_qmm(x, exp, p["gu_packed"], p["gu_scale"], p["gu_bias"], H)
    assert np.array_equal(gu, gu_plain)
    assert np.array_equal(h, om.swiglu(gu_plain, I, "silu", limit=7.0))


def test_awq_rows_power_of_two_scales():
    """Scales 2^j per (expert, projection) divide exactly and commute with bf16 rounding, so
    g, u and h are the unit-scale values times 2^-j: pins which half of the gate_up stack takes
    which scale row and that every row takes its own expert's scales."""
    p, x, exp, rng = _awq_case(2)
    E, I, H = 4, 128, 128
    jg = rng.integers(-3, 4, (E, 2))
    jd = rng.integers(-3, 4, E)
    s_gu = np.broadcast_to((2.0 ** jg)[:, :, None], (E, 2, H)).copy()
    s_dn = np.broadcast_to((2.0 ** jd)[:, None], (E, I)).copy()
    gu, h = om.awq_expert_rows(x, exp, dict(p, gu_awq=s_gu, dn_awq=s_dn), I, H)
    gu1, _ = om.awq_expert_rows(x, exp, dict(p, gu_awq=np.ones((E, 2, H)), dn_awq=np.ones((E, I))), I, H)
    assert np.array_equal(gu[:, :I], gu1[:, :I] * 2.0 ** -jg[exp, 0][:, None])
    assert np.array_equal(gu[:, I:], gu1[:, I:] * 2.0 ** -jg[exp, 1][:, None])
    want_h = oq.round_bf16(om.glu(gu[:, :I], gu[:, I:])) * 2.0 ** -jd[exp][:, None]
    assert np.array_equal(h, want_h)


# ----------------------------------------------------------------------------------- mixed widths


def test_mixed_proj_widths_and_slots():
    """mixed_proj against a per-row loop: each row's expert picks its width's stack and its slot in
    it (slots permuted, so a slot/expert mix-up fails); with one width and identity slots it is
    gather_qmm on that stack."""
    rng = np.random.default_rng(8)
    E, rows, K, gs = 6, 32, 256, 128
    pbits = np.array([3, 4, 4, 3, 6, 4])
    stacks, pslot = {}, np.zeros(E, np.int64)
    for b in (3, 4, 6):
        ids = np.flatnonzero(pbits == b)
        perm = rng.permutation(ids.size)
        pslot[ids] = perm
        w = rng.standard_normal((ids.size, rows, K)) * 0.05
        packed, sb, bb, _ = oq.quantize_rtn(w, b, gs)
        stacks[b] = (packed, sb, bb)
    m = {"stacks": {"gate": stacks}, "pbits": {"gate": pbits}, "pslot": {"gate": pslot}, "group_size": gs}
    x = oq.round_bf16(rng.standard_normal((9, K)))
    exp = rng.integers(0, E, 9)
    got = om.mixed_proj(x, exp, m, "gate", K)
    for r in range(9):
        e = exp[r]
        packed, sb, bb = stacks[pbits[e]]
        w = oq.dequant_exact(packed[pslot[e]], sb[pslot[e]], bb[pslot[e]], K, bits=int(pbits[e]), group_size=gs)
        assert np.array_equal(got[r], oq.round_bf16(w @ x[r]))
    uni = {"stacks": {"gate": {4: stacks[4]}}, "pbits": {"gate": np.full(2, 4)},
           "pslot": {"gate": np.arange(2)}, "group_size": gs}
    e2 = rng.integers(0, 2, 5)
    assert np.array_equal(om.mixed_proj(x[:5], e2, uni, "gate", K),
                          om.gather_qmm(x[:5], e2, *stacks[4], K, group_size=gs, bits=4))


def test_route_sqrtsoftplus_matches_torch_softplus():
    """DeepSeek-V4's scores sqrt(softplus(logits)) against torch's softplus, and the selection
    on score + bias with the bias-free, renormalised, scaled weights (src/quanta/dsv4/moe.py:37-57),
    including large logits where log(1 + e^l) must not overflow."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((7, 64))
    wr = rng.standard_normal((32, 64)) * 0.3
    wr[3] *= 400.0                      # logits of several hundred for expert 3
    bias = rng.standard_normal(32) * 0.1
    idx, w, logits, scores, choice = om.route(x, wr, k=4, scoring="sqrtsoftplus", bias=bias, scale=1.5)
    want = torch.sqrt(torch.nn.functional.softplus(torch.from_numpy(logits))).numpy()
    assert np.all(np.isfinite(scores))
    assert np.allclose(scores, want, rtol=1e-12, atol=0)
    for r in range(7):
        order = sorted(range(32), key=lambda e: (-(scores[r, e] + bias[e]), e))[:4]
        assert list(idx[r]) == order
        sel = scores[r, order]
        assert np.allclose(w[r], sel / (sel.sum() + 1e-20) * 1.5, rtol=1e-14)


def test_shared_weight_int8_triplet():
    """oracle.moe.shared_weight: an int8 shared-expert triplet becomes the bf16 matrix of its
    dequant (codes 0 and 255 at the closed forms b and 255 s + b; random codes at the rounding
    pinned by test_dequant_exact_rational), bf16 values pass through, and the block with the
    triplets equals the block with their dequantized matrices."""
    s_bits = oq.f32_to_bf16_bits(np.array([[0.0078125, 0.25]], np.float32))
    b_bits = oq.f32_to_bf16_bits(np.array([[-1.0, 3.0]], np.float32))
    codes = np.array([[0] * 32 + [255] * 32 + [0] * 32 + [255] * 32], np.uint32)
    t = {"packed": oq.pack_affine(codes, 8), "scale": s_bits, "bias": b_bits, "group_size": 64,
         "bits": 8}
    w = om.shared_weight(t)
    assert w.shape == (1, 128)
    assert np.all(w[0, :32] == -1.0) and np.all(w[0, 32:64] == 255 * 0.0078125 - 1.0)
    assert np.all(w[0, 64:96] == 3.0) and np.all(w[0, 96:] == oq.round_bf16(np.array(255 * 0.25 + 3.0)))
    plain = np.ones((2, 3))
    assert om.shared_weight(plain) is plain
    with pytest.raises(ValueError):
        om.shared_weight(dict(t, bits=4))

    rng = np.random.default_rng(29)
    E, H, I, Is, k, N = 8, 128, 64, 64, 3, 5
    p = _tiny_layer(rng, E=E, H=H, I=I, Is=Is)
    q = dict(p)
    for key in ("shared_gate_proj", "shared_up_proj", "shared_down_proj"):
        words, sb, bb, _ = oq.quantize_rtn(p[key].astype(np.float32), bits=8, group_size=64)
        q[key] = {"packed": words, "scale": sb, "bias": bb, "group_size": 64, "bits": 8}
        p[key] = oq.bf16_bits_to_f32(oq.dequant_bf16_bits(words, sb, bb, p[key].shape[1], bits=8)
                                     ).astype(np.float64)
    x = oq.round_bf16(rng.standard_normal((N, H)))
    y_t, _ = om.moe_forward(x, q, k=k, inter=I)
    y_d, _ = om.moe_forward(x, p, k=k, inter=I)
    assert np.array_equal(y_t, y_d)


def test_synth_int8_shared_layer_cpu():
    """synth.make_layer(shared_bits=8): the bake's int8 g64 triplets of the same bf16 draws (the
    rest of the layer unchanged), each weight within half a quantization step of its draw."""
    from quanta_amd import synth
    from quanta_amd.quant import unpack_affine

    s = synth.scaled_spec("c1", hidden_size=256, num_experts=4, moe_intermediate_size=128,
                          shared_expert_intermediate_size=128)
    p16 = synth.make_layer(s, device="cpu", seed=5)
    p8 = synth.make_layer(s, device="cpu", seed=5, shared_bits=8)
    assert torch.equal(p16["gate"], p8["gate"])
    assert torch.equal(p16["experts_down"]["packed"], p8["experts_down"]["packed"])
    for key in ("shared_gate_proj", "shared_up_proj", "shared_down_proj"):
        t, w = p8[key], p16[key].float()
        assert t["bits"] == 8 and t["group_size"] == 64
        q = unpack_affine(t["packed"], w.shape[1], 8).float()
        sc = t["scale"].float().repeat_interleave(64, dim=1)
        bi = t["bias"].float().repeat_interleave(64, dim=1)
        assert float((sc * q + bi - w).abs().max()) <= float((0.5 * sc + w.abs() * 2 ** -7).max())
    with pytest.raises(ValueError):
        synth.make_layer(s, device="cpu", seed=5, shared_bits=4)
