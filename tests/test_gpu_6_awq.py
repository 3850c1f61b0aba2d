"""GPU tier: DeepSeek-V4's activation-aware (AWQ) expert scales (src/quanta/dsv4/moe.py:112-137).

The block divides each routed row's activation by its expert's per-input-channel scale before
the gate, the up and the down projection (qmoe_config_t.awq; kernels in awq.hip; gate_up as one
launch whose up-half wavefronts read the rows prescaled for the up projection).

Above 256 tokens layers whose intermediate size is a multiple of 256 take the large regime
(int3 gate/up with int4 down included, test_awq_block_vs_oracle at N = 300): the hot experts' gate_up on the prefill (MFMA) kernels, each 256- or 512-row weight
block reading the fp16 copy of the gate's or the up projection's prescaled rows.

Bars: unit scales give the plain path's output bit for bit in both regimes (same per-output
arithmetic); random scales within the BASELINE gates of the oracle (max-abs 2e-2 scaled,
relative L2 5e-3) at every batch regime the AWQ path uses; batch invariance bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from quanta_amd import _lib as L
from quanta_amd.moe import MoEConfig, qwen35_moe
from tests._util import assert_close, f64, oracle_params_from_torch
from tests.test_gpu_5_formats import _inputs, _layer, _layer_widths

pytestmark = pytest.mark.gpu

LIMIT = 2.0   # DeepSeek-V4's clamped SwiGLU, small enough to bind on part of the values


def _cfg(E=8, I=256, H=512, **kw):
    return MoEConfig(H, E, 2, I, 256, scoring_func="sigmoid", norm_topk_prob=True,
                     routed_scaling_factor=1.5, hidden_act="silu", swiglu_limit=LIMIT, **kw)


def _with_awq(p, dev, seed, E=8, H=512, I=256, unit=False):
    g = torch.Generator(device="cpu").manual_seed(seed)
    if unit:
        s_gu, s_dn = torch.ones(E, 2, H), torch.ones(E, I)
    else:
        s_gu = 2.0 ** (torch.rand(E, 2, H, generator=g) * 2 - 1)
        s_dn = 2.0 ** (torch.rand(E, I, generator=g) * 2 - 1)
    q = dict(p)
    q["experts_gate_up"] = dict(p["experts_gate_up"], awq_scale=s_gu.to(torch.bfloat16).to(dev))
    q["experts_down"] = dict(p["experts_down"], awq_scale=s_dn.to(torch.bfloat16).to(dev))
    return q


@pytest.mark.parametrize("N,regime,E,I", [(1, L.REGIME_SMALL, 8, 256), (8, L.REGIME_SMALL, 8, 256),
                                          (40, L.REGIME_SMALL, 8, 256),
                                          (300, L.REGIME_SMALL, 8, 256),
                                          (300, L.REGIME_LARGE, 32, 256),
                                          (700, L.REGIME_LARGE, 32, 512)])
def test_awq_unit_scales_equal_plain_path(gpu, N, regime, E, I):
    """All-ones scales: prescaling is exact and the gated activation divides by one, so the
    bf16-epilogue gate_up launch plus the AWQ activation pass reproduce the fused SwiGLU launch
    bit for bit (the K chunks and their order depend on the shape only; in the large regime the
    prefill kernels sum each output in the same order under either epilogue, and the fp16 copy
    of a prescaled row equals that of its token's row)."""
    cfg = _cfg(E, I)
    p = _layer(gpu, 64, seed=3 * N, E=E, I=I, gated=False)
    x = _inputs(gpu, N, 512, N)
    y_plain = qwen35_moe(x[None], p, cfg, regime=regime)[0]
    y_awq = qwen35_moe(x[None], _with_awq(p, gpu, N, E=E, I=I, unit=True), cfg, regime=regime)[0]
    assert torch.equal(y_awq, y_plain)


@pytest.mark.parametrize("E,I,N,H", [(32, 256, 300, 512), (32, 512, 300, 512),
                                     (8, 512, 1100, 512), (32, 256, 300, 8704)])
def test_awq_large_regime_vs_oracle(gpu, E, I, N, H):
    """AWQ int4 layers above 256 tokens: hot experts (more than 16 rows) on the prefill kernels,
    the rest on the decode kernel beside them. I = 256 splits gate and up between 256-row blocks
    (the 256-row kernel), I = 512 between 512-row blocks (the 512-row kernel); E = 32 at 300
    tokens leaves both hot and cold experts. The prescaled rows come from one pass that writes
    hot rows as fp16 copies and cold rows as bf16 (H <= 8192), or above that from the bf16 pass
    and a separate fp16 conversion (H = 8704)."""
    cfg = _cfg(E, I, H)
    base = _layer(gpu, 64, seed=41 * N + I, H=H, E=E, I=I, gated=False)
    base.pop("shared_expert_gate", None)
    p = _with_awq(base, gpu, seed=43 * N + I, E=E, H=H, I=I)
    # (inputs scaled so the router logits keep H = 512's spread: at H = 8704 and scale 4 the
    # sigmoid scores of several experts round to 1.0 in fp32 and tie, unlike the fp64 oracle's)
    x = _inputs(gpu, N, H, N, scale=4.0 * (512 / H) ** 0.5)
    y = qwen35_moe(x[None], p, cfg)[0]
    _, it = om.moe_forward(f64(x), oracle_params_from_torch(p), k=2, inter=I, scoring="sigmoid",
                           norm_topk=True, scale=1.5, act="silu", limit=LIMIT, group_size=64)
    counts = np.bincount(it["idx"].reshape(-1), minlength=E)
    if E == 32:
        assert counts.max() > 16 and counts.min() <= 16, "the layer must hold hot and cold experts"
    assert_close(f64(y), it["y_exact"], f"awq large regime E={E} I={I} N={N} H={H}")


@pytest.mark.parametrize("gu_bits,dn_bits,I", [(3, 4, 512), (6, 4, 256), (4, 6, 256)])
def test_awq_narrow_widths_large_regime_vs_oracle(gpu, gu_bits, dn_bits, I):
    """AWQ scales on int3 and int6 stacks above 256 tokens, hot and cold experts (E = 32): int3
    gate_up at I = 512 runs the 512-row int3 kernel with its gate and up blocks reading their own
    prescaled rows (split_tile a multiple of 32); int6 gate_up, and int6 down, on the 256-row
    kernel."""
    E, N, H = 32, 300, 512
    cfg = _cfg(E, I, H)
    base = _layer_widths(gpu, 64, 47 * gu_bits + I + dn_bits, gu_bits, dn_bits, H=H, E=E, I=I)
    base.pop("shared_expert_gate", None)
    p = _with_awq(base, gpu, seed=53 * gu_bits + I, E=E, H=H, I=I)
    x = _inputs(gpu, N, H, N)
    y = qwen35_moe(x[None], p, cfg)[0]
    _, it = om.moe_forward(f64(x), oracle_params_from_torch(p), k=2, inter=I, scoring="sigmoid",
                           norm_topk=True, scale=1.5, act="silu", limit=LIMIT, group_size=64,
                           bits=gu_bits, down_bits=dn_bits)
    counts = np.bincount(it["idx"].reshape(-1), minlength=E)
    assert counts.max() > 16 and counts.min() <= 16, "the layer must hold hot and cold experts"
    assert_close(f64(y), it["y_exact"], f"awq int{gu_bits}/int{dn_bits} large regime I={I} N={N}")


@pytest.mark.parametrize("gs,gu_bits,dn_bits", [(64, 4, 4), (128, 4, 4), (128, 3, 4)])
@pytest.mark.parametrize("N", [1, 8, 40, 300])
def test_awq_block_vs_oracle(gpu, gs, gu_bits, dn_bits, N):
    cfg = _cfg()
    base = (_layer(gpu, gs, seed=5 * N + gs, gated=False) if (gu_bits, dn_bits) == (4, 4) else
            _layer_widths(gpu, gs, 5 * N + gs, gu_bits, dn_bits))
    base.pop("shared_expert_gate", None)   # DeepSeek-V4's shared expert is ungated
    p = _with_awq(base, gpu, seed=7 * N + gs)
    x = _inputs(gpu, N, 512, N)
    y = qwen35_moe(x[None], p, cfg)[0]
    _, it = om.moe_forward(f64(x), oracle_params_from_torch(p), k=2, inter=256, scoring="sigmoid",
                           norm_topk=True, scale=1.5, act="silu", limit=LIMIT, group_size=gs,
                           bits=gu_bits, down_bits=dn_bits)
    assert_close(f64(y), it["y_exact"], f"awq int{gu_bits}/int{dn_bits} g{gs} N={N}")
    if N >= 40:
        g = it["gu"][:, :256]
        assert np.any(g > LIMIT), "the clamp must bind somewhere for the test to mean anything"


@pytest.mark.parametrize("N", [1, 8, 40, 300])
def test_dsv4_block_vs_oracle(gpu, N):
    """DeepSeek-V4's block as the reference composes it (src/quanta/dsv4/moe.py:140-173):
    sqrt-softplus scores with the selection bias, normalised weights times 1.5, clamped SwiGLU,
    AWQ-scaled int4 experts and an ungated shared expert."""
    cfg = MoEConfig(512, 8, 2, 256, 256, scoring_func="sqrtsoftplus", norm_topk_prob=True,
                    routed_scaling_factor=1.5, hidden_act="silu", swiglu_limit=LIMIT)
    base = _layer(gpu, 128, seed=23 * N, gated=False)
    g = torch.Generator(device="cpu").manual_seed(N)
    base["e_score_correction_bias"] = (torch.randn(8, generator=g) * 0.05).to(gpu)
    p = _with_awq(base, gpu, seed=29 * N)
    x = _inputs(gpu, N, 512, N)
    y = qwen35_moe(x[None], p, cfg)[0]
    _, it = om.moe_forward(f64(x), oracle_params_from_torch(p), k=2, inter=256, scoring="sqrtsoftplus",
                           norm_topk=True, scale=1.5, act="silu", limit=LIMIT, group_size=128)
    assert_close(f64(y), it["y_exact"], f"dsv4 N={N}")


def test_awq_batch_invariance(gpu):
    cfg = _cfg()
    p = _with_awq(_layer(gpu, 64, seed=11, gated=False), gpu, seed=12)
    x = _inputs(gpu, 40, 512, 13)
    full = qwen35_moe(x[None], p, cfg)[0]
    for t in (0, 17, 39):
        assert torch.equal(qwen35_moe(x[t:t + 1][None], p, cfg)[0, 0], full[t]), f"token {t}"


def test_awq_argument_errors(gpu):
    cfg = _cfg()
    p = _layer(gpu, 64, seed=1, gated=False)
    q = _with_awq(p, gpu, seed=2)
    x = _inputs(gpu, 4, 512, 1)
    one_sided = dict(q, experts_down=p["experts_down"])
    with pytest.raises(ValueError, match="both experts_gate_up and experts_down"):
        qwen35_moe(x[None], one_sided, cfg)
    bad = dict(q, experts_down=dict(q["experts_down"], awq_scale=q["experts_down"]["awq_scale"][:, :128]))
    with pytest.raises(ValueError, match="awq_scale must be"):
        qwen35_moe(x[None], bad, cfg)
    # the large regime needs gate and up halves of whole 256-row blocks
    p128 = _layer(gpu, 64, seed=1, I=128, gated=False)
    with pytest.raises(ValueError, match="inter % 256 == 0"):
        qwen35_moe(x[None], _with_awq(p128, gpu, seed=2, I=128), _cfg(I=128),
                   regime=L.REGIME_LARGE)
