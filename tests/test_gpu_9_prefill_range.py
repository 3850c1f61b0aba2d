"""GPU tier: the number ranges of the prefill (large-M) kernels.

The prefill kernels multiply in fp16 on the MFMA units: each weight is dequantized as
fp16(s*q + b) and the activations come from a per-row power-of-two scaled fp16 copy. fp16 has a
narrower exponent range than the bf16 scales and activations it takes in, so these tests drive
both ends of it through the whole block in the large regime (N > 256, 512-row weight blocks) and
hold the result to the BASELINE gates of the oracle:
  - expert weights with standard deviation 1e-5 and 1e-7: every scale below 2^-14 (fp16's
    smallest normal), and with 1e-7 below 2^-24 (fp16's smallest subnormal);
  - activation rows whose elements span more than 2^28 in magnitude;
  - weights with large magnitudes (std 30, scales near 2^3).
The shared expert is left out where it would dominate the output and hide the routed experts.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from quanta_amd import _lib as L
from quanta_amd.moe import MoEConfig, qwen35_moe
from quanta_amd.quant import quantize_affine
from tests._util import assert_close, f64, oracle_params_from_torch

pytestmark = pytest.mark.gpu

H, E, K, I = 512, 8, 2, 256


def _layer(dev, seed, std, Is=0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    p = {"gate": (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(dev)}
    for key, shape in (("experts_gate_up", (E, 2 * I, H)), ("experts_down", (E, H, I))):
        w = (torch.randn(*shape, generator=g) * std).to(dev)
        packed, s, b = quantize_affine(w, 4, group_size=64)
        p[key] = {"packed": packed, "scale": s, "bias": b, "group_size": 64, "bits": 4}
    if Is:
        for key, shape in (("shared_gate_proj", (Is, H)), ("shared_up_proj", (Is, H)),
                           ("shared_down_proj", (H, Is))):
            p[key] = (torch.randn(*shape, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    return p


def _check(p, cfg, x, what, regime=L.REGIME_LARGE):
    y = qwen35_moe(x[None], p, cfg, regime=regime)[0]
    assert torch.isfinite(y.float()).all(), what
    _, it = om.moe_forward(f64(x), oracle_params_from_torch(p), k=K, inter=I)
    assert_close(f64(y), it["y_exact"], what)
    return y


@pytest.mark.parametrize("std", [1e-5, 1e-7])
@pytest.mark.parametrize("N", [300, 700])
def test_prefill_tiny_weight_scales(gpu, std, N):
    cfg = MoEConfig(H, E, K, I, 0)
    p = _layer(gpu, seed=int(N + 1 / std) % 10007, std=std)
    smax = max(float(p[k]["scale"].float().abs().max()) for k in ("experts_gate_up", "experts_down"))
    assert smax < 2.0 ** -14
    x = (torch.randn(N, H, generator=torch.Generator().manual_seed(N)) * 4).to(torch.bfloat16).to(gpu)
    y = _check(p, cfg, x, f"prefill std={std:g} N={N}")
    y_small = qwen35_moe(x[None], p, cfg, regime=L.REGIME_SMALL)[0]
    assert_close(f64(y), f64(y_small), f"prefill std={std:g} N={N}: large vs small regime",
                 want_rounded=True)


@pytest.mark.parametrize("N", [300, 700])
def test_prefill_large_weight_scales(gpu, N):
    cfg = MoEConfig(H, E, K, I, 0)
    p = _layer(gpu, seed=N + 3, std=30.0)
    x = (torch.randn(N, H, generator=torch.Generator().manual_seed(N + 1)) * 4).to(torch.bfloat16).to(gpu)
    _check(p, cfg, x, f"prefill std=30 N={N}")


@pytest.mark.parametrize("N", [300, 700])
@pytest.mark.parametrize("span", [30, 40])
def test_prefill_activation_dynamic_range(gpu, N, span):
    """Each row's elements spread over 2^span in magnitude (2^-(span-8) .. 2^8), with the shared
    expert on: the per-row fp16 copies keep the large elements exact, and the small ones' loss
    is bounded by fp16's subnormal step relative to the row maximum."""
    cfg = MoEConfig(H, E, K, I, 256)
    p = _layer(gpu, seed=N + span, std=0.02, Is=256)
    g = torch.Generator().manual_seed(N * span)
    mag = torch.exp2(torch.rand(N, H, generator=g) * span - (span - 8))
    x = (torch.randn(N, H, generator=g) * mag).to(torch.bfloat16)
    a = x.float().abs()
    spread = (a.max(dim=1).values / a.clamp_min(1e-38).min(dim=1).values).log2()
    assert float(spread.min()) > 28
    _check(p, cfg, x.to(gpu), f"prefill activations spanning 2^{span} N={N}")
