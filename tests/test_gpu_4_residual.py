"""GPU tier: the block with the decoder layer's steps either side of it, x + block(rmsnorm(x))
(qmoe_forward_residual / qwen35_moe_residual; reference src/quanta/qwen35/model.py:104-105).

Bars: the norm within one bf16 rounding of the float64 oracle (its fp32 reduction order is the
kernel's own); the fused call bit-identical to its parts (qmoe_rmsnorm, then qmoe_forward on the
normalised rows, then a bf16 add); the layer output against the oracle within the BASELINE
gates (max-abs 2e-2 scaled, relative L2 5e-3).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq
from quanta_amd import ops, synth
from quanta_amd.moe import Qwen35MoEModule, prepare, qwen35_moe, qwen35_moe_residual
from tests._util import assert_close, bf16_dev, f64, oracle_params_from_torch
from tests.test_gpu_2_block import _fixture, _layer

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _norm_weight(H, seed, dev):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (1.0 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)


def _ulp_bf16(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |v| (8 significant bits)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


@pytest.mark.parametrize("N,H,eps", [(1, 512, EPS), (37, 4096, EPS), (9, 7168, 1e-5), (4, 2048, 0.25),
                                     (6, 200, EPS)])
def test_rmsnorm_vs_oracle(gpu, N, H, eps):
    rng = np.random.default_rng(N * 7 + H)
    x = rng.standard_normal((N, H)) * 3.0
    x[0] *= 100.0                      # a large row
    if N > 2:
        x[1] *= 1e-3                   # a small row
        x[2] = 0.0                     # a zero row: eps keeps it finite, the output is zero
    x = oq.round_bf16(x)
    w = oq.round_bf16(1.0 + 0.2 * rng.standard_normal(H))
    got = f64(ops.rmsnorm(bf16_dev(oq.f32_to_bf16_bits(x.astype(np.float32)), gpu),
                          bf16_dev(oq.f32_to_bf16_bits(w.astype(np.float32)), gpu), eps))
    want = oq.round_bf16(om.rmsnorm(x, w, eps))
    diff = np.abs(got - want)
    assert np.all(np.isfinite(got))
    assert np.all(diff <= _ulp_bf16(want) + 1e-300), f"max diff {diff.max():.3e}"
    exact = float(np.mean(diff == 0))
    print(f"[parity] rmsnorm N={N} H={H}: {exact:.5f} of elements bit-exact, rest within one bf16 ulp")
    assert exact >= 0.99
    if N > 2:
        assert np.all(got[2] == 0.0)


def _parts(x, p, cfg, nw, eps):
    xn = ops.rmsnorm(x, nw, eps)
    ym = qwen35_moe(xn[None], p, cfg)[0]
    return (x.float() + ym.float()).to(torch.bfloat16)


@pytest.mark.parametrize("name,N", [("c1", 1), ("c1", 2), ("c1", 17), ("c1", 64), ("c2", 1), ("c2", 2),
                                    ("c2", 8), ("c2", 32),
                                    ("c2", 49), ("c2", 65), ("c2", 300), ("c3", 1), ("c3", 16),
                                    ("c0", 8)])
def test_residual_equals_its_parts(gpu, name, N):
    """The fused call against qmoe_rmsnorm + qmoe_forward + a bf16 add: bit for bit, in every
    regime the token count selects (up to 64 tokens the norm runs inside the router launch, one
    or two m-tiles per wavefront; above, and with c0's fp32 router, as a launch of its own;
    slot-major top-k, the top-k inside the routed gate_up and the fused down/combine tail (c1
    N=1-2, c2 N=1), auxiliary-stream shared expert, hybrid prefill); and in place."""
    cfg = synth.spec(name).cfg
    p = _layer(name, gpu)
    x = (synth.make_inputs(name, N, device=gpu, seed=N).float() * 4.0).to(torch.bfloat16)
    nw = _norm_weight(cfg.hidden_size, N, gpu)
    y = qwen35_moe_residual(x[None], p, cfg, nw, eps=EPS)[0]
    assert torch.equal(y, _parts(x, p, cfg, nw, EPS)), f"{name} N={N}"
    pr = prepare(p, cfg)
    xc = x.clone()
    ops.forward_residual(pr.cfg, pr.weights, xc, nw, EPS, out=xc)
    assert torch.equal(xc, y), f"{name} N={N} in place"


def test_residual_vs_oracle_and_module(gpu):
    """c1mini golden block: y = bf16(x + bf16(block(rmsnorm(x)))) against the oracle run on the
    kernel's normalised rows (so a last-bit norm difference cannot flip a near-tie route), and
    Qwen35MoEModule.forward_residual equal to the functional form."""
    a, cfg, p, x = _fixture("c1mini", gpu)
    H, k, I = cfg.hidden_size, cfg.num_experts_per_tok, cfg.moe_intermediate_size
    nw = _norm_weight(H, 5, gpu)
    y = qwen35_moe_residual(x[None], p, cfg, nw)[0]      # eps from cfg.norm_eps
    xn = ops.rmsnorm(x, nw, EPS)
    want_xn = oq.round_bf16(om.rmsnorm(f64(x), f64(nw), EPS))
    assert np.all(np.abs(f64(xn) - want_xn) <= _ulp_bf16(want_xn) + 1e-300)
    _, it = om.moe_forward(f64(xn), oracle_params_from_torch(p), k=k, inter=I)
    want = om.residual_add(f64(x), oq.round_bf16(it["y_exact"]))
    assert_close(f64(y), want, "c1mini residual block")
    m = Qwen35MoEModule(cfg, device=gpu)
    with torch.no_grad():
        for kk in ("gate", "shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
            getattr(m, kk).copy_(p[kk])
    m.set_experts_packed(p["experts_gate_up"], p["experts_down"])
    assert torch.equal(m.forward_residual(x[None], nw)[0], y)
    # the run-every-expert path takes the same norm and add around the dense oracle
    p16 = dict(p, experts_gate_up=ops.dequant(p["experts_gate_up"]["packed"], p["experts_gate_up"]["scale"],
                                              p["experts_gate_up"]["bias"]),
               experts_down=ops.dequant(p["experts_down"]["packed"], p["experts_down"]["scale"],
                                        p["experts_down"]["bias"]))
    y_dense = qwen35_moe_residual(x[None], p16, cfg, nw, sparse=False)[0]
    assert_close(f64(y_dense), f64(y), "dense path vs fused", want_rounded=True)


def test_residual_rejects_bad_arguments(gpu):
    cfg = synth.spec("c0").cfg
    p = synth.make_layer("c0", device=gpu)
    x = synth.make_inputs("c0", 4, device=gpu)
    with pytest.raises(ValueError, match="norm_weight"):
        qwen35_moe_residual(x[None], p, cfg, torch.ones(cfg.hidden_size - 1, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError, match="eps"):
        ops.rmsnorm(x, torch.ones(cfg.hidden_size, dtype=torch.bfloat16, device=gpu), -1.0)
    with pytest.raises(ValueError, match="H % 8"):
        ops.rmsnorm(x[:, :12].contiguous(), torch.ones(12, dtype=torch.bfloat16, device=gpu), EPS)
