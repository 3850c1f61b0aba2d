"""GPU tier: routed experts whose widths vary per (expert, projection) (Kimi's
QuantizedSparseMoE, src/quanta/modeling/quantized.py:40-84; qmoe_forward_mixed).

One stack per (projection, width) with each expert's slot in its width's stack; the block runs
each stack's launch over all routed m-tiles, the other widths' experts exiting.

Bars: one width with identity slots gives the uniform path's output bit for bit (same
per-output arithmetic); mixed widths and permuted slots within the BASELINE gates of the oracle
(max-abs 2e-2 scaled, relative L2 5e-3) at every batch regime; bad maps refused on the host.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from quanta_amd import _lib as L
from quanta_amd.moe import MoEConfig, qwen35_moe, qwen35_moe_residual
from quanta_amd.quant import quantize_affine
from tests._util import assert_close, bits_np, f64, oracle_params_from_torch, words_np
from tests.test_gpu_5_formats import _inputs, _layer

pytestmark = pytest.mark.gpu

H, E, I = 512, 8, 256
GS = 128


def _mixed(dev, seed, widths, permute=True, tie_slots=False, group_sizes=None, n_exp=E):
    """widths[proj] [E] -> (p["experts_mixed"] source dict, the oracle's "mixed" dict).
    tie_slots: up takes gate's slots (with equal widths, the layout that fuses gate and up);
    group_sizes[proj]: that projection's stacks' group size (default GS)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    rng = np.random.default_rng(seed)
    stacks, pslot, ostacks = {}, {}, {}
    for proj in ("gate", "up", "down"):
        rows, K = (I, H) if proj != "down" else (H, I)
        gs = (group_sizes or {}).get(proj, GS)
        pb = np.asarray(widths[proj])
        ps = np.zeros(n_exp, np.int64)
        stacks[proj], ostacks[proj] = {}, {}
        for b in sorted(set(pb.tolist())):
            ids = np.flatnonzero(pb == b)
            ps[ids] = rng.permutation(ids.size) if permute else np.arange(ids.size)
            w = (torch.randn(ids.size, rows, K, generator=g) * 0.02).to(dev)
            packed, s, bb = quantize_affine(w, b, group_size=gs)
            stacks[proj][b] = {"packed": packed, "scale": s, "bias": bb, "group_size": gs}
            ostacks[proj][b] = (words_np(packed), bits_np(s), bits_np(bb), gs)
        if tie_slots and proj == "up":
            ps = pslot["gate"].copy()
        pslot[proj] = ps
    pbits = {k: np.asarray(v) for k, v in widths.items()}
    src = {"stacks": stacks, "pbits": pbits, "pslot": pslot, "group_size": GS}
    return src, {"stacks": ostacks, "pbits": pbits, "pslot": pslot, "group_size": GS}


def _layer_mixed(dev, seed, widths, permute=True, n_exp=E, **kw):
    p = _layer(dev, GS, seed, E=n_exp)
    del p["experts_gate_up"], p["experts_down"]
    src, om_mixed = _mixed(dev, seed, widths, permute, n_exp=n_exp, **kw)
    p["experts_mixed"] = src
    return p, om_mixed


def _oracle(p, om_mixed):
    q = {k: v for k, v in p.items() if k != "experts_mixed"}
    q["experts_gate_up"] = {"packed": torch.zeros(1, 1, 1, dtype=torch.int32),
                            "scale": torch.zeros(1, 1, 1, dtype=torch.bfloat16),
                            "bias": torch.zeros(1, 1, 1, dtype=torch.bfloat16)}
    q["experts_down"] = q["experts_gate_up"]
    op = oracle_params_from_torch(q)
    op["mixed"] = om_mixed
    return op


def test_mixed_one_width_equals_uniform_path(gpu):
    """All experts int4 with identity slots: the gate, up and down stacks concatenated into the
    uniform gate_up / down triplets give the same output bit for bit, at every regime (the
    decode kernel up to 256 tokens, the prefill kernels above)."""
    widths = {k: np.full(E, 4) for k in ("gate", "up", "down")}
    p, _ = _layer_mixed(gpu, 3, widths, permute=False)
    st = p["experts_mixed"]["stacks"]
    q = {k: v for k, v in p.items() if k != "experts_mixed"}
    q["experts_gate_up"] = {key: torch.cat([st["gate"][4][key], st["up"][4][key]], dim=1)
                            for key in ("packed", "scale", "bias")}
    q["experts_gate_up"].update(group_size=GS, bits=4)
    q["experts_down"] = dict(st["down"][4], group_size=GS, bits=4)
    cfg = MoEConfig(H, E, 2, I, 256)
    for N in (1, 8, 40, 300):
        x = _inputs(gpu, N, H, N)
        y_uni = qwen35_moe(x[None], q, cfg, regime=L.REGIME_SMALL if N <= 256 else L.REGIME_AUTO)[0]
        y_mix = qwen35_moe(x[None], p, cfg)[0]
        assert torch.equal(y_mix, y_uni), f"N={N}"


@pytest.mark.parametrize("case", ["kimi", "random34", "with_int6"])
@pytest.mark.parametrize("N", [1, 8, 40, 300])
def test_mixed_vs_oracle(gpu, case, N):
    rng = np.random.default_rng(N)
    if case == "kimi":          # the canonical split, one expert's down at int3
        widths = {"gate": np.full(E, 3), "up": np.full(E, 3), "down": np.array([4, 4, 3, 4, 4, 4, 4, 4])}
    elif case == "random34":    # gate and up of one expert may differ
        widths = {k: rng.choice([3, 4], E) for k in ("gate", "up", "down")}
    else:
        widths = {k: rng.choice([3, 4, 6], E) for k in ("gate", "up", "down")}
    cfg = MoEConfig(H, E, 2, I, 256)
    p, om_mixed = _layer_mixed(gpu, 17 * N + len(case), widths)
    x = _inputs(gpu, N, H, N)
    y = qwen35_moe(x[None], p, cfg)[0]
    _, it = om.moe_forward(f64(x), _oracle(p, om_mixed), k=2, inter=I)
    assert_close(f64(y), it["y_exact"], f"mixed {case} N={N}")


@pytest.mark.parametrize("case", ["kimi", "with_int6"])
def test_mixed_large_regime_hot_and_cold_vs_oracle(gpu, case):
    """Mixed widths above 256 tokens with 32 experts: each (projection, width) stack's launch on
    the prefill kernels over the hot experts' m-tiles and on the decode kernel over the cold
    ones, the other widths' experts exiting in both."""
    n_exp, N = 32, 300
    rng = np.random.default_rng(5)
    if case == "kimi":
        widths = {"gate": np.full(n_exp, 3), "up": np.full(n_exp, 3),
                  "down": rng.choice([3, 4], n_exp, p=[0.2, 0.8])}
    else:
        widths = {k: rng.choice([3, 4, 6], n_exp) for k in ("gate", "up", "down")}
    cfg = MoEConfig(H, n_exp, 2, I, 256)
    p, om_mixed = _layer_mixed(gpu, 91 + len(case), widths, n_exp=n_exp)
    x = _inputs(gpu, N, H, N)
    y = qwen35_moe(x[None], p, cfg)[0]
    _, it = om.moe_forward(f64(x), _oracle(p, om_mixed), k=2, inter=I)
    counts = np.bincount(it["idx"].reshape(-1), minlength=n_exp)
    assert counts.max() > 16 and counts.min() <= 16, "the layer must hold hot and cold experts"
    assert_close(f64(y), it["y_exact"], f"mixed {case} hot+cold N={N}")


@pytest.mark.parametrize("case", ["fused34", "fused346", "g64_g128"])
@pytest.mark.parametrize("N", [1, 8, 40, 300])
def test_mixed_gate_up_drawn_together_vs_oracle(gpu, case, N):
    """gate and up share each expert's width and slot, over two or three widths: gate and up are
    then fused per width (SwiGLU in the epilogue) unless their group sizes differ, which keeps
    them apart. Both against the oracle."""
    from quanta_amd.moe import tile_experts_mixed

    rng = np.random.default_rng(100 + N)
    gu = rng.choice([3, 4, 6] if case == "fused346" else [3, 4], E)
    widths = {"gate": gu, "up": gu.copy(), "down": rng.choice([3, 4], E)}
    gsz = {"gate": 64, "up": 128} if case == "g64_g128" else None
    cfg = MoEConfig(H, E, 2, I, 256)
    p, om_mixed = _layer_mixed(gpu, 29 * N + len(case), widths, tie_slots=True, group_sizes=gsz)
    src = p["experts_mixed"]
    mx = tile_experts_mixed(src["stacks"], src["pbits"], src["pslot"])
    fused = any(proj == "gate_up" for proj, _, _ in mx["stacks"])
    assert fused == (case != "g64_g128")
    x = _inputs(gpu, N, H, N)
    y = qwen35_moe(x[None], dict(p, experts_mixed=mx), cfg)[0]
    _, it = om.moe_forward(f64(x), _oracle(p, om_mixed), k=2, inter=I)
    assert_close(f64(y), it["y_exact"], f"mixed gate/up together {case} N={N}")


def test_mixed_bf16_placeholder_formats_large_regime(gpu):
    """qmoe_forward_mixed ignores the config's expert_format / down_format (placeholders of a
    mixed layer): a C caller passing bf16 there still gets the prefill kernels' fp16 activation
    copies above 256 tokens, and the output of the int4 placeholders, bit for bit."""
    import ctypes

    from quanta_amd import ops
    from quanta_amd.moe import prepare

    n_exp, N = 32, 300
    rng = np.random.default_rng(9)
    widths = {"gate": np.full(n_exp, 3), "up": np.full(n_exp, 3),
              "down": rng.choice([3, 4], n_exp, p=[0.2, 0.8])}
    cfg = MoEConfig(H, n_exp, 2, I, 256)
    p, om_mixed = _layer_mixed(gpu, 77, widths, n_exp=n_exp)
    x = _inputs(gpu, N, H, N)
    pr = prepare(p, cfg)
    y_int4 = ops.forward(pr.cfg, pr.weights, x, mixed=pr.mixed)
    c16 = type(pr.cfg).from_buffer_copy(pr.cfg)
    c16.expert_format = c16.down_format = L.FMT_BF16
    ws = torch.full((ops.forward_workspace(c16, N),), 0x7F, dtype=torch.uint8, device=gpu)
    y_bf16 = ops.forward(c16, pr.weights, x, ws=ws, mixed=pr.mixed)
    torch.cuda.synchronize()
    _, it = om.moe_forward(f64(x), _oracle(p, om_mixed), k=2, inter=I)
    counts = np.bincount(it["idx"].reshape(-1), minlength=n_exp)
    assert counts.max() > 16 and counts.min() <= 16, "the layer must hold hot and cold experts"
    assert torch.equal(y_bf16, y_int4)
    assert_close(f64(y_bf16), it["y_exact"], f"mixed bf16 placeholders N={N}")


def test_mixed_argument_errors(gpu):
    cfg = MoEConfig(H, E, 2, I, 256)
    widths = {k: np.full(E, 4) for k in ("gate", "up", "down")}
    p, _ = _layer_mixed(gpu, 5, widths)
    x = _inputs(gpu, 4, H, 1)
    src = p["experts_mixed"]
    no_stack = dict(src, pbits=dict(src["pbits"], down=np.array([4] * 7 + [3])))
    with pytest.raises(ValueError, match="no stack"):
        qwen35_moe(x[None], dict(p, experts_mixed=no_stack), cfg)
    bad_slot = dict(src, pslot=dict(src["pslot"], up=np.arange(E) + 1))
    with pytest.raises(ValueError, match="outside its stack"):
        qwen35_moe(x[None], dict(p, experts_mixed=bad_slot), cfg)
    with pytest.raises(Exception, match="qmoe_forward_mixed"):
        qwen35_moe_residual(x[None], p, cfg, torch.ones(H, dtype=torch.bfloat16, device=gpu))


def test_module_set_experts_mixed(gpu):
    """Qwen35MoEModule.set_experts_mixed (QuantizedSparseMoE.set_experts' arguments) gives the
    functional form's output."""
    from quanta_amd.moe import Qwen35MoEModule

    cfg = MoEConfig(H, E, 2, I, 256)
    widths = {"gate": np.full(E, 3), "up": np.full(E, 3), "down": np.array([4, 4, 3, 4, 4, 4, 4, 4])}
    p, _ = _layer_mixed(gpu, 9, widths)
    x = _inputs(gpu, 12, H, 9)
    m = Qwen35MoEModule(cfg, device=gpu)
    with torch.no_grad():
        for kk in ("gate", "shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
            getattr(m, kk).copy_(p[kk])
    src = p["experts_mixed"]
    m.set_experts_mixed(src["stacks"], src["pbits"], src["pslot"])
    assert torch.equal(m(x[None])[0], qwen35_moe(x[None], p, cfg)[0])
