"""GPU tier: the shared expert as the bake stores it, int8 g64 (src/quanta/qwen35/bake.py:106-110,
150-151), read by the kernels as int8 and dequantized in registers.

The reference's loader dequantizes it to bf16 at load (src/quanta/qwen35/artifact.py:105-115,
171-184) and runs the bf16 chain; the int8 kernels build the same bf16 weights in registers
(bf16(fmaf(s, q, b)), the qmoe_dequant convention) and sum in the same order as the bf16 kernels,
so the bars are:
  - bit-identical to the same block with the shared expert given as its bf16 dequant, at every
    batch size and through every path (pair launch with and without the fused RMSNorm, the
    fused combine + shared down, the unfused small-regime launches above 64 tokens, the expanded
    bf16 copy of the large regime above 256 tokens, the allocation-free entry point);
  - the block against the oracle (oracle.moe.shared_weight dequantizes the triplets) within the
    BASELINE gates, with the shared expert carrying most of the output.
"""

from __future__ import annotations

import pytest
import torch

from oracle import moe as om
from quanta_amd import _lib as L
from quanta_amd import ops, synth
from quanta_amd.moe import prepare, qwen35_moe, qwen35_moe_residual
from quanta_amd.quant import quantize_affine
from tests._util import assert_close, f64, oracle_params_from_torch

pytestmark = pytest.mark.gpu

SHARED = ("shared_gate_proj", "shared_up_proj", "shared_down_proj")


def _dequant_shared(p: dict) -> dict:
    """The layer with its int8 shared triplets replaced by their bf16 dequant (the reference's
    load-time form)."""
    q = dict(p)
    for key in SHARED:
        t = p[key]
        q[key] = ops.dequant(t["packed"], t["scale"], t["bias"], bits=8, group_size=t["group_size"])
    return q


def _spec(name="c1", **dims):
    return synth.scaled_spec(name, **dims) if dims else synth.spec(name)


def _pair(spec, dev, seed):
    p8 = synth.make_layer(spec, device=dev, seed=seed, shared_bits=8)
    return p8, _dequant_shared(p8)


def test_tiled_int8_products_match_bf16(gpu):
    """grouped_qmm on tiled int8 == on tiled bf16 of the dequantized matrix, bit for bit, for each
    epilogue, one to many m-tiles (two m-tiles per wavefront from 4), K with 1-16 chunks."""
    g = torch.Generator(device="cpu").manual_seed(3)
    for rows, K in ((64, 256), (512, 1024), (256, 4096), (128, 7168)):
        w = (torch.randn(rows, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
        pk, sc, bi = quantize_affine(w, 8, group_size=64)
        c8, sb8 = ops.tile_int8(pk, sc, bi)
        w16 = ops.tile_bf16(ops.dequant(pk, sc, bi, bits=8))
        for n in (1, 5, 16, 40, 70):
            x = (torch.randn(n, K, generator=g)).to(torch.bfloat16).to(gpu)
            for epi in (L.EPI_BF16, L.EPI_F32, L.EPI_SWIGLU):
                kw = dict(K=K, n_rows=rows, epilogue=epi, out_rows=n, regime=L.REGIME_SMALL,
                          dense_rows=n)
                y8 = ops.grouped_qmm(x, weight_format=L.FMT_INT8_G64, codes=c8, sb=sb8, **kw)
                y16 = ops.grouped_qmm(x, weight_format=L.FMT_BF16, codes=w16, sb=None, **kw)
                assert torch.equal(y8, y16), (rows, K, n, epi)
    print("[parity] int8 tiled products == bf16 tiled products of the dequant, bit-exact", flush=True)


@pytest.mark.parametrize("N", [1, 2, 3, 8, 17, 32, 64, 65, 100, 257, 300])
def test_block_int8_shared_equals_bf16_dequant(gpu, N):
    """c1-shaped block (H 2048, Is 512): the int8 shared expert gives the bf16-dequant block's
    outputs bit for bit through the decode launches (N <= 64 fused, 65-256 unfused small regime)
    and the large regime's expanded copy (N > 256)."""
    s = _spec("c1")
    p8, p16 = _pair(s, gpu, seed=21)
    x = synth.make_inputs(s, N, device=gpu, seed=N)[None]
    y8 = qwen35_moe(x, p8, s.cfg)
    y16 = qwen35_moe(x, p16, s.cfg)
    assert prepare(p8, s.cfg).cfg.shared_format == L.FMT_INT8_G64
    assert prepare(p16, s.cfg).cfg.shared_format == L.FMT_BF16
    assert torch.equal(y8, y16), f"N={N}: max diff {(y8.float() - y16.float()).abs().max().item()}"


@pytest.mark.parametrize("N", [1, 4, 8, 32])
def test_residual_and_noalloc_int8_shared(gpu, N):
    """The fused-RMSNorm pair launch and the allocation-free entry point with an int8 shared
    expert: equal to the bf16-dequant block."""
    s = _spec("c1")
    p8, p16 = _pair(s, gpu, seed=22)
    x = synth.make_inputs(s, N, device=gpu, seed=100 + N)[None]
    g = torch.Generator(device="cpu").manual_seed(N)
    nw = (1.0 + 0.1 * torch.randn(s.cfg.hidden_size, generator=g)).to(torch.bfloat16).to(gpu)
    r8 = qwen35_moe_residual(x, p8, s.cfg, nw, eps=1e-6)
    r16 = qwen35_moe_residual(x, p16, s.cfg, nw, eps=1e-6)
    assert torch.equal(r8, r16), f"residual N={N}"
    pr = prepare(p8, s.cfg)
    out = torch.empty(N, s.cfg.hidden_size, dtype=torch.bfloat16, device=gpu)
    ops.forward_noalloc(pr.cfg, pr.weights, x[0].contiguous(), out)
    assert torch.equal(out, qwen35_moe(x, p16, s.cfg)[0]), f"noalloc N={N}"


@pytest.mark.parametrize("name,N", [("c2", 1), ("c2", 8), ("c2", 32), ("c3", 1), ("c3", 16), ("c3", 64)])
def test_full_size_int8_shared(gpu, name, N):
    """Full-size c2 (Is 1024) and c3 (Is 2048, ungated) layers: int8 == bf16-dequant block. At c3
    the int8 shared down (eight K chunks, four wavefronts of two) rides in the routed gate_up
    launch (slot-major with the top-k at N=1, sorted at 16 and 64), the bf16 one in the combine."""
    s = _spec(name)
    p8, p16 = _pair(s, gpu, seed=23)
    x = synth.make_inputs(s, N, device=gpu, seed=N)[None]
    y8, y16 = qwen35_moe(x, p8, s.cfg), qwen35_moe(x, p16, s.cfg)
    assert torch.equal(y8, y16), f"{name} N={N}"
    del p8, p16
    torch.cuda.empty_cache()


@pytest.mark.parametrize("N", [1, 8, 40, 300])
def test_int8_shared_vs_oracle(gpu, N):
    """The block against the oracle, whose shared_weight dequantizes the int8 triplets, with the
    shared expert's weights scaled up so it carries most of the output."""
    s = _spec("c1", hidden_size=512, num_experts=16, moe_intermediate_size=256,
              shared_expert_intermediate_size=256)
    p = synth.make_layer(s, device=gpu, seed=24)
    for key in SHARED:
        w = p[key].float() * 8.0
        pk, sc, bi = quantize_affine(w.to(torch.bfloat16), 8, group_size=64)
        p[key] = {"packed": pk, "scale": sc, "bias": bi, "group_size": 64, "bits": 8}
    x = synth.make_inputs(s, N, device=gpu, seed=7 + N)
    y = qwen35_moe(x[None], p, s.cfg)[0]
    c = s.cfg
    _, it = om.moe_forward(f64(x), oracle_params_from_torch(p), k=c.num_experts_per_tok,
                           inter=c.moe_intermediate_size)
    share = float(abs(it["shared"]).mean() / abs(it["y_exact"]).mean())
    print(f"[parity] int8 shared N={N}: shared part {share:.2f} of |y|", flush=True)
    assert share > 0.5
    assert_close(f64(y), it["y_exact"], f"int8 shared N={N}")
