"""GPU tier: other expert formats on the same kernels.

- int6 expert stacks (MiniMax M3, src/quanta/minimax/model_m3.py:414-450) on the decode kernel:
  dequant bit-exact, the grouped matmul and the block against the oracle.
- int3 expert stacks, alone and as Kimi's per-projection widths (gate/up int3 + down int4, group
  128; src/quanta/modeling/quantized.py:4-7) on the decode kernel: dequant bit-exact, the grouped
  matmul and the block against the oracle.
- int4 (and int8) stacks with 128-column groups (Kimi's QuantizedSparseMoE layout,
  src/quanta/modeling/quantized.py:29-34): dequant bit-exact, the tiled layout lossless, and the
  block against the oracle at decode and prefill sizes.
- the clamped gated activations of the SwiGLU epilogue: DeepSeek-V4's clamped silu
  (src/quanta/dsv4/moe.py:74-77) and MiniMax M3's SwiGLU-OAI (src/quanta/minimax/
  model_m3.py:112-128), on routed and shared experts, against the oracle in every regime.

Bars: dequant and tiling bit-exact; the block within the BASELINE gates (max-abs 2e-2 scaled,
relative L2 5e-3).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq
from quanta_amd import _lib as L
from quanta_amd import ops
from quanta_amd.moe import MoEConfig, qwen35_moe
from quanta_amd.quant import quantize_affine
from tests._util import (assert_close, bf16_dev, bits_np, f64, oracle_params_from_torch, words_dev,
                         words_np)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_group128_bit_exact(gpu, bits):
    rng = np.random.default_rng(bits)
    rows, K = 48, 512
    codes = rng.integers(0, 1 << bits, size=(rows, K))
    words = oq.pack_affine(codes, bits)
    s = oq.f32_to_bf16_bits((rng.random((rows, K // 128)) * 0.05 + 1e-3).astype(np.float32))
    b = oq.f32_to_bf16_bits((rng.standard_normal((rows, K // 128)) * 0.3).astype(np.float32))
    got = ops.dequant(words_dev(words, gpu), bf16_dev(s, gpu), bf16_dev(b, gpu), bits=bits,
                      group_size=128)
    want = oq.dequant_bf16_bits(words, s, b, K, bits=bits, group_size=128)
    assert np.array_equal(bits_np(got), want)


def test_tile_group128_lossless(gpu):
    rng = np.random.default_rng(5)
    E, rows, K = 3, 32, 384
    w = torch.from_numpy(rng.standard_normal((E, rows, K)).astype(np.float32) * 0.02).to(gpu)
    packed, s, b = quantize_affine(w, 4, group_size=128)
    codes, sb = ops.tile_int4(packed, s, b, group_size=128)
    back = ops.dequant_tiled(codes, sb, E, rows, K)
    assert torch.equal(back, ops.dequant(packed, s, b, bits=4, group_size=128))


def _layer(dev, gs, seed, H=512, E=8, I=256, Is=256, gated=True):
    g = torch.Generator(device="cpu").manual_seed(seed)
    nrm = lambda *shape: torch.randn(*shape, generator=g) * 0.02
    p = {"gate": nrm(E, H).to(torch.bfloat16).to(dev)}
    for key, shape in (("experts_gate_up", (E, 2 * I, H)), ("experts_down", (E, H, I))):
        packed, s, b = quantize_affine(nrm(*shape).to(dev), 4, group_size=gs)
        p[key] = {"packed": packed, "scale": s, "bias": b, "group_size": gs, "bits": 4}
    for key, shape in (("shared_gate_proj", (Is, H)), ("shared_up_proj", (Is, H)),
                       ("shared_down_proj", (H, Is))):
        p[key] = nrm(*shape).to(torch.bfloat16).to(dev)
    if gated:
        p["shared_expert_gate"] = nrm(1, H).to(torch.bfloat16).to(dev)
    return p


def _inputs(dev, N, H, seed, scale=4.0):
    g = torch.Generator(device="cpu").manual_seed(1000 + seed)
    return (torch.randn(N, H, generator=g) * scale).to(torch.bfloat16).to(dev)


def _check(p, cfg, x, what, *, act="silu", alpha=1.702, limit=0.0, gs=64, bits=4, down_bits=None):
    y = qwen35_moe(x[None], p, cfg)[0]
    _, it = om.moe_forward(f64(x), oracle_params_from_torch(p), k=cfg.num_experts_per_tok,
                           inter=cfg.moe_intermediate_size, act=act, alpha=alpha, limit=limit,
                           group_size=gs, bits=bits, down_bits=down_bits)
    assert_close(f64(y), it["y_exact"], what)
    return y, it


@pytest.mark.parametrize("N", [1, 2, 8, 40])
def test_block_wide_shared_expert_vs_oracle(gpu, N):
    """A shared expert wider than the fused decode down takes (4096 features: 16 chunks of K,
    as Qwen2-MoE's 20480-wide one): its gate_up still rides in the router launch, and its down
    product must run after that launch, on the rows it wrote."""
    cfg = MoEConfig(512, 8, 2, 256, 4096)
    p = _layer(gpu, 64, seed=70 + N, Is=4096)
    _check(p, cfg, _inputs(gpu, N, 512, N), f"shared expert 4096 wide N={N}")


@pytest.mark.parametrize("N", [1, 5, 40, 300])
def test_block_group128_vs_oracle(gpu, N):
    """128-column groups through every regime (slot-major, decode, hybrid prefill)."""
    cfg = MoEConfig(512, 8, 2, 256, 256)
    p = _layer(gpu, 128, seed=N)
    _check(p, cfg, _inputs(gpu, N, 512, N), f"group 128 N={N}", gs=128)


@pytest.mark.parametrize("act,alpha,limit", [("swigluoai", 1.702, 1.5), ("silu", 1.0, 0.75),
                                             ("swigluoai", 1.702, 0.0)])
@pytest.mark.parametrize("N", [2, 20, 70, 300])
def test_block_gated_activation_vs_oracle(gpu, act, alpha, limit, N):
    """The clamped activations on routed and shared experts: slot-major (N <= 2), fused shared
    expert (N <= 64), auxiliary-stream shared expert and hybrid prefill (N > 256). The limits are
    small enough that the clamps bind on part of the gate/up values."""
    cfg = MoEConfig(512, 8, 2, 256, 256, hidden_act=act, swiglu_alpha=alpha, swiglu_limit=limit)
    p = _layer(gpu, 64, seed=7 * N)
    x = _inputs(gpu, N, 512, N)
    _, it = _check(p, cfg, x, f"{act} limit={limit} N={N}", act=act, alpha=alpha, limit=limit)
    if limit > 0 and N >= 20:
        gu = it["gu"]
        assert np.any(gu > limit), "the clamp must bind somewhere for the test to mean anything"


def test_gated_activation_dense_path_and_errors(gpu):
    """sparse=False (bf16 stacks, run-every-expert) takes the same activation; unknown
    activations and a non-positive clamp are refused."""
    cfg = MoEConfig(512, 8, 2, 256, 256, hidden_act="swigluoai", swiglu_alpha=1.702, swiglu_limit=1.5)
    p = _layer(gpu, 64, seed=3)
    x = _inputs(gpu, 9, 512, 3)
    gu, dn = p["experts_gate_up"], p["experts_down"]
    p16 = dict(p, experts_gate_up=ops.dequant(gu["packed"], gu["scale"], gu["bias"]),
               experts_down=ops.dequant(dn["packed"], dn["scale"], dn["bias"]))
    y_sparse = f64(qwen35_moe(x[None], p16, cfg))
    y_dense = f64(qwen35_moe(x[None], p16, cfg, sparse=False))
    assert_close(y_dense, y_sparse, "swigluoai dense vs sparse", want_rounded=True)
    with pytest.raises(ValueError, match="hidden_act"):
        qwen35_moe(x[None], p, MoEConfig(512, 8, 2, 256, 256, hidden_act="gelu"))
    codes, sb = ops.tile_int4(gu["packed"], gu["scale"], gu["bias"])
    with pytest.raises(ValueError, match="act_limit"):
        ops.grouped_qmm(x, K=512, n_rows=512, weight_format=L.FMT_INT4_G64, codes=codes, sb=sb,
                        epilogue=L.EPI_SWIGLU, out_rows=9, regime=L.REGIME_SMALL, dense_rows=9,
                        glu=L.ACT_SILU_CLAMP, glu_limit=0.0)


# ------------------------------------------------------------------------------------ int6
@pytest.mark.parametrize("gs", [64, 128])
def test_dequant_int6_bit_exact(gpu, gs):
    rng = np.random.default_rng(gs + 6)
    rows, K = 40, 384
    codes = rng.integers(0, 64, size=(rows, K))
    words = oq.pack_affine(codes, 6)
    s = oq.f32_to_bf16_bits((rng.random((rows, K // gs)) * 0.05 + 1e-3).astype(np.float32))
    b = oq.f32_to_bf16_bits((rng.standard_normal((rows, K // gs)) * 0.3).astype(np.float32))
    got = ops.dequant(words_dev(words, gpu), bf16_dev(s, gpu), bf16_dev(b, gpu), bits=6, group_size=gs)
    assert np.array_equal(bits_np(got), oq.dequant_bf16_bits(words, s, b, K, bits=6, group_size=gs))


@pytest.mark.parametrize("regime", [L.REGIME_SMALL, L.REGIME_LARGE])
@pytest.mark.parametrize("epi", [L.EPI_SWIGLU, L.EPI_BF16])
@pytest.mark.parametrize("N,k,E,H,rows", [(1, 4, 8, 4096, 256), (7, 3, 6, 256, 256),
                                          (200, 4, 4, 1024, 128), (1024, 4, 32, 256, 512),
                                          (300, 3, 5, 768, 768)])
def test_grouped_qmm_int6_vs_oracle(gpu, regime, epi, N, k, E, H, rows):
    """int6 (tiled nibble + high-bit planes) against the oracle's exact affine weights: the
    decode kernel through several launch shapes (chunks per wavefront, tiles per wavefront), and
    the 256-row prefill kernel (nibble plane staged in LDS as int4's, high-bit words in registers,
    fp16 dequant under per-row exponents computed for 6-bit codes)."""
    if regime == L.REGIME_LARGE and rows % 256:
        pytest.skip("the large regime tiles 256 weight rows")
    rng = np.random.default_rng(N + E + H + rows)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    x = oq.round_bf16(rng.standard_normal((N, H)))
    w = torch.from_numpy(rng.standard_normal((E, rows, H)).astype(np.float32) * 0.05).to(gpu)
    packed, s, b = quantize_affine(w, 6, group_size=64)
    dense = oq.dequant_exact(words_np(packed), bits_np(s), bits_np(b), H, bits=6)
    m_tile = L.SMALL_M_TILE if regime == L.REGIME_SMALL else L.LARGE_M_TILE
    counts, offsets, tile_off, sorted_slot, inv, tile_map = ops.permute(torch.from_numpy(idx).to(gpu), E,
                                                                        m_tile)
    codes, sb = ops.tile_int6(packed, s, b)
    rexp = None
    if regime == L.REGIME_LARGE:
        rexp = ops.row_exponents(s, b, bits=6)
        # each row's largest dequantized magnitude (codes 0..63) times 2^rexp lies in [2^13, 2^14)
        peak = np.abs(dense).max(axis=-1) * np.exp2(rexp.cpu().numpy().astype(np.float64))
        assert np.all((peak >= 2.0 ** 13) & (peak < 2.0 ** 14))
    out = ops.grouped_qmm(bf16_dev(oq.f32_to_bf16_bits(x.astype(np.float32)), gpu), K=H, n_rows=rows,
                          weight_format=L.FMT_INT6_G64, codes=codes, sb=sb, epilogue=epi,
                          out_rows=N * k, regime=regime, slot_of=sorted_slot, slot_div=k,
                          n_slots=N * k, offsets=offsets, tile_off=tile_off, tile_map=tile_map,
                          n_experts=E, row_exp=rexp)
    order = sorted_slot.cpu().numpy()
    full = np.einsum("mh,moh->mo", x[order // k], dense[idx.reshape(-1)[order]])
    want = oq.round_bf16(full)
    if epi == L.EPI_SWIGLU:
        want = om.swiglu(want, rows // 2)
    assert_close(f64(out), want, f"int6 qmm regime={regime} epi={epi} N={N} E={E} H={H} rows={rows}",
                 rel_l2=4e-3)


def _layer6(dev, gs, seed, H=512, E=8, I=256, Is=256):
    p = _layer(dev, gs, seed, H, E, I, Is)
    g = torch.Generator(device="cpu").manual_seed(seed + 1)
    for key, shape in (("experts_gate_up", (E, 2 * I, H)), ("experts_down", (E, H, I))):
        packed, s, b = quantize_affine((torch.randn(*shape, generator=g) * 0.02).to(dev), 6, group_size=gs)
        p[key] = {"packed": packed, "scale": s, "bias": b, "group_size": gs, "bits": 6}
    return p


@pytest.mark.parametrize("gs,act", [(64, "silu"), (64, "swigluoai"), (128, "swigluoai")])
@pytest.mark.parametrize("N", [1, 8, 40, 300])
def test_block_int6_vs_oracle(gpu, gs, act, N):
    """int6 experts through the block (MiniMax M3's combination is int6 + SwiGLU-OAI): slot-major,
    fused shared expert, auxiliary-stream shared expert, and above 256 tokens the large regime
    (the 256-row prefill kernel)."""
    limit = 1.5 if act == "swigluoai" else 0.0
    cfg = MoEConfig(512, 8, 2, 256, 256, hidden_act=act, swiglu_alpha=1.702, swiglu_limit=limit)
    p = _layer6(gpu, gs, seed=11 * N + gs)
    _check(p, cfg, _inputs(gpu, N, 512, N), f"int6 g{gs} {act} N={N}", act=act, limit=limit,
           gs=gs, bits=6)


@pytest.mark.parametrize("E,I,N", [(32, 256, 300), (8, 512, 1100)])
def test_block_int6_large_regime_vs_oracle(gpu, E, I, N):
    """int6 layers above 256 tokens: hot experts (more than 16 rows) on the 256-row prefill
    kernel, the rest on the decode kernel (E = 32 at 300 tokens holds both); the large regime's
    output against the oracle and against the decode kernel's."""
    cfg = MoEConfig(512, E, 2, I, 256, hidden_act="swigluoai", swiglu_alpha=1.702,
                    swiglu_limit=1.5)
    p = _layer6(gpu, 64, seed=5 * N + I, E=E, I=I)
    x = _inputs(gpu, N, 512, N)
    y, it = _check(p, cfg, x, f"int6 large regime E={E} I={I} N={N}", act="swigluoai",
                   limit=1.5, bits=6)
    counts = np.bincount(it["idx"].reshape(-1), minlength=E)
    if E == 32:
        assert counts.max() > 16 and counts.min() <= 16, "the layer must hold hot and cold experts"
    y_small = qwen35_moe(x[None], p, cfg, regime=L.REGIME_SMALL)[0]
    assert_close(f64(y), f64(y_small), f"int6 large vs decode kernel E={E} N={N}", want_rounded=True)



# ------------------------------------------------------------------------------------ int3
@pytest.mark.parametrize("gs", [64, 128])
def test_dequant_int3_bit_exact(gpu, gs):
    rng = np.random.default_rng(gs + 3)
    rows, K = 40, 384
    codes = rng.integers(0, 8, size=(rows, K))
    words = oq.pack_affine(codes, 3)
    s = oq.f32_to_bf16_bits((rng.random((rows, K // gs)) * 0.05 + 1e-3).astype(np.float32))
    b = oq.f32_to_bf16_bits((rng.standard_normal((rows, K // gs)) * 0.3).astype(np.float32))
    got = ops.dequant(words_dev(words, gpu), bf16_dev(s, gpu), bf16_dev(b, gpu), bits=3, group_size=gs)
    assert np.array_equal(bits_np(got), oq.dequant_bf16_bits(words, s, b, K, bits=3, group_size=gs))


@pytest.mark.parametrize("regime", [L.REGIME_SMALL, L.REGIME_LARGE])
@pytest.mark.parametrize("epi", [L.EPI_SWIGLU, L.EPI_BF16])
@pytest.mark.parametrize("N,k,E,H,rows", [(1, 4, 8, 4096, 256), (7, 3, 6, 256, 256),
                                          (200, 4, 4, 1024, 128), (1024, 4, 32, 256, 512),
                                          (300, 3, 5, 768, 768)])
def test_grouped_qmm_int3_vs_oracle(gpu, regime, epi, N, k, E, H, rows):
    """int3 (three code words per lane per tile superblock) against the oracle's exact affine
    weights: the decode kernel through several launch shapes, and the 256-row prefill kernel
    (768-byte superblocks staged in LDS by dword copies, fp16 dequant under row exponents for
    3-bit codes, one more power of two of headroom than int4)."""
    if regime == L.REGIME_LARGE and rows % 256:
        pytest.skip("the large regime tiles 256 weight rows")
    rng = np.random.default_rng(3 * N + E + H + rows)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    x = oq.round_bf16(rng.standard_normal((N, H)))
    w = torch.from_numpy(rng.standard_normal((E, rows, H)).astype(np.float32) * 0.05).to(gpu)
    packed, s, b = quantize_affine(w, 3, group_size=64)
    dense = oq.dequant_exact(words_np(packed), bits_np(s), bits_np(b), H, bits=3)
    m_tile = L.SMALL_M_TILE if regime == L.REGIME_SMALL else L.LARGE_M_TILE
    counts, offsets, tile_off, sorted_slot, inv, tile_map = ops.permute(torch.from_numpy(idx).to(gpu), E,
                                                                        m_tile)
    codes, sb = ops.tile_int3(packed, s, b)
    rexp = None
    if regime == L.REGIME_LARGE:
        rexp = ops.row_exponents(s, b, bits=3)
        # each row's largest dequantized magnitude (codes 0..7) times 2^rexp lies in [2^13, 2^14)
        peak = np.abs(dense).max(axis=-1) * np.exp2(rexp.cpu().numpy().astype(np.float64))
        assert np.all((peak >= 2.0 ** 13) & (peak < 2.0 ** 14))
    out = ops.grouped_qmm(bf16_dev(oq.f32_to_bf16_bits(x.astype(np.float32)), gpu), K=H, n_rows=rows,
                          weight_format=L.FMT_INT3_G64, codes=codes, sb=sb, epilogue=epi,
                          out_rows=N * k, regime=regime, slot_of=sorted_slot, slot_div=k,
                          n_slots=N * k, offsets=offsets, tile_off=tile_off, tile_map=tile_map,
                          n_experts=E, row_exp=rexp)
    order = sorted_slot.cpu().numpy()
    full = np.einsum("mh,moh->mo", x[order // k], dense[idx.reshape(-1)[order]])
    want = oq.round_bf16(full)
    if epi == L.EPI_SWIGLU:
        want = om.swiglu(want, rows // 2)
    assert_close(f64(out), want, f"int3 qmm regime={regime} epi={epi} N={N} E={E} H={H} rows={rows}",
                 rel_l2=4e-3)


def _layer_widths(dev, gs, seed, gu_bits, dn_bits, H=512, E=8, I=256, Is=256):
    p = _layer(dev, gs, seed, H, E, I, Is)
    g = torch.Generator(device="cpu").manual_seed(seed + 1)
    for key, shape, bits in (("experts_gate_up", (E, 2 * I, H), gu_bits), ("experts_down", (E, H, I), dn_bits)):
        packed, s, b = quantize_affine((torch.randn(*shape, generator=g) * 0.02).to(dev), bits, group_size=gs)
        p[key] = {"packed": packed, "scale": s, "bias": b, "group_size": gs, "bits": bits}
    return p


@pytest.mark.parametrize("gs,gu_bits,dn_bits", [(128, 3, 4), (64, 3, 3), (128, 6, 4), (64, 4, 6)])
@pytest.mark.parametrize("N", [1, 8, 40, 300])
def test_block_mixed_widths_vs_oracle(gpu, gs, gu_bits, dn_bits, N):
    """Per-projection widths through the block: Kimi's gate/up int3 + down int4 at group 128, int3
    throughout, and the other mixes of the decode kernel's formats. Slot-major, fused shared
    expert, auxiliary-stream shared expert, and above 256 tokens the large regime (the 256-row
    prefill kernel for int3 and int6 stacks)."""
    cfg = MoEConfig(512, 8, 2, 256, 256)
    p = _layer_widths(gpu, gs, 13 * N + gs + gu_bits, gu_bits, dn_bits)
    _check(p, cfg, _inputs(gpu, N, 512, N), f"gate_up int{gu_bits} down int{dn_bits} g{gs} N={N}",
           gs=gs, bits=gu_bits, down_bits=dn_bits)


@pytest.mark.parametrize("gs,gu_bits,dn_bits,E,N,I", [(128, 3, 4, 32, 300, 256), (64, 3, 3, 8, 1100, 256),
                                                      (128, 3, 4, 32, 300, 512), (64, 3, 3, 32, 300, 512)])
def test_block_int3_large_regime_vs_oracle(gpu, gs, gu_bits, dn_bits, E, N, I):
    """int3 layers above 256 tokens (Kimi's gate/up int3 + down int4 at group 128, and int3
    throughout): hot experts on the prefill kernels, the rest on the decode kernel (E = 32 at 300
    tokens holds both); against the oracle and against the decode kernel's output. I = 256 runs
    the int3 stacks on the 256-row kernel; I = 512 gives gate_up 1024 rows, a multiple of 512, so
    the 512-row int3 kernel (qmm_wide_int3_kernel) takes it, and with int3 down (H = 512 rows)
    the down projection too, both over the hybrid regime's tile maps."""
    cfg = MoEConfig(512, E, 2, I, 256)
    p = _layer_widths(gpu, gs, 13 * N + gs + I, gu_bits, dn_bits, E=E, I=I)
    x = _inputs(gpu, N, 512, N)
    y, it = _check(p, cfg, x, f"int{gu_bits}/int{dn_bits} g{gs} large regime E={E} N={N}", gs=gs,
                   bits=gu_bits, down_bits=dn_bits)
    counts = np.bincount(it["idx"].reshape(-1), minlength=E)
    if E == 32:
        assert counts.max() > 16 and counts.min() <= 16, "the layer must hold hot and cold experts"
    y_small = qwen35_moe(x[None], p, cfg, regime=L.REGIME_SMALL)[0]
    assert_close(f64(y), f64(y_small), f"int3 large vs decode kernel E={E} N={N}", want_rounded=True)


@pytest.mark.parametrize("fmt", [dict(bits=3, down_bits=4, group_size=128), dict(bits=6)],
                         ids=["int3+int4-g128", "int6"])
def test_narrow_formats_batch_invariance_full_size(gpu, fmt):
    """The K-chunk count of the int3/int6 decode kernel follows the weight shape only, so a token's
    output at 128 tokens (few wavefronts per job, two chunks each) is bit-identical to its output
    alone (one chunk per wavefront), at the c2 shapes (K = 4096 gate_up, K = 1024 down)."""
    from quanta_amd import synth
    from quanta_amd.moe import TiledExperts, tile_experts_packed

    cfg = synth.spec("c2").cfg
    p = synth.make_layer("c2", device=gpu, **fmt)
    p["experts_gate_up"] = TiledExperts(**tile_experts_packed(p["experts_gate_up"]))
    p["experts_down"] = TiledExperts(**tile_experts_packed(p["experts_down"]))
    N = 128
    x = synth.make_inputs("c2", N, device=gpu, seed=N)
    full = qwen35_moe(x[None], p, cfg)[0]
    for t in (0, N // 3, N - 1):
        single = qwen35_moe(x[t:t + 1][None], p, cfg)[0, 0]
        assert torch.equal(single, full[t]), f"token {t} of {N}"


# ------------------------------------------------------------------------------ edge sizes
@pytest.mark.parametrize("E,k,N", [(1024, 16, 2), (64, 64, 3), (16, 16, 5), (1024, 8, 300),
                                   (16, 16, 2), (64, 64, 2), (64, 64, 1), (16, 12, 2)])
def test_block_router_limits_vs_oracle(gpu, E, k, N):
    """The router's limits through the whole block: the largest expert count (1024), the
    largest top-k (64), k = E (every expert on every token), at decode and prefill sizes. One
    or two tokens route slot-major, one m-tile per slot: with k > E / 2 that is more tiles than
    the permute's bound, so the tile map is sized for N * k."""
    cfg = MoEConfig(256, E, k, 128, 128)
    p = _layer(gpu, 64, seed=E + k + N, H=256, E=E, I=128, Is=128)
    x = _inputs(gpu, N, 256, N)
    y = qwen35_moe(x[None], p, cfg)[0]
    _, it = om.moe_forward(f64(x), oracle_params_from_torch(p), k=k, inter=128)
    assert_close(f64(y), it["y_exact"], f"E={E} k={k} N={N}")


def test_block_empty_input(gpu):
    cfg = MoEConfig(512, 8, 2, 256, 256)
    p = _layer(gpu, 64, seed=2)
    x = torch.empty(1, 0, 512, dtype=torch.bfloat16, device=gpu)
    y = qwen35_moe(x, p, cfg)
    assert y.shape == (1, 0, 512) and y.dtype == torch.bfloat16
