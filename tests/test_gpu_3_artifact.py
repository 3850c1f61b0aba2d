"""GPU tier: the artifact path. int8-g64 dequant (the bake's shared-expert format) bit-exact
against the oracle, and the golden c1mini block read back from an artifact written in the
reference's layout, with its shared expert stored dense and as int8 g64.

Bars: dequant bit-exact; the block output equal (torch.equal) to the same block fed from the
fixture tensors directly, and within the BASELINE gates of the golden float64 output.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quant as oq
from quanta_amd import ops
from quanta_amd.artifact import LM_PREFIX, QuantaArtifact
from quanta_amd.moe import MoEConfig, qwen35_moe
from tests._artifact import ArtifactBuilder, bf16_from_bits, moe_config_json, u32
from tests._util import assert_close, bf16_dev, bits_np, f64, words_dev

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("rows,K", [(16, 64), (96, 512), (300, 1024)])
def test_dequant_int8_bit_exact(gpu, rows, K):
    rng = np.random.default_rng(rows + K)
    w = rng.standard_normal((rows, K)).astype(np.float32) * 0.05
    w[0, :64] = 0.25                       # a constant group (scale 1e-8)
    words, s_bits, b_bits, _ = oq.quantize_rtn(w, bits=8, group_size=64)
    want = oq.dequant_bf16_bits(words, s_bits, b_bits, K, bits=8)
    got = ops.dequant(words_dev(words, gpu), bf16_dev(s_bits, gpu), bf16_dev(b_bits, gpu), bits=8)
    assert np.array_equal(bits_np(got), want)


def _c1mini():
    a = dict(np.load(GOLDEN / "c1mini.npz"))
    H, E, k, I, Is, ng, tg, norm, sig = a["dims"].tolist()
    assert not sig and ng == 1
    return a, (H, E, k, I, Is, bool(norm))


def _write(a, dims, d: Path, shared_int8: bool):
    H, E, k, I, Is, norm = dims
    p = LM_PREFIX + "layers.0.mlp."
    b = ArtifactBuilder()
    b.add_dense(p + "gate.weight", bf16_from_bits(a["gate"]))
    b.add_dense(p + "shared_expert_gate.weight", bf16_from_bits(a["shared_expert_gate"]))
    deq = {}
    for proj in ("gate_proj", "up_proj", "down_proj"):
        w_bits = a[f"shared_{proj}"]
        if shared_int8:
            w = oq.bf16_bits_to_f32(w_bits)
            words, s_bits, b_bits, _ = oq.quantize_rtn(w, bits=8, group_size=64)
            b.add_quantized(p + f"shared_expert.{proj}", u32(words), bf16_from_bits(s_bits),
                            bf16_from_bits(b_bits), bits=8, group_size=64)
            deq[proj] = oq.dequant_bf16_bits(words, s_bits, b_bits, w.shape[-1], bits=8)
        else:
            b.add_dense(p + f"shared_expert.{proj}.weight", bf16_from_bits(w_bits))
            deq[proj] = w_bits
    for key, pre in (("experts.gate_up_proj", "gu"), ("experts.down_proj", "dn")):
        b.add_quantized(p + key, u32(a[f"{pre}_packed"]), bf16_from_bits(a[f"{pre}_scale"]),
                        bf16_from_bits(a[f"{pre}_bias"]), bits=4, group_size=64)
    b.write(d, moe_config_json(H, E, k, I, Is, norm), n_shards=2)
    return deq


def _direct(a, dims, deq, dev):
    """The same block fed from the fixture tensors directly (the test_gpu_2_block path)."""
    H, E, k, I, Is, norm = dims
    p = {"gate": bf16_dev(a["gate"], dev),
         "shared_expert_gate": bf16_dev(a["shared_expert_gate"], dev)}
    for pre, key in (("gu", "experts_gate_up"), ("dn", "experts_down")):
        p[key] = {"packed": words_dev(a[f"{pre}_packed"], dev), "scale": bf16_dev(a[f"{pre}_scale"], dev),
                  "bias": bf16_dev(a[f"{pre}_bias"], dev), "group_size": 64, "bits": 4}
    for proj, w in deq.items():
        p[f"shared_{proj}"] = bf16_dev(w, dev)
    cfg = MoEConfig(H, E, k, I, Is, norm_topk_prob=norm)
    return p, cfg


@pytest.mark.parametrize("shared_int8", [False, True])
def test_block_from_artifact(gpu, tmp_path, shared_int8):
    a, dims = _c1mini()
    deq = _write(a, dims, tmp_path / "art", shared_int8)
    art = QuantaArtifact(tmp_path / "art")
    p = art.moe_packed(0, gpu)
    for proj, w in deq.items():   # the int8 shared expert dequantized on the GPU, bit-exact
        assert np.array_equal(bits_np(p[f"shared_{proj}"]), w), proj
    x = bf16_dev(a["x"], gpu)
    y = qwen35_moe(x[None], p, art.moe_config())[0]
    p2, cfg2 = _direct(a, dims, deq, gpu)
    y2 = qwen35_moe(x[None], p2, cfg2)[0]
    assert torch.equal(y, y2)
    if not shared_int8:
        assert_close(f64(y), a["y_exact"], "c1mini from artifact")
    m = art.moe_module(0, gpu)
    assert torch.equal(m(x[None])[0], y)
    # the int8 shared expert handed over as its triplets (read at half the bytes): same outputs
    p8 = art.moe_packed(0, gpu, shared="int8")
    for proj in deq:
        assert isinstance(p8[f"shared_{proj}"], dict) == shared_int8, proj
    for n in (1, 9, 16):
        assert torch.equal(qwen35_moe(x[None, :n], p8, art.moe_config()),
                           qwen35_moe(x[None, :n], p, art.moe_config())), n


def test_sigmoid_router_from_artifact(gpu, tmp_path):
    """A bake whose config.json declares a sigmoid router with groups and a routed scale (the
    c3mini golden block: sigmoid + correction bias, 8 groups keep 4, x2.5): moe_config reads
    scoring_func (src/quanta/qwen35/config.py:361) and the DeepSeek/GLM fields, moe_packed picks
    up the stored selection bias, and the block matches the golden output. With scoring_func
    left out of the config, the same weights route with softmax and the output differs."""
    a = dict(np.load(GOLDEN / "c3mini.npz"))
    H, E, k, I, Is, ng, tg, norm, sig = a["dims"].tolist()
    assert sig and ng > 1
    p = LM_PREFIX + "layers.0.mlp."
    b = ArtifactBuilder()
    b.add_dense(p + "gate.weight", bf16_from_bits(a["gate"]))
    b.add_dense(p + "gate.e_score_correction_bias", torch.from_numpy(a["e_score_correction_bias"]))
    for proj in ("gate_proj", "up_proj", "down_proj"):
        b.add_dense(p + f"shared_expert.{proj}.weight", bf16_from_bits(a[f"shared_{proj}"]))
    for key, pre in (("experts.gate_up_proj", "gu"), ("experts.down_proj", "dn")):
        b.add_quantized(p + key, u32(a[f"{pre}_packed"]), bf16_from_bits(a[f"{pre}_scale"]),
                        bf16_from_bits(a[f"{pre}_bias"]), bits=4, group_size=64)
    cfg_json = moe_config_json(H, E, k, I, Is, bool(norm))
    cfg_json["text_config"].update(scoring_func="sigmoid", n_group=ng, topk_group=tg,
                                   routed_scaling_factor=float(a["routed_scale"][0]))
    art = QuantaArtifact(b.write(tmp_path / "sig", cfg_json))
    cfg = art.moe_config()
    assert (cfg.scoring_func, cfg.n_group, cfg.topk_group, cfg.routed_scaling_factor) == \
        ("sigmoid", ng, tg, float(a["routed_scale"][0]))
    x = bf16_dev(a["x"], gpu)
    pk = art.moe_packed(0, gpu)
    assert "e_score_correction_bias" in pk and "shared_expert_gate" not in pk
    y = qwen35_moe(x[None], pk, cfg)[0]
    assert_close(f64(y), a["y_exact"], "c3mini (sigmoid router) from artifact")
    assert torch.equal(art.moe_module(0, gpu)(x[None])[0], y)
    del cfg_json["text_config"]["scoring_func"]
    soft = QuantaArtifact(b.write(tmp_path / "soft", cfg_json))
    assert soft.moe_config().scoring_func == "softmax"
    y_soft = qwen35_moe(x[None], soft.moe_packed(0, gpu), soft.moe_config())[0]
    assert not torch.equal(y_soft, y)
