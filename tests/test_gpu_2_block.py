"""GPU tier: the whole block through the reference surface (qwen35_moe / Qwen35MoEModule) and the
C ABI's qmoe_forward, against the golden fixtures and, at the BASELINE configurations' full sizes
and every batch they name, every token against a float64 GPU restatement of the oracle that is
itself checked against the oracle on sampled tokens, plus size-independent properties.

Bars (BASELINE parity gates): top-k expert ids bit-exact outside float32 near-ties; layer output
bf16 within max-abs 2e-2 and relative L2 5e-3.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq
from quanta_amd import _lib as L
from quanta_amd import ops, synth
from quanta_amd.moe import MoEConfig, Qwen35MoEModule, qwen35_moe, qwen35_route
from tests import _gpu_ref as gpu_ref
from tests._util import (RAW_GATE_PEAK_BASELINE, assert_close, bf16_dev, bits_np, f64,
                         oracle_params_from_torch, words_dev, words_np)

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


# ----------------------------------------------------------------------------------- fixtures


def _fixture(name, dev):
    a = dict(np.load(GOLDEN / f"{name}.npz"))
    H, E, k, I, Is, ng, tg, norm, sig = a["dims"].tolist()
    cfg = MoEConfig(H, E, k, I, Is, scoring_func="sigmoid" if sig else "softmax",
                    norm_topk_prob=bool(norm), n_group=ng, topk_group=tg,
                    routed_scaling_factor=float(a["routed_scale"][0]))
    p = {"gate": torch.from_numpy(a["gate_f32"]).to(dev) if "gate_f32" in a else bf16_dev(a["gate"], dev)}
    for pre, key in (("gu", "experts_gate_up"), ("dn", "experts_down")):
        p[key] = {"packed": words_dev(a[f"{pre}_packed"], dev), "scale": bf16_dev(a[f"{pre}_scale"], dev),
                  "bias": bf16_dev(a[f"{pre}_bias"], dev), "group_size": 64, "bits": 4}
    for kk in ("shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
        if kk in a:
            p[kk] = bf16_dev(a[kk], dev)
    if "e_score_correction_bias" in a:
        p["e_score_correction_bias"] = torch.from_numpy(a["e_score_correction_bias"]).to(dev)
    x = bf16_dev(a["x"], dev)
    return a, cfg, p, x


@pytest.mark.parametrize("name", ["c0", "c1mini", "c3mini"])
def test_block_golden(gpu, name):
    a, cfg, p, x = _fixture(name, gpu)
    y = qwen35_moe(x[None], p, cfg)[0]
    assert_close(f64(y), a["y_exact"], f"golden {name}", raw_peak=RAW_GATE_PEAK_BASELINE)
    idx, w = qwen35_route(x, p["gate"], cfg,
                          e_score_correction_bias=p.get("e_score_correction_bias"))
    ok = a["margin"] > 1e-6
    assert np.array_equal(idx.cpu().numpy()[ok], a["idx"][ok])
    assert np.allclose(w.cpu().numpy()[ok], a["w"][ok], rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("name", ["c0", "c1mini"])
@pytest.mark.parametrize("regime", [L.REGIME_SMALL, L.REGIME_LARGE])
def test_block_golden_both_regimes(gpu, name, regime):
    a, cfg, p, x = _fixture(name, gpu)
    y = qwen35_moe(x[None], p, cfg, regime=regime)[0]
    assert_close(f64(y), a["y_exact"], f"golden {name} regime={regime}")


def test_module_equals_function(gpu):
    a, cfg, p, x = _fixture("c1mini", gpu)
    mod = Qwen35MoEModule(cfg, device=gpu)
    mod.gate = p["gate"]
    for kk in ("shared_gate_proj", "shared_up_proj", "shared_down_proj", "shared_expert_gate"):
        setattr(mod, kk, p[kk])
    mod.set_experts_packed(p["experts_gate_up"], p["experts_down"])
    y_mod = mod(x[None])
    y_fn = qwen35_moe(x[None], p, cfg)
    assert torch.equal(y_mod, y_fn)
    assert isinstance(mod.experts_gate_up, dict)   # packed auto-detection still sees a dict


def test_topk_override_and_errors(gpu):
    a, cfg, p, x = _fixture("c1mini", gpu)
    op = oracle_params_from_torch(p)
    xf = f64(x)
    for k in (1, 2):
        y = qwen35_moe(x[None], p, cfg, topk_override=k)[0]
        _, it = om.moe_forward(xf, op, k=k, inter=cfg.moe_intermediate_size)
        assert_close(f64(y), it["y_exact"], f"topk_override={k}")
    for bad in (0, cfg.num_experts_per_tok + 1):
        with pytest.raises(ValueError, match="topk_override"):
            qwen35_moe(x[None], p, cfg, topk_override=bad)
    with pytest.raises(ValueError, match="sparse=False"):
        qwen35_moe(x[None], p, cfg, sparse=False)
    with pytest.raises(TypeError):
        qwen35_moe(x[None].half(), p, cfg)
    # float32 activations take the reference-dtype path: float32 out, the bf16 block's routing
    # and (x being bf16-valued) the same values to the bf16 output's rounding
    y32 = qwen35_moe(x[None].float(), p, cfg)[0]
    assert y32.dtype == torch.float32
    assert_close(f64(y32), f64(qwen35_moe(x[None], p, cfg)[0]), "float32 x", want_rounded=True)
    # a group size that does not match the stored scales fails loud
    bad = dict(p["experts_gate_up"], group_size=32)
    with pytest.raises(ValueError, match="group_size"):
        qwen35_moe(x[None], dict(p, experts_gate_up=bad), cfg)


def test_topk_override_one_moegate_keeps_score(gpu):
    """A sigmoid + correction-bias router (MoEGate) at k = 1 keeps the expert's score times the
    routed scale instead of renormalising it to 1 (`topk > 1 and norm_topk_prob`,
    src/quanta/modeling/moe.py:41, src/quanta/glm/moe.py:53)."""
    a, cfg, p, x = _fixture("c3mini", gpu)
    assert cfg.scoring_func == "sigmoid" and cfg.norm_topk_prob
    op = oracle_params_from_torch(p)
    xf = f64(x)
    kw = dict(k=1, inter=cfg.moe_intermediate_size, scoring="sigmoid", norm_topk=True,
              n_group=cfg.n_group, topk_group=cfg.topk_group, scale=cfg.routed_scaling_factor)
    _, keep = om.moe_forward(xf, op, norm_single=False, **kw)
    _, renorm = om.moe_forward(xf, op, norm_single=True, **kw)
    assert not np.allclose(keep["w"], renorm["w"])
    y = qwen35_moe(x[None], p, cfg, topk_override=1)[0]
    assert_close(f64(y), keep["y_exact"], "c3mini MoEGate k=1")
    idx, w = qwen35_route(x, p["gate"], cfg, topk_override=1,
                          e_score_correction_bias=p["e_score_correction_bias"])
    ok = om.route_margin(keep["choice"], 1) > 1e-5
    assert np.array_equal(idx.cpu().numpy()[ok], keep["idx"][ok])
    assert np.allclose(w.cpu().numpy()[ok], keep["w"][ok], rtol=1e-5, atol=1e-7)
    # the explicit override restores qwen35_route's rule
    cfg1 = MoEConfig(**{**cfg.__dict__, "norm_topk_single": True})
    y1 = qwen35_moe(x[None], p, cfg1, topk_override=1)[0]
    assert_close(f64(y1), renorm["y_exact"], "c3mini k=1 renormalised")


def test_token_chunking_and_batch_invariance(gpu):
    a, cfg, p, x = _fixture("c1mini", gpu)
    full = qwen35_moe(x[None], p, cfg, token_chunk=8192)
    chunked = qwen35_moe(x[None], p, cfg, token_chunk=3)
    assert torch.equal(full, chunked)   # per-token work is independent of the batch
    for t in (0, 5, 15):
        single = qwen35_moe(x[t:t + 1][None], p, cfg)
        assert torch.equal(single[0, 0], full[0, t])


def test_dense_oracle_path_matches_sparse(gpu):
    """bf16 expert stacks: sparse gather path == run-every-expert path (sparse=False), and both
    match the packed path on the same (dequantized) codes, as the reference's
    _moe_packed_parity gate checks (parity/qwen35_forward_test.py:216-271)."""
    a, cfg, p, x = _fixture("c1mini", gpu)
    gu, dn = p["experts_gate_up"], p["experts_down"]
    p16 = dict(p, experts_gate_up=ops.dequant(gu["packed"], gu["scale"], gu["bias"]),
               experts_down=ops.dequant(dn["packed"], dn["scale"], dn["bias"]))
    y_sparse = f64(qwen35_moe(x[None], p16, cfg))
    y_dense = f64(qwen35_moe(x[None], p16, cfg, sparse=False))
    y_packed = f64(qwen35_moe(x[None], p, cfg))
    assert_close(y_dense, y_sparse, "dense vs sparse (bf16 stacks)", want_rounded=True)
    assert_close(y_packed, y_sparse, "packed vs bf16-dequant stacks", want_rounded=True)


def test_forward_capi_rejects_bad_workspace(gpu):
    a, cfg, p, x = _fixture("c0", gpu)
    from quanta_amd.moe import prepare

    pr = prepare(p, cfg)
    small = torch.empty(16, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError, match="workspace too small"):
        L.check(L.load().qmoe_forward(__import__("ctypes").byref(pr.cfg),
                                      __import__("ctypes").byref(pr.weights), x.data_ptr(),
                                      x.shape[0], x.data_ptr(), small.data_ptr(), 16, None),
                "qmoe_forward")


# ----------------------------------------------------------------------------------- full size

_LAYERS: dict = {}


def _layer(name, dev):
    if name not in _LAYERS:
        _LAYERS.clear()
        torch.cuda.empty_cache()
        _LAYERS[name] = synth.make_layer(name, device=dev)
    return _LAYERS[name]


def _oracle_tokens(p, cfg, x64, toks, idx, w):
    """Oracle output for the sampled tokens only, fetching just the routed experts."""
    H, I = cfg.hidden_size, cfg.moe_intermediate_size
    gu, dn = p["experts_gate_up"], p["experts_down"]
    cache = {}

    def expert(e):
        if e not in cache:
            cache[e] = (oq.dequant_exact(words_np(gu["packed"][e]), bits_np(gu["scale"][e]),
                                         bits_np(gu["bias"][e]), H),
                        oq.dequant_exact(words_np(dn["packed"][e]), bits_np(dn["scale"][e]),
                                         bits_np(dn["bias"][e]), I))
        return cache[e]

    out = np.zeros((len(toks), H))
    sh = None
    if p.get("shared_gate_proj") is not None:
        sh, _, _ = om.shared_expert(x64[toks], f64(p["shared_gate_proj"]), f64(p["shared_up_proj"]),
                                    f64(p["shared_down_proj"]),
                                    f64(p["shared_expert_gate"]) if p.get("shared_expert_gate") is not None else None)
    for i, t in enumerate(toks):
        for s in range(idx.shape[1]):
            wg, wd = expert(int(idx[t, s]))
            gu_v = oq.round_bf16(x64[t] @ wg.T)
            h = oq.round_bf16(gu_v[:I] / (1 + np.exp(-gu_v[:I])) * gu_v[I:])
            d = oq.round_bf16(h @ wd.T)
            out[i] += w[t, s] * d
    if sh is not None:
        out += sh
    return out     # unrounded: the GPU's bf16 output then carries one rounding


def _full_parity(gpu, name, p, cfg, x, y, *, sample=3, tie_tol=1e-5):
    """Every token of y against the float64 GPU restatement of the oracle (tests/_gpu_ref.py),
    itself pinned to the oracle on sampled tokens.

    Routing: the top-k ids must equal the oracle's wherever the k-th and (k+1)-th choice values
    are further apart than float32 evaluation error; on the rows within that margin (near-ties)
    either choice is correct, so the reference takes the GPU's ids, checks that each is within
    the margin of the oracle's k-th choice, and weighs them with the oracle's float64 scores."""
    N = x.shape[0]
    k = cfg.num_experts_per_tok
    x64 = f64(x)
    bias = f64(p["e_score_correction_bias"]) if p.get("e_score_correction_bias") is not None else None
    moegate = cfg.scoring_func == "sigmoid" and bias is not None
    idx_o, w_o, logits_o, scores_o, choice_o = om.route(
        x64, f64(p["gate"]), k=k, scoring=cfg.scoring_func, norm_topk=cfg.norm_topk_prob,
        bias=bias, n_group=cfg.n_group, topk_group=cfg.topk_group,
        scale=cfg.routed_scaling_factor, norm_single=not moegate)
    idx, _ = qwen35_route(x, p["gate"], cfg, e_score_correction_bias=p.get("e_score_correction_bias"))
    idx = idx.cpu().numpy()
    sel = logits_o if cfg.scoring_func == "softmax" and bias is None else choice_o
    tol = tie_tol * np.max(np.abs(x64) @ np.abs(f64(p["gate"])).T, axis=1)
    tie = om.route_margin(sel, k) <= tol
    # the ids as sets: the reference's argpartition leaves the order within the top k open, and
    # two selected experts closer than float32 error may swap places in the canonical order
    order_diff = int((idx[~tie] != idx_o[~tie]).any(axis=1).sum())
    print(f"[parity] {name} N={N}: {int(tie.sum())} near-tie rows of {N}, {order_diff} rows "
          "ordered differently within the top k", flush=True)
    assert np.array_equal(np.sort(idx[~tie], axis=1), np.sort(idx_o[~tie], axis=1))
    idx_ref, w_ref = idx_o.copy(), w_o.copy()
    for t in np.flatnonzero(tie):
        kth = np.sort(sel[t])[::-1][k - 1]
        assert np.all(sel[t, idx[t]] >= kth - tol[t]), f"token {t}: GPU ids outside the tie margin"
        ws = scores_o[t, idx[t]]
        if cfg.norm_topk_prob and (k > 1 or not moegate):
            ws = ws / (ws.sum() + 1e-20)
        idx_ref[t], w_ref[t] = idx[t], ws * cfg.routed_scaling_factor
    y_ref = gpu_ref.block_reference(p, cfg, x, idx_ref, w_ref).cpu().numpy()
    toks = sorted({0, N // 2, N - 1})[:sample] if N > 2 else list(range(N))
    gpu_ref.pin_to_oracle(y_ref[toks], _oracle_tokens(p, cfg, x64, toks, idx_ref, w_ref),
                          f"{name} N={N} tokens {toks}")
    assert_close(f64(y), y_ref, f"{name} N={N}, all {N} tokens", raw_peak=RAW_GATE_PEAK_BASELINE)


@pytest.mark.parametrize("name,N", [("c1", 1), ("c1", 8), ("c1", 32), ("c1", 64),
                                    ("c2", 1), ("c2", 8), ("c2", 32), ("c2", 128),
                                    ("c3", 1), ("c3", 16), ("c3", 64)])
def test_block_full_size(gpu, name, N):
    """BASELINE configs 1-3 at every batch they name: every token against the reference."""
    cfg = synth.spec(name).cfg
    p = _layer(name, gpu)
    x = synth.make_inputs(name, N, device=gpu, seed=N)
    y = qwen35_moe(x[None], p, cfg)[0]
    assert torch.isfinite(y.float()).all()
    _full_parity(gpu, name, p, cfg, x, y)


@pytest.mark.parametrize("name,N", [("c2", 128), ("c3", 64)])
def test_batch_invariance_full_size(gpu, name, N):
    """Large decode batches stream each job's K chunks on fewer wavefronts than single tokens do;
    the chunk sums are still added in one fixed order, so every token's output is bit-identical
    to its output when it is the only token of the call."""
    cfg = synth.spec(name).cfg
    p = _layer(name, gpu)
    x = synth.make_inputs(name, N, device=gpu, seed=N)
    full = qwen35_moe(x[None], p, cfg)[0]
    for t in (0, N // 3, N - 1):
        single = qwen35_moe(x[t:t + 1][None], p, cfg)[0, 0]
        assert torch.equal(single, full[t]), f"{name} token {t} of {N}"


@pytest.mark.parametrize("name", ["c1", "c2", "c3"])
def test_fused_shared_expert_matches_unfused(gpu, name):
    """Up to 64 tokens the shared expert runs inside the router and combine launches; above, as
    its own launches. Up to a few tokens (3 at c3, 5 at c2, 11 at c1) the batch is routed
    slot-major in place of the permute; for one or two tokens the top-k runs inside the routed
    gate_up launch, and the routed down, the shared down and the combine run as one launch per
    16 output features (c2 N=1, c1 N<=2). The summation order is the same on every path, so the first N
    tokens of a 65-token call equal an N-token call bit for bit, on every repeat."""
    cfg = synth.spec(name).cfg
    p = _layer(name, gpu)
    x = synth.make_inputs(name, 65, device=gpu, seed=65)
    y65 = qwen35_moe(x[None], p, cfg)[0]
    for N in (64, 17, 11, 8, 6, 4, 3, 2, 1):
        for rep in range(8 if N == 64 else 2):
            yN = qwen35_moe(x[:N][None], p, cfg)[0]
            assert torch.equal(yN, y65[:N]), f"{name} N={N} repeat {rep}"


def test_prefill_zipf_c4(gpu):
    """all 4096 tokens of the Zipf prefill (hybrid large-M regime) against the
    reference, and the large and small regimes against each other."""
    cfg = synth.spec("c4").cfg
    p = _layer("c4", gpu)
    N = 4096
    x = synth.make_inputs("c4", N, device=gpu, seed=1)
    y_large = qwen35_moe(x[None], p, cfg)[0]                       # auto: large-M regime
    y_small = qwen35_moe(x[None], p, cfg, regime=L.REGIME_SMALL)[0]
    assert torch.isfinite(y_large.float()).all()
    assert_close(f64(y_large), f64(y_small), "c4 large vs small regime", want_rounded=True)
    idx, w = qwen35_route(x, p["gate"], cfg)
    counts = torch.bincount(idx.reshape(-1).long(), minlength=cfg.num_experts).cpu().numpy()
    print(f"[parity] c4 routing: max {counts.max()} median {int(np.median(counts))} "
          f"empty {(counts == 0).sum()}")
    assert counts.sum() == N * cfg.num_experts_per_tok and counts.max() > 500 and (counts == 0).any()
    _full_parity(gpu, "c4", p, cfg, x, y_large, tie_tol=1e-5)
    _full_parity(gpu, "c4 small regime", p, cfg, x, y_small, tie_tol=1e-5)


def test_prefill_chunking_contract_c4(gpu):
    """Above 256 tokens (the hybrid large-M regime) a token's output depends on which kernel ran
    each of its experts: experts routed more than 16 rows of the call run on the MFMA prefill
    kernels (fp16-dequantized weights), the others on the decode kernel (bf16 codes, the affine
    map on the products). Chunking the call changes those row counts, so the reference's batch
    invariance (src/quanta/qwen35/moe.py:97-100; its chunk gate, parity/moe_chunk_test.py:47-62)
    holds here within the parity gates, not bit for bit. The whole 4096-token Zipf call and the
    same tokens with token_chunk 1024 (four large-regime calls) and 300 (thirteen, then 196 tokens
    on the decode regime) each meet the gates against the reference on every token, lie within
    the gates of each other, and repeat bit for bit."""
    cfg = synth.spec("c4").cfg
    p = _layer("c4", gpu)
    N = 4096
    x = synth.make_inputs("c4", N, device=gpu, seed=1)
    whole = qwen35_moe(x[None], p, cfg)[0]
    assert torch.equal(qwen35_moe(x[None], p, cfg)[0], whole), "whole call not deterministic"
    for chunk in (1024, 300):
        y = qwen35_moe(x[None], p, cfg, token_chunk=chunk)[0]
        assert torch.equal(qwen35_moe(x[None], p, cfg, token_chunk=chunk)[0], y), f"chunk {chunk}"
        differ = float((y != whole).float().mean())
        print(f"[parity] c4 token_chunk={chunk}: {differ:.2%} of outputs differ from the whole "
              "call", flush=True)
        assert_close(f64(y), f64(whole), f"c4 token_chunk={chunk} vs whole", want_rounded=True)
        _full_parity(gpu, f"c4 token_chunk={chunk}", p, cfg, x, y, tie_tol=1e-5)
