"""GPU tier, step by step: each C-ABI entry point against the oracle.

Bars: bit-exact for dequant, tiling, permutation/offsets and (outside float32 near-ties) the
top-k expert ids; float32 routing weights within 1e-5 relative; bf16 expert matmuls within the
BASELINE output tolerance (max-abs 2e-2, relative L2 5e-3), in practice about one bf16 ulp.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import quant as oq
from quanta_amd import _lib as L
from quanta_amd import ops
from tests._util import assert_close, bf16_dev, bits_np, f64, words_dev

pytestmark = pytest.mark.gpu


def _rand_stack(rng, E, rows, K, std=0.02):
    w = (rng.standard_normal((E, rows, K)) * std).astype(np.float32)
    packed, s, b, _ = oq.quantize_rtn(w, 4, 64)
    return packed, s, b


# ----------------------------------------------------------------------------------- formats


@pytest.mark.parametrize("E,rows,K", [(1, 16, 128), (3, 48, 384), (16, 512, 512), (2, 64, 7168)])
def test_dequant_bit_exact(gpu, E, rows, K):
    rng = np.random.default_rng(E * 7 + K)
    packed, s, b = _rand_stack(rng, E, rows, K, std=0.05)
    got = ops.dequant(words_dev(packed, gpu), bf16_dev(s, gpu), bf16_dev(b, gpu))
    want = oq.dequant_bf16_bits(packed, s, b, K)
    assert np.array_equal(bits_np(got), want)


@pytest.mark.parametrize("E,rows,K", [(1, 16, 128), (3, 48, 384), (4, 256, 1024)])
def test_tile_int4_lossless(gpu, E, rows, K):
    rng = np.random.default_rng(rows + K)
    packed, s, b = _rand_stack(rng, E, rows, K, std=0.05)
    codes, sb = ops.tile_int4(words_dev(packed, gpu), bf16_dev(s, gpu), bf16_dev(b, gpu))
    got = ops.dequant_tiled(codes, sb, E, rows, K)
    assert np.array_equal(bits_np(got), oq.dequant_bf16_bits(packed, s, b, K))


def test_tile_bf16_layout(gpu):
    E, rows, K = 2, 32, 96
    w = torch.arange(E * rows * K, dtype=torch.float32).remainder(251).to(torch.bfloat16)
    w = w.reshape(E, rows, K).to(gpu)
    t = ops.tile_bf16(w).cpu().reshape(E, rows // 16, K // 32, 64, 8)
    wc = w.cpu()
    for e, R, c, lane in [(0, 0, 0, 0), (1, 1, 2, 63), (0, 1, 1, 17), (1, 0, 0, 40)]:
        row = 16 * R + lane % 16
        k0 = 32 * c + 8 * (lane // 16)
        assert torch.equal(t[e, R, c, lane], wc[e, row, k0:k0 + 8])


# ----------------------------------------------------------------------------------- router


def _route_case(rng, N, E, H, k, scoring, bias=False, n_group=1, topk_group=1, scale=1.0,
                norm=True, norm_single=True):
    x = oq.round_bf16(rng.standard_normal((N, H)))
    wr = oq.round_bf16(rng.standard_normal((E, H)) * 0.02)
    bvec = rng.standard_normal(E) * 0.01 if bias else None
    return x, wr, bvec, dict(k=k, scoring=scoring, bias=bvec, n_group=n_group,
                             topk_group=topk_group, scale=scale, norm_topk=norm,
                             norm_single=norm_single)


def _route_kw(gpu, kw) -> dict:
    """ops.router / ops.router_topk keyword arguments of an oracle routing case."""
    return dict(scoring={"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}[kw["scoring"]],
                bias=None if kw["bias"] is None else
                torch.tensor(kw["bias"], dtype=torch.float32, device=gpu),
                n_group=kw["n_group"], topk_group=kw["topk_group"],
                norm_topk=(L.NORM_NONE if not kw["norm_topk"] else
                           L.NORM_ALWAYS if kw["norm_single"] else L.NORM_MULTI),
                routed_scale=kw["scale"])


def _check_route(gpu, x, wr, kw, logits_dev, E, got=None):
    """GPU routing vs the oracle: the top-k over `logits_dev`, or `got` = (idx, w) from a
    one-call router."""
    idx_o, w_o, logits_o, scores_o, choice_o = om.route(x, wr, **kw)
    k = kw["k"]
    if got is None:
        idx, w, _ = ops.router_topk(logits_dev, E, k, **_route_kw(gpu, kw))
    else:
        idx, w = got
    idx, w = idx.cpu().numpy(), w.cpu().numpy().astype(np.float64)
    # float32 logits carry ~|x||w| * 2^-24 * sqrt(H) error: rows whose selection gap is below a
    # generous bound of that are reported and compared as sets only.
    sel = logits_o if (kw["scoring"] == "softmax" and kw["bias"] is None) else choice_o
    margin = om.route_margin(sel, k)
    scale_l = np.abs(x) @ np.abs(wr).T
    tie = margin <= 1e-5 * np.maximum(scale_l.max(axis=1), 1.0)
    if kw["n_group"] > 1:   # the group selection has its own boundary gap
        n, e = choice_o.shape
        g = np.sort(choice_o.reshape(n, kw["n_group"], -1), axis=-1)[..., -2:].sum(-1)
        gm = om.route_margin(g, kw["topk_group"])
        tie |= gm <= 1e-5 * np.maximum(scale_l.max(axis=1), 1.0)
    ok = ~tie
    print(f"[parity] router: {ok.sum()}/{len(ok)} rows compared exactly ({tie.sum()} near-ties)")
    assert np.array_equal(idx[ok], idx_o[ok]), "top-k ids differ outside near-ties"
    assert all(set(a) == set(b) for a, b in zip(idx.tolist(), idx_o.tolist())) or tie.any()
    assert np.allclose(w[ok], w_o[ok], rtol=1e-5, atol=1e-7)
    return idx, w


@pytest.mark.parametrize("case", [
    dict(N=8, E=16, H=512, k=2, scoring="softmax"),
    dict(N=64, E=512, H=4096, k=10, scoring="softmax"),
    dict(N=33, E=256, H=2048, k=8, scoring="softmax"),
    dict(N=20, E=128, H=1024, k=6, scoring="sigmoid"),
    dict(N=64, E=256, H=7168, k=8, scoring="sigmoid", bias=True, n_group=8, topk_group=4, scale=2.5),
    dict(N=5, E=64, H=256, k=1, scoring="sigmoid", bias=True, norm=False),
    # k = 1 with renormalisation: a MoEGate keeps the score (x 2.5), qwen35_route gives 1
    dict(N=7, E=64, H=256, k=1, scoring="sigmoid", bias=True, scale=2.5, norm_single=False),
    dict(N=6, E=64, H=256, k=1, scoring="softmax"),
    dict(N=3, E=1024, H=256, k=16, scoring="softmax"),
    dict(N=40, E=256, H=1024, k=6, scoring="sqrtsoftplus", bias=True, scale=1.5),
    dict(N=9, E=384, H=512, k=8, scoring="sqrtsoftplus"),
])
def test_router_topk_vs_oracle(gpu, case):
    rng = np.random.default_rng(case["N"] * 31 + case["E"])
    x, wr, bvec, kw = _route_case(rng, case["N"], case["E"], case["H"], case["k"], case["scoring"],
                                  case.get("bias", False), case.get("n_group", 1),
                                  case.get("topk_group", 1), case.get("scale", 1.0),
                                  case.get("norm", True), case.get("norm_single", True))
    logits = ops.router_logits_f32(bf16_dev(oq.f32_to_bf16_bits(x.astype(np.float32)), gpu),
                                   torch.tensor(wr, dtype=torch.float32, device=gpu))
    lg = f64(logits)[:, :case["E"]]
    assert np.allclose(lg, x @ wr.T, rtol=1e-4, atol=1e-4)
    _check_route(gpu, x, wr, kw, logits, case["E"])


@pytest.mark.parametrize("case", [
    dict(N=1, E=512, H=2048, k=10, scoring="softmax"),
    dict(N=32, E=512, H=2048, k=10, scoring="softmax"),
    dict(N=7, E=256, H=2048, k=8, scoring="softmax"),
    dict(N=64, E=256, H=7168, k=8, scoring="sigmoid", bias=True, n_group=8, topk_group=4, scale=2.5),
    dict(N=5, E=64, H=256, k=1, scoring="sigmoid", bias=True, norm=False),
    dict(N=3, E=1024, H=264, k=16, scoring="softmax"),
    dict(N=40, E=256, H=1024, k=6, scoring="sqrtsoftplus", bias=True, scale=1.5),
])
@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_router_one_call_vs_oracle(gpu, case, wdt):
    """qmoe_router from the gate as stored (bf16 or fp32 [E, H], no tiling) against the oracle:
    ids exact outside float32 near-ties, weights within 1e-5 relative, the shared-expert gate
    sigmoid(x . g) alongside, and the same routing without the shared gate."""
    rng = np.random.default_rng(case["N"] * 37 + case["E"])
    x, wr, bvec, kw = _route_case(rng, case["N"], case["E"], case["H"], case["k"], case["scoring"],
                                  case.get("bias", False), case.get("n_group", 1),
                                  case.get("topk_group", 1), case.get("scale", 1.0),
                                  case.get("norm", True), case.get("norm_single", True))
    sgate = oq.round_bf16(rng.standard_normal(case["H"]) * 0.02)
    xd = bf16_dev(oq.f32_to_bf16_bits(x.astype(np.float32)), gpu)
    wd = torch.tensor(wr, dtype=torch.float32, device=gpu).to(wdt)
    sd = torch.tensor(sgate, dtype=torch.float32, device=gpu).to(wdt)
    idx, w, sg = ops.router(xd, wd, case["k"], shared_gate=sd, **_route_kw(gpu, kw))
    _check_route(gpu, x, wr, kw, None, case["E"], got=(idx, w))
    want_sg = 1.0 / (1.0 + np.exp(-(x @ sgate)))
    assert np.allclose(f64(sg), want_sg, rtol=1e-5, atol=1e-7)
    idx2, w2, sg2 = ops.router(xd, wd, case["k"], **_route_kw(gpu, kw))
    assert torch.equal(idx2, idx) and torch.equal(w2, w) and sg2 is None


def test_router_one_call_rejects():
    lib = L.load()
    rc = lib.qmoe_router(None, None, 0, None, None, 4, 100, 16, 2, 0, 1, 1, 1, 1.0, None, None, None,
                         None, 0, None)
    assert rc == L.QMOE_EINVAL


def test_router_bf16_mfma_logits(gpu):
    """bf16 router through the MFMA grouped-qmm (EPI_F32): logits equal x . Wr^T in float."""
    rng = np.random.default_rng(5)
    for N, E, H in ((1, 512, 4096), (40, 256, 2048), (300, 512, 4096)):
        x = oq.round_bf16(rng.standard_normal((N, H)))
        wr = oq.round_bf16(rng.standard_normal((E, H)) * 0.02)
        rows = ((E + 1 + 255) // 256) * 256
        full = np.zeros((rows, H))
        full[:E] = wr
        tiled = ops.tile_bf16(bf16_dev(oq.f32_to_bf16_bits(full.astype(np.float32)), gpu))
        for regime in (L.REGIME_SMALL, L.REGIME_LARGE):
            lg = ops.grouped_qmm(bf16_dev(oq.f32_to_bf16_bits(x.astype(np.float32)), gpu), K=H,
                                 n_rows=rows, weight_format=L.FMT_BF16, codes=tiled, sb=None,
                                 epilogue=L.EPI_F32, out_rows=N, regime=regime, dense_rows=N)
            got = f64(lg)[:, :E]
            ref = x @ wr.T
            err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
            print(f"[parity] bf16 router logits N={N} regime={regime}: rel max err {err:.2e}")
            assert err < 1e-5
            assert np.all(f64(lg)[:, E:] == 0.0)


# ----------------------------------------------------------------------------------- permute


@pytest.mark.parametrize("N,k,E,m_tile", [
    (1, 10, 512, 16), (8, 2, 16, 16), (128, 10, 512, 16), (300, 8, 256, 16), (4096, 10, 512, 128),
    (5, 1, 1, 16), (64, 64, 64, 16), (8192, 8, 256, 128), (1000, 3, 1024, 128),
    (2500, 4, 64, 16),
])
def test_permute_bit_exact(gpu, N, k, E, m_tile):
    rng = np.random.default_rng(N + k + E)
    if N >= 1000:   # skewed popularity: a few hot experts, many empty
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        p /= p.sum()
        idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(N)])
    else:
        idx = np.stack([rng.permutation(E)[:k] for _ in range(N)])
    idx = idx.astype(np.int32)
    counts, offsets, tile_off, sorted_slot, inv, tile_map = ops.permute(
        torch.from_numpy(idx).to(gpu), E, m_tile)
    c_o, off_o, order_o, inv_o = om.permute(idx, E)
    assert np.array_equal(counts.cpu().numpy(), c_o)
    assert np.array_equal(offsets.cpu().numpy(), off_o)
    assert np.array_equal(sorted_slot.cpu().numpy(), order_o)
    assert np.array_equal(inv.cpu().numpy(), inv_o)
    tiles = (c_o + m_tile - 1) // m_tile
    assert np.array_equal(tile_off.cpu().numpy(), np.concatenate([[0], np.cumsum(tiles)]))
    want = [[e, off_o[e] + i * m_tile, min(m_tile, c_o[e] - i * m_tile), 0]
            for e in range(E) for i in range(tiles[e])]
    tm = tile_map.cpu().numpy()
    assert np.array_equal(tm[:len(want)], np.array(want, dtype=np.int32).reshape(-1, 4))
    assert np.all(tm[len(want):, 0] == -1)


def test_permute_ignores_out_of_range_ids(gpu):
    idx = np.array([[0, 3], [5, 1], [-1, 2]], np.int32)   # 5 and -1 are outside [0, 4)
    counts, offsets, _, sorted_slot, inv, _ = ops.permute(torch.from_numpy(idx).to(gpu), 4, 16)
    assert counts.cpu().tolist() == [1, 1, 1, 1]
    assert offsets.cpu().tolist() == [0, 1, 2, 3, 4]
    inv = inv.cpu().numpy()
    assert inv[2] == -1 and inv[4] == -1
    assert sorted(sorted_slot.cpu().numpy()[:4].tolist()) == [0, 1, 3, 5]


# ----------------------------------------------------------------------------------- grouped qmm


def _qmm_problem(rng, N, k, E, H, rows, fmt):
    idx = np.stack([rng.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    x = oq.round_bf16(rng.standard_normal((N, H)))
    if fmt == L.FMT_INT4_G64:
        packed, s, b = _rand_stack(rng, E, rows, H)
        dense = oq.dequant_exact(packed, s, b, H)
        return idx, x, (packed, s, b), dense
    w = oq.round_bf16(rng.standard_normal((E, rows, H)) * 0.02)
    return idx, x, w, w


@pytest.mark.parametrize("fmt", [L.FMT_INT4_G64, L.FMT_BF16])
@pytest.mark.parametrize("regime", [L.REGIME_SMALL, L.REGIME_LARGE])
@pytest.mark.parametrize("epi", [L.EPI_SWIGLU, L.EPI_BF16])
# (1024, 4, 32, 256, 1024): enough m-tiles that the small kernel runs several jobs per
# wavefront (2 for SwiGLU, 4 otherwise)
@pytest.mark.parametrize("N,k,E,H,rows,use_map", [(7, 3, 6, 256, 256, True), (40, 2, 5, 512, 384, False),
                                                  (1, 4, 8, 4096, 256, True), (200, 4, 4, 1024, 128, True),
                                                  (300, 3, 5, 768, 512, True), (129, 2, 3, 256, 768, False),
                                                  (1024, 4, 32, 256, 1024, True)])
def test_grouped_qmm_vs_oracle(gpu, fmt, regime, epi, N, k, E, H, rows, use_map):
    if regime == L.REGIME_LARGE and rows % 256:
        pytest.skip("the large regime tiles 256 weight rows")
    rng = np.random.default_rng(N * 13 + E + H + rows + fmt)
    idx, x, w, dense = _qmm_problem(rng, N, k, E, H, rows, fmt)
    m_tile = L.SMALL_M_TILE if regime == L.REGIME_SMALL else L.LARGE_M_TILE
    counts, offsets, tile_off, sorted_slot, inv, tile_map = ops.permute(
        torch.from_numpy(idx).to(gpu), E, m_tile)
    rexp = None
    if fmt == L.FMT_INT4_G64:
        codes, sb = ops.tile_int4(words_dev(w[0], gpu), bf16_dev(w[1], gpu), bf16_dev(w[2], gpu))
        rexp = ops.row_exponents(bf16_dev(w[1], gpu), bf16_dev(w[2], gpu))
        # the defining property: each row's largest dequantized magnitude times 2^rexp lies in
        # [2^13, 2^14)
        peak = np.abs(dense).max(axis=-1) * np.exp2(rexp.cpu().numpy().astype(np.float64))
        assert np.all((peak >= 2.0 ** 13) & (peak < 2.0 ** 14))
    else:
        codes, sb = ops.tile_bf16(bf16_dev(oq.f32_to_bf16_bits(w.astype(np.float32)), gpu)), None
    xd = bf16_dev(oq.f32_to_bf16_bits(x.astype(np.float32)), gpu)
    out = ops.grouped_qmm(xd, K=H, n_rows=rows, weight_format=fmt, codes=codes, sb=sb,
                          row_exp=rexp,
                          epilogue=epi, out_rows=N * k, regime=regime, slot_of=sorted_slot,
                          slot_div=k, n_slots=N * k, offsets=offsets, tile_off=tile_off,
                          tile_map=tile_map if use_map else None, n_experts=E)
    order = sorted_slot.cpu().numpy()
    exp_sorted = idx.reshape(-1)[order]
    tok_sorted = order // k
    full = np.einsum("mh,moh->mo", x[tok_sorted], dense[exp_sorted])
    want = oq.round_bf16(full)
    if epi == L.EPI_SWIGLU:
        want = om.swiglu(want, rows // 2)
    # intermediate activations reach |h| ~ 10, so the absolute bound scales with the magnitude
    assert_close(f64(out), want, f"qmm fmt={fmt} regime={regime} epi={epi} N={N} E={E} H={H}",
                 rel_l2=4e-3)


def test_combine_vs_oracle(gpu):
    rng = np.random.default_rng(77)
    N, k, E, H = 9, 4, 12, 384
    idx = np.stack([rng.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    c_o, off_o, order, inv = om.permute(idx, E)
    d_sorted = oq.round_bf16(rng.standard_normal((N * k, H)))
    w = rng.random((N, k)).astype(np.float32)
    sh = oq.round_bf16(rng.standard_normal((N, H)))
    sg = rng.random(N).astype(np.float32)
    y = ops.combine(bf16_dev(oq.f32_to_bf16_bits(d_sorted.astype(np.float32)), gpu),
                    torch.from_numpy(inv).to(gpu), torch.from_numpy(w).to(gpu),
                    bf16_dev(oq.f32_to_bf16_bits(sh.astype(np.float32)), gpu),
                    torch.from_numpy(sg).to(gpu))
    d_slot = d_sorted[inv]
    want = oq.round_bf16(om.combine(d_slot, w.astype(np.float64)) + sh * sg[:, None])
    assert_close(f64(y), want, "combine", max_abs=1e-2, rel_l2=4e-3, want_rounded=True)
