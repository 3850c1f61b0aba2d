"""CPU tier: the committed golden fixtures are consistent with the oracle (regression pin of the
oracle and of the fixtures the GPU parity tests compare against)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import moe as om
from oracle import quant as oq
from tests.golden.make_golden import oracle_params

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = ["c0", "c1mini", "c3mini"]


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz"))


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    a = load(name)
    H, E, k, I, Is, ng, tg, norm, sig = a["dims"].tolist()
    xf = oq.bf16_bits_to_f32(a["x"]).astype(np.float64)
    y, it = om.moe_forward(xf, oracle_params(a), k=k, inter=I,
                           scoring="sigmoid" if sig else "softmax", norm_topk=bool(norm),
                           n_group=ng, topk_group=tg, scale=float(a["routed_scale"][0]))
    assert np.array_equal(it["idx"], a["idx"])
    assert np.allclose(it["w"], a["w"], rtol=1e-12)
    assert np.array_equal(oq.f32_to_bf16_bits(y.astype(np.float32)), a["y"])
    counts, offsets, order, inv = om.permute(a["idx"], E)
    for got, key in ((counts, "counts"), (offsets, "offsets"), (order, "order"), (inv, "inv")):
        assert np.array_equal(got, a[key])


@pytest.mark.parametrize("name", NAMES)
def test_fixture_dequant_matches_format(name):
    a = load(name)
    H = int(a["dims"][0])
    got = oq.dequant_bf16_bits(a["gu_packed"][0], a["gu_scale"][0], a["gu_bias"][0], H)
    assert np.array_equal(got, a["deq_gu_e0"])
    # every expert's ids are distinct within a token (top-k) and cover [0, E)
    E = int(a["dims"][1])
    assert all(len(set(r)) == len(r) for r in a["idx"].tolist())
    assert a["idx"].min() >= 0 and a["idx"].max() < E
