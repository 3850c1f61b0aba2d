"""GPU tier: the decode dataflow launch (flow.hip) against the multi-launch chain.

Slot-major decode batches with int4 experts, a bf16 router and a shared expert can run everything
after the router launch as one launch whose units hand data to each other through coherent loads
and stores and wait on counters in the workspace. Every product keeps its
standalone launch's chunking and summation order and the combine sums as combine_kernel, so the
output must equal the chain's (qmoe_set_decode_flow(0)) bit for bit, at both BASELINE decode
shapes (c1, c2), at every slot-major batch the kernel covers (forced with mode 2; by default it
runs for one and two tokens), on repeated calls (a missed handoff would show as a changed value),
with the residual add, through the allocation-free entry, and with no in-kernel wait running out
of its bound.
"""

from __future__ import annotations

import pytest
import torch

from quanta_amd import _lib as L
from quanta_amd import ops, synth
from quanta_amd.moe import prepare, qwen35_moe, qwen35_moe_residual
from tests.test_gpu_2_block import _layer

pytestmark = pytest.mark.gpu


def _mode(mode, fn):
    prev = L.load().qmoe_set_decode_flow(mode)
    try:
        return fn()
    finally:
        L.load().qmoe_set_decode_flow(prev)


def _chain(fn):
    return _mode(0, fn)


@pytest.mark.parametrize("name", ["c2", "c1"])
def test_flow_equals_chain_every_slot_major_batch(gpu, name):
    """The dataflow launch forced (mode 2) at every batch it covers (the slot-major sizes: up to
    6 tokens at c2, 11 at c1) equals the chain bit for bit, three calls in a row; the default mode
    (the dataflow launch for one and two tokens only) as well, at those and larger batches."""
    cfg = synth.spec(name).cfg
    p = _layer(name, gpu)
    before = L.load().qmoe_flow_timeouts()
    x = synth.make_inputs(name, 64, device=gpu, seed=7)
    for N in (1, 2, 3, 4, 5, 6, 7, 8, 9, 11, 12, 16, 33, 64):
        xn = x[:N][None]
        want = _chain(lambda: qwen35_moe(xn, p, cfg))
        for rep in range(3):
            got = _mode(2, lambda: qwen35_moe(xn, p, cfg))
            assert torch.equal(got, want), f"{name} N={N} forced, call {rep}"
        assert torch.equal(qwen35_moe(xn, p, cfg), want), f"{name} N={N} default mode"
    torch.cuda.synchronize()
    assert L.load().qmoe_flow_timeouts() == before, "an in-kernel wait ran out of its bound"


def test_flow_residual_and_noalloc(gpu):
    """The residual entry (norm fused in the router launch, residual added in the flow's
    combine) and the allocation-free entry (counters in the fixed scratch) equal the chain."""
    cfg = synth.spec("c2").cfg
    p = _layer("c2", gpu)
    g = torch.Generator(device="cpu").manual_seed(3)
    nw = (1.0 + 0.1 * torch.randn(cfg.hidden_size, generator=g)).to(torch.bfloat16).to(gpu)
    before = L.load().qmoe_flow_timeouts()
    for N in (1, 2, 4, 6):
        x = synth.make_inputs("c2", N, device=gpu, seed=100 + N)
        want = _chain(lambda: qwen35_moe_residual(x[None], p, cfg, nw))
        got = _mode(2, lambda: qwen35_moe_residual(x[None], p, cfg, nw))
        assert torch.equal(got, want), f"residual N={N}"
        pr = prepare(p, cfg)
        want = _chain(lambda: ops.forward(pr.cfg, pr.weights, x))
        got = _mode(2, lambda: ops.forward_noalloc(pr.cfg, pr.weights, x, torch.empty_like(x)))
        got2 = _mode(2, lambda: ops.forward_noalloc(pr.cfg, pr.weights, x, torch.empty_like(x)))
        assert torch.equal(got, want) and torch.equal(got2, want), f"noalloc N={N}"
    torch.cuda.synchronize()
    assert L.load().qmoe_flow_timeouts() == before, "an in-kernel wait ran out of its bound"
