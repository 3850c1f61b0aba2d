"""GPU tier: the routing tail of the router pair launch against the top-k and permute launches.

Decode batches sorted by expert (above the slot-major sizes) with a bf16 router and a shared
expert run the router logits and the shared gate_up in one launch; its last router workgroups to
finish can also rank the tokens (the top-k launch's arithmetic, on coherent loads of the logits;
one token per workgroup, up to 32 workgroups, once the count is complete) and the last of them
sorts the slots by expert (the permute launch's outputs). The block's output must equal the
separate launches' (qmoe_set_route_tail(0)) bit for bit at both BASELINE decode shapes, from
7 ranking workgroups to 32 (two tokens each at 64), on repeated calls (the arrival counter resets
itself), with the residual add (the RMSNorm fused into the same launch), through the
allocation-free entry and over a workspace whose bytes start as garbage (the counter needs no
clearing).
"""

from __future__ import annotations

import pytest
import torch

from quanta_amd import _lib as L
from quanta_amd import ops, synth
from quanta_amd.moe import prepare, qwen35_moe, qwen35_moe_residual
from tests.test_gpu_2_block import _layer

pytestmark = pytest.mark.gpu


def _tail(mode, fn):
    prev = L.load().qmoe_set_route_tail(mode)
    try:
        return fn()
    finally:
        L.load().qmoe_set_route_tail(prev)


def test_route_tail_switch_returns_previous():
    lib = L.load()
    prev = lib.qmoe_set_route_tail(0)
    try:
        assert prev == 1   # the default
        assert lib.qmoe_set_route_tail(7) == 0   # unknown: no change
        assert lib.qmoe_set_route_tail(1) == 0
        assert lib.qmoe_set_route_tail(1) == 1
    finally:
        lib.qmoe_set_route_tail(prev)


@pytest.mark.parametrize("name", ["c2", "c1"])
def test_route_tail_equals_separate_launches(gpu, name):
    """Every batch from the first sorted size to 64 tokens (and past it, where the tail is off),
    three calls in a row, equals the top-k + permute launches bit for bit."""
    cfg = synth.spec(name).cfg
    p = _layer(name, gpu)
    before = L.load().qmoe_flow_timeouts()
    x = synth.make_inputs(name, 80, device=gpu, seed=11)
    for N in (6, 7, 8, 12, 13, 16, 17, 31, 32, 33, 48, 63, 64, 65, 80):
        xn = x[:N][None]
        want = _tail(0, lambda: qwen35_moe(xn, p, cfg))
        for rep in range(3):
            got = _tail(1, lambda: qwen35_moe(xn, p, cfg))
            assert torch.equal(got, want), f"{name} N={N}, call {rep}"
    torch.cuda.synchronize()
    assert L.load().qmoe_flow_timeouts() == before, "a ranker's wait ran out of its bound"


def test_route_tail_residual_noalloc_and_garbage_workspace(gpu):
    """The residual entry (norm fused in the router launch), the allocation-free entry and a
    workspace filled with 0xFF bytes before the first call equal the separate launches."""
    cfg = synth.spec("c2").cfg
    p = _layer("c2", gpu)
    pr = prepare(p, cfg)
    g = torch.Generator(device="cpu").manual_seed(5)
    nw = (1.0 + 0.1 * torch.randn(cfg.hidden_size, generator=g)).to(torch.bfloat16).to(gpu)
    for N in (8, 32, 64):
        x = synth.make_inputs("c2", N, device=gpu, seed=200 + N)
        want = _tail(0, lambda: qwen35_moe_residual(x[None], p, cfg, nw))
        got = _tail(1, lambda: qwen35_moe_residual(x[None], p, cfg, nw))
        assert torch.equal(got, want), f"residual N={N}"
        want = _tail(0, lambda: ops.forward(pr.cfg, pr.weights, x))
        for rep in range(2):
            got = _tail(1, lambda: ops.forward_noalloc(pr.cfg, pr.weights, x, torch.empty_like(x)))
            assert torch.equal(got, want), f"noalloc N={N}, call {rep}"
        ws = torch.full((ops.forward_workspace(pr.cfg, N),), 255, dtype=torch.uint8, device=gpu)
        for rep in range(2):
            got = _tail(1, lambda: ops.forward(pr.cfg, pr.weights, x, ws=ws))
            assert torch.equal(got, want), f"0xFF workspace N={N}, call {rep}"


@pytest.mark.parametrize("n", [8, 32])
def test_route_tail_graph_replay(gpu, n):
    """Captured into a HIP graph and replayed after eager calls on the same workspace, every
    replay equals the stream launches: the arrival counter is back at its tagged zero after each
    call, so a replay (same kernel arguments) counts from zero again."""
    cfg = synth.spec("c2").cfg
    pr = prepare(_layer("c2", gpu), cfg)
    xs = [synth.make_inputs("c2", n, device=gpu, seed=60 + i) for i in range(2)]
    ws = torch.empty(ops.forward_workspace(pr.cfg, n), dtype=torch.uint8, device=gpu)
    outs = [torch.empty_like(x) for x in xs]

    def run():
        want = [_tail(0, lambda: ops.forward(pr.cfg, pr.weights, x)) for x in xs]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for x, o in zip(xs, outs):
                ops.forward(pr.cfg, pr.weights, x, out=o, ws=ws)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for x, o in zip(xs, outs):
                ops.forward(pr.cfg, pr.weights, x, out=o, ws=ws)
        other = synth.make_inputs("c2", n, device=gpu, seed=98)
        for r in range(3):
            for o in outs:
                o.fill_(float("nan"))
            ops.forward(pr.cfg, pr.weights, other, ws=ws)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for i, (o, w) in enumerate(zip(outs, want)):
                assert torch.equal(o, w), f"N={n}: replay {r}, call {i}"
        del g

    _tail(1, run)
