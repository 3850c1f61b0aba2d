"""GPU tier: the block captured into a HIP graph (torch.cuda.CUDAGraph around qmoe_forward on the
capture stream) and replayed, against the same calls launched on a stream. The forward records
kernel launches only (no memset or copy nodes), and above the fused-shared-expert batch sizes its
auxiliary stream joins the capture through the fork and join events. Each replay follows eager
work on the same workspace and a synchronisation, and every replay's outputs must equal the
stream results bit for bit."""

from __future__ import annotations

import pytest
import torch

from quanta_amd import ops, synth
from quanta_amd.moe import prepare

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def c1_layer(gpu):
    spec = synth.spec("c1")
    return spec, prepare(synth.make_layer("c1", device=gpu, seed=31), spec.cfg)


# 1: slot-major, top-k inside the routed gate_up, fused down/shared/combine tail; 8: slot-major
# with the top-k launch; 32: permute, shared expert fused into the router and combine launches;
# 128: the shared expert on the auxiliary stream (fork/join events inside the capture)
@pytest.mark.parametrize("n", [1, 8, 32, 128])
def test_graph_replay_matches_stream(gpu, c1_layer, n):
    spec, pr = c1_layer
    xs = [synth.make_inputs(spec, n, device=gpu, seed=40 + i) for i in range(3)]
    ws = torch.empty(ops.forward_workspace(pr.cfg, n), dtype=torch.uint8, device=gpu)
    want = [ops.forward(pr.cfg, pr.weights, x) for x in xs]
    outs = [torch.empty_like(x) for x in xs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # torch's pre-capture warm-up on a side stream
        for x, o in zip(xs, outs):
            ops.forward(pr.cfg, pr.weights, x, out=o, ws=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for x, o in zip(xs, outs):
            ops.forward(pr.cfg, pr.weights, x, out=o, ws=ws)
    other = synth.make_inputs(spec, n, device=gpu, seed=99)
    for r in range(3):
        for o in outs:
            o.fill_(float("nan"))
        ops.forward(pr.cfg, pr.weights, other, ws=ws)   # eager work on the same workspace
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), f"N={n}: replay {r}, call {i} differs from the stream launch"
    print(f"[graph] c1 N={n}: 3 replays of 3 captured calls bit-identical to stream launches",
          flush=True)
    del g
