"""GPU tier: qmoe_forward_noalloc, the entry point that allocates nothing (its workspace is the
library's fixed per-GPU scratch, every launch on the caller's stream), against qmoe_forward with a
caller workspace: bit-identical outputs on two calls in a row, the second with fewer tokens (the
scratch keeps the first call's contents), in the decode, slot-major and hybrid prefill regimes;
a batch whose workspace exceeds the scratch is refused."""

from __future__ import annotations

import pytest
import torch

from quanta_amd import _lib as L
from quanta_amd import ops, synth
from quanta_amd.moe import prepare

pytestmark = pytest.mark.gpu


def _pair(dev, spec, p, n_first, n_second, seed):
    pr = prepare(p, spec.cfg)
    for n in (n_first, n_second):
        x = synth.make_inputs(spec, n, device=dev, seed=seed + n)
        want = ops.forward(pr.cfg, pr.weights, x)
        got = torch.full_like(x, float("nan"))
        torch.cuda.synchronize()
        before = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
        ops.forward_noalloc(pr.cfg, pr.weights, x, got)
        after = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
        torch.cuda.synchronize()
        assert after == before, "the no-allocation call allocated through torch"
        assert torch.equal(got, want), f"N={n}"
        print(f"[noalloc] N={n}: bit-identical to qmoe_forward "
              f"(workspace {ops.forward_workspace(pr.cfg, n)} of {L.NOALLOC_SCRATCH_BYTES} bytes)",
              flush=True)


def test_noalloc_decode_c2(gpu):
    """c2 at 32 then 8 tokens (fused shared expert), then 2 tokens (slot-major routing, the
    top-k inside the routed gate_up), then 4 and 1 (the fused down/combine tail)."""
    spec = synth.spec("c2")
    p = synth.make_layer("c2", device=gpu, seed=21)
    _pair(gpu, spec, p, 32, 8, 1)
    _pair(gpu, spec, p, 128, 2, 2)   # shared expert on its own launches, then slot-major
    _pair(gpu, spec, p, 4, 1, 3)


def test_noalloc_hybrid_prefill(gpu):
    """A small layer at 600 tokens (hybrid large-M regime: hot experts on the wide kernel, cold
    ones on the small kernel, here on one stream) then 40 tokens."""
    spec = synth.scaled_spec("c1", hidden_size=512, num_experts=16, moe_intermediate_size=256,
                             shared_expert_intermediate_size=256)
    p = synth.make_layer(spec, device=gpu, seed=22)
    _pair(gpu, spec, p, 600, 40, 3)


def test_noalloc_rejects_oversized_batch(gpu):
    spec = synth.spec("c2")
    p = synth.make_layer(synth.scaled_spec("c2", num_experts=16), device=gpu, seed=23)
    pr = prepare(p, synth.scaled_spec("c2", num_experts=16).cfg)
    N = 4096
    assert ops.forward_workspace(pr.cfg, N) > L.NOALLOC_SCRATCH_BYTES
    x = synth.make_inputs(spec, N, device=gpu, seed=5)
    out = torch.empty_like(x)
    with pytest.raises(ValueError, match="scratch"):
        ops.forward_noalloc(pr.cfg, pr.weights, x, out)
