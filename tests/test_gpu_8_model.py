"""GPU tier: the functional drop-in at model scale.

A decode step calls qwen35_moe once per layer with that layer's parameter dict
(src/quanta/qwen35/batched_runtime.py:595-616 through Qwen35MoEModule.__call__,
src/quanta/qwen35/model.py:68-70; calibration builds the dict afresh per call,
src/quanta/qwen35/calibrate.py:114-119). Each layer's weights must be converted to their tiled
resident form once, however many layers the model has, and a caller that keeps the resident
form must be able to drop its native copy.
"""

from __future__ import annotations

import gc
import weakref

import pytest
import torch

from quanta_amd import moe as qm
from quanta_amd import ops, synth

pytestmark = pytest.mark.gpu

N_LAYERS = 60


def _spec():
    return synth.scaled_spec("c1", hidden_size=512, num_experts=32, moe_intermediate_size=256,
                             shared_expert_intermediate_size=256)


def _native_bytes(p) -> int:
    return sum(t.numel() * t.element_size() for key in ("experts_gate_up", "experts_down")
               for t in (p[key]["packed"], p[key]["scale"], p[key]["bias"]))


def test_sixty_layers_tile_once(gpu, monkeypatch):
    """60 distinct layers cycled three times through qwen35_moe, each call with a fresh copy of the
    layer's dict (as calibration builds it): one tiling per expert stack, router and shared
    expert, no memory growth after the first cycle, bit-identical outputs on every cycle."""
    qm.clear_cache()
    s = _spec()
    counts = {"int4": 0, "bf16": 0}
    real4, real16 = ops.tile_int4, ops.tile_bf16

    def tile4(*a, **kw):
        counts["int4"] += 1
        return real4(*a, **kw)

    def tile16(*a, **kw):
        counts["bf16"] += 1
        return real16(*a, **kw)

    monkeypatch.setattr(ops, "tile_int4", tile4)
    monkeypatch.setattr(ops, "tile_bf16", tile16)
    layers = [synth.make_layer(s, device=gpu, seed=11, layer=i) for i in range(N_LAYERS)]
    x = synth.make_inputs(s, 4, device=gpu, seed=3)[None]
    first, mem = {}, []
    for cycle in range(3):
        for i, p in enumerate(layers):
            y = qm.qwen35_moe(x, dict(p), s.cfg)
            if cycle == 0:
                first[i] = y
            elif i % 7 == 0:
                assert torch.equal(y, first[i]), f"layer {i} cycle {cycle}"
            del y
        torch.cuda.synchronize()
        mem.append(torch.cuda.memory_allocated())
        print(f"[model] cycle {cycle}: tilings {counts}, allocated {mem[-1] / 2**20:.1f} MiB",
              flush=True)
    # gate_up + down per layer; router (with the shared gate row) + shared gate_up + shared down
    assert counts == {"int4": 2 * N_LAYERS, "bf16": 3 * N_LAYERS}
    assert mem[1] == mem[0] and mem[2] == mem[0]


def test_resident_params_drop_native_copy(gpu):
    """resident_params hands the caller the tiled stacks; once the caller drops the native
    triplets the library holds no reference to them (their device memory is released), the layer
    is resident once, and the outputs are unchanged."""
    qm.clear_cache()
    s = _spec()
    layers = [synth.make_layer(s, device=gpu, seed=12, layer=i) for i in range(8)]
    x = synth.make_inputs(s, 5, device=gpu, seed=4)[None]
    want = [qm.qwen35_moe(x, p, s.cfg) for p in layers]
    resident = [qm.resident_params(p) for p in layers]
    native = sum(_native_bytes(p) for p in layers)
    refs = [weakref.ref(p["experts_gate_up"]["packed"]) for p in layers]
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    for p in layers:
        del p["experts_gate_up"], p["experts_down"]
    gc.collect()
    torch.cuda.synchronize()
    after = torch.cuda.memory_allocated()
    assert all(r() is None for r in refs), "the library still holds a native triplet"
    assert before - after >= native, (before, after, native)
    for q, w in zip(resident, want):
        assert torch.equal(qm.qwen35_moe(x, q, s.cfg), w)
