"""CPU oracle for the quantized sparse-MoE block.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (`quanta_amd`) imports this
package. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may use it, and only as the checker / the timed CPU baseline, never as the thing measured
or shipped.

Modules:
  quant      -- affine int-N pack/unpack (LSB-first bitstream), RTN quantizer, dequant,
                bf16 rounding helpers (numpy, exact integer/bit work).
  moe        -- float64 restatement of the reference block: routers (softmax, sigmoid +
                correction bias, group-limited), stable permute, gather-qmm, SwiGLU,
                weighted combine, gated shared expert, and the run-every-expert oracle.
  torch_cpu  -- a torch-CPU float32 port of the same algorithm, used as the timed CPU
                baseline in bench.py (the reference's MLX CPU backend cannot run here).

Reference being restated (pmrjge/quanta, read-only):
  src/quanta/qwen35/moe.py:32-202, src/quanta/modeling/moe.py:33-44,81-97,
  src/quanta/glm/moe.py:44-55, src/quanta/dsv4/moe.py:93-137,
  src/quanta/bake/quant.py:48-73, src/quanta/qwen35/artifact.py:187-229.
Group-limited routing follows transformers 5.15.0
  models/deepseek_v3/modeling_deepseek_v3.py:144-170 (third party, not in the reference).

Parity pins (what each oracle function is checked against) live in tests/test_oracle.py.
Functions whose MLX-internal behaviour could only be pinned by importing MLX (absent here)
are marked "parity unpinned at the MLX boundary" in their docstrings: the exact codes
`mx.quantize` would choose, MLX's bf16 rounding inside gather_qmm, and argpartition's
within-top-k order.
"""
