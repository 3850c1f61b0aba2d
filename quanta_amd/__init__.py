"""quanta_amd: MI355X-native (gfx950) quantized sparse-MoE block.

The reference's MoE-block surface (pmrjge/quanta `qwen35_moe`, `qwen35_route`,
`Qwen35MoEModule`) on PyTorch-ROCm, computed by hand-written HIP kernels behind the C ABI in
include/quanta_moe.h (`quanta_amd/_qmoe.so`, built by `python -m quanta_amd.build`).
"""

from quanta_amd.moe import (MoEConfig, Qwen35MoEModule, TiledExperts, prepare, qwen35_moe,
                            qwen35_moe_residual, qwen35_route, tile_experts_bf16,
                            tile_experts_packed)
from quanta_amd.quant import pack_affine, quantize_affine, unpack_affine

__all__ = [
    "MoEConfig", "Qwen35MoEModule", "TiledExperts", "prepare", "qwen35_moe", "qwen35_moe_residual",
    "qwen35_route",
    "tile_experts_bf16", "tile_experts_packed", "pack_affine", "quantize_affine", "unpack_affine",
]
