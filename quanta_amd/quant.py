"""Affine integer quantization format (torch, any device): RTN quantizer and the LSB-first
pack/unpack of the reference's bake.

Reference: src/quanta/bake/quant.py:18-73 (`quantize_affine` with optional bf16 scale dtype,
`pack_affine` / `unpack_affine` LSB-first bitstream: code i occupies stream bits
[i*bits, i*bits+bits)); routed experts are int4 g64 with bf16 scale and bias
(src/quanta/qwen35/bake.py:113-124). Packed words are returned as torch.int32 tensors holding the
uint32 bit patterns.

The quantizer is this build's own RTN (per-group min/max; the codes MLX's `mx.quantize` would
pick are not restated in the reference). Every kernel consumes whatever codes it is given.
"""

from __future__ import annotations

import torch

GROUP_SIZE = 128   # the reference's default group for non-expert weights (bake/quant.py:15)


def _to_int32_bits(v: torch.Tensor) -> torch.Tensor:
    """int64 values in [0, 2^32) -> int32 tensor with the same 32-bit pattern."""
    v = torch.where(v >= 2 ** 31, v - 2 ** 32, v)
    return v.to(torch.int32)


def pack_affine(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack integer codes [..., in] (0 .. 2^bits-1) into 32-bit words [..., in*bits/32]."""
    *lead, n_in = codes.shape
    if (n_in * bits) % 32:
        raise ValueError("in*bits must be a multiple of 32")
    c = codes.to(torch.int64)
    if bits in (2, 4, 8):
        per = 32 // bits
        c = c.reshape(*lead, n_in // per, per)
        shifts = torch.arange(per, device=c.device, dtype=torch.int64) * bits
        return _to_int32_bits((c << shifts).sum(dim=-1))
    bitpos = torch.arange(bits, device=c.device, dtype=torch.int64)
    stream = ((c[..., None] >> bitpos) & 1).reshape(*lead, (n_in * bits) // 32, 32)
    wordpos = torch.arange(32, device=c.device, dtype=torch.int64)
    return _to_int32_bits((stream << wordpos).sum(dim=-1))


def unpack_affine(words: torch.Tensor, in_features: int, bits: int) -> torch.Tensor:
    """Inverse of :func:`pack_affine`: words [..., n_words] -> codes [..., in] (int32)."""
    *lead, n_words = words.shape
    if n_words * 32 != in_features * bits:
        raise ValueError("word count does not match in_features*bits/32")
    w = words.to(torch.int64) & 0xFFFFFFFF
    if bits in (2, 4, 8):
        per = 32 // bits
        shifts = torch.arange(per, device=w.device, dtype=torch.int64) * bits
        c = (w[..., None] >> shifts) & ((1 << bits) - 1)
        return c.reshape(*lead, in_features).to(torch.int32)
    wordpos = torch.arange(32, device=w.device, dtype=torch.int64)
    stream = ((w[..., None] >> wordpos) & 1).reshape(*lead, in_features, bits)
    bitpos = torch.arange(bits, device=w.device, dtype=torch.int64)
    return (stream << bitpos).sum(dim=-1).to(torch.int32)


def quantize_affine(w: torch.Tensor, bits: int, group_size: int = GROUP_SIZE, *,
                    scale_dtype: torch.dtype | None = torch.bfloat16):
    """RTN affine-quantize w [..., in] -> (packed int32 words, scale, bias).

    Mirrors the signature of `quantize_affine` (src/quanta/bake/quant.py:18-29): with a
    `scale_dtype` the weight is first cast to it, and scale/bias come back in it. Per group:
    scale = (max - min) / (2^bits - 1) (1e-8 for a constant group), bias = min, both rounded to
    `scale_dtype`; code = clamp(round((w - bias) / scale), 0, 2^bits - 1) in float32 against the
    rounded scale/bias, round-half-to-even.
    """
    if scale_dtype is not None:
        w = w.to(scale_dtype)
    out_dtype = w.dtype
    wf = w.to(torch.float32)
    *lead, n_in = wf.shape
    if n_in % group_size:
        raise ValueError("in_features must be a multiple of group_size")
    g = wf.reshape(*lead, n_in // group_size, group_size)
    wmin = g.amin(dim=-1)
    wmax = g.amax(dim=-1)
    levels = float((1 << bits) - 1)
    scale = (wmax - wmin) / levels
    scale = torch.where(scale == 0, torch.full_like(scale, 1e-8), scale)
    s = scale.to(out_dtype)
    b = wmin.to(out_dtype)
    q = torch.round((g - b.to(torch.float32)[..., None]) / s.to(torch.float32)[..., None])
    q = q.clamp_(0, levels).to(torch.int32).reshape(*lead, n_in)
    return pack_affine(q, bits), s, b
