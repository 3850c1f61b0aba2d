"""Oracle: affine integer quantization format and bf16 helpers (numpy, exact bit work).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Format (reference `src/quanta/bake/quant.py:48-73`, `src/quanta/qwen35/bake.py:113-124`):
  * codes c in [0, 2^bits) for a weight W[out, in]; packed LSB-first as one contiguous
    bitstream per row: code i occupies stream bits [i*bits, i*bits+bits), and stream word j is
    bits [32j, 32j+32). For bits=4, code i sits in word i//8 at bits 4*(i%8)..4*(i%8)+3.
  * per group of `group_size` consecutive codes along `in`: a scale s and bias b (bf16 for the
    routed experts), with dequantized value w = s*c + b.
  * stacks keep the leading expert axis: packed [E, out, in*bits/32] uint32,
    scale/bias [E, out, in/group_size].
"""

from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------------------- bf16 helpers


def f32_to_bf16_bits(a) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even), return the uint16 bit patterns.

    NaN maps to the canonical quiet NaN 0x7FC0. Standard IEEE-style RNE on the top 16 bits.
    """
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint32)
    r = np.where(np.isnan(a), np.uint32(0x7FC0), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32 values (exact)."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """Round to bf16 precision, returned as float64 values. float64 input is first rounded to
    float32 (the GPU keeps float32 accumulators and then rounds to bf16: two roundings)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, dtype=np.float64).astype(np.float32))
                            ).astype(np.float64)


# ----------------------------------------------------------------------------- pack / unpack


def pack_affine(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack integer codes [..., in] into uint32 words [..., in*bits/32], LSB-first bitstream.

    Restates `pack_affine` (`src/quanta/bake/quant.py:48-63`): expand every code into its
    `bits` bits LSB-first, lay the bits out as one stream, then cut the stream into 32-bit words
    whose bit j is stream bit 32*w + j. Requires in*bits % 32 == 0.
    """
    codes = np.asarray(codes)
    *lead, n_in = codes.shape
    if (n_in * bits) % 32:
        raise ValueError(f"in*bits must be a multiple of 32 (in={n_in}, bits={bits})")
    c = codes.astype(np.uint64)
    if np.any(c >> bits):
        raise ValueError(f"codes out of range for {bits} bits")
    bitpos = np.arange(bits, dtype=np.uint64)
    stream = ((c[..., None] >> bitpos) & 1).reshape(*lead, (n_in * bits) // 32, 32)
    wordpos = np.arange(32, dtype=np.uint64)
    return (stream << wordpos).sum(axis=-1).astype(np.uint32)


def unpack_affine(words: np.ndarray, in_features: int, bits: int) -> np.ndarray:
    """Inverse of :func:`pack_affine`: uint32 words [..., n_words] -> codes [..., in] (uint32).

    Restates `unpack_affine` (`src/quanta/bake/quant.py:66-73`).
    """
    words = np.asarray(words, dtype=np.uint32)
    *lead, n_words = words.shape
    if n_words * 32 != in_features * bits:
        raise ValueError("word count does not match in_features*bits/32")
    wordpos = np.arange(32, dtype=np.uint64)
    stream = (words.astype(np.uint64)[..., None] >> wordpos) & 1
    grouped = stream.reshape(*lead, in_features, bits)
    bitpos = np.arange(bits, dtype=np.uint64)
    return (grouped << bitpos).sum(axis=-1).astype(np.uint32)


def unpack_int4_fast(words: np.ndarray, in_features: int) -> np.ndarray:
    """bits=4 special case of :func:`unpack_affine` by shifts (same result, vectorised)."""
    words = np.asarray(words, dtype=np.uint32)
    shifts = (4 * np.arange(8, dtype=np.uint32))
    c = (words[..., None] >> shifts) & np.uint32(0xF)
    return c.reshape(*words.shape[:-1], in_features)


def _unpack(words, in_features, bits):
    return unpack_int4_fast(words, in_features) if bits == 4 else unpack_affine(words, in_features, bits)


# ----------------------------------------------------------------------------- quantize


def quantize_rtn(w: np.ndarray, bits: int = 4, group_size: int = 64):
    """This build's own RTN affine quantizer (min/max per group).

    The weight is first rounded to bf16 (the reference quantizes the bf16 weight when
    `scale_dtype=bf16`, `src/quanta/bake/quant.py:27-29`). Per group of `group_size` along the
    last axis: scale = bf16((max-min)/(2^bits-1)), bias = bf16(min),
    code = clip(rint((w - bias)/scale), 0, 2^bits-1) evaluated in float32.
    A constant group (max == min) gets scale = bf16(1e-8) so the division is defined.

    parity unpinned at the MLX boundary: `mx.quantize` may pick different codes/scales for
    the same weight; every gate compares GPU and oracle on the SAME codes, so this is a
    choice of test data, not a parity input. Returns (packed uint32, scale bf16 bits,
    bias bf16 bits, codes uint32).
    """
    w = bf16_bits_to_f32(f32_to_bf16_bits(w))
    *lead, n_in = w.shape
    if n_in % group_size:
        raise ValueError("in_features must be a multiple of group_size")
    g = w.reshape(*lead, n_in // group_size, group_size)
    wmin = g.min(axis=-1)
    wmax = g.max(axis=-1)
    levels = np.float32((1 << bits) - 1)
    scale = ((wmax - wmin) / levels).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1e-8), scale)
    s_bits = f32_to_bf16_bits(scale)
    b_bits = f32_to_bf16_bits(wmin)
    s = bf16_bits_to_f32(s_bits)[..., None]
    b = bf16_bits_to_f32(b_bits)[..., None]
    q = np.rint(((g - b) / s).astype(np.float32))
    q = np.clip(q, 0, levels).astype(np.uint32).reshape(*lead, n_in)
    return pack_affine(q, bits), s_bits, b_bits, q


# ----------------------------------------------------------------------------- dequantize


def quantize_rtn_f32(w: np.ndarray, bits: int = 4, group_size: int = 32):
    """quantize_rtn with float32 scale and bias (the layout mx.quantize gives float32 weights,
    `parity/qwen35_forward_test.py:236-237`): per group, scale = f32((max-min)/(2^bits-1)),
    bias = f32(min), code = clip(rint((w - bias)/scale)). Test data, like quantize_rtn.
    Returns (packed uint32, scale float32, bias float32, codes uint32)."""
    w = np.asarray(w, dtype=np.float32)
    *lead, n_in = w.shape
    if n_in % group_size:
        raise ValueError("in_features must be a multiple of group_size")
    g = w.reshape(*lead, n_in // group_size, group_size)
    wmin = g.min(axis=-1)
    levels = np.float32((1 << bits) - 1)
    scale = ((g.max(axis=-1) - wmin) / levels).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1e-8), scale)
    q = np.rint(((g - wmin[..., None]) / scale[..., None]).astype(np.float32))
    q = np.clip(q, 0, levels).astype(np.uint32).reshape(*lead, n_in)
    return pack_affine(q, bits), scale, wmin.astype(np.float32), q


def dequant_bf16_bits(words: np.ndarray, scale_bits: np.ndarray, bias_bits: np.ndarray,
                      in_features: int, bits: int = 4, group_size: int = 64) -> np.ndarray:
    """Dequantize to bf16 under this build's declared rounding convention (bit patterns out).

    Value w = s*c + b (`src/quanta/qwen35/artifact.py:105-115` via mx.dequantize). Declared
    convention: bf16( fp32(s)*c + fp32(b) ) with the product exact in float32 (an 8-bit bf16
    mantissa times a code below 2^8), one float32 rounding for the add, then round-to-nearest-
    even to bf16. FMA and mul+add are therefore identical. parity unpinned at the MLX
    boundary: MLX's own bf16 operator sequence inside `dequantize` is not restated anywhere
    in the reference.
    """
    codes = _unpack(words, in_features, bits).astype(np.float32)
    s = bf16_bits_to_f32(scale_bits).astype(np.float32)
    b = bf16_bits_to_f32(bias_bits).astype(np.float32)
    s = np.repeat(s, group_size, axis=-1)
    b = np.repeat(b, group_size, axis=-1)
    val = (s * codes).astype(np.float32) + b      # float32 product (exact) + float32 add
    return f32_to_bf16_bits(val.astype(np.float32))


def dequant_exact(words: np.ndarray, scale_bits: np.ndarray, bias_bits: np.ndarray,
                  in_features: int, bits: int = 4, group_size: int = 64) -> np.ndarray:
    """Exact (float64, unrounded) dequantized weights s*c + b, as used inside gather-qmm.

    The reference's fused qmm never materialises a rounded weight: it evaluates
    sum_k x_k*(s*c_k + b) with float accumulation, so the oracle keeps the exact value.
    """
    codes = _unpack(words, in_features, bits).astype(np.float64)
    s = np.repeat(bf16_bits_to_f32(scale_bits).astype(np.float64), group_size, axis=-1)
    b = np.repeat(bf16_bits_to_f32(bias_bits).astype(np.float64), group_size, axis=-1)
    return s * codes + b


def dequant_float(words: np.ndarray, scale: np.ndarray, bias: np.ndarray, in_features: int,
                  bits: int = 4, group_size: int = 64) -> np.ndarray:
    """dequant_exact for float-valued scale/bias (float32 or bf16 values as float arrays): the
    float64 value s*c + b of every weight, groups of `group_size` along the in-features. The
    reference's float32 parity gates bake float32 scales (mx.quantize of float32 weights,
    `parity/qwen35_forward_test.py:236-237`) at group 32."""
    codes = _unpack(words, in_features, bits).astype(np.float64)
    s = np.repeat(np.asarray(scale, dtype=np.float64), group_size, axis=-1)
    b = np.repeat(np.asarray(bias, dtype=np.float64), group_size, axis=-1)
    return s * codes + b
