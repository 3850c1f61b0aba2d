// Weight-format kernels: bit-exact dequant of the native affine int4 stack, and the one-time
// transform of native stacks into the MFMA-tiled layouts the grouped-qmm kernels stream.
//
// Reference format: src/quanta/bake/quant.py:48-73 (LSB-first nibbles, code i of a row in word
// i/8 at bits 4*(i%8)), src/quanta/qwen35/bake.py:113-124 (stacks [E, out, in], bf16 scale and
// bias per 64 along `in`), src/quanta/qwen35/artifact.py:187-229 (the {packed, scale, bias}
// triplet the resident runtime holds); group 128 along `in`: Kimi's QuantizedSparseMoE stacks
// (src/quanta/modeling/quantized.py:29-34).
#include "qmoe_internal.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

// ---------------------------------------------------------------------------------- dequant
// One thread per packed word: 8 codes -> 8 bf16 written as one 16-byte store. Rounding
// convention: bf16(fma(s, c, b)) in float32; s*c is exact in float32 (8-bit x 4-bit
// mantissas), so fma == mul+add.
__global__ void __launch_bounds__(256) dequant_native_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ bias, int64_t n_words, int words_per_row, int groups_per_row,
    int words_per_group, uint4* __restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_words) return;
  int64_t row = i / words_per_row;
  int wr = static_cast<int>(i - row * words_per_row);
  int64_t g = row * groups_per_row + wr / words_per_group;   // 8 words per 64-code group
  float s = bf16_to_f32(scale[g]);
  float b = bf16_to_f32(bias[g]);
  uint32_t w = packed[i];
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v0 = fmaf(s, static_cast<float>((w >> (8 * j)) & 0xFu), b);
    float v1 = fmaf(s, static_cast<float>((w >> (8 * j + 4)) & 0xFu), b);
    o[j] = pack_bf16x2(v0, v1);
  }
  out[i] = make_uint4(o[0], o[1], o[2], o[3]);
}

// int8: one thread per packed word, 4 byte codes -> 4 bf16 (one 8-byte store), same rounding
// (s*c exact in float32: 8-bit x 8-bit mantissas). Reference: the int8 g64 shared expert and
// non-expert weights of the bake (src/quanta/qwen35/bake.py:106-110, 143-151).
__global__ void __launch_bounds__(256) dequant_native8_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ bias, int64_t n_words, int words_per_row, int groups_per_row,
    int words_per_group, uint2* __restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_words) return;
  int64_t row = i / words_per_row;
  int wr = static_cast<int>(i - row * words_per_row);
  int64_t g = row * groups_per_row + wr / words_per_group;   // 16 words per 64-code group
  float s = bf16_to_f32(scale[g]);
  float b = bf16_to_f32(bias[g]);
  uint32_t w = packed[i];
  uint32_t o[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float v0 = fmaf(s, static_cast<float>((w >> (16 * j)) & 0xFFu), b);
    float v1 = fmaf(s, static_cast<float>((w >> (16 * j + 8)) & 0xFFu), b);
    o[j] = pack_bf16x2(v0, v1);
  }
  out[i] = make_uint2(o[0], o[1]);
}

// Code k (6 bits) of a native int6 row (LSB-first bitstream: code k at bits 6k .. 6k+5).
__device__ __forceinline__ uint32_t int6_code(const uint32_t* __restrict__ row_words, int k) {
  const int bit = 6 * k, w = bit >> 5, sh = bit & 31;
  uint32_t v = row_words[w] >> sh;
  if (sh > 26) v |= row_words[w + 1] << (32 - sh);
  return v & 63u;
}

// int6: one thread per 3 packed words = 16 codes of one row, written as two 16-byte stores;
// same rounding (s*c exact in float32: 8-bit x 6-bit mantissas). Reference: the int6 expert
// stacks of MiniMax M3 (src/quanta/minimax/model_m3.py:414-450), packed as the bake's bitstream
// (src/quanta/bake/quant.py:48-63).
__global__ void __launch_bounds__(256) dequant_native6_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ bias, int64_t n_chunks, int chunks_per_row, int groups_per_row,
    int chunks_per_group, uint4* __restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_chunks) return;
  int64_t row = i / chunks_per_row;
  int cr = static_cast<int>(i - row * chunks_per_row);
  int64_t g = row * groups_per_row + cr / chunks_per_group;
  float s = bf16_to_f32(scale[g]);
  float b = bf16_to_f32(bias[g]);
  const uint32_t w[3] = {packed[3 * i], packed[3 * i + 1], packed[3 * i + 2]};
  uint32_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    o[j] = pack_bf16x2(fmaf(s, static_cast<float>(int6_code(w, 2 * j)), b),
                       fmaf(s, static_cast<float>(int6_code(w, 2 * j + 1)), b));
  out[2 * i] = make_uint4(o[0], o[1], o[2], o[3]);
  out[2 * i + 1] = make_uint4(o[4], o[5], o[6], o[7]);
}

// Code k (3 bits) of a native int3 row (LSB-first bitstream: code k at bits 3k .. 3k+2).
__device__ __forceinline__ uint32_t int3_code(const uint32_t* __restrict__ row_words, int k) {
  const int bit = 3 * k, w = bit >> 5, sh = bit & 31;
  uint32_t v = row_words[w] >> sh;
  if (sh > 29) v |= row_words[w + 1] << (32 - sh);
  return v & 7u;
}

// int3: one thread per 3 packed words = 32 codes of one row (Kimi's int3 expert stacks,
// src/quanta/modeling/quantized.py:29-84, packed as the bake's bitstream,
// src/quanta/bake/quant.py:48-63), written as four 16-byte stores; same rounding.
__global__ void __launch_bounds__(256) dequant_native3_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ bias, int64_t n_chunks, int chunks_per_row, int groups_per_row,
    int chunks_per_group, uint4* __restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_chunks) return;
  int64_t row = i / chunks_per_row;
  int cr = static_cast<int>(i - row * chunks_per_row);
  int64_t g = row * groups_per_row + cr / chunks_per_group;
  float s = bf16_to_f32(scale[g]);
  float b = bf16_to_f32(bias[g]);
  const uint32_t w[3] = {packed[3 * i], packed[3 * i + 1], packed[3 * i + 2]};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16x2(fmaf(s, static_cast<float>(int3_code(w, 8 * q + 2 * j)), b),
                         fmaf(s, static_cast<float>(int3_code(w, 8 * q + 2 * j + 1)), b));
    out[4 * i + q] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Native int3 -> tiled int3: per 16-row tile and 128-deep superblock 768 B, three words per lane
// (lane l: row l%16, the codes 16g .. 16g+15 of each 64-column group, g = l/16). The lane's 32
// codes form 16 pairs, pair q = 8c + 4h + j being codes 2j and 2j + 1 of half h (codes 8h .. 8h+7)
// of group c; pair q < 15 sits in word q / 5 at bits 3(q % 5) and 16 + 3(q % 5), pair 15 keeps bit
// i of its two codes in bits 15 and 31 of word i. Scale/bias as the int4 tiling. One thread per
// lane slot.
__global__ void __launch_bounds__(256) tile_int3_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ bias, int64_t n_lanes_total, int K, int rows,
    int halves_per_group, uint32_t* __restrict__ codes, uint16_t* __restrict__ sb) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_lanes_total) return;
  const int nsb = K / 128, wpr = K * 3 / 32, gpr = K / (64 * halves_per_group);
  int lane = static_cast<int>(i & 63);
  int64_t blk = i >> 6;
  int p = static_cast<int>(blk % nsb);
  int64_t mr = blk / nsb;
  int rt = rows / 16;
  int64_t mat = mr / rt;
  int R = static_cast<int>(mr - mat * rt);
  int r = lane & 15, g = lane >> 4;
  int64_t row = mat * rows + R * 16 + r;
  const uint32_t* src = packed + row * wpr;
  uint32_t w[3] = {0u, 0u, 0u};
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int c = q >> 3, h = (q >> 2) & 1, j = q & 3;
    const int k0 = 128 * p + 64 * c + 16 * g + 8 * h + 2 * j;
    const uint32_t lo = int3_code(src, k0), hi = int3_code(src, k0 + 1);
    if (q < 15) {
      w[q / 5] |= (lo << (3 * (q % 5))) | (hi << (16 + 3 * (q % 5)));
    } else {
#pragma unroll
      for (int b = 0; b < 3; ++b) w[b] |= (((lo >> b) & 1u) << 15) | (((hi >> b) & 1u) << 31);
    }
  }
  uint32_t* blkp = codes + blk * 192 + 3 * lane;
  blkp[0] = w[0];
  blkp[1] = w[1];
  blkp[2] = w[2];
  if (g == 0) {
    uint16_t* d = sb + ((blk * 16 + r) * 2) * 2;
    const int64_t g0 = row * gpr + (2 * p) / halves_per_group;
    const int64_t g1 = row * gpr + (2 * p + 1) / halves_per_group;
    d[0] = scale[g0];
    d[1] = bias[g0];
    d[2] = scale[g1];
    d[3] = bias[g1];
  }
}

// Native int6 -> tiled int6: per 16-row tile and 128-deep superblock, a 1 KiB plane of the codes'
// low nibbles laid out exactly as the int4 tiles (lane l: row l%16, words {2g, 2g+1} of each of
// the two 64-column groups, g = l/16, nibbles interleaved) and a 512-byte plane of their high two
// bits, lane l's 8 bytes being one word per group: the high bits of the lane's 8-code half h,
// pair j (codes 2j, 2j+1 of the half) at bits 2j + 8h and 16 + 2j + 8h, so a shift by 2j + 8h and a
// mask of 0x00030003 puts them beside the pair's nibbles. Scale/bias as the int4 tiling. One
// thread per 16-byte lane slot of the nibble plane.
__global__ void __launch_bounds__(256) tile_int6_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ bias, int64_t n_lanes_total, int K, int rows,
    int halves_per_group, uint32_t* __restrict__ codes, uint16_t* __restrict__ sb) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_lanes_total) return;
  const int nsb = K / 128, wpr = K * 6 / 32, gpr = K / (64 * halves_per_group);
  int lane = static_cast<int>(i & 63);
  int64_t blk = i >> 6;
  int p = static_cast<int>(blk % nsb);
  int64_t mr = blk / nsb;
  int rt = rows / 16;
  int64_t mat = mr / rt;
  int R = static_cast<int>(mr - mat * rt);
  int r = lane & 15, g = lane >> 4;
  int64_t row = mat * rows + R * 16 + r;
  const uint32_t* src = packed + row * wpr;
  uint32_t nib[4], hi[2];
#pragma unroll
  for (int grp = 0; grp < 2; ++grp) {
    hi[grp] = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t w = 0;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t code = int6_code(src, 128 * p + 64 * grp + 16 * g + 8 * h + c);
        w |= (code & 15u) << (4 * c);                 // natural order, interleaved below
        const int j = c >> 1;
        hi[grp] |= (code >> 4) << ((c & 1) ? 16 + 2 * j + 8 * h : 2 * j + 8 * h);
      }
      nib[2 * grp + h] = interleave_nibbles(w);
    }
  }
  // superblock tile block: 1 KiB nibble plane then 512 B high-bit plane
  uint32_t* blkp = codes + blk * 384;
  reinterpret_cast<uint4*>(blkp)[lane] = make_uint4(nib[0], nib[1], nib[2], nib[3]);
  reinterpret_cast<uint2*>(blkp + 256)[lane] = make_uint2(hi[0], hi[1]);
  if (g == 0) {
    uint16_t* d = sb + ((blk * 16 + r) * 2) * 2;
    const int64_t g0 = row * gpr + (2 * p) / halves_per_group;
    const int64_t g1 = row * gpr + (2 * p + 1) / halves_per_group;
    d[0] = scale[g0];
    d[1] = bias[g0];
    d[2] = scale[g1];
    d[3] = bias[g1];
  }
}

// Tiled int4 -> natural bf16 [mats][rows][K]; checks the tiled transform is lossless (it undoes
// the nibble interleave of the stored words).
__global__ void __launch_bounds__(256) dequant_tiled_kernel(
    const uint4* __restrict__ codes, const uint16_t* __restrict__ sb, int64_t n_lanes_total,
    int K, int rows, uint4* __restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // one 16B lane slot
  if (i >= n_lanes_total) return;
  const int nsb = K / 128;
  int lane = static_cast<int>(i & 63);
  int64_t blk = i >> 6;                       // (mat, R, p)
  int p = static_cast<int>(blk % nsb);
  int64_t mr = blk / nsb;                     // mat * rows/16 + R
  int rt = rows / 16;
  int64_t mat = mr / rt;
  int R = static_cast<int>(mr - mat * rt);
  int r = lane & 15, g = lane >> 4;
  int row = R * 16 + r;
  uint4 q = codes[i];
  uint32_t words[4] = {q.x, q.y, q.z, q.w};
  const uint16_t* sbp = sb + ((blk * 16 + r) * 2) * 2;   // [blk][16 rows][2 groups][2]
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    int gg = t >> 1, wi = 2 * g + (t & 1);
    float s = bf16_to_f32(sbp[gg * 2 + 0]);
    float b = bf16_to_f32(sbp[gg * 2 + 1]);
    const uint32_t w = deinterleave_nibbles(words[t]);
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v0 = fmaf(s, static_cast<float>((w >> (8 * j)) & 0xFu), b);
      float v1 = fmaf(s, static_cast<float>((w >> (8 * j + 4)) & 0xFu), b);
      o[j] = pack_bf16x2(v0, v1);
    }
    int64_t kk = static_cast<int64_t>(p) * 128 + gg * 64 + wi * 8;   // first code of this word
    int64_t off = ((mat * rows + row) * K + kk) / 8;                  // in uint4 units
    out[off] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Native int4 -> tiled codes (nibble-interleaved words) + tiled scale/bias. One thread per
// 16-byte lane slot.
__global__ void __launch_bounds__(256) tile_int4_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ bias, int64_t n_lanes_total, int K, int rows,
    int halves_per_group, uint4* __restrict__ codes, uint16_t* __restrict__ sb) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_lanes_total) return;
  const int nsb = K / 128, wpr = K / 8, gpr = K / (64 * halves_per_group);
  int lane = static_cast<int>(i & 63);
  int64_t blk = i >> 6;
  int p = static_cast<int>(blk % nsb);
  int64_t mr = blk / nsb;
  int rt = rows / 16;
  int64_t mat = mr / rt;
  int R = static_cast<int>(mr - mat * rt);
  int r = lane & 15, g = lane >> 4;
  int64_t row = mat * rows + R * 16 + r;
  const uint32_t* src = packed + row * wpr + p * 16;   // 16 words = groups 2p, 2p+1
  codes[i] = make_uint4(interleave_nibbles(src[2 * g]), interleave_nibbles(src[2 * g + 1]),
                        interleave_nibbles(src[8 + 2 * g]), interleave_nibbles(src[8 + 2 * g + 1]));
  if (g == 0) {
    // one (scale, bias) per 64 columns: a 128-column group's pair serves both of its halves
    uint16_t* d = sb + ((blk * 16 + r) * 2) * 2;
    const int64_t g0 = row * gpr + (2 * p) / halves_per_group;
    const int64_t g1 = row * gpr + (2 * p + 1) / halves_per_group;
    d[0] = scale[g0];
    d[1] = bias[g0];
    d[2] = scale[g1];
    d[3] = bias[g1];
  }
}

// Row-major bf16 [mats][rows][K] -> tiled [mats][rows/16][K/32][64][8].
__global__ void __launch_bounds__(256) tile_bf16_kernel(const uint16_t* __restrict__ w,
                                                        int64_t n_lanes_total, int K, int rows,
                                                        uint4* __restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_lanes_total) return;
  const int nk = K / 32;
  int lane = static_cast<int>(i & 63);
  int64_t blk = i >> 6;
  int c = static_cast<int>(blk % nk);
  int64_t mr = blk / nk;
  int rt = rows / 16;
  int64_t mat = mr / rt;
  int R = static_cast<int>(mr - mat * rt);
  int64_t row = mat * rows + R * 16 + (lane & 15);
  const uint4* src = reinterpret_cast<const uint4*>(w + row * K + c * 32 + (lane >> 4) * 8);
  out[i] = *src;
}

// Native int8 [mats][rows][K] (code k in byte k%4 of word k/4, so a row's bytes are its codes in
// order) -> tiled codes [mats][rows/16][K/32][64 lanes][8 codes], lane l holding row l%16's codes
// 32c + 8(l/16) .. +8, and sb [mats][rows/16][K/64][16 rows][scale, bias]. One thread per 8-byte
// lane slot; the lanes of the even steps' first lane group also write the scale/bias pairs.
__global__ void __launch_bounds__(256) tile_int8_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ bias, int64_t n_lanes_total, int K, int rows,
    int halves_per_group, uint2* __restrict__ codes, uint32_t* __restrict__ sb) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_lanes_total) return;
  const int nk = K / 32, gpr = K / (64 * halves_per_group);
  const int lane = static_cast<int>(i & 63);
  const int64_t blk = i >> 6;                 // (mat, R, c)
  const int c = static_cast<int>(blk % nk);
  const int64_t mr = blk / nk;                // mat * rows/16 + R
  const int rt = rows / 16;
  const int64_t mat = mr / rt;
  const int R = static_cast<int>(mr - mat * rt);
  const int r = lane & 15;
  const int64_t row = mat * rows + R * 16 + r;
  codes[i] = *reinterpret_cast<const uint2*>(packed + row * (K / 4) + c * 8 + (lane >> 4) * 2);
  if ((c & 1) == 0 && lane < 16) {
    const int64_t g = row * gpr + (c / 2) / halves_per_group;
    sb[(mr * (K / 64) + c / 2) * 16 + r] =
        static_cast<uint32_t>(scale[g]) | (static_cast<uint32_t>(bias[g]) << 16);
  }
}

// Tiled int8 -> tiled bf16 [mats][rows/16][K/32][64][8]: every lane slot's 8 codes become the 8
// bf16 weights the dense kernels make of them in registers (dense_bf16).
__global__ void __launch_bounds__(256) expand_int8_kernel(const u32x2* __restrict__ codes,
                                                          const uint16_t* __restrict__ sb,
                                                          int64_t n_lanes_total, int K,
                                                          u32x4* __restrict__ out) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_lanes_total) return;
  const int nk = K / 32;
  const int lane = static_cast<int>(i & 63);
  const int64_t blk = i >> 6;
  const int c = static_cast<int>(blk % nk);
  const int64_t tile = blk / nk;
  DenseTile<FMT_INT8> t;
  t.init(codes, sb, tile, K, lane);
  out[i] = dense_bf16<FMT_INT8>(t.load(c));
}

int launch_expand_int8(const uint32_t* codes, const uint16_t* sb, int64_t rows, int K,
                       uint16_t* out, hipStream_t stream) {
  if (rows <= 0 || rows % 16 || K <= 0 || K % 64) return fail("expand int8: rows % 16, K % 64 == 0");
  const int64_t lanes = rows * (K / 32) * 4;
  expand_int8_kernel<<<static_cast<unsigned>((lanes + 255) / 256), 256, 0, stream>>>(
      reinterpret_cast<const u32x2*>(codes), sb, lanes, K, reinterpret_cast<u32x4*>(out));
  return check_launch("expand int8");
}

// ---------------------------------------------------------------------------- row exponents
// One wavefront per weight row: M = the row's largest dequantized magnitude, max over its groups of
// max(|b|, |qmax * s + b|) (the affine map is monotone in the code, so its extremes sit at codes
// 0 and qmax), and row_exp = 14 - ex with 2^(ex-1) <= M < 2^ex, so every weight of the row times
// 2^row_exp lies below 2^14 and fp16 holds it at full precision down to 2^-14 of that (2^28 of
// dynamic range within the row). 0 for an all-zero or non-finite row; clamped to [-100, 100].
__global__ void __launch_bounds__(256) row_exp_kernel(const uint16_t* __restrict__ scale,
                                                      const uint16_t* __restrict__ bias,
                                                      int64_t n_rows, int groups, float qmax,
                                                      int8_t* __restrict__ row_exp) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= n_rows) return;   // the whole wavefront
  const uint16_t* sr = scale + r * groups;
  const uint16_t* br = bias + r * groups;
  float m = 0.f;
  for (int g = lane; g < groups; g += 64) {
    const float sv = bf16_to_f32(sr[g]), bv = bf16_to_f32(br[g]);
    m = fmaxf(m, fmaxf(fabsf(bv), fabsf(fmaf(qmax, sv, bv))));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (lane) return;
  int ex = 0;
  if (m > 0.f && m <= 3.4e38f) {
    frexpf(m, &ex);
    ex = 14 - ex;
    ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
  }
  row_exp[r] = static_cast<int8_t>(ex);
}

static inline unsigned grid_for(int64_t n, int block) {
  return static_cast<unsigned>((n + block - 1) / block);
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int qmoe_dequant(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                            int64_t rows, int64_t in_features, int bits, int group_size,
                            uint16_t* out, void* stream) {
  if ((bits != 3 && bits != 4 && bits != 6 && bits != 8) || (group_size != 64 && group_size != 128))
    return fail("qmoe_dequant: bits 3, 4, 6 or 8 with group_size 64 or 128 only");
  if (rows <= 0 || in_features <= 0 || in_features % group_size)
    return fail("qmoe_dequant: rows > 0 and in_features % group_size == 0 required");
  if (!packed || !scale || !bias || !out) return fail("qmoe_dequant: null pointer");
  if (bits == 3) {
    const int64_t n_chunks = rows * (in_features / 32);
    if (in_features % 32) return fail("qmoe_dequant: int3 needs in_features % 32 == 0");
    if (n_chunks >= (int64_t(1) << 40)) return fail("qmoe_dequant: tensor too large");
    dequant_native3_kernel<<<grid_for(n_chunks, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        packed, scale, bias, n_chunks, static_cast<int>(in_features / 32),
        static_cast<int>(in_features / group_size), group_size / 32, reinterpret_cast<uint4*>(out));
    return check_launch("qmoe_dequant");
  }
  if (bits == 6) {
    const int64_t n_chunks = rows * (in_features / 16);
    if (n_chunks >= (int64_t(1) << 40)) return fail("qmoe_dequant: tensor too large");
    dequant_native6_kernel<<<grid_for(n_chunks, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        packed, scale, bias, n_chunks, static_cast<int>(in_features / 16),
        static_cast<int>(in_features / group_size), group_size / 16, reinterpret_cast<uint4*>(out));
    return check_launch("qmoe_dequant");
  }
  const int per_word = 32 / bits;
  int64_t n_words = rows * (in_features / per_word);
  if (n_words >= (int64_t(1) << 40)) return fail("qmoe_dequant: tensor too large");
  if (bits == 4)
    dequant_native_kernel<<<grid_for(n_words, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        packed, scale, bias, n_words, static_cast<int>(in_features / 8),
        static_cast<int>(in_features / group_size), group_size / 8, reinterpret_cast<uint4*>(out));
  else
    dequant_native8_kernel<<<grid_for(n_words, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        packed, scale, bias, n_words, static_cast<int>(in_features / 4),
        static_cast<int>(in_features / group_size), group_size / 4, reinterpret_cast<uint2*>(out));
  return check_launch("qmoe_dequant");
}

extern "C" int qmoe_row_exponents(const uint16_t* scale, const uint16_t* bias, int64_t n_mats,
                                  int64_t rows, int64_t in_features, int bits, int group_size,
                                  int8_t* row_exp, void* stream) {
  if (!scale || !bias || !row_exp) return fail("qmoe_row_exponents: null pointer");
  if (n_mats <= 0 || rows <= 0 || in_features <= 0) return fail("qmoe_row_exponents: bad dims");
  if (bits < 2 || bits > 8) return fail("qmoe_row_exponents: 2 <= bits <= 8");
  if (group_size <= 0 || in_features % group_size) return fail("qmoe_row_exponents: in % group_size != 0");
  const int64_t n = n_mats * rows;
  row_exp_kernel<<<grid_for(n, 4), 256, 0, static_cast<hipStream_t>(stream)>>>(
      scale, bias, n, static_cast<int>(in_features / group_size), static_cast<float>((1 << bits) - 1),
      row_exp);
  return check_launch("row_exponents");
}

extern "C" int qmoe_tile_int4(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                              int64_t n_mats, int64_t rows, int64_t in_features, int group_size,
                              uint32_t* tiled_codes, uint16_t* tiled_sb, void* stream) {
  if (group_size != 64 && group_size != 128) return fail("qmoe_tile_int4: group_size must be 64 or 128");
  if (n_mats <= 0 || rows <= 0 || rows % 16 || in_features <= 0 || in_features % 128)
    return fail("qmoe_tile_int4: need rows % 16 == 0 and in_features % 128 == 0");
  if (!packed || !scale || !bias || !tiled_codes || !tiled_sb)
    return fail("qmoe_tile_int4: null pointer");
  if (rows > (1 << 30) || in_features > (1 << 30)) return fail("qmoe_tile_int4: dims too large");
  int64_t lanes = n_mats * rows * (in_features / 128) * 4;   // 16 rows x 64 lanes per 16 rows
  tile_int4_kernel<<<grid_for(lanes, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      packed, scale, bias, lanes, static_cast<int>(in_features), static_cast<int>(rows),
      group_size / 64, reinterpret_cast<uint4*>(tiled_codes), tiled_sb);
  return check_launch("qmoe_tile_int4");
}

extern "C" int qmoe_tile_int3(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                              int64_t n_mats, int64_t rows, int64_t in_features, int group_size,
                              uint32_t* tiled_codes, uint16_t* tiled_sb, void* stream) {
  if (group_size != 64 && group_size != 128) return fail("qmoe_tile_int3: group_size must be 64 or 128");
  if (n_mats <= 0 || rows <= 0 || rows % 16 || in_features <= 0 || in_features % 128)
    return fail("qmoe_tile_int3: need rows % 16 == 0 and in_features % 128 == 0");
  if (!packed || !scale || !bias || !tiled_codes || !tiled_sb)
    return fail("qmoe_tile_int3: null pointer");
  if (rows > (1 << 30) || in_features > (1 << 30)) return fail("qmoe_tile_int3: dims too large");
  int64_t lanes = n_mats * rows * (in_features / 128) * 4;
  tile_int3_kernel<<<grid_for(lanes, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      packed, scale, bias, lanes, static_cast<int>(in_features), static_cast<int>(rows),
      group_size / 64, tiled_codes, tiled_sb);
  return check_launch("qmoe_tile_int3");
}

extern "C" int qmoe_tile_int6(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                              int64_t n_mats, int64_t rows, int64_t in_features, int group_size,
                              uint32_t* tiled_codes, uint16_t* tiled_sb, void* stream) {
  if (group_size != 64 && group_size != 128) return fail("qmoe_tile_int6: group_size must be 64 or 128");
  if (n_mats <= 0 || rows <= 0 || rows % 16 || in_features <= 0 || in_features % 128)
    return fail("qmoe_tile_int6: need rows % 16 == 0 and in_features % 128 == 0");
  if (!packed || !scale || !bias || !tiled_codes || !tiled_sb)
    return fail("qmoe_tile_int6: null pointer");
  if (rows > (1 << 30) || in_features > (1 << 30)) return fail("qmoe_tile_int6: dims too large");
  int64_t lanes = n_mats * rows * (in_features / 128) * 4;
  tile_int6_kernel<<<grid_for(lanes, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      packed, scale, bias, lanes, static_cast<int>(in_features), static_cast<int>(rows),
      group_size / 64, tiled_codes, tiled_sb);
  return check_launch("qmoe_tile_int6");
}

extern "C" int qmoe_tile_int8(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                              int64_t n_mats, int64_t rows, int64_t in_features, int group_size,
                              uint32_t* tiled_codes, uint16_t* tiled_sb, void* stream) {
  if (group_size != 64 && group_size != 128) return fail("qmoe_tile_int8: group_size must be 64 or 128");
  if (n_mats <= 0 || rows <= 0 || rows % 16 || in_features <= 0 || in_features % 64 ||
      in_features % group_size)
    return fail("qmoe_tile_int8: need rows % 16 == 0 and in_features % 64 == 0 (and % group_size)");
  if (!packed || !scale || !bias || !tiled_codes || !tiled_sb)
    return fail("qmoe_tile_int8: null pointer");
  if (rows > (1 << 30) || in_features > (1 << 30)) return fail("qmoe_tile_int8: dims too large");
  const int64_t lanes = n_mats * rows * (in_features / 32) * 4;   // 64 lanes per 16 rows x 32
  tile_int8_kernel<<<grid_for(lanes, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      packed, scale, bias, lanes, static_cast<int>(in_features), static_cast<int>(rows),
      group_size / 64, reinterpret_cast<uint2*>(tiled_codes), reinterpret_cast<uint32_t*>(tiled_sb));
  return check_launch("qmoe_tile_int8");
}

extern "C" int qmoe_dequant_tiled(const uint32_t* tiled_codes, const uint16_t* tiled_sb,
                                  int64_t n_mats, int64_t rows, int64_t in_features,
                                  uint16_t* out, void* stream) {
  if (n_mats <= 0 || rows <= 0 || rows % 16 || in_features <= 0 || in_features % 128)
    return fail("qmoe_dequant_tiled: need rows % 16 == 0 and in_features % 128 == 0");
  if (!tiled_codes || !tiled_sb || !out) return fail("qmoe_dequant_tiled: null pointer");
  if (rows > (1 << 30) || in_features > (1 << 30)) return fail("qmoe_dequant_tiled: dims too large");
  int64_t lanes = n_mats * rows * (in_features / 128) * 4;
  dequant_tiled_kernel<<<grid_for(lanes, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint4*>(tiled_codes), tiled_sb, lanes, static_cast<int>(in_features),
      static_cast<int>(rows), reinterpret_cast<uint4*>(out));
  return check_launch("qmoe_dequant_tiled");
}

extern "C" int qmoe_tile_bf16(const uint16_t* w, int64_t n_mats, int64_t rows, int64_t in_features,
                              uint16_t* tiled, void* stream) {
  if (n_mats <= 0 || rows <= 0 || rows % 16 || in_features <= 0 || in_features % 32)
    return fail("qmoe_tile_bf16: need rows % 16 == 0 and in_features % 32 == 0");
  if (!w || !tiled) return fail("qmoe_tile_bf16: null pointer");
  if (rows > (1 << 30) || in_features > (1 << 30)) return fail("qmoe_tile_bf16: dims too large");
  int64_t lanes = n_mats * rows * (in_features / 32) * 4;
  tile_bf16_kernel<<<grid_for(lanes, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w, lanes, static_cast<int>(in_features), static_cast<int>(rows),
      reinterpret_cast<uint4*>(tiled));
  return check_launch("qmoe_tile_bf16");
}
