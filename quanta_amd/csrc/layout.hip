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

static inline unsigned grid_for(int64_t n, int block) {
  return static_cast<unsigned>((n + block - 1) / block);
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int qmoe_dequant(const uint32_t* packed, const uint16_t* scale, const uint16_t* bias,
                            int64_t rows, int64_t in_features, int bits, int group_size,
                            uint16_t* out, void* stream) {
  if ((bits != 4 && bits != 8) || (group_size != 64 && group_size != 128))
    return fail("qmoe_dequant: bits 4 or 8 with group_size 64 or 128 only");
  if (rows <= 0 || in_features <= 0 || in_features % group_size)
    return fail("qmoe_dequant: rows > 0 and in_features % group_size == 0 required");
  if (!packed || !scale || !bias || !out) return fail("qmoe_dequant: null pointer");
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
