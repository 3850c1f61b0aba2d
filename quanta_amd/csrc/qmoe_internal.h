// Internal helpers shared by the quantized-MoE HIP sources (gfx950 / CDNA4 only).
//
// Layout vocabulary used throughout:
//   * "native" int4 stack  : packed u32 [mats][rows][K/8], scale/bias bf16 [mats][rows][K/64]
//                            (the reference's affine_packed triplet, LSB-first nibbles).
//   * "tiled" int4 stack   : codes u32 [mats][rows/16][K/128][64 lanes][4 words] and
//                            sb bf16 [mats][rows/16][K/128][16 rows][2 groups][scale,bias].
//                            One 16-row x 128-K superblock is 1 KiB of codes, read by one
//                            wavefront as a single contiguous dwordx4 load per lane.
//                            Lane l (row l%16, lane group g=l/16) holds words {2g,2g+1} of
//                            group 2p followed by words {2g,2g+1} of group 2p+1. Each stored
//                            word carries its 8 codes c0..c7 with nibbles interleaved as
//                            [c0 c2 c4 c6 c1 c3 c5 c7] (nibble 0 lowest), so (w >> 4j) & 0x000F000F
//                            yields the natural-order pair (c_2j, c_2j+1) in one mask.
//   * "tiled" bf16 matrix  : [mats][rows/16][K/32][64 lanes][8 bf16]; lane l holds
//                            W[16R + l%16][32c + 8(l/16) .. +8).
// Both tiled layouts put each lane's MFMA B-fragment (weight row = l%16, 8 consecutive K of
// one 64-wide scale group) in 16 contiguous bytes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>
#include "../../include/quanta_moe.h"

namespace qmoe {

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
// Native 16-byte vector (HIP's uint4 is a struct whose copies lower to memcpy, which can
// pin arrays of it in scratch); used for all raw 16-byte global/LDS traffic in the kernels.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------ error reporting
void set_error(const std::string& msg);
int fail(const std::string& msg);           // set_error + return QMOE_EINVAL
int check_launch(const char* what);         // hipGetLastError -> QMOE_EHIP on failure

// ------------------------------------------------------------------ bf16 helpers
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float bf16lo_to_f32(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16hi_to_f32(uint32_t pair) {
  return __uint_as_float(pair & 0xFFFF0000u);
}
// Round-to-nearest-even float -> bf16 (NaN -> quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}
// The same round-to-nearest-even pack in one instruction (gfx950's v_cvt_pk_bf16_f32): equal to
// pack_bf16x2 for every non-NaN input (a NaN stays a NaN, its payload may differ). Used where the
// conversion is the hot loop (the RMSNorm paths, which both use it, so they agree bit for bit).
typedef __bf16 bf16x2_hw_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_hw_t));
}

// Native word (nibble i = code i) <-> stored tiled word (nibbles [c0 c2 c4 c6 c1 c3 c5 c7]).
__host__ __device__ __forceinline__ uint32_t interleave_nibbles(uint32_t w) {
  uint32_t o = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    o |= ((w >> (8 * j)) & 0xFu) << (4 * j);            // c_2j   -> nibble j
    o |= ((w >> (8 * j + 4)) & 0xFu) << (4 * j + 16);   // c_2j+1 -> nibble j+4
  }
  return o;
}
__host__ __device__ __forceinline__ uint32_t deinterleave_nibbles(uint32_t o) {
  uint32_t w = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    w |= ((o >> (4 * j)) & 0xFu) << (8 * j);
    w |= ((o >> (4 * j + 16)) & 0xFu) << (8 * j + 4);
  }
  return w;
}

// Nibble unpack of a stored (interleaved) word for the decode MFMA path. Register j holds the
// bf16 pair (128 + c_2j, 128 + c_2j+1): 128 + c is exact in bf16 (7 mantissa bits span 128..255
// in steps of 1), and the pairs come out in natural k order, matching the activation fragment.
__device__ __forceinline__ bf16x8_t unpack_q128(uint32_t w) {
  const uint32_t m = 0x000F000Fu, o = 0x43004300u;
  uint32_t r0 = (w & m) | o;
  uint32_t r1 = ((w >> 4) & m) | o;
  uint32_t r2 = ((w >> 8) & m) | o;
  uint32_t r3 = ((w >> 12) & m) | o;
  bf16x8_t v;
  uint32_t* p = reinterpret_cast<uint32_t*>(&v);
  p[0] = r0; p[1] = r1; p[2] = r2; p[3] = r3;
  return v;
}

// int6 tiles: the low nibbles as unpack_q128, the high two bits from the lane's high-bit word of
// the group (the word's half h holds pair j's two high-bit pairs at bits 2j + 8h and 16 + 2j + 8h).
// 128 + q (q < 64) is exact in bf16.
__device__ __forceinline__ bf16x8_t unpack_q128_6(uint32_t w, uint32_t hw, int h) {
  const uint32_t m = 0x000F000Fu, o = 0x43004300u, mh = 0x00030003u;
  bf16x8_t v;
  uint32_t* p = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    p[j] = ((w >> (4 * j)) & m) | (((hw >> (2 * j + 8 * h)) & mh) << 4) | o;
  return v;
}

// int3 tiles: the lane's three words w0..w2 hold its 32 codes as 16 pairs; pair q = 8c + 4h + j
// (group c, half h, pair j of the half: codes 2j and 2j + 1) sits, for q < 15, in word q / 5 at
// bits 3(q % 5) .. +2 and 16 + 3(q % 5) .. +2, so one shift and one and-or make the bf16 pair
// 128 + code; pair 15 keeps bit i of each code in bit 15 / bit 31 of word i. 128 + q (q < 8) is
// exact in bf16.
__device__ __forceinline__ bf16x8_t unpack_q128_3(uint32_t w0, uint32_t w1, uint32_t w2, int c,
                                                  int h) {
  const uint32_t o = 0x43004300u;
  const uint32_t w[3] = {w0, w1, w2};
  bf16x8_t v;
  uint32_t* p = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int q = 8 * c + 4 * h + j;
    if (q < 15)
      p[j] = ((w[q / 5] >> (3 * (q % 5))) & 0x00070007u) | o;
    else
      p[j] = ((w0 >> 15) & 0x00010001u) | ((w1 >> 14) & 0x00020002u) | ((w2 >> 13) & 0x00040004u) | o;
  }
  return v;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 q) {
  bf16x8_t v;
  __builtin_memcpy(&v, &q, 16);
  return v;
}
__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 q) { return __builtin_bit_cast(bf16x8_t, q); }

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

__device__ __forceinline__ f32x16_t mfma32_f16(u32x4 a, u32x4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32_bf16(u32x4 a, u32x4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// x * sigmoid(x) with the hardware exp and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each);
// every kernel's SwiGLU goes through it, so they all agree bit for bit.
__device__ __forceinline__ float silu_f(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
}
// The gated activation on (bf16-valued) gate/up values, fp32 (QMOE_ACT_*: silu(g)*u; its clamped
// form, src/quanta/dsv4/moe.py:74-77; SwiGLU-OAI, src/quanta/minimax/model_m3.py:112-128).
__device__ __forceinline__ float glu_f(float g, float u, int act, float alpha, float limit) {
  if (act == QMOE_ACT_SILU) return silu_f(g) * u;
  const float gc = fminf(g, limit);
  const float uc = fminf(fmaxf(u, -limit), limit);
  return (act == QMOE_ACT_SILU_CLAMP) ? silu_f(gc) * uc
                                      : (uc + 1.0f) * (gc * __builtin_amdgcn_rcpf(1.0f + __expf(-alpha * gc)));
}

// Upper bound on the number of m-tiles a permuted (token, slot) list can produce.
inline int64_t mtile_upper_bound(int64_t mc, int64_t n_experts, int64_t m_tile) {
  int64_t active = mc < n_experts ? mc : n_experts;
  return (mc + m_tile - 1) / m_tile + active;
}

// Launchers shared between entry points (defined in the .hip files).
int launch_router_f32(const uint16_t* x, const float* wr, const float* shared_gate, int N, int H,
                      int E, float* logits, int ld_logits, hipStream_t stream);
// With tile_map: slot-major routing (each slot its own one-row m-tile, identity sorted/inv)
// in place of the permute; max_tiles >= N*k.
int launch_topk(const float* logits, int ld_logits, const float* bias, int N, int E, int k,
                int scoring, int n_group, int topk_group, int norm_topk, float scale, int has_sg,
                int32_t* idx, float* w, float* sg_out, hipStream_t stream,
                int32_t* tile_map = nullptr, int64_t max_tiles = 0, int32_t* sorted = nullptr,
                int32_t* inv = nullptr);
// With tile_map_big: experts of more than split_rows rows get m_tile_big-row tiles there and
// none in tile_map (the hybrid regime); without it, every expert's tiles go to tile_map.
int launch_permute(const int32_t* idx, int N, int k, int E, int m_tile, int32_t* counts,
                   int32_t* offsets, int32_t* tile_off, int32_t* sorted_slot, int32_t* inv,
                   int32_t* tile_map, int64_t max_tiles, hipStream_t stream, int split_rows = 0,
                   int m_tile_big = 0, int32_t* tile_map_big = nullptr, int64_t max_tiles_big = 0);

struct QmmArgs {
  const uint16_t* act;        // activation rows (bf16), row stride K (or act_stride)
  int64_t act_rows;           // number of activation rows (bounds check)
  const int32_t* slot_of;     // sorted position -> slot id (nullable: identity)
  int slot_div;               // activation row = slot / slot_div
  int64_t n_slots;            // total sorted positions (bounds check on slot ids)
  const int32_t* offsets;     // [E+1] segment offsets (nullable: dense, one segment of M rows)
  const int32_t* tile_off;    // [E+1] m-tile prefix per segment (nullable in dense mode)
  const int4* tile_map;       // per m-tile {expert, m0, rows} from permute (nullable: search)
  int64_t dense_rows;         // M for dense mode
  int n_experts;              // E (1 in dense mode)
  int K;                      // reduction length
  int n_rows;                 // weight rows per expert (2I for SwiGLU)
  const void* codes;          // tiled int4 codes or tiled bf16 weights
  const uint16_t* sb;         // tiled scale/bias (int4 only)
  void* out;                  // output rows by sorted position
  int ld_out;                 // output row stride (elements)
  const uint16_t* act16;      // large int4 regime: fp16 copy of act, row r scaled by 1/row_sinv[r]
  const float* row_sinv;      // large int4 regime: per activation row inverse scale (2^e)
  int mtiles;                 // large regime: m-tiles in the grid (entries of tile_map it reads)
  int glu;                    // SwiGLU epilogue: gated activation (QMOE_ACT_*)
  float glu_alpha;            // SWIGLU_OAI alpha
  float glu_limit;            // clamp of SILU_CLAMP / SWIGLU_OAI
  const uint16_t* act_hi;     // small quantized regime, nullable: the activation rows of the
                              // weight tiles from split_tile on (AWQ: the up half of gate_up
                              // reads rows prescaled for the up projection)
  int split_tile;             // first 16-row tile that reads act_hi (a multiple of 4; large
                              // regime: of 16, of 32 for the 512-row kernel)
  const uint16_t* act16_hi;   // large int4 regime, nullable: act16 and row_sinv of act_hi, read
  const float* row_sinv_hi;   // by the weight-row blocks from split_tile on
  const int32_t* expert_map;  // small regime, nullable: expert -> its slot in this launch's
                              // weight stack, -1 when it is not in the stack (its m-tiles exit)
  const int8_t* row_exp;      // large int4 regime, nullable: per weight row [n_experts][n_rows]
                              // the power of two 2^row_exp that brings the row's dequantized
                              // weights into fp16's normal range (undone in the epilogue)
  const uint16_t* norm_w;     // dense bf16 pair launch, nullable: the rows of `act` are RMSNorm'd
                              // on the fly, bf16(norm_w * (x * r)), r = 1/sqrt(mean(x^2) + eps)
                              // summed in the canonical order of rmsnorm_row (norm.hip)
  float norm_eps;
  uint16_t* norm_out;         // nullable: the normalised rows, written by job 0's wavefronts
  int dense_mtile;            // large regime, one dense segment: rows per m-tile (16..128, a
                              // multiple of 16; 0 = 128), so a short product still spreads
                              // over enough workgroups
  const uint32_t* act_ready;  // decode dataflow kernel: per m-tile counters (kSyncStride words
  uint32_t act_ready_target;  // apart) of the activation rows' producers; complete at the target
  uint32_t* timeouts;         // where a bounded wait that ran out is counted
  uint32_t* zero_words;       // dense pair launch, nullable: n_zero counters (kSyncStride words
  int n_zero;                 // apart) its first workgroup clears for the dataflow kernel after it
  int act_stride;             // elements from one activation row to the next (0: K)
};

enum { FMT_INT4 = 0, FMT_BF16 = 1, FMT_INT6 = 2, FMT_INT3 = 3, FMT_INT8 = 4 };
// affine-quantized weight formats summed as codes (int3, int4 or int6 codes with per-64
// scale/bias, the affine part applied to the products). int8 weights are not among them: they
// are dequantized to bf16 in registers and run the bf16 products (dense formats).
constexpr bool fmt_quant(int fmt) { return fmt == FMT_INT4 || fmt == FMT_INT6 || fmt == FMT_INT3; }
constexpr bool fmt_dense(int fmt) { return fmt == FMT_BF16 || fmt == FMT_INT8; }

// One lane's weight fragment of a 32-deep step of a dense product: 8 bf16 weights (tiled bf16),
// or 8 int8 codes with their row's (scale, bias) pair of the 64-column group (tiled int8).
template <int FMT> struct DenseFrag { u32x4 w; };
template <> struct DenseFrag<FMT_INT8> { u32x2 q; uint32_t sb; };

// Streams of a tiled dense matrix for one lane: bf16 [rows/16][K/32][64][8] or int8 codes
// [rows/16][K/32][64][8 B] + sb [rows/16][K/64][16][scale, bias]; `tile` = 16-row tile index of
// the whole stack (expert * rows/16 + tile of the expert).
template <int FMT>
struct DenseTile {
  const void* p;
  const uint32_t* sb;
  __device__ __forceinline__ void init(const void* codes, const uint16_t* sbase, int64_t tile, int K,
                                       int lane) {
    const int nks = K / 32;
    if constexpr (FMT == FMT_INT8) {
      p = static_cast<const u32x2*>(codes) + tile * nks * 64 + lane;
      sb = reinterpret_cast<const uint32_t*>(sbase) + tile * (K / 64) * 16 + (lane & 15);
    } else {
      p = static_cast<const u32x4*>(codes) + tile * nks * 64 + lane;
      sb = nullptr;
    }
  }
  // fragment of step c
  __device__ __forceinline__ DenseFrag<FMT> load(int c) const {
    if constexpr (FMT == FMT_INT8)
      return DenseFrag<FMT>{static_cast<const u32x2*>(p)[c * 64], sb[(c >> 1) * 16]};
    else
      return DenseFrag<FMT>{static_cast<const u32x4*>(p)[c * 64]};
  }
};

// bf16 fragment of a dense weight fragment. int8: code byte j (LSB-first) becomes
// bf16(fmaf(s, c_j, b)), the product exact in fp32 (8-bit x 8-bit mantissas), rounded to nearest
// even: the same bits as the dequant of the native int8 matrix (qmoe_dequant), so the int8 and
// bf16 forms of a matrix give identical products.
template <int FMT>
__device__ __forceinline__ u32x4 dense_bf16(const DenseFrag<FMT>& f) {
  if constexpr (FMT == FMT_INT8) {
    const float s = __uint_as_float(f.sb << 16), b = __uint_as_float(f.sb & 0xFFFF0000u);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = f.q[j >> 1] >> (16 * (j & 1));
      const float lo = static_cast<float>(w & 0xFFu), hi = static_cast<float>((w >> 8) & 0xFFu);
      o[j] = pack_bf16x2_rne(fmaf(s, lo, b), fmaf(s, hi, b));
    }
    return o;
  } else {
    return f.w;
  }
}
enum { EPI_SWIGLU = 0, EPI_BF16 = 1, EPI_F32 = 2 };

int launch_qmm(const QmmArgs& a, int fmt, int epi, int regime, int64_t mtile_bound,
               hipStream_t stream);
// Chunk count of the small-regime bf16 products over K: ~8 32-deep steps per chunk, one
// wavefront per chunk, chunk sums added in chunk order.
inline int bf16_chunks(int K) {
  const int nks = K / 32;
  return (nks >= 128) ? 16 : (nks >= 64) ? 8 : (nks >= 32) ? 4 : (nks >= 16) ? 2 : 1;
}
// One launch of two dense small-regime products over the same rows and K: a1 (tiled bf16) with
// the fp32 epilogue (router logits), a2 (tiled bf16 or int8, fmt2) with SwiGLU (shared expert
// gate_up), or with `split` the gate and up halves as bf16 [gate | up] rows (a2.ld_out >= its
// rows) for a consumer that forms the gated activation itself (the decode dataflow launch).
int launch_qmm_pair_bf16(const QmmArgs& a1, const QmmArgs& a2, hipStream_t stream,
                         int fmt2 = FMT_BF16, bool split = false);
// Whether the pair launch over `rows` rows of K normalises them itself (QmmArgs::norm_w): one
// job per workgroup (K >= 1024), and each wavefront's K chunk one load batch (8 32-wide steps
// with one m-tile per wavefront, 4 with two), or up to 16 steps for one or two rows.
bool pair_norm_fusable(int K, int64_t rows);
// Decode combine with the shared expert's down projection fused in (wd: tiled bf16 [H, Is], or
// tiled int8 codes with their scale/bias wd_sb when fmt is FMT_INT8).
// resid (nullable): the decoder layer's residual row, y = bf16(resid + bf16(block output)).
int launch_combine_shared(const uint16_t* d, const int32_t* inv, const float* w, int N, int k,
                          int H, const uint16_t* sh_h, int Is, const void* wd,
                          const uint16_t* wd_sb, int fmt, const float* shared_gate, uint16_t* y,
                          hipStream_t stream, const uint16_t* resid = nullptr);
// Tiled int8 [rows/16][K/32][64][8 B] + sb -> tiled bf16 [rows/16][K/32][64][8], each weight
// bf16(s*q + b) as dense_bf16 makes it.
int launch_expand_int8(const uint32_t* codes, const uint16_t* sb, int64_t rows, int K,
                       uint16_t* out, hipStream_t stream);
// act [rows][K] bf16 -> act16 fp16 with a per-row power-of-two scale (exact for bf16 values
// within 2^28 of the row's largest magnitude); row_sinv[r] = the inverse scale.
int launch_act_to_f16(const uint16_t* act, int64_t rows, int K, uint16_t* act16, float* row_sinv,
                      hipStream_t stream);
inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }
inline size_t act16_ws_bytes(int64_t rows, int K) {
  return align256(static_cast<size_t>(rows) * K * 2) + align256(static_cast<size_t>(rows) * 4);
}
int launch_combine(const uint16_t* d, const int32_t* inv, const float* w, int N, int k, int H,
                   const uint16_t* shared_out, const float* shared_gate, uint16_t* y,
                   hipStream_t stream, const uint16_t* resid = nullptr);
// RMSNorm rows: out = bf16(w * (x * rsqrt(mean(x^2) + eps))) in fp32 (norm.hip).
// Activation-aware (AWQ) expert scales (src/quanta/dsv4/moe.py:112-137): per sorted row m of
// expert e (offsets), xg[m] = bf16(x[tok] / s_gu[e][0]) and xu[m] = bf16(x[tok] / s_gu[e][1]),
// tok = sorted[m] / k; s_gu bf16 [E][2][H].
int launch_awq_prescale(const uint16_t* x, const int32_t* sorted, const int32_t* offsets, int E,
                        int k, int64_t mc, int H, const uint16_t* s_gu, uint16_t* xg, uint16_t* xu,
                        hipStream_t stream);
// The same quotients for the hybrid regime, in one pass: rows of experts with at most split_rows
// rows as bf16 into xgu [2][mc][H] (gate rows, then up rows), the others only as fp16 copies
// x16 [2][mc][H] with row scales x_sinv [2][mc] (launch_act_to_f16's conversion). H <= 8192.
constexpr int kAwqSplitMaxH = 8192;
int launch_awq_prescale_split(const uint16_t* x, const int32_t* sorted, const int32_t* offsets,
                              int E, int k, int64_t mc, int H, const uint16_t* s_gu,
                              int split_rows, uint16_t* xgu, uint16_t* x16, float* x_sinv,
                              hipStream_t stream);
// h[m] = bf16(glu(g, u) / s_dn[e]) over gu [mc][2I] (gate | up, bf16) with s_dn bf16 [E][I];
// s_dn NULL: h[m] = bf16(glu(g, u)) (offsets unused).
int launch_awq_glu(const uint16_t* gu, const int32_t* offsets, int E, int64_t mc, int I,
                   const uint16_t* s_dn, int act, float alpha, float limit, uint16_t* h,
                   hipStream_t stream);
// For H % 32 == 0 the sum of squares follows the canonical order that the fused-norm pair launch
// also follows: H cut into bf16_chunks(H) chunks of 32-wide steps; within a chunk, lane group g
// (0..3) sums the elements 32 s + 8 g + j (steps s in order, j = 0..7 in order) with fmaf from
// zero; the four group sums combine as (g0 + g1) + (g2 + g3); the chunk sums add in chunk order.
int launch_rmsnorm(const uint16_t* x, const uint16_t* w, int64_t N, int H, float eps, uint16_t* out,
                   hipStream_t stream);

// Slot-major routed gate_up with the top-k done in the launch (qmm.hip): int4 weights, SwiGLU
// epilogue, a.act the N token rows (no slot_of/offsets); writes idx/w/sg and the slot-major
// tile map, sorted and inv exactly as launch_topk does with a tile map.
// The routed int4 SwiGLU gate_up (small regime, a1 with its tile map over mtiles1 m-tiles) and a
// dense int8 product (a2: the shared expert's down projection) in one launch, each with the
// arithmetic of its own launch. Returns 1 without launching when the two shapes have no
// compiled combination.
int launch_gate_up_shared_down(const QmmArgs& a1, int64_t mtiles1, const QmmArgs& a2,
                               hipStream_t stream);
bool route_gate_up_fits(int E, int k);
// Workgroups of that launch for mc slots (each ranks its token's logits once).
int64_t route_gate_up_workgroups(int K, int n_rows, int64_t mc);
int launch_route_gate_up(const QmmArgs& a, int N, const float* logits, int ld, const float* bias,
                         int E, int k, int scoring, int n_group, int topk_group, int norm_topk,
                         float scale, int has_sg, int32_t* idx, float* w, float* sg,
                         int32_t* tile_map, int64_t max_tiles, int32_t* sorted, int32_t* inv,
                         hipStream_t stream, const QmmArgs* sdn = nullptr);
// (sdn: the shared expert's int8 down projection, one dense segment, in the same launch; returns 1
// without launching when that pair has no compiled shape)
// Slot-major decode tail (fused.hip): routed int4 down, shared down (tiled bf16 or int8 as sfmt)
// and the combine in one launch; h/idx/w in slot order. down_combine_fits: the shapes it takes
// (I = 512 or 1024, a shared expert of <= 8 bf16 chunks, at most 24 units of work per
// workgroup: one or two tokens). sh_out (with sh_h null): the bf16 shared output, computed
// earlier, added in the combine.
bool down_combine_fits(int N, int k, int H, int I, int Is);
int launch_down_combine(const uint16_t* h, const int32_t* idx, const float* w, const float* sg,
                        int N, int k, int H, int I, const void* codes, const uint16_t* sb,
                        const uint16_t* sh_h, int Is, const void* wd, const uint16_t* wd_sb,
                        int sfmt, const uint16_t* resid, uint16_t* y, hipStream_t stream,
                        const uint16_t* sh_out = nullptr);

// Counters of the decode dataflow kernel sit kSyncStride words apart (256 bytes): polls and
// atomics of one counter then never queue behind another's on the same cache line.
constexpr int kSyncStride = 64;

constexpr int kSmallMTile = 16;
constexpr int kLargeMTile = 128;
// Large-M (prefill) regime: experts routed more rows than this use 128-row tiles on the large
// kernel, the others 16-row tiles on the small kernel.
constexpr int kHybridSplitRows = 16;

}  // namespace qmoe
