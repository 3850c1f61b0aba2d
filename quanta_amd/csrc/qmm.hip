// Grouped quantized matmul over expert segments (the gather-qmm of the MoE block), for gfx950.
//
// out[p, n] = sum_k act[row(p), k] * W_e[n, k]  for every sorted position p in expert e's
// segment, where W_e is affine int4 g64 (w = s*q + b, bf16 s/b per 64 along k) or bf16.
// Epilogues: fused SwiGLU over the gate|up row halves (-> bf16 h), plain bf16, or float32.
//
// Reference: mx.gather_qmm(x, packed, scale, bias, rhs_indices=exp, transpose=True,
// group_size=64, bits=4) at src/quanta/qwen35/moe.py:117-123 and the sorted variant
// src/quanta/dsv4/moe.py:114-124; SwiGLU src/quanta/qwen35/moe.py:59-63 (gate = first I rows,
// up = last I rows); bf16 sibling mx.gather_mm src/quanta/qwen35/moe.py:66-82; the shared
// expert's dense bf16 matmuls src/quanta/qwen35/moe.py:145-151; router logits
// src/quanta/qwen35/moe.py:47.
//
// Two regimes, both on v_mfma_f32_16x16x32_bf16 with activations as the A operand
// (16 token rows) and weights as the B operand (16 weight rows as columns):
//  * small-M ("decode"): 16-token m-tiles; each wavefront streams one 16-row weight tile (two
//    for SwiGLU) straight from HBM into registers with one contiguous 1 KiB dwordx4 load per
//    superblock, and never materialises a dequantised weight. For int4 it multiplies the raw
//    codes (as bf16 128+q, exact) and applies the per-group affine map on the 16x16 result:
//      sum_k x_k (s q_k + b) = s * sum_k x_k (128+q_k) + (b - 128 s) * sum_k x_k,
//    with sum_k x_k from one extra MFMA against a ones fragment. Optional split-K across the
//    workgroup's wavefronts, reduced through LDS.
//  * large-M ("prefill"): 128x128 workgroup tiles; each 128-deep k-step is dequantised
//    cooperatively into LDS as bf16 (one dequant per weight element per workgroup, shared by
//    128 tokens), activations gathered by token id into LDS, then 2x2 wavefronts of 64x64.
#include "qmoe_internal.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

__device__ __forceinline__ int find_segment(const int32_t* __restrict__ tile_off, int E, int mt) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tile_off[mid] <= mt) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Resolve the m-tile handled by this workgroup. Returns false when the tile is past the end
// (the grid is sized by an upper bound); uniform across the workgroup.
__device__ __forceinline__ bool resolve_mtile(const QmmArgs& a, int mt, int m_tile, int& e,
                                              int& m0, int& m_cnt) {
  if (a.tile_map) {
    const int4 t = a.tile_map[mt];
    if (t.x < 0) return false;
    e = t.x;
    m0 = t.y;
    m_cnt = t.z;
  } else if (a.offsets) {
    if (mt >= a.tile_off[a.n_experts]) return false;
    e = find_segment(a.tile_off, a.n_experts, mt);
    m0 = a.offsets[e] + (mt - a.tile_off[e]) * m_tile;
    m_cnt = min(m_tile, a.offsets[e + 1] - m0);
  } else {
    e = 0;
    m0 = mt * m_tile;
    m_cnt = static_cast<int>(min<int64_t>(m_tile, a.dense_rows - m0));
  }
  return m_cnt > 0;
}

// Activation row for sorted position pos, or -1 when it must read as zeros.
__device__ __forceinline__ int64_t act_row(const QmmArgs& a, int pos) {
  int64_t r = pos;
  if (a.slot_of) {
    const int s = a.slot_of[pos];
    if (s < 0 || s >= a.n_slots) return -1;
    r = s / a.slot_div;
  }
  return (r >= 0 && r < a.act_rows) ? r : -1;
}

template <int EPI>
__device__ __forceinline__ void store_out(const QmmArgs& a, int row, int col, float v, float v_up) {
  const int64_t off = static_cast<int64_t>(row) * a.ld_out + col;
  if (EPI == EPI_SWIGLU) {
    // gate/up are bf16 tensors in the reference's flow; SwiGLU then rounds once to bf16.
    const float g = bf16_to_f32(f32_to_bf16(v));
    const float u = bf16_to_f32(f32_to_bf16(v_up));
    static_cast<uint16_t*>(a.out)[off] = f32_to_bf16(silu_f(g) * u);
  } else if (EPI == EPI_BF16) {
    static_cast<uint16_t*>(a.out)[off] = f32_to_bf16(v);
  } else {
    static_cast<float*>(a.out)[off] = v;
  }
}

// ============================================================================ small-M kernel
// One wavefront = one 16-row weight tile job (two tiles, gate and up, for SwiGLU) over one
// k-range of one 16-position m-tile. KSPLIT wavefronts of a workgroup share a job and split K;
// their partial tiles are summed through LDS. WAVES = max(4, KSPLIT) wavefronts per workgroup.
template <int FMT, int KSPLIT>
struct SmallStage {
  static constexpr int NT = 2;
  u32x4 q[NT];    // int4: raw codes of one superblock / bf16: weight fragments of one 32-k step
  uint2 sb[NT];   // int4 scale/bias of the superblock's two groups
  u32x4 x[4];     // activation fragments
};

template <int FMT, int EPI, int KSPLIT>
__global__ void __launch_bounds__(KSPLIT > 4 ? 64 * KSPLIT : 256)
qmm_small_kernel(QmmArgs a, int n_jobs) {
  constexpr int WAVES = KSPLIT > 4 ? KSPLIT : 4;
  constexpr int JOBS_PER_WG = WAVES / KSPLIT;
  constexpr int NT = (EPI == EPI_SWIGLU) ? 2 : 1;
  __shared__ f32x4_t red[(KSPLIT > 1) ? WAVES * NT * 64 : 1];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int e, m0, m_cnt;
  if (!resolve_mtile(a, blockIdx.y, kSmallMTile, e, m0, m_cnt)) return;

  const int job = blockIdx.x * JOBS_PER_WG + wave / KSPLIT;
  const int kpart = wave % KSPLIT;
  const bool job_ok = job < n_jobs;
  const int mrow = lane & 15, lg = lane >> 4;

  int64_t arow = -1;
  if (mrow < m_cnt) arow = act_row(a, m0 + mrow);
  const bool row_ok = arow >= 0;
  const uint16_t* xrow = a.act + (row_ok ? arow : 0) * static_cast<int64_t>(a.K);

  f32x4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int tiles_per_expert = a.n_rows / 16;
  int tile[NT];
  tile[0] = job;
  if (NT == 2) tile[NT - 1] = job + a.n_rows / 32;   // up half starts at row I = n_rows/2

  if (job_ok) {
    if (FMT == FMT_INT4) {
      const int nsb = a.K / 128;
      const int p0 = kpart * nsb / KSPLIT, p1 = (kpart + 1) * nsb / KSPLIT;
      const u32x4* cp[NT];
      const uint2* sp[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t tb = (static_cast<int64_t>(e) * tiles_per_expert + tile[t]) * nsb;
        cp[t] = static_cast<const u32x4*>(a.codes) + tb * 64 + lane;
        sp[t] = reinterpret_cast<const uint2*>(a.sb) + tb * 16 + (lane & 15);
      }
      const u32x4* xp = reinterpret_cast<const u32x4*>(xrow) + 2 * lg;   // 16 lg bf16
      bf16x8_t ones;
      {
        uint32_t* o = reinterpret_cast<uint32_t*>(&ones);
        o[0] = o[1] = o[2] = o[3] = 0x3F803F80u;
      }
      const f32x4_t zero4{0.f, 0.f, 0.f, 0.f};
      // Two register stages: the loads of superblock p+1 are in flight while p is computed.
      SmallStage<FMT, KSPLIT> st[2];
      auto load = [&](SmallStage<FMT, KSPLIT>& s, int p) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          s.q[t] = cp[t][p * 64];
          s.sb[t] = sp[t][p * 16];
        }
        // group 2p: k 16lg + 0..7 (step 0) and + 8..15 (step 1); group 2p+1 likewise, +64.
        // Only rows of the segment load; the rest of the 16-row tile is zeros.
        if (row_ok) {
          s.x[0] = xp[p * 16 + 0];
          s.x[1] = xp[p * 16 + 1];
          s.x[2] = xp[p * 16 + 8];
          s.x[3] = xp[p * 16 + 9];
        } else {
          s.x[0] = s.x[1] = s.x[2] = s.x[3] = u32x4{0u, 0u, 0u, 0u};
        }
      };
      auto compute = [&](const SmallStage<FMT, KSPLIT>& s) __attribute__((always_inline)) {
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
          const bf16x8_t A0 = as_bf16x8(s.x[2 * gg]);
          const bf16x8_t A1 = as_bf16x8(s.x[2 * gg + 1]);
          f32x4_t xs = mfma16(A0, ones, zero4);
          xs = mfma16(A1, ones, xs);
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const uint32_t w0 = gg ? s.q[t].z : s.q[t].x;
            const uint32_t w1 = gg ? s.q[t].w : s.q[t].y;
            f32x4_t r = mfma16(A0, unpack_q128(w0), zero4);
            r = mfma16(A1, unpack_q128(w1), r);
            const uint32_t sbw = gg ? s.sb[t].y : s.sb[t].x;
            const float sc = bf16lo_to_f32(sbw);
            const float bi = bf16hi_to_f32(sbw) - 128.0f * sc;
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][j] = fmaf(sc, r[j], fmaf(bi, xs[j], acc[t][j]));
          }
        }
      };
      int p = p0;
      if (p < p1) load(st[0], p);
      while (p < p1) {
        if (p + 1 < p1) load(st[1], p + 1);
        compute(st[0]);
        if (++p >= p1) break;
        if (p + 1 < p1) load(st[0], p + 1);
        compute(st[1]);
        ++p;
      }
    } else {  // FMT_BF16
      const int nks = a.K / 32;
      const int k0 = kpart * nks / KSPLIT, k1 = (kpart + 1) * nks / KSPLIT;
      const u32x4* wp[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t tb = (static_cast<int64_t>(e) * tiles_per_expert + tile[t]) * nks;
        wp[t] = static_cast<const u32x4*>(a.codes) + tb * 64 + lane;
      }
      const u32x4* xp = reinterpret_cast<const u32x4*>(xrow) + lg;   // 8 lg bf16
#pragma unroll 4
      for (int c = k0; c < k1; ++c) {
        u32x4 wv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) wv[t] = wp[t][c * 64];
        u32x4 xv = u32x4{0u, 0u, 0u, 0u};
        if (row_ok) xv = xp[c * 4];
        const bf16x8_t A = as_bf16x8(xv);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = mfma16(A, as_bf16x8(wv[t]), acc[t]);
      }
    }
  }

  if (KSPLIT > 1) {
    const int jl = wave / KSPLIT;
    if (kpart > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) red[(wave * NT + t) * 64 + lane] = acc[t];
    }
    __syncthreads();
    if (kpart == 0) {
#pragma unroll
      for (int kp = 1; kp < KSPLIT; ++kp)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const f32x4_t o = red[((jl * KSPLIT + kp) * NT + t) * 64 + lane];
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[t][j] += o[j];
        }
    }
  }
  if (!job_ok || kpart != 0) return;

  const int col = job * 16 + (lane & 15);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int mr = 4 * lg + j;
    if (mr < m_cnt) store_out<EPI>(a, m0 + mr, col, acc[0][j], acc[NT - 1][j]);
  }
}

// ============================================================================ large-M kernel
// Workgroup tile: 128 sorted positions x 256 weight rows (SwiGLU: 128 gate + 128 up rows ->
// 128 h columns), one 128-deep k-step (one int4 superblock) per iteration. 4 wavefronts in a
// 2x2 arrangement, each owning 64 positions x 128 weight rows as 2x4 blocks of
// v_mfma_f32_32x32x16 (f16 for int4 weights, bf16 for bf16 weights).
//
// int4 weights are dequantized in registers, right after their global load and while the
// previous step's MFMAs run, with packed fp16 FMAs (fp16(s*q + b), one rounding; 11-bit
// mantissa), and activations come from the fp16 per-row-scaled copy (act16), so the step is an
// exact-input fp16 product with fp32 accumulation. Outputs are rescaled per row by row_sinv.
// bf16 weights (shared expert, router) are copied as they are, against bf16 activations.
//
// LDS (dynamic, 96 KiB): A [4 m-blocks of 32][8 k-steps of 16][64 lanes] and
// B [8 n-blocks of 32][8][64], 16 B per entry, each entry one lane's MFMA fragment (lane l:
// row l%32, k 8*(l/32)..+8 of the 16-k step), so fragment reads are conflict-free 16-byte loads.
constexpr int kLgThreads = 256;
constexpr size_t kLgLdsBytes = (2048 + 4096) * 16;

template <int FMT, int EPI>
__global__ void __launch_bounds__(kLgThreads) qmm_large_kernel(QmmArgs a) {
  extern __shared__ u32x4 lds[];
  u32x4* la = lds;
  u32x4* lb = lds + 2048;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int e, m0, m_cnt;
  if (!resolve_mtile(a, blockIdx.y, kLargeMTile, e, m0, m_cnt)) return;
  const int cb = blockIdx.x;
  const int tiles_per_expert = a.n_rows / 16;
  const int64_t ebase = static_cast<int64_t>(e) * tiles_per_expert;
  const int nsb = a.K / 128;
  const int nks32 = a.K / 32;

  // 16-row global tile of local tile lt (0..15)
  auto gtile = [&](int lt) -> int {
    if (EPI == EPI_SWIGLU) return (lt < 8) ? 8 * cb + lt : a.n_rows / 32 + 8 * cb + (lt - 8);
    return 16 * cb + lt;
  };

  // ---- activation staging: thread -> row ar (0..127), 64-wide k half ah
  const int ar = tid & 127, ah = tid >> 7;
  int64_t arow = -1;
  if (ar < m_cnt) arow = act_row(a, m0 + ar);
  const uint32_t xmask = (arow >= 0) ? 0xFFFFFFFFu : 0u;
  const uint16_t* abase = (FMT == FMT_INT4) ? a.act16 : a.act;
  const u32x4* asrc =
      reinterpret_cast<const u32x4*>(abase + (arow >= 0 ? arow : 0) * static_cast<int64_t>(a.K)) +
      ah * 8;
  // chunk i covers k 64ah + 8i: 16-k step 4ah + i/2, half (i&1)
  u32x4* adst = la + ((ar >> 5) * 8 + 4 * ah) * 64 + (ar & 31);

  // ---- weight staging pointers
  const u32x4* cptr[4];
  const uint2* sptr[4];
  int bdst[4];
  if (FMT == FMT_INT4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int slot = tid + 256 * i, lt = slot >> 6, L = slot & 63;
      const int64_t tb = (ebase + gtile(lt)) * nsb;
      cptr[i] = static_cast<const u32x4*>(a.codes) + tb * 64 + L;
      sptr[i] = reinterpret_cast<const uint2*>(a.sb) + tb * 16 + (L & 15);
      const int rb = 16 * lt + (L & 15), g = L >> 4;
      bdst[i] = ((rb >> 5) * 8 + g) * 64 + (rb & 31);   // + word-dependent offsets below
    }
  }
  const u32x4* wbase = nullptr;
  if (FMT == FMT_BF16) {
    // thread owns lane slot (k32 chunk (tid>>6)&3, lane tid&63) of local tiles 0..15
    wbase = static_cast<const u32x4*>(a.codes) + ((tid >> 6) & 3) * 64 + (tid & 63);
  }

  f32x16_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int wm = wave >> 1, wn = wave & 1;
  int wtl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    wtl[j] = (EPI == EPI_SWIGLU) ? ((j < 2) ? 2 * wn + j : 4 + 2 * wn + (j - 2)) : 4 * wn + j;

  u32x4 xv[8];
  u32x4 bq[FMT == FMT_INT4 ? 4 : 16];   // raw codes (int4) or bf16 weight fragments
  uint2 bs[4];
  u32x4 dq[16];                         // dequantized fp16 weights (int4)

  auto load_step = [&](int p) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = asrc[p * 16 + i] & xmask;
    if (FMT == FMT_INT4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bq[i] = cptr[i][p * 64];
        bs[i] = sptr[i][p * 16];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        bq[i] = wbase[((ebase + gtile(i)) * nks32 + 4 * p) * 64];
    }
  };
  auto dequant_step = [&]() __attribute__((always_inline)) {
    if (FMT == FMT_INT4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
          const uint32_t sbw = gg ? bs[i].y : bs[i].x;
          const _Float16 s = static_cast<_Float16>(bf16lo_to_f32(sbw));
          const _Float16 b = static_cast<_Float16>(bf16hi_to_f32(sbw));
          const f16x2_t s2 = {s, s}, b2 = {b, b};
          dq[4 * i + 2 * gg + 0] = dequant_word_f16(gg ? bq[i].z : bq[i].x, s2, b2);
          dq[4 * i + 2 * gg + 1] = dequant_word_f16(gg ? bq[i].w : bq[i].y, s2, b2);
        }
      }
    }
  };

  load_step(0);
  dequant_step();
  for (int p = 0; p < nsb; ++p) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) adst[(i >> 1) * 64 + 32 * (i & 1)] = xv[i];
    if (FMT == FMT_INT4) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          // word t: group gg = t>>1 (k 64gg..), step s = t&1 -> 16-k step 4gg + g, half s
          const int gg = t >> 1, s = t & 1;
          lb[bdst[i] + (4 * gg) * 64 + 32 * s] = dq[4 * i + t];
        }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // tile i, k32 chunk cc = (tid>>6)&3, lane L = tid&63: row 16i + L%16, k 32cc + 8(L/16)
        const int L = tid & 63, cc = (tid >> 6) & 3;
        const int rb = 16 * i + (L & 15), kk = 32 * cc + 8 * (L >> 4);
        lb[((rb >> 5) * 8 + (kk >> 4)) * 64 + 32 * ((kk >> 3) & 1) + (rb & 31)] = bq[i];
      }
    }
    __syncthreads();
    const bool more = p + 1 < nsb;
    if (more) load_step(p + 1);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      u32x4 A[2], B[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) A[i] = la[((2 * wm + i) * 8 + ks) * 64 + lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) B[j] = lb[(wtl[j] * 8 + ks) * 64 + lane];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = (FMT == FMT_INT4) ? mfma32_f16(A[i], B[j], acc[i][j])
                                        : mfma32_bf16(A[i], B[j], acc[i][j]);
    }
    if (more) dequant_step();
  }

  // ---- epilogue: lane holds C[row 8(r/4) + 4(lane/32) + r%4][col lane%32] of each block
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mr = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (mr >= m_cnt) continue;
      float rs = 1.0f;
      if (FMT == FMT_INT4) {
        const int64_t ar2 = act_row(a, m0 + mr);
        rs = (ar2 >= 0) ? a.row_sinv[ar2] : 0.0f;
      }
      if (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = 128 * cb + 64 * wn + 32 * t + (lane & 31);
          store_out<EPI>(a, m0 + mr, col, acc[i][t][r] * rs, acc[i][2 + t][r] * rs);
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int col = 256 * cb + 32 * (4 * wn + t) + (lane & 31);
          store_out<EPI>(a, m0 + mr, col, acc[i][t][r] * rs, 0.f);
        }
      }
    }
  }
}

// ---------------------------------------------------------------- fp16 activation copy
// One workgroup per row: absmax, then act16 = fp16(act * 2^(14 - e)) with 2^(e-1) <= absmax < 2^e,
// so every value sits below 2^14 and all bf16 values within 2^28 of the row maximum convert
// exactly. row_sinv = 2^(e - 14) undoes it on the product (a power of two: exact).
__global__ void __launch_bounds__(256) act_to_f16_kernel(const uint16_t* __restrict__ act, int K,
                                                         uint16_t* __restrict__ act16,
                                                         float* __restrict__ row_sinv) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(act + row * K);
  const int n8 = K / 8;
  float m = 0.f;
  for (int i = threadIdx.x; i < n8; i += 256) {
    const u32x4 v = src[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m = fmaxf(m, fabsf(bf16lo_to_f32(v[j])));
      m = fmaxf(m, fabsf(bf16hi_to_f32(v[j])));
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int ex = 0;
  if (m > 0.f && m <= 3.4e38f) frexpf(m, &ex);   // m = f * 2^ex, f in [0.5, 1)
  const int sh = (m > 0.f && m <= 3.4e38f) ? 14 - ex : 0;
  if (threadIdx.x == 0) row_sinv[row] = ldexpf(1.0f, -sh);
  u32x4* dst = reinterpret_cast<u32x4*>(act16 + row * K);
  for (int i = threadIdx.x; i < n8; i += 256) {
    const u32x4 v = src[i];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2_t h = {static_cast<_Float16>(ldexpf(bf16lo_to_f32(v[j]), sh)),
                         static_cast<_Float16>(ldexpf(bf16hi_to_f32(v[j]), sh))};
      o[j] = __builtin_bit_cast(uint32_t, h);
    }
    dst[i] = o;
  }
}

int launch_act_to_f16(const uint16_t* act, int64_t rows, int K, uint16_t* act16, float* row_sinv,
                      hipStream_t stream) {
  if (rows <= 0) return 0;
  if (K % 8) return fail("act_to_f16: K % 8 == 0 required");
  if (rows > 0x7fffffff) return fail("act_to_f16: too many rows");
  act_to_f16_kernel<<<static_cast<unsigned>(rows), 256, 0, stream>>>(act, K, act16, row_sinv);
  return check_launch("act_to_f16");
}


// ============================================================================ launcher
template <int FMT, int EPI, int KSPLIT>
static void launch_small_k(const QmmArgs& a, int64_t mtiles, hipStream_t stream) {
  constexpr int WAVES = KSPLIT > 4 ? KSPLIT : 4;
  const int n_jobs = (EPI == EPI_SWIGLU) ? a.n_rows / 32 : a.n_rows / 16;
  const int jobs_per_wg = WAVES / KSPLIT;
  dim3 grid((n_jobs + jobs_per_wg - 1) / jobs_per_wg, static_cast<unsigned>(mtiles));
  qmm_small_kernel<FMT, EPI, KSPLIT><<<grid, 64 * WAVES, 0, stream>>>(a, n_jobs);
}

template <int FMT, int EPI>
static void launch_small(const QmmArgs& a, int ksplit, int64_t mtiles, hipStream_t stream) {
  switch (ksplit) {
    case 16: launch_small_k<FMT, EPI, 16>(a, mtiles, stream); break;
    case 8: launch_small_k<FMT, EPI, 8>(a, mtiles, stream); break;
    case 4: launch_small_k<FMT, EPI, 4>(a, mtiles, stream); break;
    case 2: launch_small_k<FMT, EPI, 2>(a, mtiles, stream); break;
    default: launch_small_k<FMT, EPI, 1>(a, mtiles, stream); break;
  }
}

template <int FMT, int EPI>
static int launch_large(const QmmArgs& a, int64_t mtiles, hipStream_t stream) {
  // 96 KiB of dynamic LDS is above the default per-kernel limit; set it for the current device
  const hipError_t err =
      hipFuncSetAttribute(reinterpret_cast<const void*>(qmm_large_kernel<FMT, EPI>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLgLdsBytes));
  if (err != hipSuccess) return fail(std::string("qmm(large): LDS attribute: ") + hipGetErrorString(err));
  dim3 grid(a.n_rows / 256, static_cast<unsigned>(mtiles));
  qmm_large_kernel<FMT, EPI><<<grid, kLgThreads, kLgLdsBytes, stream>>>(a);
  return 0;
}

int launch_qmm(const QmmArgs& a, int fmt, int epi, int regime, int64_t mtile_bound,
               hipStream_t stream) {
  if (a.K <= 0 || a.n_rows <= 0) return fail("qmm: empty problem");
  if (mtile_bound <= 0) return 0;
  if (mtile_bound > 65535) return fail("qmm: too many m-tiles for one launch");
  if (regime == QMOE_REGIME_SMALL) {
    if (fmt == FMT_INT4 && a.K % 128) return fail("qmm: int4 needs K % 128 == 0");
    if (fmt == FMT_BF16 && a.K % 32) return fail("qmm: bf16 needs K % 32 == 0");
    if (a.n_rows % (epi == EPI_SWIGLU ? 32 : 16)) return fail("qmm: weight rows not a tile multiple");
    // Split-K depends on the shape only (never on the token count), so a row's summation
    // order, and therefore its result, is the same at every batch size (batch invariance).
    // int4 wavefronts keep >= 8 superblocks each; bf16 (router, shared expert) wavefronts
    // keep ~8 32-deep steps, which spreads the few dense row tiles over enough wavefronts.
    int ksplit;
    if (fmt == FMT_INT4) {
      ksplit = (a.K >= 4096) ? 4 : (a.K >= 2048) ? 2 : 1;
    } else {
      const int nks = a.K / 32;
      ksplit = (nks >= 128) ? 16 : (nks >= 64) ? 8 : (nks >= 32) ? 4 : (nks >= 16) ? 2 : 1;
    }
#define QMOE_SMALL(F, P) launch_small<F, P>(a, ksplit, mtile_bound, stream)
    if (fmt == FMT_INT4) {
      if (epi == EPI_SWIGLU) QMOE_SMALL(FMT_INT4, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_SMALL(FMT_INT4, EPI_BF16);
      else QMOE_SMALL(FMT_INT4, EPI_F32);
    } else {
      if (epi == EPI_SWIGLU) QMOE_SMALL(FMT_BF16, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_SMALL(FMT_BF16, EPI_BF16);
      else QMOE_SMALL(FMT_BF16, EPI_F32);
    }
#undef QMOE_SMALL
  } else {
    if (a.K % 128) return fail("qmm(large): K % 128 == 0 required");
    if (a.n_rows % 256) return fail("qmm(large): weight rows % 256 == 0 required");
    if (fmt == FMT_INT4 && (!a.act16 || !a.row_sinv))
      return fail("qmm(large): int4 weights need the fp16 activation copy");
    int rc;
#define QMOE_LARGE(F, P) rc = launch_large<F, P>(a, mtile_bound, stream)
    if (fmt == FMT_INT4) {
      if (epi == EPI_SWIGLU) QMOE_LARGE(FMT_INT4, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_LARGE(FMT_INT4, EPI_BF16);
      else QMOE_LARGE(FMT_INT4, EPI_F32);
    } else {
      if (epi == EPI_SWIGLU) QMOE_LARGE(FMT_BF16, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_LARGE(FMT_BF16, EPI_BF16);
      else QMOE_LARGE(FMT_BF16, EPI_F32);
    }
#undef QMOE_LARGE
    if (rc) return rc;
  }
  return check_launch("qmm");
}

}  // namespace qmoe
