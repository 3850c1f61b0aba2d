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
  if (a.offsets) {
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
template <int FMT, int EPI, int KSPLIT>
__global__ void __launch_bounds__(256) qmm_small_kernel(QmmArgs a, int n_jobs) {
  constexpr int JOBS_PER_WG = 4 / KSPLIT;
  constexpr int NT = (EPI == EPI_SWIGLU) ? 2 : 1;
  __shared__ f32x4_t red[(KSPLIT > 1) ? 4 * NT * 64 : 1];

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
      const uint4* cp[NT];
      const uint2* sp[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t tb = (static_cast<int64_t>(e) * tiles_per_expert + tile[t]) * nsb;
        cp[t] = static_cast<const uint4*>(a.codes) + tb * 64 + lane;
        sp[t] = reinterpret_cast<const uint2*>(a.sb) + tb * 16 + (lane & 15);
      }
      const uint4* xp = reinterpret_cast<const uint4*>(xrow) + 2 * lg;   // 16 lg bf16
      bf16x8_t ones;
      {
        uint32_t* o = reinterpret_cast<uint32_t*>(&ones);
        o[0] = o[1] = o[2] = o[3] = 0x3F803F80u;
      }
      const f32x4_t zero4{0.f, 0.f, 0.f, 0.f};

      for (int p = p0; p < p1; ++p) {
        uint4 q[NT];
        uint2 sbv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          q[t] = cp[t][p * 64];
          sbv[t] = sp[t][p * 16];
        }
        uint4 xv[4] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0),
                       make_uint4(0, 0, 0, 0)};
        if (row_ok) {
          xv[0] = xp[p * 16 + 0];   // group 2p, k 16lg + 0..7
          xv[1] = xp[p * 16 + 1];   // group 2p, k 16lg + 8..15
          xv[2] = xp[p * 16 + 8];   // group 2p+1
          xv[3] = xp[p * 16 + 9];
        }
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
          const bf16x8_t A0 = pair_permute(xv[2 * gg]);
          const bf16x8_t A1 = pair_permute(xv[2 * gg + 1]);
          f32x4_t xs = mfma16(A0, ones, zero4);
          xs = mfma16(A1, ones, xs);
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const uint32_t w0 = gg ? q[t].z : q[t].x;
            const uint32_t w1 = gg ? q[t].w : q[t].y;
            f32x4_t r = mfma16(A0, unpack_q128(w0), zero4);
            r = mfma16(A1, unpack_q128(w1), r);
            const uint32_t sbw = gg ? sbv[t].y : sbv[t].x;
            const float s = bf16lo_to_f32(sbw);
            const float b = bf16hi_to_f32(sbw) - 128.0f * s;
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][j] = fmaf(s, r[j], fmaf(b, xs[j], acc[t][j]));
          }
        }
      }
    } else {  // FMT_BF16
      const int nks = a.K / 32;
      const int k0 = kpart * nks / KSPLIT, k1 = (kpart + 1) * nks / KSPLIT;
      const uint4* wp[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t tb = (static_cast<int64_t>(e) * tiles_per_expert + tile[t]) * nks;
        wp[t] = static_cast<const uint4*>(a.codes) + tb * 64 + lane;
      }
      const uint4* xp = reinterpret_cast<const uint4*>(xrow) + lg;   // 8 lg bf16
#pragma unroll 4
      for (int c = k0; c < k1; ++c) {
        uint4 wv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) wv[t] = wp[t][c * 64];
        const uint4 xv = row_ok ? xp[c * 4] : make_uint4(0, 0, 0, 0);
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
      for (int t = 0; t < NT; ++t) red[((wave) * NT + t) * 64 + lane] = acc[t];
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
// Workgroup tile: 128 sorted positions x 128 weight rows (SwiGLU: 64 gate + 64 up rows).
// LDS holds one 128-deep k-step of both operands in MFMA fragment order:
//   X[mtile 8][kstep 4][lane 64] and W[wtile 8][kstep 4][lane 64], 16 B per entry.
template <int FMT, int EPI>
__global__ void __launch_bounds__(256) qmm_large_kernel(QmmArgs a) {
  __shared__ u32x4 lds_x[8 * 4 * 64];
  __shared__ u32x4 lds_w[8 * 4 * 64];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int e, m0, m_cnt;
  if (!resolve_mtile(a, blockIdx.y, kLargeMTile, e, m0, m_cnt)) return;
  const int cb = blockIdx.x;
  const int tiles_per_expert = a.n_rows / 16;
  const int64_t ebase = static_cast<int64_t>(e) * tiles_per_expert;

  auto global_tile = [&](int wt) -> int {
    if (EPI == EPI_SWIGLU) return (wt < 4) ? 4 * cb + wt : a.n_rows / 32 + 4 * cb + (wt - 4);
    return 8 * cb + wt;
  };

  // activation row owned by this thread for the global->LDS copy
  const int xr_row = tid >> 1, xr_half = tid & 1;
  int64_t arow = -1;
  if (xr_row < m_cnt) arow = act_row(a, m0 + xr_row);
  const bool xr_ok = arow >= 0;
  const uint32_t xmask = xr_ok ? 0xFFFFFFFFu : 0u;   // rows past the segment read as zeros
  const u32x4* xsrc =
      reinterpret_cast<const u32x4*>(a.act + (xr_ok ? arow : 0) * static_cast<int64_t>(a.K)) +
      xr_half * 8;

  const int nsb = a.K / 128;
  const int wm = wave >> 1, wn = wave & 1;

  // weight slots for int4: two 16B lane slots per thread
  const u32x4* cptr[2] = {nullptr, nullptr};
  const uint2* sptr[2] = {nullptr, nullptr};
  // bf16: thread owns lane slot (tile i, kstep (tid>>6)&3, lane tid&63) for i = 0..7; tiles
  // 0..3 and 4..7 are each contiguous runs of global tiles.
  const int nks = a.K / 32;
  const u32x4* wlo = nullptr;
  const u32x4* whi = nullptr;
  if (FMT == FMT_INT4) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int slot = tid + 256 * i, wt = slot >> 6, ln = slot & 63;
      const int64_t tb = (ebase + global_tile(wt)) * nsb;
      cptr[i] = static_cast<const u32x4*>(a.codes) + tb * 64 + ln;
      sptr[i] = reinterpret_cast<const uint2*>(a.sb) + tb * 16 + (ln & 15);
    }
  } else {
    const int ks = (tid >> 6) & 3, ln = tid & 63;
    wlo = static_cast<const u32x4*>(a.codes) + ((ebase + global_tile(0)) * nks + ks) * 64 + ln;
    whi = static_cast<const u32x4*>(a.codes) + ((ebase + global_tile(4)) * nks + ks) * 64 + ln;
  }

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  u32x4 xv[8];
  u32x4 qv[2];
  uint2 sv[2];
  u32x4 wv[8];
#define QMOE_LOAD_STEP(P)                                                                     \
  do {                                                                                        \
    _Pragma("unroll") for (int i = 0; i < 8; ++i) {                                           \
      xv[i] = xsrc[(P) * 16 + i] & xmask;                                                     \
    }                                                                                         \
    if (FMT == FMT_INT4) {                                                                    \
      _Pragma("unroll") for (int i = 0; i < 2; ++i) {                                         \
        qv[i] = cptr[i][(P) * 64];                                                            \
        sv[i] = sptr[i][(P) * 16];                                                            \
      }                                                                                       \
    } else {                                                                                  \
      const int64_t tstride = static_cast<int64_t>(nks) * 64;                                 \
      _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                         \
        wv[i] = wlo[i * tstride + (P) * 4 * 64];                                              \
        wv[4 + i] = whi[i * tstride + (P) * 4 * 64];                                          \
      }                                                                                       \
    }                                                                                         \
  } while (0)

  // LDS column of each wavefront's weight tiles
  int wtl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (EPI == EPI_SWIGLU) wtl[j] = (j < 2) ? 2 * wn + j : 4 + 2 * wn + (j - 2);
    else wtl[j] = 4 * wn + j;
  }

  QMOE_LOAD_STEP(0);
  for (int p = 0; p < nsb; ++p) {
    __syncthreads();
    // activations -> LDS (fragment order)
    {
      // element i of this thread's 64-wide half row: kstep 2*half + i/4, lane group i%4
      u32x4* xd = lds_x + ((xr_row >> 4) * 4 + 2 * xr_half) * 64 + (xr_row & 15);
      xd[0 * 16] = xv[0];
      xd[1 * 16] = xv[1];
      xd[2 * 16] = xv[2];
      xd[3 * 16] = xv[3];
      xd[64 + 0 * 16] = xv[4];
      xd[64 + 1 * 16] = xv[5];
      xd[64 + 2 * 16] = xv[6];
      xd[64 + 3 * 16] = xv[7];
    }
    if (FMT == FMT_INT4) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int slot = tid + 256 * i, wt = slot >> 6, ln = slot & 63;
        const int r = ln & 15, g = ln >> 4;
        const uint32_t words[4] = {qv[i].x, qv[i].y, qv[i].z, qv[i].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int gg = t >> 1, wi = 2 * g + (t & 1);
          const uint32_t sbw = gg ? sv[i].y : sv[i].x;
          const float s = bf16lo_to_f32(sbw), b = bf16hi_to_f32(sbw);
          const uint32_t w = words[t];
          uint32_t o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float v0 = fmaf(s, static_cast<float>((w >> (8 * j)) & 0xFu), b);
            const float v1 = fmaf(s, static_cast<float>((w >> (8 * j + 4)) & 0xFu), b);
            o[j] = pack_bf16x2(v0, v1);
          }
          const int kl = 64 * gg + 8 * wi;   // first k of this word within the 128-deep step
          lds_w[(wt * 4 + (kl >> 5)) * 64 + ((kl >> 3) & 3) * 16 + r] = u32x4{o[0], o[1], o[2], o[3]};
        }
      }
    } else {
      lds_w[tid + 0 * 256] = wv[0];
      lds_w[tid + 1 * 256] = wv[1];
      lds_w[tid + 2 * 256] = wv[2];
      lds_w[tid + 3 * 256] = wv[3];
      lds_w[tid + 4 * 256] = wv[4];
      lds_w[tid + 5 * 256] = wv[5];
      lds_w[tid + 6 * 256] = wv[6];
      lds_w[tid + 7 * 256] = wv[7];
    }
    __syncthreads();
    if (p + 1 < nsb) QMOE_LOAD_STEP(p + 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8_t A[4], B[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) A[i] = as_bf16x8(lds_x[((4 * wm + i) * 4 + ks) * 64 + lane]);
#pragma unroll
      for (int j = 0; j < 4; ++j) B[j] = as_bf16x8(lds_w[(wtl[j] * 4 + ks) * 64 + lane]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(A[i], B[j], acc[i][j]);
    }
  }

  const int lg = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int mr = 16 * (4 * wm + i) + 4 * lg + jj;
      if (mr >= m_cnt) continue;
      if (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = 64 * cb + 16 * (2 * wn + t) + (lane & 15);
          store_out<EPI>(a, m0 + mr, col, acc[i][t][jj], acc[i][2 + t][jj]);
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int col = 128 * cb + 16 * (4 * wn + t) + (lane & 15);
          store_out<EPI>(a, m0 + mr, col, acc[i][t][jj], 0.f);
        }
      }
    }
  }
}

#undef QMOE_LOAD_STEP

// ============================================================================ launcher
template <int FMT, int EPI>
static void launch_small(const QmmArgs& a, int ksplit, int64_t mtiles, hipStream_t stream) {
  const int n_jobs = (EPI == EPI_SWIGLU) ? a.n_rows / 32 : a.n_rows / 16;
  const int jobs_per_wg = 4 / ksplit;
  dim3 grid((n_jobs + jobs_per_wg - 1) / jobs_per_wg, static_cast<unsigned>(mtiles));
  if (ksplit == 4) qmm_small_kernel<FMT, EPI, 4><<<grid, 256, 0, stream>>>(a, n_jobs);
  else if (ksplit == 2) qmm_small_kernel<FMT, EPI, 2><<<grid, 256, 0, stream>>>(a, n_jobs);
  else qmm_small_kernel<FMT, EPI, 1><<<grid, 256, 0, stream>>>(a, n_jobs);
}

template <int FMT, int EPI>
static void launch_large(const QmmArgs& a, int64_t mtiles, hipStream_t stream) {
  const int n_cb = (EPI == EPI_SWIGLU) ? a.n_rows / 128 : a.n_rows / 128;
  dim3 grid(n_cb, static_cast<unsigned>(mtiles));
  qmm_large_kernel<FMT, EPI><<<grid, 256, 0, stream>>>(a);
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
    // Split-K depends on K only (never on the token count), so a row's summation order, and
    // therefore its result, is the same at every batch size (batch invariance).
    const int ksplit = (a.K >= 4096) ? 4 : (a.K >= 2048) ? 2 : 1;
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
    if (a.n_rows % 128) return fail("qmm(large): weight rows % 128 == 0 required");
#define QMOE_LARGE(F, P) launch_large<F, P>(a, mtile_bound, stream)
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
  }
  return check_launch("qmm");
}

}  // namespace qmoe
