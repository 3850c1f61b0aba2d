// The decode (small-M) grouped-matmul body shared by the qmm kernels (qmm.hip) and the
// decode dataflow kernel (flow.hip): m-tile resolution, activation-row lookup, epilogues and
// small_body, so every launch that runs a product computes it with the same arithmetic.
//
// Reference: mx.gather_qmm(x, packed, scale, bias, rhs_indices=exp, transpose=True,
// group_size=64, bits=4) at src/quanta/qwen35/moe.py:117-123; SwiGLU
// src/quanta/qwen35/moe.py:59-63; the dense bf16 products src/quanta/qwen35/moe.py:47,145-151.
#pragma once

#include <type_traits>

#include "qmoe_internal.h"
#include "route_common.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

// Routing done inside the routed gate_up launch (slot-major batches): the logits, the top-k
// parameters and where the routing results go for the launches after it.
struct SlotRoute {
  const float* logits;
  int ld;
  TopkParams P;
  int32_t* idx;
  float* w;
  float* sg;
  int4* tile_map;
  int max_tiles;
  int32_t* sorted;
  int32_t* inv;
  int mc;      // slots (N * k): the m-tiles of the launch
  int store;   // 1: the bx == 0 workgroups store the routing for later launches; 0: rank only
};

__device__ __forceinline__ int find_segment(const int32_t* __restrict__ tile_off, int E, int mt) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tile_off[mid] <= mt) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// ---------------------------------------------------------------- in-kernel handoff
// Data that one workgroup writes and another reads within the same launch (the decode dataflow
// kernel, flow.hip) goes through agent-coherent accesses: relaxed agent-scope atomic loads and
// stores, which gfx950 issues with the sc1 cache policy, so a value stored on one XCD is seen by
// a load on any other without an L2 write-back or invalidate. The producer waits for its stores
// (s_waitcnt) before it counts itself done; the consumer reads only after it has seen that count.
__device__ __forceinline__ uint32_t coh_ld32(const void* p) {
  return __hip_atomic_load(static_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32x4 coh_ld128(const void* p) {
  const unsigned long long* q = static_cast<const unsigned long long*>(p);
  const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return u32x4{static_cast<uint32_t>(lo), static_cast<uint32_t>(lo >> 32), static_cast<uint32_t>(hi),
               static_cast<uint32_t>(hi >> 32)};
}
__device__ __forceinline__ void coh_st16(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_st32(void* p, uint32_t v) {
  __hip_atomic_store(static_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// small_body's handoff modes (template COH, a bit set): the activation rows are read coherently
// (kCohAct); outputs are stored coherently (kCohOut). With RVPL routing: kCohRowSlot: the
// activation row is the slot (m-tile `by`) itself, not its token (the down projection of a slot's
// h row); kCohWaitAct: the workgroup waits until QmmArgs::act_ready[by * kSyncStride] reaches
// act_ready_target (the rows' producers have finished) before it loads the activations; thread 0
// polls for the whole workgroup. With DEEP staging every weight load of the chunk is issued first
// and every wavefront of the workgroup must hold a job; with dense weights the wait comes first.
constexpr int kCohAct = 2, kCohOut = 4, kCohRowSlot = 16, kCohWaitAct = 32;


// One lane of the wavefront polls *p until it reaches target, sleeping longer the longer it
// waits (fewer polls of a hot counter); bounded: past kWaitLimit polls it counts a timeout in
// *timeouts and returns, so the kernel always ends.
constexpr uint32_t kWaitLimit = 1u << 18;
__device__ __forceinline__ void poll_geq(const uint32_t* p, uint32_t target, uint32_t* timeouts) {
  uint32_t n = 0;
  while (coh_ld32(p) < target) {
    if (n < 4) __builtin_amdgcn_s_sleep(1);
    else if (n < 16) __builtin_amdgcn_s_sleep(4);
    else __builtin_amdgcn_s_sleep(16);
    if (++n >= kWaitLimit) {
      __hip_atomic_fetch_add(timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
  }
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

template <int EPI, bool COH = false>
__device__ __forceinline__ void store_out(const QmmArgs& a, int row, int col, float v, float v_up) {
  const int64_t off = static_cast<int64_t>(row) * a.ld_out + col;
  if (EPI == EPI_SWIGLU) {
    // gate/up are bf16 tensors in the reference's flow; the gated activation runs on them in
    // fp32 and rounds once to bf16 (QMOE_ACT_*: the clamped forms of src/quanta/dsv4/moe.py:74-77
    // and src/quanta/minimax/model_m3.py:112-128)
    // (the hardware round-to-nearest-even conversions: a NaN stays a NaN, its payload may differ)
    const uint32_t gu = pack_bf16x2_rne(v, v_up);
    const float g = bf16lo_to_f32(gu), u = bf16hi_to_f32(gu);
    const float h = glu_f(g, u, a.glu, a.glu_alpha, a.glu_limit);
    const uint16_t o = static_cast<uint16_t>(pack_bf16x2_rne(h, h));
    if (COH) coh_st16(static_cast<uint16_t*>(a.out) + off, o);
    else static_cast<uint16_t*>(a.out)[off] = o;
  } else if (EPI == EPI_BF16) {
    const uint16_t o = static_cast<uint16_t>(pack_bf16x2_rne(v, v));
    if (COH) coh_st16(static_cast<uint16_t*>(a.out) + off, o);
    else static_cast<uint16_t*>(a.out)[off] = o;
  } else {
    if (COH) coh_st32(static_cast<float*>(a.out) + off, __float_as_uint(v));
    else static_cast<float*>(a.out)[off] = v;
  }
}

// ============================================================================ small-M kernel
// One wavefront = JPW consecutive 16-row weight tile jobs (each two tiles, gate and up, for
// SwiGLU) over one k-range of one 16-position m-tile; the jobs share the wavefront's activation
// fragments, so activation loads are amortised over JPW times the weight bytes.
//
// Summation order: K is cut into CH = W * CPW equal chunks (CH depends on K only); each chunk is
// summed from zero over its superblocks, and the chunk sums are added in chunk order,
// ((c0 + c1) + c2) + ... . W wavefronts of a workgroup share a job, each summing CPW consecutive
// chunks; chunk sums meet in LDS. How many wavefronts share the chunks (W) varies with the
// launch size, but the arithmetic does not, so every output is bit-identical at every batch size.
// WAVES = max(4, W) wavefronts per workgroup.
template <int NT, int FMT>
struct SmallStage {
  u32x4 q[NT];    // int4/int6: the codes' nibbles of one superblock / bf16: weight fragments of one 32-k step
  uint2 sb[NT];   // int4/int6 scale/bias of the superblock's two groups
  u32x2 hq[(FMT == FMT_INT6) ? NT : 1];   // int6: the codes' high two bits (one word per group)
  u32x4 x[4];     // activation fragments
};

template <int FMT, int EPI, int W, int CPW, int JPW, int MT = 1>
struct SmallCfg {
  static constexpr int WAVES = W > 4 ? W : 4;
  static constexpr int JOBS_PER_WG = WAVES / W;
  static constexpr int NT = ((EPI == EPI_SWIGLU) ? 2 : 1) * JPW;
  static constexpr int CH = W * CPW;
  // chunk sums: [wave][chunk of the wave][m-tile][tile][lane]
  static constexpr int RED = (CH > 1) ? WAVES * CPW * MT * NT * 64 : 1;
  // the four-tile variants are held to 3 wavefronts per SIMD (168 VGPRs)
  static constexpr int WPE = (fmt_quant(FMT) && NT >= 4) ? 3 : 1;
};

// Body of one workgroup: job block `bx` of m-tile `by` (MT > 1, dense bf16 products only:
// m-tiles by*MT .. by*MT+MT-1, every weight fragment feeding MT MFMAs), chunk sums in `red`
// (LDS).
// RVPL > 0 (slot-major routing in the launch, int4 SwiGLU): m-tile `by` is slot m = t*k + s,
// one row; every wavefront ranks token t's logits (topk_token with RVPL experts per lane, the
// top-k kernel's arithmetic) and takes lane s's expert; workgroups with bx == 0 store the slot's
// expert, weight and tile (and slot 0 the token's shared-expert gate) for the later launches.
// DEEP > 0 (with RVPL, one chunk per wavefront of exactly DEEP superblocks): the wavefront
// stages its K range of the token row in its own LDS range (xlds, DEEP * 256 bytes) and issues
// every weight load of its chunk at once, then multiplies superblock by superblock.
// COH (a set of kCoh* bits): the handoff modes of the decode dataflow kernel (flow.hip); 0 for
// every other launch.
template <int FMT, int EPI, int W, int CPW, int JPW, int MT = 1, bool NORM = false, int RVPL = 0,
          int DEEP = 0, int COH = 0>
__device__ __forceinline__ void small_body(const QmmArgs& a, int n_jobs, int bx, int by,
                                           f32x4_t* red, const SlotRoute* route = nullptr,
                                           u32x4* xlds = nullptr, int* route_e = nullptr) {
  using C = SmallCfg<FMT, EPI, W, CPW, JPW, MT>;
  constexpr bool kOutC = (COH & kCohOut) != 0;
  // one activation fragment (16 bytes): coherent when the rows were written in this launch
  auto ldx = [](const u32x4* p) __attribute__((always_inline)) {
    if constexpr ((COH & kCohAct) != 0) return coh_ld128(p); else return *p;
  };
  static_assert(MT == 1 || fmt_dense(FMT), "several m-tiles per wavefront: dense weights only");
  constexpr int JOBS_PER_WG = C::JOBS_PER_WG;
  constexpr int NT = C::NT;
  constexpr int CH = C::CH;
  constexpr bool kRed = CH > 1;

  // wave index as a scalar, so per-wavefront quantities (job, k-range) stay in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  int e, mt0[MT], mtc[MT];
  int route_tok = -1;
  if constexpr (RVPL > 0) {
    static_assert(MT == 1, "slot-major routing: one m-tile per wavefront");
    const SlotRoute& R = *route;
    const int m = by, t = m / R.P.k, s = m - t * R.P.k;
    const float* lrow = R.logits + static_cast<int64_t>(t) * R.ld;
    int id = 0;
    float wsel = 0.f;
    // Every wavefront of the workgroup serves slot m: wavefront 0 ranks the logits and shares
    // the expert through LDS. Only the storing workgroup needs the routing weights; the others
    // rank by logit up to the slot's own rank.
    if (wave == 0) {
      if (bx == 0 && R.store)
        topk_token<RVPL>(lrow, R.P, lane, id, wsel);
      else
        topk_token<RVPL, true>(lrow, R.P, lane, id, wsel, s + 1);
      if (lane == 0) *route_e = __builtin_amdgcn_readlane(id, s);
    }
    __syncthreads();
    e = __builtin_amdgcn_readfirstlane(*route_e);
    mt0[0] = m;
    mtc[0] = 1;
    route_tok = (COH & kCohRowSlot) ? m : t;
    if (bx == 0 && wave == 0 && R.store) {
      if (lane == s) {
        R.idx[m] = id;
        R.w[m] = wsel;
        R.tile_map[m] = make_int4(id, m, 1, 0);
        R.sorted[m] = m;
        R.inv[m] = m;
      }
      if (s == 0 && lane == 0 && R.P.has_sg) R.sg[t] = 1.0f / (1.0f + expf(-lrow[R.P.E]));
      if (m == 0) {
        const int mc = R.mc;
        for (int i = mc + lane; i < R.max_tiles; i += 64) R.tile_map[i] = make_int4(-1, 0, 0, 0);
      }
    }
  } else if (MT == 1) {
    if (!resolve_mtile(a, by, kSmallMTile, e, mt0[0], mtc[0])) return;
    // (one stack of a projection whose experts have different widths: the others' m-tiles exit;
    // every wavefront of the workgroup resolves the same m-tile)
    if (a.expert_map) {
      e = a.expert_map[e];
      if (e < 0) return;
    }
  } else {   // dense rows (the launcher guarantees no segments)
    e = 0;
#pragma unroll
    for (int u = 0; u < MT; ++u) {
      mt0[u] = (by * MT + u) * kSmallMTile;
      mtc[u] = static_cast<int>(max<int64_t>(0, min<int64_t>(kSmallMTile, a.dense_rows - mt0[u])));
    }
    if (mtc[0] <= 0) return;
  }

  const int job = bx * JOBS_PER_WG + wave / W;
  const int kpart = wave % W;
  const bool job_ok = job < n_jobs;
  const int mrow = lane & 15, lg = lane >> 4;

  // Rows past the segment and rows whose slot is invalid read activation row 0, so every load
  // is unconditional (a load under a branch makes the compiler wait for all loads in flight);
  // the former are never stored, the latter are stored as zeros.
  // (act_hi: the wavefront's JPW tiles lie on one side of split_tile, a multiple of 4)
  const uint16_t* act = (fmt_quant(FMT) && a.act_hi && job * JPW >= a.split_tile) ? a.act_hi : a.act;
  const uint16_t* xrows[MT];
  uint32_t rows_okm[MT];
#pragma unroll
  for (int u = 0; u < MT; ++u) {
    int64_t arow = -1;
    if (RVPL > 0) arow = (mrow == 0 && route_tok < a.act_rows) ? route_tok : -1;
    else if (mrow < mtc[u]) arow = act_row(a, mt0[u] + mrow);
    const bool row_ok = arow >= 0;
    xrows[u] = act + (row_ok ? arow : 0) * static_cast<int64_t>(a.act_stride ? a.act_stride : a.K);
    rows_okm[u] = static_cast<uint32_t>(__ballot(row_ok)) & 0xFFFFu;   // lanes 0-15
  }
  const uint16_t* xrow = xrows[0];
  if constexpr ((COH & kCohWaitAct) != 0 && !fmt_quant(FMT)) {
    // dense weights: the whole workgroup waits for the activation rows' producers first
    if (threadIdx.x == 0)
      poll_geq(a.act_ready + static_cast<int64_t>(by) * kSyncStride, a.act_ready_target, a.timeouts);
    __syncthreads();
  }

  f32x4_t accm[MT][NT];
#pragma unroll
  for (int u = 0; u < MT; ++u)
#pragma unroll
    for (int t = 0; t < NT; ++t) accm[u][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  f32x4_t (&acc)[NT] = accm[0];

  const int tiles_per_expert = a.n_rows / 16;
  // tiles of this wavefront's jobs: job j covers tile j (SwiGLU: gate tile j and up tile
  // j + n_rows/32, the up half starting at row I = n_rows/2); SwiGLU keeps gates first
  int tile[NT];
#pragma unroll
  for (int jp = 0; jp < JPW; ++jp) {
    tile[jp] = job * JPW + jp;
    if (EPI == EPI_SWIGLU) tile[JPW + jp] = job * JPW + jp + a.n_rows / 32;
  }

  if (job_ok) {
    if (fmt_quant(FMT)) {
      // tile superblock: int4 1 KiB of codes; int6 1 KiB of nibbles + 512 B of high bits; int3
      // 768 B, three words per lane
      constexpr int SBB = (FMT == FMT_INT6) ? 1536 : (FMT == FMT_INT3) ? 768 : 1024;
      const int nsb = a.K / 128;
      // chunk c = superblocks [c * nsb / CH, (c + 1) * nsb / CH); this wavefront: CPW chunks
      const int p0 = kpart * CPW * nsb / CH, p1 = (kpart + 1) * CPW * nsb / CH;
      const int pmid = (kpart * CPW + 1) * nsb / CH;   // end of the first chunk (CPW == 2)
      // tile bases are wave-uniform (scalar registers); every stream adds one shared per-lane
      // offset, so the loads use scalar-base + 32-bit vector-offset addressing
      const char* cb[NT];
      const char* sbb[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t tb = (static_cast<int64_t>(e) * tiles_per_expert + tile[t]) * nsb;
        cb[t] = static_cast<const char*>(a.codes) + tb * SBB;
        sbb[t] = reinterpret_cast<const char*>(a.sb) + tb * 128;
      }
      const uint32_t lane_c = static_cast<uint32_t>(lane) * 16u;
      const uint32_t lane_s = static_cast<uint32_t>(lane & 15) * 8u;
      const u32x4* xp = reinterpret_cast<const u32x4*>(xrow) + 2 * lg;   // 16 lg bf16
      bf16x8_t ones;
      {
        uint32_t* o = reinterpret_cast<uint32_t*>(&ones);
        o[0] = o[1] = o[2] = o[3] = 0x3F803F80u;
      }
      const f32x4_t zero4{0.f, 0.f, 0.f, 0.f};
      // Two register stages: the loads of superblock p+1 are in flight while p is computed.
      SmallStage<NT, FMT> st[2];
      auto load = [&](SmallStage<NT, FMT>& s, int p) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          // weights are streamed once per call: nontemporal loads keep them out of the way of
          // the activations that every job of the m-tile re-reads
          if constexpr (FMT == FMT_INT3) {
            // the lane's three code words (one dwordx3 load)
            const uint32_t* w3 = reinterpret_cast<const uint32_t*>(
                cb[t] + static_cast<int64_t>(p) * SBB + 12 * lane);
            s.q[t] = u32x4{__builtin_nontemporal_load(w3), __builtin_nontemporal_load(w3 + 1),
                           __builtin_nontemporal_load(w3 + 2), 0u};
          } else {
            s.q[t] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(cb[t] + static_cast<int64_t>(p) * SBB + lane_c));
          }
          if constexpr (FMT == FMT_INT6)
            s.hq[t] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(
                cb[t] + static_cast<int64_t>(p) * SBB + 1024 + 8 * lane));
          const u32x2 v = __builtin_nontemporal_load(
              reinterpret_cast<const u32x2*>(sbb[t] + static_cast<int64_t>(p) * 128 + lane_s));
          s.sb[t] = uint2{v.x, v.y};
        }
        // group 2p: k 16lg + 0..7 (step 0) and + 8..15 (step 1); group 2p+1 likewise, +64
        s.x[0] = ldx(xp + p * 16 + 0);
        s.x[1] = ldx(xp + p * 16 + 1);
        s.x[2] = ldx(xp + p * 16 + 8);
        s.x[3] = ldx(xp + p * 16 + 9);
      };
      auto compute = [&](const SmallStage<NT, FMT>& s) __attribute__((always_inline)) {
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
            f32x4_t r;
            if constexpr (FMT == FMT_INT6) {
              const uint32_t hw = gg ? s.hq[t].y : s.hq[t].x;
              r = mfma16(A0, unpack_q128_6(w0, hw, 0), zero4);
              r = mfma16(A1, unpack_q128_6(w1, hw, 1), r);
            } else if constexpr (FMT == FMT_INT3) {
              r = mfma16(A0, unpack_q128_3(s.q[t].x, s.q[t].y, s.q[t].z, gg, 0), zero4);
              r = mfma16(A1, unpack_q128_3(s.q[t].x, s.q[t].y, s.q[t].z, gg, 1), r);
            } else {
              r = mfma16(A0, unpack_q128(w0), zero4);
              r = mfma16(A1, unpack_q128(w1), r);
            }
            const uint32_t sbw = gg ? s.sb[t].y : s.sb[t].x;
            const float sc = bf16lo_to_f32(sbw);
            const float bi = bf16hi_to_f32(sbw) - 128.0f * sc;
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][j] = fmaf(sc, r[j], fmaf(bi, xs[j], acc[t][j]));
          }
        }
      };
      // the first chunk's sum goes to LDS and the accumulators restart from zero
      auto chunk_end = [&](int pdone) __attribute__((always_inline)) {
        if (CPW == 2 && pdone == pmid) {
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            red[((wave * CPW) * NT + t) * 64 + lane] = acc[t];
            acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          }
        }
      };
      if constexpr (DEEP > 0) {
        static_assert(RVPL > 0 && CPW == 1, "deep prefetch: slot-major routed launches");
        // the chunk's activations (one token row, the same for every lane), first, so the
        // weight loads behind them stay in flight when the compiler waits for them
        constexpr int XV = DEEP * 16 / 64;
        const u32x4* xg = reinterpret_cast<const u32x4*>(a.act + static_cast<int64_t>(route_tok) * a.K) +
                          p0 * 16;
        u32x4 xv[XV];
        u32x4 qd[DEEP][NT];
        uint2 sd[DEEP][NT];
        auto load_w = [&]() __attribute__((always_inline)) {
#pragma unroll
          for (int pp = 0; pp < DEEP; ++pp)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              qd[pp][t] = __builtin_nontemporal_load(
                  reinterpret_cast<const u32x4*>(cb[t] + static_cast<int64_t>(p0 + pp) * SBB + lane_c));
              const u32x2 v = __builtin_nontemporal_load(
                  reinterpret_cast<const u32x2*>(sbb[t] + static_cast<int64_t>(p0 + pp) * 128 + lane_s));
              sd[pp][t] = uint2{v.x, v.y};
            }
        };
        if constexpr ((COH & kCohWaitAct) != 0) {
          // weights in flight first; the activation rows only once their producers are done
          load_w();
          __builtin_amdgcn_sched_barrier(0);
          if (threadIdx.x == 0)
            poll_geq(a.act_ready + static_cast<int64_t>(by) * kSyncStride, a.act_ready_target, a.timeouts);
          __syncthreads();
#pragma unroll
          for (int i = 0; i < XV; ++i) xv[i] = ldx(xg + lane + 64 * i);
        } else {
#pragma unroll
          for (int i = 0; i < XV; ++i) xv[i] = ldx(xg + lane + 64 * i);
          load_w();
        }
        // (keeps the loads issued together: the scheduler would otherwise sink each one down to
        // its superblock)
        __builtin_amdgcn_sched_barrier(0);
        u32x4* xl = xlds + wave * (DEEP * 16);
#pragma unroll
        for (int i = 0; i < XV; ++i) xl[lane + 64 * i] = xv[i];
        const u32x4* xr = xl + 2 * lg;
#pragma unroll
        for (int pp = 0; pp < DEEP; ++pp) {
          SmallStage<NT, FMT> sg;
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            sg.q[t] = qd[pp][t];
            sg.sb[t] = sd[pp][t];
          }
          sg.x[0] = xr[pp * 16 + 0];
          sg.x[1] = xr[pp * 16 + 1];
          sg.x[2] = xr[pp * 16 + 8];
          sg.x[3] = xr[pp * 16 + 9];
          compute(sg);
        }
      } else {
      // Steady state: two superblocks per iteration with every load unconditional, so the
      // compiler waits only for the stage about to be computed; then a one- or two-superblock
      // tail (p1 - p0 >= 1).
      // (the scheduling barriers keep each stage's loads issued before the MFMAs that wait for
      // the previous stage)
      int p = p0;
      // (the guard is always true, p1 > p0; with it the compiler allocates 140 VGPRs and no
      // scratch to the four-tile int4 kernels, against 168 and 20 bytes of spills without it,
      // which measured 2-3% faster layers at N = 8 to 128)
      if (p < p1) {
        load(st[0], p);
        for (; p + 2 < p1; p += 2) {
          load(st[1], p + 1);
          __builtin_amdgcn_sched_barrier(0);
          compute(st[0]);
          chunk_end(p + 1);
          load(st[0], p + 2);
          __builtin_amdgcn_sched_barrier(0);
          compute(st[1]);
          chunk_end(p + 2);
        }
        if (p + 1 < p1) {
          load(st[1], p + 1);
          __builtin_amdgcn_sched_barrier(0);
          compute(st[0]);
          chunk_end(p + 1);
          compute(st[1]);
          chunk_end(p + 2);
        } else {
          compute(st[0]);
          chunk_end(p + 1);
        }
      }
      }
    } else {  // dense: bf16 weights, or int8 codes dequantized to bf16 in registers
      // (CPW == 2: the wavefront's two chunks [k0, kmid) and [kmid, k1), the first one's sums
      // set aside in LDS at the boundary as the int4 path does, one m-tile, no fused norm)
      static_assert(CPW == 1 || (CPW == 2 && MT == 1 && !NORM), "dense: two chunks per wavefront need one m-tile");
      const int nks = a.K / 32;
      const int k0 = kpart * nks / W, k1 = (kpart + 1) * nks / W;
      const int kmid = (CPW == 2) ? (kpart * 2 + 1) * nks / (2 * W) : k1;
      int kend = (CPW == 2) ? kmid : k1;   // the current chunk's end (loads are clamped to it)
      using Frag = DenseFrag<FMT>;
      DenseTile<FMT> wt[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wt[t].init(a.codes, a.sb, static_cast<int64_t>(e) * tiles_per_expert + tile[t], a.K, lane);
      const u32x4* xp[MT];
#pragma unroll
      for (int u = 0; u < MT; ++u) xp[u] = reinterpret_cast<const u32x4*>(xrows[u]) + lg;   // 8 lg bf16
      // Batches of steps: all loads of a batch issue before its MFMAs (indices clamped into
      // the range, so no load is conditional); the MFMAs run in step order.
      constexpr int BS = (MT > 1) ? 4 : 8;
      auto load_batch = [&](int cb, Frag (&wv)[BS][NT], u32x4 (&xv)[BS][MT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < BS; ++i) {
          const int c = min(cb + i, kend - 1);
#pragma unroll
          for (int t = 0; t < NT; ++t) wv[i][t] = wt[t].load(c);
#pragma unroll
          for (int u = 0; u < MT; ++u) xv[i][u] = ldx(xp[u] + c * 4);
        }
      };
      // RMSNorm on the fly (NORM, the pair launch; the launcher guarantees W >= 4, so the
      // workgroup is one job and every wavefront reaches the barrier): the rows' sums of squares
      // over the job's W chunks in the canonical order of rmsnorm_row (lane group sums over the
      // chunk's steps in order, then (g0 + g1) + (g2 + g3), then the chunks in order), taken while
      // the first batch's weights are already in flight; each activation fragment is then
      // normalised, bf16(w * (x * r)), and job 0 writes the normalised rows for later launches.
      // The norm weights come to LDS (the launch's dynamic LDS, a.K * 2 bytes; the workgroup's
      // threads load one 16-byte piece each, issued before the activations, so the sums' wait
      // covers them) and are read from there after the barrier.
      float rn[MT];
      u32x4* outp[MT];
      extern __shared__ u32x4 norm_g[];
      const u32x4* wnp = norm_g + lg;
      auto mma_batch = [&](int cb, const Frag (&wv)[BS][NT], const u32x4 (&xv)[BS][MT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < BS; ++i) {
          if (cb + i < kend) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              const bf16x8_t B = as_bf16x8(dense_bf16<FMT>(wv[i][t]));
#pragma unroll
              for (int u = 0; u < MT; ++u) accm[u][t] = mfma16(as_bf16x8(xv[i][u]), B, accm[u][t]);
            }
          }
        }
      };
      // NORM: each step's fragments normalised right before its MFMAs (short register lives)
      auto norm_mma_batch = [&](int cb, const Frag (&wv)[BS][NT], const u32x4 (&xv)[BS][MT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < BS; ++i) {
          const int c = min(cb + i, k1 - 1);
          const u32x4 g = wnp[c * 4];
          bf16x8_t B[NT];
#pragma unroll
          for (int t = 0; t < NT; ++t) B[t] = as_bf16x8(dense_bf16<FMT>(wv[i][t]));
#pragma unroll
          for (int u = 0; u < MT; ++u) {
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              o[j] = pack_bf16x2_rne(bf16lo_to_f32(g[j]) * (bf16lo_to_f32(xv[i][u][j]) * rn[u]),
                                     bf16hi_to_f32(g[j]) * (bf16hi_to_f32(xv[i][u][j]) * rn[u]));
            if (outp[u]) outp[u][c * 4] = o;
            if (cb + i < k1) {
#pragma unroll
              for (int t = 0; t < NT; ++t)
                accm[u][t] = mfma16(as_bf16x8(o), B[t], accm[u][t]);
            }
          }
        }
      };
      int cb = k0;
      if constexpr (NORM) {
        auto sq = [&](float acc, u32x4 v) __attribute__((always_inline)) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float lo = bf16lo_to_f32(v[j]), hi = bf16hi_to_f32(v[j]);
            acc = fmaf(lo, lo, acc);
            acc = fmaf(hi, hi, acc);
          }
          return acc;
        };
        float ssl[MT];
#pragma unroll
        for (int u = 0; u < MT; ++u) ssl[u] = 0.f;
        // (pair_norm_fusable bounds a.K / 8 by the workgroup's threads)
        const bool g_mine = static_cast<int>(threadIdx.x) < a.K / 8;
        u32x4 g_piece{};
        if (g_mine) g_piece = reinterpret_cast<const u32x4*>(a.norm_w)[threadIdx.x];
        Frag wv[BS][NT];
        u32x4 xv[BS][MT];
        const bool one_batch = k1 - k0 <= BS;
        if (one_batch) {
          // the batch's activations, then its weights: loads complete in issue order, so the
          // sums wait only for the activations and the weights stay in flight over the barrier
#pragma unroll
          for (int i = 0; i < BS; ++i) {
            const int c = min(cb + i, k1 - 1);
#pragma unroll
            for (int u = 0; u < MT; ++u) xv[i][u] = xp[u][c * 4];
          }
#pragma unroll
          for (int i = 0; i < BS; ++i) {
            const int c = min(cb + i, k1 - 1);
#pragma unroll
            for (int t = 0; t < NT; ++t) wv[i][t] = wt[t].load(c);
          }
#pragma unroll
          for (int i = 0; i < BS; ++i)
            if (cb + i < k1) {
#pragma unroll
              for (int u = 0; u < MT; ++u) ssl[u] = sq(ssl[u], xv[i][u]);
            }
        } else {
          // a longer chunk (pair_norm_fusable: at most NS steps): all its activations at once,
          // summed in step order; the products re-read them (L1/L2 hits)
          constexpr int NS = (MT > 1) ? 8 : 16;
          u32x4 xs[NS][MT];
#pragma unroll
          for (int i = 0; i < NS; ++i) {
            const int c = min(k0 + i, k1 - 1);
#pragma unroll
            for (int u = 0; u < MT; ++u) xs[i][u] = xp[u][c * 4];
          }
#pragma unroll
          for (int i = 0; i < NS; ++i)
            if (k0 + i < k1) {
#pragma unroll
              for (int u = 0; u < MT; ++u) ssl[u] = sq(ssl[u], xs[i][u]);
            }
        }
        if (g_mine) norm_g[threadIdx.x] = g_piece;
        float* nred = reinterpret_cast<float*>(red + SmallCfg<FMT, EPI, W, CPW, JPW, MT>::RED);
#pragma unroll
        for (int u = 0; u < MT; ++u) {
          ssl[u] += __shfl_xor(ssl[u], 16);
          ssl[u] += __shfl_xor(ssl[u], 32);
          if (lg == 0) nred[(wave * MT + u) * 16 + mrow] = ssl[u];
        }
        __syncthreads();
        const bool wr_norm = a.norm_out && job == 0;
#pragma unroll
        for (int u = 0; u < MT; ++u) {
          float ss = nred[u * 16 + mrow];
          for (int c = 1; c < W; ++c) ss += nred[(c * MT + u) * 16 + mrow];
          rn[u] = 1.0f / sqrtf(ss / static_cast<float>(a.K) + a.norm_eps);
          outp[u] = (wr_norm && mrow < mtc[u])
                        ? reinterpret_cast<u32x4*>(a.norm_out + static_cast<int64_t>(mt0[u] + mrow) * a.K) + lg
                        : nullptr;
        }
        if (one_batch) {
          norm_mma_batch(cb, wv, xv);
          cb += BS;
        }
      }
      if constexpr (CPW == 2) {
        for (; cb < kmid; cb += BS) {
          Frag wv[BS][NT];
          u32x4 xv[BS][MT];
          load_batch(cb, wv, xv);
          mma_batch(cb, wv, xv);
        }
        // the first chunk's sums to LDS, where the reduction below adds them in chunk order
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          red[((wave * CPW) * NT + t) * 64 + lane] = acc[t];
          acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        cb = kmid;
        kend = k1;
      }
      for (; cb < k1; cb += BS) {
        Frag wv[BS][NT];
        u32x4 xv[BS][MT];
        load_batch(cb, wv, xv);
        if constexpr (NORM)
          norm_mma_batch(cb, wv, xv);
        else
          mma_batch(cb, wv, xv);
      }
    }
  }

  if (kRed) {
    // the wavefront's last chunk stays in registers for kpart 0 and goes to LDS for the others;
    // kpart 0 then adds the chunks in order: its own first chunk (CPW == 2) + its last, then
    // every chunk of wavefronts 1 .. W-1
    const int jl = wave / W;
    auto ri = [&](int wc, int u, int t) { return ((wc * MT + u) * NT + t) * 64 + lane; };
    if (kpart > 0) {
#pragma unroll
      for (int u = 0; u < MT; ++u)
#pragma unroll
        for (int t = 0; t < NT; ++t) red[ri(wave * CPW + CPW - 1, u, t)] = accm[u][t];
    }
    if (W > 1) __syncthreads();
    if (kpart == 0) {
      if (CPW == 2) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const f32x4_t o = red[ri(wave * CPW, 0, t)];
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[t][j] = o[j] + acc[t][j];
        }
      }
#pragma unroll
      for (int kp = 1; kp < W; ++kp)
#pragma unroll
        for (int ci = 0; ci < CPW; ++ci)
#pragma unroll
          for (int u = 0; u < MT; ++u)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              const f32x4_t o = red[ri((jl * W + kp) * CPW + ci, u, t)];
#pragma unroll
              for (int j = 0; j < 4; ++j) accm[u][t][j] += o[j];
            }
    }
  }
  if (!job_ok || kpart != 0) return;

#pragma unroll
  for (int u = 0; u < MT; ++u) {
#pragma unroll
    for (int jp = 0; jp < JPW; ++jp) {
      const int col = (job * JPW + jp) * 16 + (lane & 15);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int mr = 4 * lg + j;
        const bool ok = (rows_okm[u] >> mr) & 1u;
        if (mr < mtc[u])
          store_out<EPI, kOutC>(a, mt0[u] + mr, col, ok ? accm[u][jp][j] : 0.f,
                         ok ? accm[u][(EPI == EPI_SWIGLU) ? JPW + jp : jp][j] : 0.f);
      }
    }
  }
}

}  // namespace qmoe
