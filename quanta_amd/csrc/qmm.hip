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
// Two regimes, both on 16x16x32 MFMAs with activations as the A operand (16 token rows) and
// weights as the B operand (16 weight rows as columns):
//  * small-M ("decode"): 16-token m-tiles; each wavefront streams one 16-row weight tile (two
//    for SwiGLU) straight from HBM into registers with one contiguous 1 KiB dwordx4 load per
//    superblock, and never materialises a dequantised weight. For int4 it multiplies the raw
//    codes (as bf16 128+q, exact) on v_mfma_f32_16x16x32_bf16 and applies the per-group affine
//    map on the 16x16 result:
//      sum_k x_k (s q_k + b) = s * sum_k x_k (128+q_k) + (b - 128 s) * sum_k x_k,
//    with sum_k x_k from one extra MFMA against a ones fragment. Optional split-K across the
//    workgroup's wavefronts, reduced through LDS.
//  * large-M ("prefill"): int4 weights are dequantised to fp16 in registers from an LDS copy of
//    their tiled layout and multiplied on v_mfma_f32_16x16x32_f16 against an exactly scaled fp16
//    copy of the activations, staged through LDS. Weight-row counts in 512-row blocks take the
//    wide kernel (128-position x 512-weight-row workgroup tiles, each wavefront 128 x 64);
//    others, and bf16 weights, the 128 x 256 kernel (each wavefront 128 x 32).
#include <type_traits>

#include "qmoe_internal.h"
#include "route_common.h"
#include "small_body.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

// (SlotRoute, resolve_mtile, act_row, store_out and small_body live in small_body.h)

template <int FMT, int EPI, int W, int CPW, int JPW, int MT>
__global__ void __launch_bounds__(W > 4 ? 64 * W : 256)
__attribute__((amdgpu_waves_per_eu(SmallCfg<FMT, EPI, W, CPW, JPW>::WPE)))
qmm_small_kernel(QmmArgs a, int n_jobs) {
  __shared__ f32x4_t red[SmallCfg<FMT, EPI, W, CPW, JPW, MT>::RED];
  small_body<FMT, EPI, W, CPW, JPW, MT>(a, n_jobs, blockIdx.x, blockIdx.y, red);
}

// The routed gate_up of a slot-major batch with its routing (grid.y = N*k slots).
template <int W, int JPW, int VPL, int DEEP>
__global__ void __launch_bounds__(W > 4 ? 64 * W : 256)
__attribute__((amdgpu_waves_per_eu(SmallCfg<FMT_INT4, EPI_SWIGLU, W, 1, JPW>::WPE)))
qmm_route_gate_up_kernel(QmmArgs a, int n_jobs, SlotRoute route) {
  __shared__ f32x4_t red[SmallCfg<FMT_INT4, EPI_SWIGLU, W, 1, JPW, 1>::RED];
  __shared__ u32x4 xlds[DEEP > 0 ? (W > 4 ? W : 4) * DEEP * 16 : 1];
  __shared__ int route_e;
  small_body<FMT_INT4, EPI_SWIGLU, W, 1, JPW, 1, false, VPL, DEEP>(a, n_jobs, blockIdx.x, blockIdx.y,
                                                                    red, &route, xlds, &route_e);
}

// The same with the shared expert's int8 down projection (a2: W2 * CPW2 chunks, W2 wavefronts
// per job each summing CPW2 of them, one m-tile per wavefront) in the launch, on a flat grid of
// 4-wavefront workgroups: the routed gate_up's job blocks x slots first, then the shared down's
// job blocks x m-tiles.
template <int W, int JPW, int VPL, int DEEP, int W2, int CPW2 = 1>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(SmallCfg<FMT_INT4, EPI_SWIGLU, W, 1, JPW>::WPE)))
qmm_route_gate_up_shdown_kernel(QmmArgs a, int n_jobs, SlotRoute route, int gx1, int64_t n1,
                                QmmArgs a2, int n_jobs2, int gx2) {
  static_assert(W <= 4 && W2 <= 4, "one 4-wavefront workgroup shape for both products");
  constexpr int R1 = SmallCfg<FMT_INT4, EPI_SWIGLU, W, 1, JPW, 1>::RED;
  constexpr int R2 = SmallCfg<FMT_INT8, EPI_BF16, W2, CPW2, 1, 1>::RED;
  __shared__ f32x4_t red[R1 > R2 ? R1 : R2];
  __shared__ u32x4 xlds[DEEP > 0 ? 4 * DEEP * 16 : 1];
  __shared__ int route_e;
  const int64_t b = blockIdx.x;
  if (b < n1) {
    small_body<FMT_INT4, EPI_SWIGLU, W, 1, JPW, 1, false, VPL, DEEP>(
        a, n_jobs, static_cast<int>(b % gx1), static_cast<int>(b / gx1), red, &route, xlds, &route_e);
  } else {
    const int64_t b2 = b - n1;
    small_body<FMT_INT8, EPI_BF16, W2, CPW2, 1, 1>(a2, n_jobs2, static_cast<int>(b2 % gx2),
                                                   static_cast<int>(b2 / gx2), red);
  }
}

// The routing tail (RouteTail). Counts go on tagged workspace words, (kRouteTailTag << 20) |
// count: an atomic add, and a word found without the tag (a fresh workspace) is replaced by a
// tagged count of 1 (compare-and-swap), or counted on once another workgroup has tagged it; the
// add that landed on the untagged word is discarded with it. Returns the count after this one.
__device__ __forceinline__ int tail_count(unsigned long long* w) {
  constexpr unsigned long long kMask = (1ull << 20) - 1;
  const unsigned long long old = __hip_atomic_fetch_add(w, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if ((old >> 20) == kRouteTailTag) return static_cast<int>((old & kMask) + 1);
  unsigned long long cur = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned long long want;
  do {
    want = ((cur >> 20) == kRouteTailTag) ? cur + 1 : ((kRouteTailTag << 20) | 1ull);
  } while (!__hip_atomic_compare_exchange_strong(w, &cur, want, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT));
  return static_cast<int>(want & kMask);
}

// This workgroup's stores are complete (s_waitcnt 0, then the barrier); thread 0 counts it on
// *w and the workgroup learns the count.
__device__ __forceinline__ int tail_arrive(unsigned long long* w) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int s_cnt;
  if (threadIdx.x == 0) s_cnt = tail_count(w);
  __syncthreads();
  return s_cnt;
}

// Bounded wait of the workgroup until *w holds a tagged count of at least `target`; a wait that
// runs out adds to *timeouts and returns (the kernel always ends).
__device__ __forceinline__ void tail_wait(const unsigned long long* w, int target, uint32_t* timeouts) {
  if (threadIdx.x == 0) {
    uint32_t n = 0;
    for (;;) {
      const unsigned long long v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((v >> 20) == kRouteTailTag && static_cast<int>(v & ((1ull << 20) - 1)) >= target) break;
      __builtin_amdgcn_s_sleep(2);
      if (++n >= kWaitLimit) {
        __hip_atomic_fetch_add(timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
}

// Ranker r of R: tokens r, r + R, ... one wavefront each, with coherent loads of the logits; the
// top-k launch's outputs (idx coherently, read by the last ranker), and the ids into `ids` (LDS)
// when one workgroup ranks every token.
template <int VPL>
__device__ __forceinline__ void route_tail_rank(const RouteTail& T, int r, int R, int32_t* ids) {
  const int lane = threadIdx.x & 63;
  const int nw = blockDim.x >> 6;
  const int k = T.P.k;
  for (int t = r + R * (threadIdx.x >> 6); t < T.N; t += R * nw) {
    const float* row = T.logits + static_cast<int64_t>(t) * T.ld;
    // (the shared gate's logit is loaded before the ranking, so its latency overlaps it)
    const float sgl = (T.P.has_sg && lane == 0) ? logit_ld<true>(row + T.P.E) : 0.f;
    int id;
    float wsel;
    topk_token<VPL, false, true>(row, T.P, lane, id, wsel);
    if (lane < k) {
      __hip_atomic_store(T.idx + t * k + lane, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      T.w[t * k + lane] = wsel;
      if (ids) ids[t * k + lane] = id;
    }
    if (T.P.has_sg && lane == 0) T.sg[t] = 1.0f / (1.0f + expf(-sgl));
  }
}

// Exclusive scan of one value per thread across the workgroup (1 to 16 wavefronts); tmp holds
// 33 ints and is free again on return.
__device__ __forceinline__ int tail_scan(int v, int* tmp, int& total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == 63) tmp[wid] = incl;
  __syncthreads();
  if (wid == 0) {
    const int s = lane < nw ? tmp[lane] : 0;
    int si = s;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const int o = __shfl_up(si, off);
      if (lane >= off) si += o;
    }
    if (lane < nw) tmp[16 + lane] = si - s;
    if (lane == nw - 1) tmp[32] = si;
  }
  __syncthreads();
  const int r = tmp[16 + wid] + incl - v;
  total = tmp[32];
  __syncthreads();
  return r;
}

// The stable permute of the N * k slots by expert (N <= 64), the permute launch's outputs for
// 16-row m-tiles: counts, offsets and the m-tile prefix (E + 1 entries each with the totals),
// the tile descriptors {expert, first sorted position, rows, 0} with -1 sentinels up to
// max_tiles, and sorted / inv. A slot's stable rank within its expert is the number of earlier
// tokens that chose the expert (top-k experts of a token are distinct): the popcount of the
// expert's 64-bit token mask below the token. Thread i owns experts [i * ve, i * ve + ve).
__device__ __forceinline__ void route_tail_permute(const RouteTail& T, const int32_t* ids,
                                                   unsigned long long* mask, int* hist, int* offs,
                                                   int* tmp) {
  const int E = T.P.E, k = T.P.k, mc = T.N * k, tid = threadIdx.x, nthr = blockDim.x;
  for (int e = tid; e < E; e += nthr) {
    hist[e] = 0;
    mask[e] = 0ull;
  }
  __syncthreads();
  for (int m = tid; m < mc; m += nthr) {
    const int e = ids[m];
    atomicAdd(&hist[e], 1);
    atomicOr(&mask[e], 1ull << (m / k));
  }
  __syncthreads();
  const int ve = (E + nthr - 1) / nthr;   // at most 2 (E <= 512 and 256 threads or more)
  int c[2], rows = 0, tiles = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = tid * ve + j;
    c[j] = (j < ve && e < E) ? hist[e] : 0;
    rows += c[j];
    tiles += (c[j] + kSmallMTile - 1) / kSmallMTile;
  }
  int rows_total, tiles_total;
  int ex = tail_scan(rows, tmp, rows_total);
  int tex = tail_scan(tiles, tmp, tiles_total);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = tid * ve + j;
    if (j >= ve || e >= E) break;
    T.counts[e] = c[j];
    T.offsets[e] = ex;
    T.tile_off[e] = tex;
    offs[e] = ex;
    const int nt = (c[j] + kSmallMTile - 1) / kSmallMTile;
    for (int i = 0; i < nt; ++i)
      reinterpret_cast<int4*>(T.tile_map)[tex + i] =
          make_int4(e, ex + i * kSmallMTile, min(kSmallMTile, c[j] - i * kSmallMTile), 0);
    ex += c[j];
    tex += nt;
  }
  if (tid == 0) {
    T.offsets[E] = rows_total;
    T.tile_off[E] = tiles_total;
  }
  for (int t = tiles_total + tid; t < T.max_tiles; t += nthr)
    reinterpret_cast<int4*>(T.tile_map)[t] = make_int4(-1, 0, 0, 0);
  __syncthreads();
  for (int m = tid; m < mc; m += nthr) {
    const int e = ids[m], t = m / k;
    const int pos = offs[e] + __popcll(mask[e] & ((1ull << t) - 1ull));
    T.sorted[pos] = m;
    T.inv[m] = pos;
  }
}

// The rankers' part of the tail; the last ranker to finish then sorts the slots by expert and
// resets the counters.
__device__ __forceinline__ void route_tail_run(const RouteTail& T, int r, int R) {
  // dynamic LDS: token masks [E] (8 bytes each), histogram [E], offsets [E], scan scratch [34],
  // slot ids [N * k]
  extern __shared__ unsigned long long tail_lds[];
  unsigned long long* mask = tail_lds;
  int* hist = reinterpret_cast<int*>(mask + T.P.E);
  int* offs = hist + T.P.E;
  int* tmp = offs + T.P.E;
  int32_t* ids = tmp + 34;
  int32_t* own = (R == 1) ? ids : nullptr;
  switch (T.vpl) {
    case 1: route_tail_rank<1>(T, r, R, own); break;
    case 2: route_tail_rank<2>(T, r, R, own); break;
    case 4: route_tail_rank<4>(T, r, R, own); break;
    default: route_tail_rank<8>(T, r, R, own); break;
  }
  if (R > 1) {
    if (tail_arrive(T.ctr + 1) != R) return;
    // the last ranker: every slot's expert, from the rankers' coherent stores
    for (int m = threadIdx.x; m < T.N * T.P.k; m += blockDim.x)
      ids[m] = static_cast<int32_t>(__hip_atomic_load(T.idx + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  }
  __syncthreads();
  route_tail_permute(T, ids, mask, hist, offs, tmp);
  if (threadIdx.x == 0) {
    __hip_atomic_store(T.ctr, kRouteTailTag << 20, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(T.ctr + 1, kRouteTailTag << 20, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Two dense products over the same activation rows in one launch (the router logits, tiled
// bf16, and the shared expert's gate_up, tiled bf16 or int8 as FMT2): job blocks [0, gx1) run
// the first, the rest the second. Both use the same K, so the same chunking W, and each keeps the
// arithmetic of its own launch.
// NORM: both products RMSNorm their activation rows on the fly (QmmArgs::norm_w), and the first
// product's job 0 writes the normalised rows (norm_out).
// TAIL: the routing tail (RouteTail) after the router workgroups' products.
template <int EPI1, int EPI2, int W, int MT, bool NORM = false, int FMT2 = FMT_BF16, bool TAIL = false>
__global__ void __launch_bounds__(W > 4 ? 64 * W : 256)
qmm_small_pair_kernel(QmmArgs a1, int n_jobs1, int gx1, QmmArgs a2, int n_jobs2, RouteTail T) {
  constexpr int R1 = SmallCfg<FMT_BF16, EPI1, W, 1, 1, MT>::RED;
  constexpr int R2 = SmallCfg<FMT2, EPI2, W, 1, 1, MT>::RED;
  constexpr int RR = R1 > R2 ? R1 : R2;
  // (NORM: behind the chunk sums, the norm's chunk sums [WAVES][MT][16] floats)
  constexpr int WAVES = W > 4 ? W : 4;
  __shared__ f32x4_t red[RR + (NORM ? (WAVES * MT * 16 + 3) / 4 : 0)];
  // the decode dataflow kernel's counters (kSyncStride words apart), cleared for the launch that
  // follows this one
  if (a1.zero_words && blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = threadIdx.x; i < a1.n_zero; i += blockDim.x) a1.zero_words[i * kSyncStride] = 0u;
  if (static_cast<int>(blockIdx.x) < gx1) {
    // (TAIL: the logits go out with coherent stores, read by the last router workgroup)
    small_body<FMT_BF16, EPI1, W, 1, 1, MT, NORM, 0, 0, TAIL ? kCohOut : 0>(a1, n_jobs1, blockIdx.x,
                                                                          blockIdx.y, red);
    if constexpr (TAIL) {
      // the last R router workgroups to finish rank the tokens, the first of them once all
      // router workgroups have stored their logits
      const int arrival = tail_arrive(T.ctr);
      if (arrival > T.total - T.rankers) {
        if (T.rankers > 1) tail_wait(T.ctr, T.total, T.timeouts);
        route_tail_run(T, T.total - arrival, T.rankers);
      }
    }
  } else {
    small_body<FMT2, EPI2, W, 1, 1, MT, NORM>(a2, n_jobs2, blockIdx.x - gx1, blockIdx.y, red);
  }
}

// The routed gate_up (int4 SwiGLU over the permuted m-tiles, small-regime shape W/CPW/JPW) and
// the shared expert's down projection (int8 codes, K = its intermediate size, one dense segment
// of N rows; W2 * CPW2 chunks, W2 wavefronts per job each summing CPW2 of them, MT2 m-tiles per
// wavefront) in one launch of 4-wavefront workgroups on a flat grid: the gate_up's job blocks x
// m-tiles first, the shared down's after them. Each keeps the arithmetic of its own launch, so
// the outputs are those of the two launches bit for bit.
template <int W, int CPW, int JPW, int W2, int MT2, int CPW2 = 1>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(SmallCfg<FMT_INT4, EPI_SWIGLU, W, CPW, JPW>::WPE)))
qmm_gate_up_shdown_kernel(QmmArgs a1, int n_jobs1, int gx1, int64_t n1, QmmArgs a2, int n_jobs2,
                          int gx2) {
  constexpr int R1 = SmallCfg<FMT_INT4, EPI_SWIGLU, W, CPW, JPW, 1>::RED;
  constexpr int R2 = SmallCfg<FMT_INT8, EPI_BF16, W2, CPW2, 1, MT2>::RED;
  __shared__ f32x4_t red[R1 > R2 ? R1 : R2];
  const int64_t b = blockIdx.x;
  if (b < n1) {
    small_body<FMT_INT4, EPI_SWIGLU, W, CPW, JPW, 1>(a1, n_jobs1, static_cast<int>(b % gx1),
                                                     static_cast<int>(b / gx1), red);
  } else {
    const int64_t b2 = b - n1;
    small_body<FMT_INT8, EPI_BF16, W2, CPW2, 1, MT2>(a2, n_jobs2, static_cast<int>(b2 % gx2),
                                                     static_cast<int>(b2 / gx2), red);
  }
}

// ============================================================================ large-M kernel
// Workgroup tile: 128 sorted positions x 256 weight rows (SwiGLU: 128 gate + 128 up rows ->
// 128 h columns), one 128-deep k superblock per iteration. 8 wavefronts side by side along the
// weight rows: wavefront w owns all 128 positions (8 m-blocks of 16) and two 16-row weight tiles
// (SwiGLU: gate tile w and its up tile), on v_mfma_f32_16x16x32 (f16 for int4 weights, bf16 for
// bf16 weights). Every weight is dequantized exactly once per workgroup; two wavefronts per SIMD.
//
// All streaming loads go global -> LDS directly (global_load_lds_dwordx4 / _dword), two
// superblocks ahead of the MFMAs, into rings of three LDS slots:
//  * A (activations): 32 KiB per slot, [m-block][step][64 lanes] x 16 B; wavefront w loads
//    m-block w, lane l fetching row l%16's 8-k chunk that MFMA lane l consumes, so fragment
//    reads are 64 consecutive 16-byte slots.
//  * int4 weights: per wavefront and slot, its two tiles' 1 KiB code blocks (verbatim copies of
//    the tiled layout, each lane's 16 bytes being its B fragments for the superblock's four
//    32-k steps) and their 2 x 128 B of scale/bias.
// Every wavefront waits for its own loads of the next superblock (explicit vmcnt: the loads are
// issued from inline assembly, so the compiler neither tracks them nor serialises LDS reads
// behind them), then one barrier publishes the superblock. Weights are dequantized from the
// LDS copy in registers with packed fp16 FMAs (fp16(s*q + b), one rounding); activations come
// from the fp16 per-row-scaled copy (act16), so each step is an exact-input fp16 product with
// fp32 accumulation; the epilogue rescales rows by row_sinv. bf16 weights (shared expert,
// router) are read into registers one superblock ahead, against bf16 activations.
// A partly filled tile computes only its first 2, 4 or 8 m-blocks (three compiled variants of
// the loop, chosen once per workgroup).
constexpr int kLgThreads = 512;
constexpr int kLgNBuf = 3;
constexpr int kLgABytes = 8 * 4 * 64 * 16;                // one A slot: 32 KiB
constexpr int kLgBWaveBytes = 2 * 1024 + 2 * 128;         // one wavefront's int4 weight slot
constexpr int kLgBBytes = 8 * kLgBWaveBytes;              // 18 KiB
constexpr int kLgRowTabBytes = 128 * 4;   // after the slots: per-row scales (as the wide kernel)
constexpr size_t kLgLdsBytes = kLgNBuf * (kLgABytes + kLgBBytes) + kLgRowTabBytes;   // 150.5 KiB
// int6: a wavefront's slot adds the tiles' high-bit planes (2 x 512 B); two slots, 116 KiB
constexpr int kLg6BWaveBytes = 2 * 1024 + 2 * 128 + 2 * 512;
constexpr size_t kLg6LdsBytes = 2 * (kLgABytes + 8 * kLg6BWaveBytes) + kLgRowTabBytes;
// int3: 768 B of codes per tile superblock; three slots, 138 KiB
constexpr int kLg3BWaveBytes = 2 * 768 + 2 * 128;
constexpr size_t kLg3LdsBytes = kLgNBuf * (kLgABytes + 8 * kLg3BWaveBytes) + kLgRowTabBytes;

// 16-byte k-chunk (of 16 in a superblock) that MFMA step s consumes in lane group g: int4 weight
// fragments follow the tiled code words, bf16 ones the natural 32-k chunks.
template <int FMT>
__device__ __forceinline__ int lg_chunk(int s, int g) {
  return FMT == FMT_INT4 ? 8 * (s >> 1) + 2 * g + (s & 1) : 4 * s + g;
}
__device__ __forceinline__ f32x4_t mfma16_f16(u32x4 a, u32x4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
// LDS byte offset of a pointer into the kernel's dynamic LDS (the low 32 bits of its generic
// address), made wave-uniform for M0
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}
// Global -> LDS copy: each lane's 16 (or 4) bytes at src land at lds_off + 16 (or 4) * lane.
// M0 is saved and restored around the copy.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_off) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
               "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(src), "s"(lds_off) : "memory");
}
__device__ __forceinline__ void dma4(const void* src, uint32_t lds_off) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
               "global_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(src), "s"(lds_off) : "memory");
}
// Wait until at most n of this wavefront's vector-memory operations are outstanding (they
// complete in issue order).
// The same copies from a wave-uniform base address (a scalar register pair) plus a 32-bit
// per-lane offset: the base costs no vector registers.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_off) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
               "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(voff), "s"(sbase), "s"(lds_off) : "memory");
}
__device__ __forceinline__ void dma4s(const void* sbase, uint32_t voff, uint32_t lds_off) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
               "global_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(voff), "s"(sbase), "s"(lds_off) : "memory");
}
// A byte loaded and waited for in one asm block, before any DMA of the kernel is issued: the
// compiler then sees a ready value and never guards its later uses with a vmcnt wait, which it
// cannot tell from the DMA prefetch's own (those waits would drain the prefetch every superblock).
__device__ __forceinline__ int load_i8_now(const int8_t* p) {
  int v;
  asm volatile("global_load_sbyte %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}

// A lane's row data for the prologue of the prefill kernels, loaded and waited for in one asm
// block before any DMA is issued (as load_i8_now, one memory round trip for all of it): the
// four weight-row exponent bytes of its tiles and the row scale of its activation row.
struct RowLoads {
  int ex[4];
  float rs;
};
__device__ __forceinline__ RowLoads load_rows_now(const int8_t* e0, const int8_t* e1,
                                                  const int8_t* e2, const int8_t* e3,
                                                  const float* rs) {
  int v0, v1, v2, v3;
  float f;
  asm volatile("global_load_sbyte %0, %5, off\n\tglobal_load_sbyte %1, %6, off\n\t"
               "global_load_sbyte %2, %7, off\n\tglobal_load_sbyte %3, %8, off\n\t"
               "global_load_dword %4, %9, off\n\ts_waitcnt vmcnt(0)"
               : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3), "=&v"(f)
               : "v"(e0), "v"(e1), "v"(e2), "v"(e3), "v"(rs)
               : "memory");
  return RowLoads{{v0, v1, v2, v3}, f};
}

__device__ __forceinline__ RowLoads load_rows_now2(const int8_t* e0, const int8_t* e1, const float* rs) {
  int v0, v1;
  float f;
  asm volatile("global_load_sbyte %0, %3, off\n\tglobal_load_sbyte %1, %4, off\n\t"
               "global_load_dword %2, %5, off\n\ts_waitcnt vmcnt(0)"
               : "=&v"(v0), "=&v"(v1), "=&v"(f)
               : "v"(e0), "v"(e1), "v"(rs)
               : "memory");
  return RowLoads{{v0, v1, 0, 0}, f};
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// Workgroup barrier for the load rings: this wavefront's LDS reads drained (lgkmcnt 0), then
// s_barrier. Unlike __syncthreads() it carries no release fence, whose vmcnt(0) would also wait
// for the loads still in flight for later superblocks; the data each barrier publishes has been
// waited for explicitly (wait_vmcnt) by the wavefront that loaded it.
__device__ __forceinline__ void lg_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// bf16-weight superblock registers of a wavefront: 2 tiles x 4 steps of B fragments.
// Weight data a wavefront holds in registers one superblock ahead: bf16, the B fragments of its
// two tiles; int4 and int6 (staged in LDS), none.
template <int FMT>
struct LgStage {
  u32x4 q[2][4];
};
template <>
struct LgStage<FMT_INT6> {};
template <>
struct LgStage<FMT_INT4> {};
template <>
struct LgStage<FMT_INT3> {};

// int4 -> fp16 dequant of the prefill kernels, one packed register (two weights) per VALU FMA.
// A code nibble masked in place is an fp16 subnormal: at bits 0-3 of a half it reads q * 2^-24,
// at bits 4-7 q * 2^-20, so fma(code, s * 2^(e+24) or s * 2^(e+20), b * 2^e) yields
// fp16(2^e (s q + b)) with a single rounding (the product is exact inside the FMA). e = row_exp
// - kDeqShift: row_exp puts the row's largest magnitude in [2^13, 2^14), which bounds
// s * 2^row_exp below 2^15 / 15 (15 s = (15 s + b) - b), so the larger scale factor, s *
// 2^(row_exp + 4), stays below 2^15.1 < 65504; the weights themselves lie below 2^-6 and keep
// fp16's full precision down to 2^-8 of the row maximum, below that an absolute 2^-20 of it
// (fp16 subnormals; the MFMAs take them exactly). Pairs 2 and 3 share one 8-bit shift.
constexpr int kDeqShift = 20;
struct DeqSb {
  f16x2_t s_lo, s_hi, b;   // scale for nibbles at bits 0-3 / 4-7 of each half, bias
};
__device__ __forceinline__ DeqSb deq_sb(uint32_t sbw, int e) {
  const float sv = bf16lo_to_f32(sbw), bv = bf16hi_to_f32(sbw);
  const _Float16 lo = static_cast<_Float16>(ldexpf(sv, e + 24));
  const _Float16 hi = static_cast<_Float16>(ldexpf(sv, e + 20));
  const _Float16 b = static_cast<_Float16>(ldexpf(bv, e));
  return DeqSb{f16x2_t{lo, lo}, f16x2_t{hi, hi}, f16x2_t{b, b}};
}
// nibble pair j (0..3) of code word w: weights k = j and j+4 of the word's two 16-bit halves
__device__ __forceinline__ uint32_t deq_pair(uint32_t w, int j, const DeqSb& d) {
  const uint32_t src = (j >= 2) ? (w >> 8) : w;
  const f16x2_t q = __builtin_bit_cast(f16x2_t, src & ((j & 1) ? 0x00F000F0u : 0x000F000Fu));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, (j & 1) ? d.s_hi : d.s_lo, d.b));
}

// int6 pair j (0..3) of step half h: the nibble pair of word w as deq_pair takes it (even j at
// bits 0-3 of each half, odd j in place at bits 4-7, pairs 2 and 3 sharing one 8-bit shift), its
// two high bits from the group's high-bit word hw (bits 2j + 8h and 16 + 2j + 8h, as
// unpack_q128_6) moved just above the nibble: each half holds the 6-bit code q as the fp16
// subnormal q * 2^-24 (even j) or 16 q * 2^-24 (odd j, scaled by s_hi). row_exp bounds
// s * 2^row_exp below 2^15 / 63, so both scale factors stay below 2^19 / 63.
__device__ __forceinline__ uint32_t deq_pair6(uint32_t w, uint32_t hw, int h, int j, const DeqSb& d) {
  const uint32_t src = (j >= 2) ? (w >> 8) : w;
  const bool odd = (j & 1) != 0;
  const int hs = 2 * j + 8 * h - (odd ? 8 : 4);   // right shift of the high bits (left if < 0)
  const uint32_t hb = (hs >= 0) ? (hw >> hs) : (hw << -hs);
  const uint32_t v = (src & (odd ? 0x00F000F0u : 0x000F000Fu)) | (hb & (odd ? 0x03000300u : 0x00300030u));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2_t, v),
                                                                odd ? d.s_hi : d.s_lo, d.b));
}

// int3 pair q (0..15) of the lane's three code words, as unpack_q128_3: the 3-bit codes at bits
// 0-2 of each half, the fp16 subnormal q * 2^-24. (int3 dequantizes with a shift one larger than
// kDeqShift: row_exp bounds s * 2^row_exp below 2^15 / 7, so s * 2^(e+24) stays below 2^18 / 7.)
__device__ __forceinline__ uint32_t deq_pair3(uint32_t w0, uint32_t w1, uint32_t w2, int q,
                                             const DeqSb& d) {
  const uint32_t w = (q < 5) ? w0 : (q < 10) ? w1 : w2;
  const uint32_t v = (q < 15) ? (w >> (3 * (q % 5))) & 0x00070007u
                              : ((w0 >> 15) & 0x00010001u) | ((w1 >> 14) & 0x00020002u) |
                                    ((w2 >> 13) & 0x00040004u);
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_fma(__builtin_bit_cast(f16x2_t, v), d.s_lo, d.b));
}

template <int FMT, int EPI>
__global__ void __launch_bounds__(kLgThreads) qmm_large_kernel(QmmArgs a) {
  // QF: int4 or int6 codes, dequantized to fp16 (int6: the nibble plane staged as int4's and
  // the high-bit plane after the scale/bias copy, in two slots instead of three)
  constexpr bool QF = (FMT == FMT_INT4 || FMT == FMT_INT6 || FMT == FMT_INT3);
  // bytes of a tile superblock, and of its codes in a wavefront's LDS slot (int6: the nibble
  // plane; its high-bit plane follows the scale/bias copy)
  constexpr int SBB = (FMT == FMT_INT6) ? 1536 : (FMT == FMT_INT3) ? 768 : 1024;
  constexpr int CB = (FMT == FMT_INT3) ? 768 : 1024;
  constexpr int NBUF = (FMT == FMT_INT6) ? 2 : kLgNBuf;
  constexpr int BWAVE = (FMT == FMT_INT6) ? kLg6BWaveBytes
                        : (FMT == FMT_INT3) ? kLg3BWaveBytes : kLgBWaveBytes;
  constexpr int DS = (FMT == FMT_INT3) ? kDeqShift + 1 : kDeqShift;   // row_exp - e
  constexpr int LDS_ROWTAB = NBUF * (kLgABytes + 8 * BWAVE);            // after the slots
  extern __shared__ u32x4 lds[];
  char* lds_c = reinterpret_cast<char*>(lds);
  const int tid = threadIdx.x, lane = tid & 63;
  // wave index as a scalar: per-wave decisions are uniform (scalar) branches
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int e, m0, m_cnt;
  // XCD-aware tile order. Workgroups are dispatched round-robin over the 8 XCDs, so linear id
  // i runs on XCD i % 8 as that XCD's (i / 8)-th workgroup. Each XCD takes groups of G m-tiles
  // x all nb weight-row blocks (G * nb <= 32, one workgroup per CU of the XCD): the nb blocks
  // of an m-tile share its activation slices through the XCD's L2, and the G m-tiles share the
  // weight slices, instead of every XCD streaming every activation row from MALL.
  const int nbk = a.n_rows / 256;
  const int G = (nbk >= 32) ? 1 : 32 / nbk;
  const int wi = blockIdx.x, xcd = wi & 7, kx = wi >> 3;
  const int gk = kx / (G * nbk), rk = kx - gk * (G * nbk);
  const int mt = (gk * 8 + xcd) * G + rk / nbk;
  const int cb = rk % nbk;
  const int mrows = (a.dense_mtile > 0 && !a.offsets && !a.tile_map) ? a.dense_mtile : kLargeMTile;
  if (mt >= a.mtiles || !resolve_mtile(a, mt, mrows, e, m0, m_cnt)) return;
  // (one stack of a projection whose experts have different widths: the others' m-tiles exit)
  if (a.expert_map) {
    e = a.expert_map[e];
    if (e < 0) return;
  }
  // (AWQ: the 256-row blocks from split_tile on read the second activation copy)
  const bool hi = (QF) && a.act16_hi && 16 * cb >= a.split_tile;
  const uint16_t* act16 = hi ? a.act16_hi : a.act16;
  const float* row_sinv = hi ? a.row_sinv_hi : a.row_sinv;
  const int64_t ebase = static_cast<int64_t>(e) * (a.n_rows / 16);
  const int nsb = a.K / 128;
  const int mb_act = __builtin_amdgcn_readfirstlane((m_cnt + 15) >> 4);   // 1..8

  // ---- activation source: this wavefront loads m-block `wave`; lane -> row lane%16 of the
  // block, k-chunk lg_chunk(s, lane/16) of step s. Rows past the tile and rows whose activation
  // row is invalid read activation row 0 (the former are never stored, the latter are written
  // as zeros by the epilogue). A wavefront whose m-block lies past the tile loads no A.
  const bool a_on = wave < mb_act;
  const char* arow_ptr;
  const int arow_r = 16 * wave + (lane & 15);
  const int64_t arow = (arow_r < m_cnt) ? act_row(a, m0 + arow_r) : -1;
  {
    const uint16_t* abase = (QF) ? act16 : a.act;
    arow_ptr = reinterpret_cast<const char*>(abase + (arow >= 0 ? arow : 0) * static_cast<int64_t>(a.K)) +
               16 * lg_chunk<QF ? FMT_INT4 : FMT>(0, lane >> 4);
  }
  const uint32_t lds_base = lds_offset(lds);
  auto a_slot = [&](int p) { return (p % NBUF) * kLgABytes; };
  auto b_slot = [&](int p) { return NBUF * kLgABytes + (p % NBUF) * 8 * BWAVE + wave * BWAVE; };

  // ---- this wavefront's two weight tiles
  const char* wcode[2];
  const char* wtile[2];   // int4/int6: the tile's first superblock
  const char* wsb[2];
  const u32x4* wp[2];
  const int8_t* wexp[2] = {nullptr, nullptr};
  int rex[2] = {0, 0};   // int4/int6: the lane's weight row of each tile, its dequant exponent e
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int tl = (EPI == EPI_SWIGLU) ? (t == 0 ? 8 * cb + wave : a.n_rows / 32 + 8 * cb + wave)
                                       : 16 * cb + 2 * wave + t;
    if (QF) {
      const int64_t tb = (ebase + tl) * nsb;
      wtile[t] = static_cast<const char*>(a.codes) + tb * SBB;
      wcode[t] = wtile[t] + lane * 16;
      wsb[t] = reinterpret_cast<const char*>(a.sb) + tb * 128;
      wp[t] = nullptr;
      wexp[t] = a.row_exp + (ebase + tl) * 16 + (lane & 15);
    } else {
      wcode[t] = wtile[t] = wsb[t] = nullptr;
      wp[t] = static_cast<const u32x4*>(a.codes) + (ebase + tl) * (a.K / 32) * 64 + lane;
    }
  }
  // the exponents and the activation row's scale in one round trip (bf16 weights: no scaling);
  // wavefront w's lanes 0-15 publish m-block w's row scales for the epilogue (-1: no data)
  float* row_tab = reinterpret_cast<float*>(lds_c + LDS_ROWTAB);
  {
    float rs = 1.0f;
    if (QF) {
      const RowLoads rl = load_rows_now2(wexp[0], wexp[1], row_sinv + (arow >= 0 ? arow : 0));
      rex[0] = rl.ex[0] - DS;
      rex[1] = rl.ex[1] - DS;
      rs = rl.rs;
    }
    if (a_on && lane < 16) row_tab[arow_r] = (arow >= 0) ? rs : -1.0f;
  }
  // scale/bias copy: lanes 0-31 take tile 0's 128 B, lanes 32-63 tile 1's, 4 B each
  const char* sb_src = (QF) ? wsb[lane >> 5] + 4 * (lane & 31) : nullptr;
  // int6 high-bit planes: lanes 0-31 take tile 0's 512 B, lanes 32-63 tile 1's, 16 B each
  const char* hb_src = (FMT == FMT_INT6) ? wtile[lane >> 5] + 1024 + 16 * (lane & 31) : nullptr;

  // issue all loads of superblock p (A: 4 instructions when a_on; int4 weights: 3)
  auto issue = [&](int p) __attribute__((always_inline)) {
    if (a_on) {
      const char* src = arow_ptr + 256 * p;
      const uint32_t dst = lds_base + a_slot(p) + wave * 4 * 1024;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int off = 16 * ((QF) ? 8 * (s >> 1) + (s & 1) : 4 * s);
        dma16(src + off, dst + s * 1024);
      }
    }
    if (QF) {
      const uint32_t dst = lds_base + b_slot(p);
      if (FMT == FMT_INT3) {
        // 768 B per tile: three dword copies, lane l's 4 bytes at 256 i + 4 l of each
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 3; ++i)
            dma4(wtile[t] + static_cast<int64_t>(p) * SBB + 256 * i + 4 * lane, dst + t * CB + 256 * i);
      } else {
        dma16(wcode[0] + static_cast<int64_t>(p) * SBB, dst);
        dma16(wcode[1] + static_cast<int64_t>(p) * SBB, dst + 1024);
      }
      dma4(sb_src + static_cast<int64_t>(p) * 128, dst + 2 * CB);
      if (FMT == FMT_INT6) dma16(hb_src + static_cast<int64_t>(p) * SBB, dst + 2048 + 256);
    }
  };

  f32x4_t acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[i][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One superblock: four 32-k MFMA steps, software-pipelined by hand. Step s is MB slots; slot
  // i issues the two MFMAs of m-block i, the read of m-block i's A fragment for step s+1 and
  // 1/MB of step s+1's weight dequant, and a scheduling barrier keeps that order, so LDS reads
  // have a full step to land and the dequant VALU work is spread between the MFMAs.
  // (int4 dequant: deq_sb / deq_pair)
  auto compute = [&](int p, const LgStage<FMT>& gb, auto mbc) __attribute__((always_inline)) {
    constexpr int MB = decltype(mbc)::value;
    constexpr int UPS = 8 / MB;                 // dequant units (nibble pairs) per slot
    const u32x4* la = reinterpret_cast<const u32x4*>(lds_c + a_slot(p)) + lane;
    u32x4 q[2];
    uint2 sbv[2];
    u32x2 hq[2];   // int6: the lane's high-bit words of each tile (group 0, group 1)
    if (QF) {
      const char* lb = lds_c + b_slot(p);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (FMT == FMT_INT3) {   // the lane's three words
          const uint32_t* w3 = reinterpret_cast<const uint32_t*>(lb + t * CB) + 3 * lane;
          q[t] = u32x4{w3[0], w3[1], w3[2], 0u};
        } else {
          q[t] = reinterpret_cast<const u32x4*>(lb + t * 1024)[lane];
        }
        sbv[t] = reinterpret_cast<const uint2*>(lb + 2 * CB + t * 128)[lane & 15];
        if (FMT == FMT_INT6) hq[t] = reinterpret_cast<const u32x2*>(lb + 2304 + t * 512)[lane];
      }
    }
    DeqSb dsb[2];
    // the group's scale and bias, scaled by 2^e (exact)
    auto sb_conv = [&](int grp) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < 2; ++t) dsb[t] = deq_sb(grp ? sbv[t].y : sbv[t].x, rex[t]);
    };
    // dequant unit u (0..7) of step s: tile u/4, nibble pair u%4 -> one packed fp16 register
    auto deq_unit = [&](int s, int u, u32x4* bfo) __attribute__((always_inline)) {
      const int t = u >> 2, j = u & 3;
      if constexpr (FMT == FMT_INT6) {
        bfo[t][j] = deq_pair6(q[t][s], (s >> 1) ? hq[t].y : hq[t].x, s & 1, j, dsb[t]);
      } else if constexpr (FMT == FMT_INT3) {
        bfo[t][j] = deq_pair3(q[t].x, q[t].y, q[t].z, 4 * s + j, dsb[t]);
      } else if constexpr (FMT == FMT_INT4) {
        bfo[t][j] = deq_pair(q[t][s], j, dsb[t]);
      } else if (j == 0) {
        bfo[t] = gb.q[t][s];
      }
    };
    u32x4 bf[2][2], A[2][MB];
    if (QF) sb_conv(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) deq_unit(0, u, bf[0]);
#pragma unroll
    for (int i = 0; i < MB; ++i) A[0][i] = la[256 * i];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = s & 1;
      if (QF && s == 1) sb_conv(1);      // group 1 feeds steps 2 and 3
#pragma unroll
      for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
          acc[i][t] = (QF) ? mfma16_f16(A[c][i], bf[c][t], acc[i][t])
                                        : mfma16(as_bf16x8(A[c][i]), as_bf16x8(bf[c][t]), acc[i][t]);
        if (s < 3) {
          A[c ^ 1][i] = la[256 * i + 64 * (s + 1)];
#pragma unroll
          for (int v = 0; v < UPS; ++v) deq_unit(s + 1, i * UPS + v, bf[c ^ 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // bf16 weights: registers, one superblock ahead
  LgStage<FMT> gbf[2];
  auto load_bf = [&](int p, LgStage<FMT>& g) __attribute__((always_inline)) {
    if constexpr (FMT == FMT_BF16) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) g.q[t][s] = wp[t][(4 * p + s) * 64];
    }
  };

  // Loads in flight per wavefront and superblock: NA (A, when a_on) + NB (int4 weights).
  // Before the barrier that publishes superblock p+1, a wavefront waits until only the loads
  // of p+2 remain outstanding.
  constexpr int NB = (FMT == FMT_INT6) ? 4 : (FMT == FMT_INT3) ? 7 : (QF) ? 3 : 0;
  auto run = [&](auto mbc) __attribute__((always_inline)) {
    if constexpr (FMT == FMT_INT6) {
      // two slots (the 512-row kernel's ring): at the end of superblock p each wavefront waits
      // for its own loads of p+1, the barrier publishes slot p+1 and retires slot p, and the
      // loads of p+2 go into slot p
      issue(0);
      if (nsb > 1) {
        issue(1);
        if (a_on) wait_vmcnt<4 + NB>(); else wait_vmcnt<NB>();
      } else {
        wait_vmcnt<0>();
      }
      lg_barrier();
      for (int p = 0; p < nsb; ++p) {
        compute(p, gbf[0], mbc);
        if (p + 1 < nsb) {
          wait_vmcnt<0>();
          lg_barrier();
          if (p + 2 < nsb) issue(p + 2);
        }
      }
      return;
    }
    auto wait_next = [&](bool far) __attribute__((always_inline)) {
      // loads of the superblock after the next one, if issued, may stay in flight
      if (a_on) {
        if (far) wait_vmcnt<4 + NB>(); else wait_vmcnt<0>();
      } else {
        if (far) wait_vmcnt<NB>(); else wait_vmcnt<0>();
      }
    };
    issue(0);
    if (nsb > 1) issue(1);
    load_bf(0, gbf[0]);
    wait_next(nsb > 1);
    lg_barrier();
    auto iter = [&](int p, const LgStage<FMT>& cur, LgStage<FMT>& nxt) __attribute__((always_inline)) {
      const bool far = p + 2 < nsb;
      if (far) issue(p + 2);
      load_bf(p + 1, nxt);
      compute(p, cur, mbc);
      wait_next(far);
      lg_barrier();
    };
    int p = 0;
    for (; p + 2 < nsb; p += 2) {
      iter(p, gbf[0], gbf[1]);
      iter(p + 1, gbf[1], gbf[0]);
    }
    if (p + 1 < nsb) {
      iter(p, gbf[0], gbf[1]);
      compute(p + 1, gbf[1], mbc);
    } else {
      compute(p, gbf[0], mbc);
    }
  };
  if (mb_act <= 2) run(std::integral_constant<int, 2>{});
  else if (mb_act <= 4) run(std::integral_constant<int, 4>{});
  else run(std::integral_constant<int, 8>{});

  // ---- epilogue: lane holds C[row 4(lane/16) + j][col lane%16] of each 16x16 block
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i >= mb_act) break;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int mr = 16 * i + 4 * (lane >> 4) + j;
      if (mr >= m_cnt) continue;
      // rows whose activation row is invalid read as zeros (their A data was row 0's)
      const float rs = row_tab[mr];
      const bool ok = rs >= 0.f;
      // undo both power-of-two scalings (activation row, int4 weight row): exact
      auto val = [&](int t) { return ok ? ldexpf(acc[i][t][j] * rs, -rex[t]) : 0.f; };
      if (EPI == EPI_SWIGLU) {
        const int col = 128 * cb + 16 * wave + (lane & 15);
        store_out<EPI>(a, m0 + mr, col, val(0), val(1));
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = 256 * cb + 32 * wave + 16 * t + (lane & 15);
          store_out<EPI>(a, m0 + mr, col, val(t), 0.f);
        }
      }
    }
  }
}

// ============================================================================ wide prefill kernel
// int4 weights, large-M regime, for weight-row counts that are multiples of 512 (SwiGLU: gate
// halves that are multiples of 256). Workgroup tile: 128 sorted positions x 512 weight rows
// (SwiGLU: 256 gate + 256 up rows -> 256 h columns), 8 wavefronts side by side along the
// weight rows. Wavefront w owns all 128 positions (8 m-blocks of 16) and four 16-row weight
// tiles (SwiGLU: two gate tiles and their up tiles), so each A fragment read from LDS feeds four
// MFMAs and every dequantised B fragment feeds eight: half the LDS bytes per MFMA of the
// 256-row tile, at the same dequant cost per MFMA. Accumulators: 8 x 4 16x16 blocks (128 VGPRs).
//
// LDS: two slots of one superblock each, A 32 KiB ([m-block][step][64 lanes] x 16 B, as in the
// 256-row kernel) + int4 weights 8 x 4.5 KiB (per wavefront its four tiles' 1 KiB code blocks
// and 4 x 128 B of scale/bias), 136 KiB in all. One barrier per superblock: at the end of
// superblock p every wavefront waits for its own loads of p+1 (the only ones in flight), the
// barrier publishes slot p+1 and retires slot p, and the loads of p+2 are issued into slot p at
// once, landing while p+1 is computed.
//
// Per output the summation is the 256-row kernel's (k-steps in order within a superblock,
// superblocks in order, one fp32 accumulator), so both kernels give identical results.
constexpr int kWdThreads = 512;
constexpr int kWdABytes = 8 * 4 * 64 * 16;                 // 32 KiB
constexpr int kWdBWaveBytes = 4 * 1024 + 4 * 128;          // 4.5 KiB
constexpr int kWdSlotBytes = kWdABytes + 8 * kWdBWaveBytes; // 68 KiB
// after the two slots: the m-tile's per-row activation scales (-1 marks a row without data)
constexpr int kWdRowTabBytes = 128 * 4;
constexpr size_t kWdLdsBytes = 2 * kWdSlotBytes + kWdRowTabBytes;   // 136.5 KiB
// int3 (qmm_wide_int3_kernel): 768 B of codes per tile superblock, 3.5 KiB per wavefront, 120 KiB
constexpr int kWd3BWaveBytes = 4 * 768 + 4 * 128;
constexpr int kWd3SlotBytes = kWdABytes + 8 * kWd3BWaveBytes;
constexpr size_t kWd3LdsBytes = 2 * kWd3SlotBytes + kWdRowTabBytes;

// FMT: int4 (qmm_wide_kernel) or int3 (qmm_wide_int3_kernel, the tile superblocks staged by dword
// copies as in qmm_large_kernel)
template <int FMT, int EPI>
__device__ __forceinline__ void wide_body(const QmmArgs& a) {
  constexpr int SBB = (FMT == FMT_INT3) ? 768 : 1024;   // code bytes of a tile superblock
  constexpr int BWAVE = (FMT == FMT_INT3) ? kWd3BWaveBytes : kWdBWaveBytes;
  constexpr int SLOT = (FMT == FMT_INT3) ? kWd3SlotBytes : kWdSlotBytes;
  constexpr int DS = (FMT == FMT_INT3) ? kDeqShift + 1 : kDeqShift;   // row_exp - e
  constexpr int NB = (FMT == FMT_INT3) ? 14 : 6;   // weight loads per superblock
  extern __shared__ u32x4 lds[];
  char* lds_c = reinterpret_cast<char*>(lds);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int e, m0, m_cnt;
  // XCD-aware tile order, as in the 256-row kernel (groups of G m-tiles x all nbk weight-row
  // blocks per XCD, G * nbk <= 32)
  const int nbk = a.n_rows / 512;
  const int G = (nbk >= 32) ? 1 : 32 / nbk;
  const int wi = blockIdx.x, xcd = wi & 7, kx = wi >> 3;
  const int gk = kx / (G * nbk), rk = kx - gk * (G * nbk);
  const int mt = (gk * 8 + xcd) * G + rk / nbk;
  const int cb = rk % nbk;
  if (mt >= a.mtiles || !resolve_mtile(a, mt, kLargeMTile, e, m0, m_cnt)) return;
  if (a.expert_map) {   // (as qmm_large_kernel)
    e = a.expert_map[e];
    if (e < 0) return;
  }
  const int64_t ebase = static_cast<int64_t>(e) * (a.n_rows / 16);
  const int nsb = a.K / 128;
  const int mb_act = __builtin_amdgcn_readfirstlane((m_cnt + 15) >> 4);   // 1..8
  // (AWQ: the 512-row blocks from split_tile on read the second activation copy)
  const bool hi = a.act16_hi && 32 * cb >= a.split_tile;
  const uint16_t* act16 = hi ? a.act16_hi : a.act16;
  const float* row_sinv = hi ? a.row_sinv_hi : a.row_sinv;

  // activation source: wavefront w loads m-block w (see qmm_large_kernel)
  const bool a_on = wave < mb_act;
  const char* arow_ptr;
  const int arow_r = 16 * wave + (lane & 15);
  const int64_t arow = (arow_r < m_cnt) ? act_row(a, m0 + arow_r) : -1;
  arow_ptr = reinterpret_cast<const char*>(act16 + (arow >= 0 ? arow : 0) * static_cast<int64_t>(a.K)) +
             16 * lg_chunk<FMT_INT4>(0, lane >> 4);
  const uint32_t lds_base = lds_offset(lds);
  auto a_slot = [&](int p) { return (p & 1) * SLOT; };
  auto b_slot = [&](int p) { return (p & 1) * SLOT + kWdABytes + wave * BWAVE; };

  // this wavefront's four weight tiles (SwiGLU: gate tiles first, then their up tiles)
  // (tile bases are wave-uniform: the copies take them from scalar registers)
  const char* wtile[4];   // the tile's first superblock
  const char* wsb[4];
  const int8_t* wexp[4];
  int rex[4];   // the lane's weight row of each tile: its dequant exponent e (deq_sb)
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int tl = (EPI == EPI_SWIGLU)
                       ? ((t < 2) ? 16 * cb + 2 * wave + t : a.n_rows / 32 + 16 * cb + 2 * wave + (t - 2))
                       : 32 * cb + 4 * wave + t;
    const int64_t tb = (ebase + tl) * nsb;
    wtile[t] = static_cast<const char*>(a.codes) + tb * SBB;
    wsb[t] = reinterpret_cast<const char*>(a.sb) + tb * 128;
    wexp[t] = a.row_exp + (ebase + tl) * 16 + (lane & 15);
  }
  // the exponents and the activation row's scale in one round trip; wavefront w's lanes 0-15
  // publish the scales of m-block w for the epilogue (-1: no data), before the first barrier
  float* row_tab = reinterpret_cast<float*>(lds_c + 2 * SLOT);
  {
    const RowLoads rl = load_rows_now(wexp[0], wexp[1], wexp[2], wexp[3], row_sinv + (arow >= 0 ? arow : 0));
#pragma unroll
    for (int t = 0; t < 4; ++t) rex[t] = rl.ex[t] - DS;
    if (a_on && lane < 16) row_tab[arow_r] = (arow >= 0) ? rl.rs : -1.0f;
  }
  // scale/bias copies: lanes 0-31 take the first tile's 128 B, lanes 32-63 the second's (tiles
  // 0, 1 and 2, 3 are consecutive, nsb * 128 bytes apart)
  const uint32_t sb_voff = static_cast<uint32_t>((lane >> 5) * nsb * 128 + 4 * (lane & 31));

  // all loads of superblock p: A 4 (when a_on) + codes 4 + scale/bias 2
  auto issue = [&](int p) __attribute__((always_inline)) {
    if (a_on) {
      const char* src = arow_ptr + 256 * p;
      const uint32_t dst = lds_base + a_slot(p) + wave * 4 * 1024;
#pragma unroll
      for (int s = 0; s < 4; ++s) dma16(src + 16 * (8 * (s >> 1) + (s & 1)), dst + s * 1024);
    }
    const uint32_t dst = lds_base + b_slot(p);
    if (FMT == FMT_INT3) {
      // 768 B per tile: three dword copies, lane l's 4 bytes at 256 i + 4 l of each
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 3; ++i)
          dma4s(wtile[t] + static_cast<int64_t>(p) * SBB + 256 * i, 4 * lane, dst + t * SBB + 256 * i);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) dma16s(wtile[t] + static_cast<int64_t>(p) * SBB, 16 * lane, dst + t * SBB);
    }
    dma4s(wsb[0] + static_cast<int64_t>(p) * 128, sb_voff, dst + 4 * SBB);
    dma4s(wsb[2] + static_cast<int64_t>(p) * 128, sb_voff, dst + 4 * SBB + 256);
  };

  f32x4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[i][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One superblock: four 32-k steps. Step s is MB slots; slot i issues the four MFMAs of
  // m-block i, the LDS read of the A fragment two slots ahead, and step s+1's weight dequant
  // units [16i/MB, 16(i+1)/MB) (tile u/4, nibble pair u%4), in that order (scheduling barriers).
  auto compute = [&](int p, auto mbc) __attribute__((always_inline)) {
    constexpr int MB = decltype(mbc)::value;
    constexpr int NI = 4 * MB;                 // A fragments (slots) per superblock
    const u32x4* la = reinterpret_cast<const u32x4*>(lds_c + a_slot(p)) + lane;
    const char* lb = lds_c + b_slot(p);
    u32x4 q[4];
    uint2 sbv[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (FMT == FMT_INT3) {   // the lane's three words
        const uint32_t* w3 = reinterpret_cast<const uint32_t*>(lb + t * SBB) + 3 * lane;
        q[t] = u32x4{w3[0], w3[1], w3[2], 0u};
      } else {
        q[t] = reinterpret_cast<const u32x4*>(lb + t * 1024)[lane];
      }
      sbv[t] = reinterpret_cast<const uint2*>(lb + 4 * SBB + t * 128)[lane & 15];
    }
    DeqSb dsb[4];
    // the group's scale and bias, scaled by 2^e (exact)
    auto sb_conv = [&](int grp) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < 4; ++t) dsb[t] = deq_sb(grp ? sbv[t].y : sbv[t].x, rex[t]);
    };
    auto deq_unit = [&](int s, int u, u32x4* bfo) __attribute__((always_inline)) {
      const int t = u >> 2, j = u & 3;
      if constexpr (FMT == FMT_INT3)
        bfo[t][j] = deq_pair3(q[t].x, q[t].y, q[t].z, 4 * s + j, dsb[t]);
      else
        bfo[t][j] = deq_pair(q[t][s], j, dsb[t]);
    };
    u32x4 bf[2][4];
    u32x4 A[NI];
    sb_conv(0);
#pragma unroll
    for (int u = 0; u < 16; ++u) deq_unit(0, u, bf[0]);
    A[0] = la[0];
    if (NI > 1) A[1] = la[(MB > 1) ? 256 : 64];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = s & 1;
      if (s == 1) sb_conv(1);      // group 1 feeds steps 2 and 3
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const int n = s * MB + i;
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[i][t] = mfma16_f16(A[n], bf[c][t], acc[i][t]);
        if (n + 2 < NI) {
          const int n2 = n + 2, s2i = n2 / MB, i2 = n2 % MB;
          A[n2] = la[256 * i2 + 64 * s2i];
        }
        if (s < 3) {
#pragma unroll
          for (int u = i * 16 / MB; u < (i + 1) * 16 / MB; ++u) deq_unit(s + 1, u, bf[c ^ 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  auto run = [&](auto mbc) __attribute__((always_inline)) {
    issue(0);
    if (nsb > 1) {
      issue(1);
      if (a_on) wait_vmcnt<4 + NB>(); else wait_vmcnt<NB>();
    } else {
      wait_vmcnt<0>();
    }
    lg_barrier();
    for (int p = 0; p < nsb; ++p) {
      compute(p, mbc);
      if (p + 1 < nsb) {
        wait_vmcnt<0>();
        lg_barrier();
        if (p + 2 < nsb) issue(p + 2);
      }
    }
  };
  switch (mb_act) {
    case 1:
    case 2: run(std::integral_constant<int, 2>{}); break;
    case 3: run(std::integral_constant<int, 3>{}); break;
    case 4: run(std::integral_constant<int, 4>{}); break;
    case 5: run(std::integral_constant<int, 5>{}); break;
    case 6: run(std::integral_constant<int, 6>{}); break;
    case 7: run(std::integral_constant<int, 7>{}); break;
    default: run(std::integral_constant<int, 8>{}); break;
  }

  // epilogue: lane holds C[row 4(lane/16) + j][col lane%16] of each 16x16 block
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i >= mb_act) break;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int mr = 16 * i + 4 * (lane >> 4) + j;
      if (mr >= m_cnt) continue;
      const float rs = row_tab[mr];
      const bool ok = rs >= 0.f;
      // undo both power-of-two scalings (activation row, weight row): exact
      auto val = [&](int t) { return ok ? ldexpf(acc[i][t][j] * rs, -rex[t]) : 0.f; };
      if (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = 256 * cb + 32 * wave + 16 * t + (lane & 15);
          store_out<EPI>(a, m0 + mr, col, val(t), val(t + 2));
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int col = 512 * cb + 64 * wave + 16 * t + (lane & 15);
          store_out<EPI>(a, m0 + mr, col, val(t), 0.f);
        }
      }
    }
  }
}

template <int EPI>
__global__ void __launch_bounds__(kWdThreads, 1) qmm_wide_kernel(QmmArgs a) {
  wide_body<FMT_INT4, EPI>(a);
}
template <int EPI>
__global__ void __launch_bounds__(kWdThreads, 1) qmm_wide_int3_kernel(QmmArgs a) {
  wide_body<FMT_INT3, EPI>(a);
}

// ---------------------------------------------------------------- fp16 activation copy
// One wavefront per row, the row held in registers (RPL 16-byte pieces per lane): absmax by a
// wavefront reduction, then act16 = fp16(act * 2^(14 - e)) with 2^(e-1) <= absmax < 2^e, so every
// value sits below 2^14 and all bf16 values within 2^28 of the row maximum convert exactly.
// row_sinv = 2^(e - 14) undoes it on the product (a power of two: exact). The maximum is exact in
// any order, so the result does not depend on the launch shape.
template <int RPL>
__global__ void __launch_bounds__(256) act_to_f16_kernel(const uint16_t* __restrict__ act, int K,
                                                         int64_t rows,
                                                         uint16_t* __restrict__ act16,
                                                         float* __restrict__ row_sinv) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;   // whole wavefront
  const u32x4* src = reinterpret_cast<const u32x4*>(act + row * K);
  const int n8 = K / 8;
  u32x4 v[RPL];
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = (c < n8) ? src[c] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m = fmaxf(m, fabsf(bf16lo_to_f32(v[i][j])));
      m = fmaxf(m, fabsf(bf16hi_to_f32(v[i][j])));
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  int ex = 0;
  if (m > 0.f && m <= 3.4e38f) frexpf(m, &ex);   // m = f * 2^ex, f in [0.5, 1)
  const int sh = (m > 0.f && m <= 3.4e38f) ? 14 - ex : 0;
  if (lane == 0) row_sinv[row] = ldexpf(1.0f, -sh);
  u32x4* dst = reinterpret_cast<u32x4*>(act16 + row * K);
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int c = lane + 64 * i;
    if (c < n8) {
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f16x2_t h = {static_cast<_Float16>(ldexpf(bf16lo_to_f32(v[i][j]), sh)),
                           static_cast<_Float16>(ldexpf(bf16hi_to_f32(v[i][j]), sh))};
        o[j] = __builtin_bit_cast(uint32_t, h);
      }
      dst[c] = o;
    }
  }
}

// Rows longer than 8192: one workgroup per row, the row read twice (absmax, then convert).
__global__ void __launch_bounds__(256) act_to_f16_wide_kernel(const uint16_t* __restrict__ act, int K,
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
  if (K > 8 * 64 * 16) {
    if (rows > 0x7fffffff) return fail("act_to_f16: too many rows");
    act_to_f16_wide_kernel<<<static_cast<unsigned>(rows), 256, 0, stream>>>(act, K, act16, row_sinv);
    return check_launch("act_to_f16");
  }
  if (rows > (int64_t(1) << 32)) return fail("act_to_f16: too many rows");
  const unsigned grid = static_cast<unsigned>((rows + 3) / 4);
  const int rpl = (K / 8 + 63) / 64;   // 16-byte pieces per lane
#define QMOE_A16(R) act_to_f16_kernel<R><<<grid, 256, 0, stream>>>(act, K, rows, act16, row_sinv)
  if (rpl <= 2) QMOE_A16(2);
  else if (rpl <= 4) QMOE_A16(4);
  else if (rpl <= 8) QMOE_A16(8);
  else if (rpl <= 14) QMOE_A16(14);
  else QMOE_A16(16);
#undef QMOE_A16
  return check_launch("act_to_f16");
}


// ============================================================================ launcher
// Small-kernel launch shape. The chunk count CH depends on K only (the summation order); the
// launch picks how many 16-row tiles a wavefront streams (JPW) and how many wavefronts share a
// job's chunks (W = CH or CH / 2, so CPW = 1 or 2): the most work per wavefront that still
// leaves kSmallMinWaves wavefronts, else the most wavefronts.
constexpr int64_t kSmallMinWaves = 5120;
// Fewest m-tiles for which dense bf16 products run two m-tiles per wavefront.
constexpr int64_t kSmallMt2MinTiles = 4;
template <int FMT, int EPI, int W, int CPW, int JPW>
static void launch_small_k(const QmmArgs& a, int64_t mtiles, hipStream_t stream) {
  constexpr int WAVES = W > 4 ? W : 4;
  const int n_jobs = ((EPI == EPI_SWIGLU) ? a.n_rows / 32 : a.n_rows / 16) / JPW;
  const int jobs_per_wg = WAVES / W;
  // dense products over kSmallMt2MinTiles or more m-tiles: two per wavefront (weights read, and
  // int8 weights dequantized, once per 32 rows; below that, halving the grid leaves CUs idle)
  if constexpr (fmt_dense(FMT)) {
    if (mtiles >= kSmallMt2MinTiles && !a.offsets && !a.tile_map) {
      dim3 grid((n_jobs + jobs_per_wg - 1) / jobs_per_wg, static_cast<unsigned>((mtiles + 1) / 2));
      qmm_small_kernel<FMT, EPI, W, CPW, JPW, 2><<<grid, 64 * WAVES, 0, stream>>>(a, n_jobs);
      return;
    }
  }
  dim3 grid((n_jobs + jobs_per_wg - 1) / jobs_per_wg, static_cast<unsigned>(mtiles));
  qmm_small_kernel<FMT, EPI, W, CPW, JPW, 1><<<grid, 64 * WAVES, 0, stream>>>(a, n_jobs);
}

struct SmallShape {
  int jpw, w, cpw;
};

// (SwiGLU wavefronts hold two tiles per job: JPW 4 would exceed the register budget)
// (int6 wavefronts hold at most two tiles: four spill at the three-wavefront register budget)
static SmallShape pick_small_shape(int fmt, int epi, int ch, int64_t mtiles, int jobs) {
  if (!fmt_quant(fmt)) return SmallShape{1, ch, 1};
  const int jmax = (fmt == FMT_INT6) ? ((epi == EPI_SWIGLU) ? 1 : 2) : ((epi == EPI_SWIGLU) ? 2 : 4);
  SmallShape best{1, ch, 1};
  int64_t best_waves = mtiles * jobs * ch, best_work = 1;
  bool best_ok = best_waves >= kSmallMinWaves;
  for (int jpw = 1; jpw <= jmax; jpw *= 2) {
    if (jobs % jpw) continue;
    for (int cpw = 1; cpw <= 2 && cpw <= ch; cpw *= 2) {
      const int w = ch / cpw;
      const int64_t waves = mtiles * (jobs / jpw) * w;
      const int64_t work = static_cast<int64_t>(jpw) * cpw;
      const bool ok = waves >= kSmallMinWaves;
      const bool better = ok ? (!best_ok || work > best_work || (work == best_work && jpw > best.jpw))
                             : (!best_ok && waves > best_waves);
      if (better) {
        best = SmallShape{jpw, w, cpw};
        best_waves = waves;
        best_work = work;
        best_ok = ok;
      }
    }
  }
  return best;
}

template <int FMT, int EPI, int W, int CPW>
static void launch_small_j(const QmmArgs& a, int jpw, int64_t mtiles, hipStream_t stream) {
  if constexpr (FMT == FMT_INT6) {
    if (EPI != EPI_SWIGLU && jpw == 2)
      launch_small_k<FMT, EPI, W, CPW, (EPI == EPI_SWIGLU) ? 1 : 2>(a, mtiles, stream);
    else
      launch_small_k<FMT, EPI, W, CPW, 1>(a, mtiles, stream);
  } else if constexpr (FMT == FMT_INT4 || FMT == FMT_INT3) {
    if (EPI != EPI_SWIGLU && jpw == 4)
      launch_small_k<FMT, EPI, W, CPW, (EPI == EPI_SWIGLU) ? 2 : 4>(a, mtiles, stream);
    else if (jpw == 2)
      launch_small_k<FMT, EPI, W, CPW, 2>(a, mtiles, stream);
    else
      launch_small_k<FMT, EPI, W, CPW, 1>(a, mtiles, stream);
  } else {
    launch_small_k<FMT, EPI, W, 1, 1>(a, mtiles, stream);
  }
}

template <int FMT, int EPI>
static void launch_small(const QmmArgs& a, const SmallShape& sh, int64_t mtiles,
                         hipStream_t stream) {
  if constexpr (fmt_quant(FMT)) {
    if (sh.cpw == 2) {
      if (sh.w == 2) launch_small_j<FMT, EPI, 2, 2>(a, sh.jpw, mtiles, stream);
      else launch_small_j<FMT, EPI, 1, 2>(a, sh.jpw, mtiles, stream);
    } else {
      if (sh.w == 4) launch_small_j<FMT, EPI, 4, 1>(a, sh.jpw, mtiles, stream);
      else if (sh.w == 2) launch_small_j<FMT, EPI, 2, 1>(a, sh.jpw, mtiles, stream);
      else launch_small_j<FMT, EPI, 1, 1>(a, sh.jpw, mtiles, stream);
    }
  } else {
    switch (sh.w) {
      case 16: launch_small_j<FMT, EPI, 16, 1>(a, sh.jpw, mtiles, stream); break;
      case 8: launch_small_j<FMT, EPI, 8, 1>(a, sh.jpw, mtiles, stream); break;
      case 4: launch_small_j<FMT, EPI, 4, 1>(a, sh.jpw, mtiles, stream); break;
      case 2: launch_small_j<FMT, EPI, 2, 1>(a, sh.jpw, mtiles, stream); break;
      default: launch_small_j<FMT, EPI, 1, 1>(a, sh.jpw, mtiles, stream); break;
    }
  }
}

template <int FMT, int EPI>
static int launch_large(const QmmArgs& a, int64_t mtiles, hipStream_t stream) {
  // 150 KiB (int6: 116 KiB) of dynamic LDS is above the default per-kernel limit; set it for
  // the current device
  const size_t lds_bytes = (FMT == FMT_INT6) ? kLg6LdsBytes
                           : (FMT == FMT_INT3) ? kLg3LdsBytes : kLgLdsBytes;
  const hipError_t err =
      hipFuncSetAttribute(reinterpret_cast<const void*>(qmm_large_kernel<FMT, EPI>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_bytes));
  if (err != hipSuccess) return fail(std::string("qmm(large): LDS attribute: ") + hipGetErrorString(err));
  // 1-D grid in the XCD-grouped order the kernel decodes: m-tiles padded to whole groups of
  // 8 XCDs x G m-tiles; workgroups past `mtiles` exit at once
  const int nbk = a.n_rows / 256;
  const int G = (nbk >= 32) ? 1 : 32 / nbk;
  const int64_t mpad = (mtiles + 8 * G - 1) / (8 * G) * (8 * G);
  QmmArgs b = a;
  b.mtiles = static_cast<int>(mtiles);
  qmm_large_kernel<FMT, EPI><<<dim3(static_cast<unsigned>(mpad * nbk)), kLgThreads, lds_bytes, stream>>>(b);
  return 0;
}

// 1-D grid in the XCD-grouped order the wide kernel decodes (as in launch_large, with 512-row
// weight blocks)
template <int FMT, int EPI>
static int launch_wide(const QmmArgs& a, int64_t mtiles, hipStream_t stream) {
  const void* fn = (FMT == FMT_INT3) ? reinterpret_cast<const void*>(qmm_wide_int3_kernel<EPI>)
                                     : reinterpret_cast<const void*>(qmm_wide_kernel<EPI>);
  const size_t lds_bytes = (FMT == FMT_INT3) ? kWd3LdsBytes : kWdLdsBytes;
  const hipError_t err =
      hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_bytes));
  if (err != hipSuccess) return fail(std::string("qmm(wide): LDS attribute: ") + hipGetErrorString(err));
  const int nbk = a.n_rows / 512;
  const int G = (nbk >= 32) ? 1 : 32 / nbk;
  const int64_t mpad = (mtiles + 8 * G - 1) / (8 * G) * (8 * G);
  QmmArgs b = a;
  b.mtiles = static_cast<int>(mtiles);
  const dim3 grid(static_cast<unsigned>(mpad * nbk));
  if (FMT == FMT_INT3) qmm_wide_int3_kernel<EPI><<<grid, kWdThreads, lds_bytes, stream>>>(b);
  else qmm_wide_kernel<EPI><<<grid, kWdThreads, lds_bytes, stream>>>(b);
  return 0;
}

// Slot-major routed gate_up with its routing (qmm_route_gate_up_kernel): int4 weights, SwiGLU,
// the decode kernel's chunking (W = CH wavefronts per job, one chunk each, one tile pair each).
template <int W, int VPL>
static void launch_route_k(const QmmArgs& a, int64_t mc, const SlotRoute& R, hipStream_t stream,
                           const QmmArgs* sdn = nullptr, int w2 = 0) {
  constexpr int WAVES = W > 4 ? W : 4;
  const int n_jobs = a.n_rows / 32;
  const int jobs_per_wg = WAVES / W;
  if (sdn) {   // (the caller checked w2 and the m-tile count)
    const int gx1 = (n_jobs + jobs_per_wg - 1) / jobs_per_wg;
    const int64_t n1 = static_cast<int64_t>(gx1) * mc;
    // (eight chunks: four wavefronts of two per job)
    const int wv2 = (w2 == 8) ? 4 : w2;
    const int n_jobs2 = sdn->n_rows / 16, gx2 = (n_jobs2 + 4 / wv2 - 1) / (4 / wv2);
    const int64_t n2 = static_cast<int64_t>(gx2) * ((sdn->dense_rows + kSmallMTile - 1) / kSmallMTile);
    const dim3 g(static_cast<unsigned>(n1 + n2));
#define QMOE_RSD(D, W2_, CPW2_)                                                                  \
  qmm_route_gate_up_shdown_kernel<W, 1, VPL, D, W2_, CPW2_><<<g, 256, 0, stream>>>(a, n_jobs, R, gx1, n1, \
                                                                                 *sdn, n_jobs2, gx2)
    // (one chunk per job, W = 1, means fewer than 8 superblocks: never the deep form)
    if constexpr (W > 1) {
      if (a.K / 128 == 8 * W) {
        if (w2 == 8) QMOE_RSD(8, 4, 2); else if (w2 == 4) QMOE_RSD(8, 4, 1); else QMOE_RSD(8, 2, 1);
        return;
      }
    }
    if (w2 == 8) QMOE_RSD(0, 4, 2); else if (w2 == 4) QMOE_RSD(0, 4, 1); else QMOE_RSD(0, 2, 1);
#undef QMOE_RSD
    return;
  }
  dim3 grid((n_jobs + jobs_per_wg - 1) / jobs_per_wg, static_cast<unsigned>(mc));
  // every weight load of a wavefront's chunk in flight at once when the chunk is 8 superblocks
  if constexpr (W > 1) {
    if (a.K / 128 == 8 * W) {
      qmm_route_gate_up_kernel<W, 1, VPL, 8><<<grid, 64 * WAVES, 0, stream>>>(a, n_jobs, R);
      return;
    }
  }
  qmm_route_gate_up_kernel<W, 1, VPL, 0><<<grid, 64 * WAVES, 0, stream>>>(a, n_jobs, R);
}
template <int W>
static void launch_route_w(const QmmArgs& a, int64_t mc, const SlotRoute& R, int vpl, hipStream_t stream,
                           const QmmArgs* sdn, int w2) {
  switch (vpl) {
    case 1: launch_route_k<W, 1>(a, mc, R, stream, sdn, w2); break;
    case 2: launch_route_k<W, 2>(a, mc, R, stream, sdn, w2); break;
    case 4: launch_route_k<W, 4>(a, mc, R, stream, sdn, w2); break;
    default: launch_route_k<W, 8>(a, mc, R, stream, sdn, w2); break;
  }
}

bool route_gate_up_fits(int E, int k) { return E <= 512 && k <= 64; }

int64_t route_gate_up_workgroups(int K, int n_rows, int64_t mc) {
  const int nsb = K / 128;
  const int W = (nsb >= 32) ? 4 : (nsb >= 8) ? 2 : 1;   // launch_route_gate_up's chunking
  const int jobs_per_wg = 4 / W, n_jobs = n_rows / 32;
  return static_cast<int64_t>((n_jobs + jobs_per_wg - 1) / jobs_per_wg) * mc;
}

int launch_route_gate_up(const QmmArgs& a, int N, const float* logits, int ld, const float* bias,
                         int E, int k, int scoring, int n_group, int topk_group, int norm_topk,
                         float scale, int has_sg, int32_t* idx, float* w, float* sg,
                         int32_t* tile_map, int64_t max_tiles, int32_t* sorted, int32_t* inv,
                         hipStream_t stream, const QmmArgs* sdn) {
  const int64_t mc = static_cast<int64_t>(N) * k;
  if (!route_gate_up_fits(E, k) || a.K % 128 || a.n_rows % 32 || mc <= 0 || mc > 65535 ||
      max_tiles < mc || max_tiles > (int64_t(1) << 30) || a.slot_of || a.offsets)
    return fail("qmm(route): outside the slot-major routed gate_up");
  SlotRoute R{logits, ld, topk_params(bias, E, k, scoring, n_group, topk_group, norm_topk, scale, has_sg),
              idx, w, sg, reinterpret_cast<int4*>(tile_map), static_cast<int>(max_tiles), sorted, inv,
              static_cast<int>(mc), 1};
  const int nsb = a.K / 128;
  const int ch = (nsb >= 32) ? 4 : (nsb >= 8) ? 2 : 1;   // the int4 chunk rule of launch_qmm
  const int vpl = topk_vpl(E);
  int w2 = 0;
  if (sdn) {
    if (sdn->K % 64 || sdn->n_rows % 16 || !sdn->sb || sdn->offsets || sdn->tile_map ||
        sdn->dense_rows <= 0)
      return fail("qmm(route): the shared down is one dense int8 segment");
    w2 = bf16_chunks(sdn->K);
    // one m-tile per wavefront below kSmallMt2MinTiles m-tiles, as its own launch would run it
    if ((w2 != 2 && w2 != 4 && w2 != 8) ||
        (sdn->dense_rows + kSmallMTile - 1) / kSmallMTile >= kSmallMt2MinTiles)
      return 1;   // no compiled combination: the caller launches the shared down apart
  }
  if (ch == 4) launch_route_w<4>(a, mc, R, vpl, stream, sdn, w2);
  else if (ch == 2) launch_route_w<2>(a, mc, R, vpl, stream, sdn, w2);
  else launch_route_w<1>(a, mc, R, vpl, stream, sdn, w2);
  return check_launch("qmm(route)");
}

// SPLIT: the second product's gate and up tiles as jobs of their own with the bf16 epilogue, the
// [gate | up] rows for a consumer that forms the gated activation (the decode dataflow launch's
// H unit): twice the workgroups, each with one tile's dequant, for the launches whose time this
// product sets.
template <int W, int FMT2, bool TAIL = false, bool SPLIT = false>
static void launch_pair_w(const QmmArgs& a1, const QmmArgs& a2, int64_t mtiles, hipStream_t stream,
                          RouteTail T = RouteTail{}) {
  constexpr int WAVES = W > 4 ? W : 4;
  constexpr int JPWG = WAVES / W;
  constexpr int EPI2 = SPLIT ? EPI_BF16 : EPI_SWIGLU;
  // fp32 epilogue jobs; SwiGLU jobs (a gate and an up tile) or, split, single tiles
  const int n1 = a1.n_rows / 16, n2 = a2.n_rows / (SPLIT ? 16 : 32);
  const int gx1 = (n1 + JPWG - 1) / JPWG, gx2 = (n2 + JPWG - 1) / JPWG;
  const bool mt2 = mtiles >= kSmallMt2MinTiles;   // two m-tiles per wavefront, as in launch_small_k
  const dim3 g(gx1 + gx2, static_cast<unsigned>(mt2 ? (mtiles + 1) / 2 : mtiles));
  size_t lds = 0;
  if (TAIL) {
    T.total = gx1 * static_cast<int>(g.y);
    lds = route_tail_lds_bytes(T.P.E, T.N, T.P.k);
    // rankers: one token per workgroup (its first wavefront), up to kRouteTailMaxRankers and
    // the router workgroups; c2 at 32 tokens: 294.1 us per layer against 299.5 with one token
    // per wavefront of two rankers (16 wavefronts ranking on one compute unit take about four
    // times as long as one)
    T.rankers = std::min(std::min(T.N, kRouteTailMaxRankers), T.total);
  }
  // (NORM: the norm weights in the same dynamic LDS, used before the tail's)
  if (a1.norm_w) lds = std::max(lds, static_cast<size_t>(a1.K) * 2);
#define QMOE_PAIR(MT, NORM) \
  qmm_small_pair_kernel<EPI_F32, EPI2, W, MT, NORM, FMT2, TAIL><<<g, 64 * WAVES, lds, stream>>>(a1, n1, gx1, a2, n2, T)
  if (a1.norm_w) {
    if (mt2) QMOE_PAIR(2, true); else QMOE_PAIR(1, true);
  } else {
    if (mt2) QMOE_PAIR(2, false); else QMOE_PAIR(1, false);
  }
#undef QMOE_PAIR
}

template <int FMT2, bool SPLIT>
static void launch_pair_f(const QmmArgs& a1, const QmmArgs& a2, int64_t mtiles, hipStream_t stream) {
  switch (bf16_chunks(a1.K)) {
    case 16: launch_pair_w<16, FMT2, false, SPLIT>(a1, a2, mtiles, stream); break;
    case 8: launch_pair_w<8, FMT2, false, SPLIT>(a1, a2, mtiles, stream); break;
    case 4: launch_pair_w<4, FMT2, false, SPLIT>(a1, a2, mtiles, stream); break;
    case 2: launch_pair_w<2, FMT2, false, SPLIT>(a1, a2, mtiles, stream); break;
    default: launch_pair_w<1, FMT2, false, SPLIT>(a1, a2, mtiles, stream); break;
  }
}

bool pair_norm_fusable(int K, int64_t rows) {
  const int W = bf16_chunks(K);
  const int64_t mtiles = (rows + kSmallMTile - 1) / kSmallMTile;
  const bool mt2 = mtiles >= kSmallMt2MinTiles;
  const int nks = K / 32, steps = (nks + W - 1) / W;
  if (K % 32 || W < 4) return false;
  // one load batch per chunk: the norm's sums overlap the first weight loads (c2, 32 tokens:
  // 16.2 us against the plain launch's 11.0); longer chunks only for one or two tokens, where
  // the separate norm launch costs a kernel boundary more than the fused pass does
  return steps <= (mt2 ? 4 : 8) || (rows <= 2 && steps <= 16);
}

int launch_qmm_pair_route(const QmmArgs& a1, const QmmArgs& a2, hipStream_t stream, int fmt2,
                          const RouteTail& tail) {
  if (a1.offsets || a2.offsets || a1.dense_rows != a2.dense_rows || a1.K != a2.K || a1.K % 32 ||
      a1.n_rows % 16 || a2.n_rows % 32 || a1.dense_rows <= 0)
    return fail("qmm pair: two dense products over the same rows and K required");
  if (fmt2 != FMT_BF16 && fmt2 != FMT_INT8) return fail("qmm pair: the second product is bf16 or int8");
  if (fmt2 == FMT_INT8 && (a1.K % 64 || !a2.sb)) return fail("qmm pair: int8 weights need K % 64 == 0 and sb");
  if ((a1.norm_w != nullptr) != (a2.norm_w != nullptr) || a2.norm_out)
    return fail("qmm pair: the fused norm applies to both products; the first writes the rows");
  if (a1.norm_w && !pair_norm_fusable(a1.K, a1.dense_rows))
    return fail("qmm pair: the fused norm needs one job per workgroup and one load batch per chunk");
  const int mc = tail.N * tail.P.k;
  if (tail.N != a1.dense_rows || tail.N > kRouteTailMaxTokens || tail.P.E <= 0 ||
      tail.P.E > kRouteTailMaxExperts || tail.P.k <= 0 || tail.P.k > 64 || tail.P.k > tail.P.E ||
      !tail.ctr || !tail.timeouts || tail.logits != a1.out ||
      tail.ld != a1.ld_out || !tail.counts || !tail.tile_map || tail.words != (tail.N + 31) / 32 ||
      tail.vpl != topk_vpl(tail.P.E) ||
      tail.max_tiles < mtile_upper_bound(mc, tail.P.E, kSmallMTile))
    return fail("qmm pair (routing tail): bad routing arguments");
  const int64_t mtiles = (a1.dense_rows + kSmallMTile - 1) / kSmallMTile;
#define QMOE_PAIR_T(W)                                                                     \
  if (fmt2 == FMT_INT8) launch_pair_w<W, FMT_INT8, true>(a1, a2, mtiles, stream, tail);     \
  else launch_pair_w<W, FMT_BF16, true>(a1, a2, mtiles, stream, tail);
  switch (bf16_chunks(a1.K)) {
    case 16: QMOE_PAIR_T(16) break;
    case 8: QMOE_PAIR_T(8) break;
    case 4: QMOE_PAIR_T(4) break;
    case 2: QMOE_PAIR_T(2) break;
    default: QMOE_PAIR_T(1) break;
  }
#undef QMOE_PAIR_T
  return check_launch("qmm pair (routing tail)");
}

__device__ uint32_t g_route_timeouts;

uint32_t* route_tail_timeouts_ptr() {
  uint32_t* p = nullptr;
  return hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(g_route_timeouts)) == hipSuccess ? p : nullptr;
}

uint32_t route_tail_timeouts() {
  uint32_t v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_route_timeouts), sizeof(v), 0, hipMemcpyDeviceToHost) != hipSuccess)
    return 0xFFFFFFFFu;
  return v;
}

int launch_qmm_pair_bf16(const QmmArgs& a1, const QmmArgs& a2, hipStream_t stream, int fmt2, bool split) {
  if (a1.offsets || a2.offsets || a1.dense_rows != a2.dense_rows || a1.K != a2.K || a1.K % 32 ||
      a1.n_rows % 16 || a2.n_rows % 32 || a1.dense_rows <= 0)
    return fail("qmm pair: two dense products over the same rows and K required");
  if (fmt2 != FMT_BF16 && fmt2 != FMT_INT8) return fail("qmm pair: the second product is bf16 or int8");
  if (fmt2 == FMT_INT8 && (a1.K % 64 || !a2.sb)) return fail("qmm pair: int8 weights need K % 64 == 0 and sb");
  if ((a1.norm_w != nullptr) != (a2.norm_w != nullptr) || a2.norm_out)
    return fail("qmm pair: the fused norm applies to both products; the first writes the rows");
  if (a1.norm_w && !pair_norm_fusable(a1.K, a1.dense_rows))
    return fail("qmm pair: the fused norm needs one job per workgroup and one load batch per chunk");
  const int64_t mtiles = (a1.dense_rows + kSmallMTile - 1) / kSmallMTile;
  if (mtiles > 65535) return fail("qmm pair: too many m-tiles for one launch");
  if (split && a2.ld_out < a2.n_rows) return fail("qmm pair: split gate_up rows hold both halves");
  if (fmt2 == FMT_INT8) {
    if (split) launch_pair_f<FMT_INT8, true>(a1, a2, mtiles, stream);
    else launch_pair_f<FMT_INT8, false>(a1, a2, mtiles, stream);
  } else {
    if (split) launch_pair_f<FMT_BF16, true>(a1, a2, mtiles, stream);
    else launch_pair_f<FMT_BF16, false>(a1, a2, mtiles, stream);
  }
  return check_launch("qmm pair");
}

template <int W, int CPW, int JPW, int W2, int MT2, int CPW2 = 1>
static int launch_gsd(const QmmArgs& a1, int64_t mtiles1, const QmmArgs& a2, int64_t mtiles2,
                      hipStream_t stream) {
  static_assert(W <= 4 && W2 <= 4, "one 4-wavefront workgroup shape for both products");
  const int n_jobs1 = a1.n_rows / 32 / JPW, gx1 = (n_jobs1 + 4 / W - 1) / (4 / W);
  const int n_jobs2 = a2.n_rows / 16, gx2 = (n_jobs2 + 4 / W2 - 1) / (4 / W2);
  const int64_t n1 = static_cast<int64_t>(gx1) * mtiles1;
  const int64_t n2 = static_cast<int64_t>(gx2) * ((MT2 == 2) ? (mtiles2 + 1) / 2 : mtiles2);
  if (n1 + n2 > 0x7fffffff) return fail("qmm(gate_up + shared down): grid too large");
  qmm_gate_up_shdown_kernel<W, CPW, JPW, W2, MT2, CPW2>
      <<<dim3(static_cast<unsigned>(n1 + n2)), 256, 0, stream>>>(a1, n_jobs1, gx1, n1, a2, n_jobs2, gx2);
  return check_launch("qmm(gate_up + shared down)");
}

int launch_gate_up_shared_down(const QmmArgs& a1, int64_t mtiles1, const QmmArgs& a2,
                               hipStream_t stream) {
  if (a1.K % 128 || a1.n_rows % 32 || !a1.tile_map || mtiles1 <= 0 || mtiles1 > 65535 ||
      a2.K % 64 || a2.n_rows % 16 || !a2.sb || a2.offsets || a2.tile_map || a2.dense_rows <= 0)
    return fail("qmm(gate_up + shared down): routed int4 gate_up and a dense int8 product required");
  const int nsb = a1.K / 128;
  const int ch = (nsb >= 32) ? 4 : (nsb >= 8) ? 2 : 1;   // launch_qmm's int4 chunk rule
  const SmallShape sh = pick_small_shape(FMT_INT4, EPI_SWIGLU, ch, mtiles1, a1.n_rows / 32);
  const int w2 = bf16_chunks(a2.K);
  const int64_t mtiles2 = (a2.dense_rows + kSmallMTile - 1) / kSmallMTile;
  const bool mt2 = mtiles2 >= kSmallMt2MinTiles;   // as launch_small_k for dense products
#define QMOE_GSD(W, CPW, JPW, W2)                                                    \
  if (sh.w == W && sh.cpw == CPW && sh.jpw == JPW && w2 == W2)                        \
    return mt2 ? launch_gsd<W, CPW, JPW, W2, 2>(a1, mtiles1, a2, mtiles2, stream)     \
               : launch_gsd<W, CPW, JPW, W2, 1>(a1, mtiles1, a2, mtiles2, stream);
  // c2-like shapes (H 4096, shared intermediate 1024). With two m-tiles per wavefront the
  // shared down does not fit beside this gate_up shape's registers (c2 N=64 461 vs 445 us), so
  // it runs one m-tile per wavefront there (the same sums: m-tiles are independent)
  if (sh.w == 2 && sh.cpw == 2 && sh.jpw == 2 && w2 == 4)
    return launch_gsd<2, 2, 2, 4, 1>(a1, mtiles1, a2, mtiles2, stream);
  QMOE_GSD(4, 1, 2, 4)
  QMOE_GSD(4, 1, 1, 4)
  QMOE_GSD(2, 1, 1, 2)   // c1-like shapes (H 2048, shared intermediate 512)
  QMOE_GSD(2, 1, 2, 2)
#undef QMOE_GSD
  // c3-like shapes (H 7168, shared intermediate 2048: eight chunks, four wavefronts of two, one
  // m-tile per wavefront)
  if (w2 == 8) {
    if (sh.w == 2 && sh.cpw == 2 && sh.jpw == 2) return launch_gsd<2, 2, 2, 4, 1, 2>(a1, mtiles1, a2, mtiles2, stream);
    if (sh.w == 4 && sh.cpw == 1 && sh.jpw == 2) return launch_gsd<4, 1, 2, 4, 1, 2>(a1, mtiles1, a2, mtiles2, stream);
    if (sh.w == 4 && sh.cpw == 1 && sh.jpw == 1) return launch_gsd<4, 1, 1, 4, 1, 2>(a1, mtiles1, a2, mtiles2, stream);
  }
  return 1;   // no compiled combination: the caller launches the two products apart
}

int launch_qmm(const QmmArgs& a, int fmt, int epi, int regime, int64_t mtile_bound,
               hipStream_t stream) {
  if (a.K <= 0 || a.n_rows <= 0) return fail("qmm: empty problem");
  if (mtile_bound <= 0) return 0;
  if (mtile_bound > 65535) return fail("qmm: too many m-tiles for one launch");
  if (a.expert_map && !fmt_quant(fmt))
    return fail("qmm: an expert map needs int3/int4/int6 weights");
  const bool two_acts = (regime == QMOE_REGIME_SMALL) ? a.act_hi != nullptr : a.act16_hi != nullptr;
  if (two_acts) {
    if (!fmt_quant(fmt) || epi == EPI_SWIGLU || a.slot_of)
      return fail("qmm: a second activation needs quantized weights, a non-SwiGLU epilogue and "
                  "rows by sorted position");
    if (a.split_tile <= 0 || a.split_tile % 4 || a.split_tile >= a.n_rows / 16)
      return fail("qmm: split_tile must be a positive multiple of 4 inside the weight tiles");
    if (regime != QMOE_REGIME_SMALL &&
        (!fmt_quant(fmt) || !a.row_sinv_hi || a.split_tile % 16))
      return fail("qmm(large): a second activation needs int3/int4/int6 weights, its row scales "
                  "and split_tile % 16 == 0");
  }
  if (regime == QMOE_REGIME_SMALL) {
    if (fmt_quant(fmt) && a.K % 128) return fail("qmm: int3/int4/int6 need K % 128 == 0");
    if (fmt == FMT_BF16 && a.K % 32) return fail("qmm: bf16 needs K % 32 == 0");
    if (fmt == FMT_INT8 && (a.K % 64 || !a.sb)) return fail("qmm: int8 needs K % 64 == 0 and sb");
    if (a.n_rows % (epi == EPI_SWIGLU ? 32 : 16)) return fail("qmm: weight rows not a tile multiple");
    // The chunk count depends on the shape only (never on the token count), so a row's
    // summation order, and therefore its result, is the same at every batch size (batch
    // invariance). int3/int4/int6 chunks hold >= 4 superblocks (int3, whose superblocks are
    // 3/4 the bytes of int4's: >= 16 at K = 4096, where two chunks measured faster than four);
    // bf16 (router, shared expert) chunks ~8 32-deep steps, one wavefront each, which spreads
    // the few dense row tiles over enough wavefronts.
    int ch;
    if (fmt_quant(fmt)) {
      const int nsb = a.K / 128;
      ch = (nsb >= (fmt == FMT_INT3 ? 64 : 32)) ? 4 : (nsb >= 8) ? 2 : 1;
    } else {
      ch = bf16_chunks(a.K);
    }
    const int jobs = (epi == EPI_SWIGLU) ? a.n_rows / 32 : a.n_rows / 16;
    const SmallShape sh = pick_small_shape(fmt, epi, ch, mtile_bound, jobs);
#define QMOE_SMALL(F, P) launch_small<F, P>(a, sh, mtile_bound, stream)
    if (fmt == FMT_INT4) {
      if (epi == EPI_SWIGLU) QMOE_SMALL(FMT_INT4, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_SMALL(FMT_INT4, EPI_BF16);
      else QMOE_SMALL(FMT_INT4, EPI_F32);
    } else if (fmt == FMT_INT6) {
      if (epi == EPI_SWIGLU) QMOE_SMALL(FMT_INT6, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_SMALL(FMT_INT6, EPI_BF16);
      else QMOE_SMALL(FMT_INT6, EPI_F32);
    } else if (fmt == FMT_INT3) {
      if (epi == EPI_SWIGLU) QMOE_SMALL(FMT_INT3, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_SMALL(FMT_INT3, EPI_BF16);
      else QMOE_SMALL(FMT_INT3, EPI_F32);
    } else if (fmt == FMT_INT8) {
      if (epi == EPI_SWIGLU) QMOE_SMALL(FMT_INT8, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_SMALL(FMT_INT8, EPI_BF16);
      else QMOE_SMALL(FMT_INT8, EPI_F32);
    } else {
      if (epi == EPI_SWIGLU) QMOE_SMALL(FMT_BF16, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_SMALL(FMT_BF16, EPI_BF16);
      else QMOE_SMALL(FMT_BF16, EPI_F32);
    }
#undef QMOE_SMALL
  } else {
    if (fmt == FMT_INT8)
      return fail("qmm(large): int8 weights run in the small regime only (expand them to bf16 "
                  "for the large kernels)");
    if (a.K % 128) return fail("qmm(large): K % 128 == 0 required");
    if (a.dense_mtile && (a.offsets || a.tile_map || a.dense_mtile % 16 || a.dense_mtile < 16 ||
                          a.dense_mtile > kLargeMTile || fmt != FMT_BF16))
      return fail("qmm(large): dense_mtile is a multiple of 16 up to 128, for one dense bf16 segment");
    if (a.n_rows % 256) return fail("qmm(large): weight rows % 256 == 0 required");
    const bool qf = fmt_quant(fmt);
    if (qf && (!a.act16 || !a.row_sinv))
      return fail("qmm(large): int3/int4/int6 weights need the fp16 activation copy");
    if (qf && !a.row_exp)
      return fail("qmm(large): int3/int4/int6 weights need their row exponents (qmoe_row_exponents)");
    int rc;
#define QMOE_LARGE(F, P) rc = launch_large<F, P>(a, mtile_bound, stream)
    // int4 weights in 512-row blocks (SwiGLU: 256-row gate and up halves; a second activation:
    // blocks on one side of its split) take the wide kernel
    if (fmt == FMT_INT4 && a.n_rows % 512 == 0 && (!two_acts || a.split_tile % 32 == 0)) {
      if (epi == EPI_SWIGLU) rc = launch_wide<FMT_INT4, EPI_SWIGLU>(a, mtile_bound, stream);
      else if (epi == EPI_BF16) rc = launch_wide<FMT_INT4, EPI_BF16>(a, mtile_bound, stream);
      else rc = launch_wide<FMT_INT4, EPI_F32>(a, mtile_bound, stream);
    } else if (fmt == FMT_INT3 && a.n_rows % 512 == 0 && (!two_acts || a.split_tile % 32 == 0)) {
      if (epi == EPI_SWIGLU) rc = launch_wide<FMT_INT3, EPI_SWIGLU>(a, mtile_bound, stream);
      else if (epi == EPI_BF16) rc = launch_wide<FMT_INT3, EPI_BF16>(a, mtile_bound, stream);
      else rc = launch_wide<FMT_INT3, EPI_F32>(a, mtile_bound, stream);
    } else if (fmt == FMT_INT4) {
      if (epi == EPI_SWIGLU) QMOE_LARGE(FMT_INT4, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_LARGE(FMT_INT4, EPI_BF16);
      else QMOE_LARGE(FMT_INT4, EPI_F32);
    } else if (fmt == FMT_INT6) {   // (1.5 KiB superblocks: the 256-row kernel only)
      if (epi == EPI_SWIGLU) QMOE_LARGE(FMT_INT6, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_LARGE(FMT_INT6, EPI_BF16);
      else QMOE_LARGE(FMT_INT6, EPI_F32);
    } else if (fmt == FMT_INT3) {
      if (epi == EPI_SWIGLU) QMOE_LARGE(FMT_INT3, EPI_SWIGLU);
      else if (epi == EPI_BF16) QMOE_LARGE(FMT_INT3, EPI_BF16);
      else QMOE_LARGE(FMT_INT3, EPI_F32);
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
