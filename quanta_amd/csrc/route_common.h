// Device building blocks of the routing stage: the per-token top-k of one wavefront and the
// stable-permute body of one workgroup (kept apart from their kernels so that any kernel
// embedding them computes bit-identical ids, weights and permutations).
//
// Reference: top-k softmax routing src/quanta/qwen35/moe.py:36-56 (softmax over all experts,
// top-k, renorm with +1e-20); sigmoid + correction bias, bias-free weights and
// routed_scaling_factor src/quanta/modeling/moe.py:33-44 and src/quanta/glm/moe.py:44-55; the
// stable permute order = argsort(exp) (stable), inv = argsort(order)
// src/quanta/modeling/moe.py:81-85.
#pragma once

#include <math.h>

#include "qmoe_internal.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

// Wavefront reductions from ROCm's device library (declared by HIP's own headers only under an
// opt-in macro); used by the group-limited selection only.
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_max_u64(
    unsigned long long);

// ---------------------------------------------------------------- wavefront reductions
// Butterfly over each 16-lane row with DPP (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror), then the four row results combined in a fixed order. Every
// step pairs two lanes that combine the same two partial results, so all lanes of a row hold
// bitwise-identical values and the result is the same on every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
// Same butterfly on unsigned integers (0 is max's identity, so the DPP moves fold into the
// max instructions).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u<0xB1>(v));
  v = max(v, dpp_u<0x4E>(v));
  v = max(v, dpp_u<0x141>(v));
  v = max(v, dpp_u<0x140>(v));
  const uint32_t r0 = __builtin_amdgcn_readlane(static_cast<int>(v), 0);
  const uint32_t r1 = __builtin_amdgcn_readlane(static_cast<int>(v), 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(static_cast<int>(v), 32);
  const uint32_t r3 = __builtin_amdgcn_readlane(static_cast<int>(v), 48);
  return max(max(r0, r1), max(r2, r3));
}

// Order-preserving map of a float onto uint32 (larger float -> larger integer).
__device__ __forceinline__ uint32_t orderable(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// Group selection key: value first, then the lower group id wins a tie.
__device__ __forceinline__ unsigned long long sel_key(float v, int id) {
  return (static_cast<unsigned long long>(orderable(v)) << 32) |
         static_cast<unsigned long long>(0xFFFFFFFFu - static_cast<uint32_t>(id));
}
__device__ __forceinline__ int key_id(unsigned long long key) {
  return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key));
}

struct TopkParams {
  const float* bias;   // [E] selection-only correction bias (nullable)
  int E, k, scoring, n_group, topk_group, norm_topk, has_sg;
  float scale;
};

// Top-k of one token's logits row, by one wavefront. Lane l holds experts l*VPL .. l*VPL+VPL-1
// (contiguous, so a group of E/n_group experts spans whole lanes when VPL divides the group
// size). Selection order is canonical: choice value descending, lower expert id first on
// ties (the reference's argpartition returns the same set in an unspecified order). Each lane
// keeps its best remaining candidate (the lowest of its ids among its largest values); a round
// takes the wavefront max of those values and the lowest lane holding it, which owns the
// lowest id of that value (a lane's candidates are taken in id order, and only a strictly
// larger value replaces the current best). Lane r < k returns the r-th expert and its final
// weight.
// IDS_ONLY: lane r < rounds returns the r-th expert and out_w is undefined; the selection is the
// same, and softmax routing without a bias (which selects by logit) then skips the
// probabilities altogether.
// A logit read; COH: an agent-scope (cross-XCD coherent) load, for logits that other
// workgroups of the same launch wrote with coherent stores.
template <bool COH>
__device__ __forceinline__ float logit_ld(const float* p) {
  if constexpr (COH)
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
  else
    return *p;
}

template <int VPL, bool IDS_ONLY = false, bool COH = false>
__device__ __forceinline__ void topk_token(const float* __restrict__ row, const TopkParams& P,
                                           int lane, int& out_id, float& out_w, int rounds = 0) {
  const float NEG_INF = -INFINITY;
  const int E = P.E;
  const int e_base = lane * VPL;
  // Branch-free throughout (per-element predicates become selects, loads are clamped in
  // bounds): the selection is a serial chain on one wavefront, so branches would dominate it.
  float lg[VPL], sc[VPL], ch[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const float v = logit_ld<COH>(row + min(e_base + i, E - 1));
    lg[i] = (e_base + i < E) ? v : NEG_INF;
  }
  const bool by_logit = (P.scoring == QMOE_SCORE_SOFTMAX);
  if (IDS_ONLY && by_logit && !P.bias) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) sc[i] = 0.f;
  } else if (P.scoring == QMOE_SCORE_SOFTMAX) {
    float m = NEG_INF;
#pragma unroll
    for (int i = 0; i < VPL; ++i) m = fmaxf(m, lg[i]);
    m = wave_max_f32(m);
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      sc[i] = (e_base + i < E) ? expf(lg[i] - m) : 0.f;
      z += sc[i];
    }
    z = wave_sum_f32(z);
    const float inv = 1.0f / z;
#pragma unroll
    for (int i = 0; i < VPL; ++i) sc[i] *= inv;
  } else if (P.scoring == QMOE_SCORE_SIGMOID) {
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      sc[i] = (e_base + i < E) ? 1.0f / (1.0f + expf(-lg[i])) : 0.f;
  } else {   // sqrt(softplus), softplus(l) = log(1 + e^l) = max(l, 0) + log1p(e^-|l|)
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      sc[i] = (e_base + i < E) ? sqrtf(fmaxf(lg[i], 0.f) + log1pf(expf(-fabsf(lg[i])))) : 0.f;
  }
  // Without a bias, softmax selection by probability equals selection by logit (monotone); the
  // logit avoids ties manufactured by rounding exp(). Sigmoid and sqrt-softplus select on the
  // score, as the reference does.
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = e_base + i;
    float c = by_logit ? lg[i] : sc[i];
    if (P.bias) c = sc[i] + P.bias[min(e, E - 1)];
    c = (e < E) ? c : NEG_INF;
    ch[i] = (c != c) ? NEG_INF : c;   // a NaN never outranks a number
  }

  if (P.n_group > 1) {
    const int gsize = E / P.n_group;
    // group score = sum of the group's two largest choice values; gkey holds one selection key
    // per group (on the lane holding the group's first expert, or on lane gamma in the generic
    // path), 0 elsewhere
    unsigned long long gkey = 0ull;
    if (gsize % VPL == 0) {
      const int lanes_per_group = gsize / VPL;   // a power of two for power-of-two E, n_group
      float b1 = NEG_INF, b2 = NEG_INF;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const float v = ch[i];
        if (v > b1) { b2 = b1; b1 = v; } else if (v > b2) { b2 = v; }
      }
      for (int off = 1; off < lanes_per_group; off <<= 1) {
        const float o1 = __shfl_xor(b1, off), o2 = __shfl_xor(b2, off);
        const float n2 = fmaxf(fminf(b1, o1), fmaxf(b2, o2));
        b1 = fmaxf(b1, o1);
        b2 = n2;
      }
      if (e_base < E && e_base % gsize == 0) gkey = sel_key(b1 + b2, e_base / gsize);
    } else {
      for (int gam = 0; gam < P.n_group; ++gam) {
        float b1 = NEG_INF, b2 = NEG_INF;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          const int e = e_base + i;
          if (e < E && e / gsize == gam) {
            const float v = ch[i];
            if (v > b1) { b2 = b1; b1 = v; } else if (v > b2) { b2 = v; }
          }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
          const float o1 = __shfl_xor(b1, off), o2 = __shfl_xor(b2, off);
          const float n2 = fmaxf(fminf(b1, o1), fmaxf(b2, o2));
          b1 = fmaxf(b1, o1);
          b2 = n2;
        }
        if (lane == gam) gkey = sel_key(b1 + b2, gam);
      }
    }
    unsigned long long keep = 0ull;
    for (int r = 0; r < P.topk_group; ++r) {
      const unsigned long long best = __ockl_wfred_max_u64(gkey);
      keep |= 1ull << key_id(best);
      if (gkey == best) gkey = 0ull;   // keys are unique (they embed the group id)
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = e_base + i;
      if (e < E && !((keep >> (e / gsize)) & 1ull)) ch[i] = NEG_INF;
    }
  }

  // Selection runs on order-preserving integer keys of the choice values (-0 folded into +0,
  // which compare equal); every real key is above 0, the "no candidate" value.
  uint32_t key[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) key[i] = orderable(ch[i] + 0.0f);
  // remaining candidates of this lane (bit i = expert e_base + i)
  uint32_t avail = 0u;
#pragma unroll
  for (int i = 0; i < VPL; ++i)
    if (e_base + i < E) avail |= 1u << i;
  int my_id = 0;
  float my_w = 0.f;
  const int n_rounds = (IDS_ONLY && rounds > 0) ? min(rounds, P.k) : P.k;
  // Two forms of the same selection. Rescan: a round's owner rescans its remaining candidates
  // after the wavefront reduction. Two heads: each lane also holds its next best candidate,
  // recomputed at the start of every round beside the reduction, and the owner promotes it.
  // Same choices in the same order; measured per use (300-step loops, same box): the two-head
  // form is faster with four or fewer experts per lane and in the routing tail's rankers (c2
  // 8-32 tokens and c1 1-8 tokens by 0.4-0.7 us per call), the rescan form in the dataflow
  // launch's units with eight (c2 one token, 0.6 us).
  constexpr bool kTwoHead = COH || VPL <= 4;
  if constexpr (kTwoHead) {
    // Best candidate of a mask: a pairwise tree in index order where the right operand wins
    // only with a strictly larger key, so equal keys keep the lowest index; key 0 = none.
    auto best = [&](uint32_t mask, uint32_t& bk, int& bi, float& bs) __attribute__((always_inline)) {
      uint32_t tk[VPL];
      int ti[VPL];
      float ts[VPL];
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        tk[i] = ((mask >> i) & 1u) ? key[i] : 0u;
        ti[i] = i;
        ts[i] = sc[i];
      }
      auto pick = [&](int i, int j) __attribute__((always_inline)) {
        const bool tb = tk[j] > tk[i];
        tk[i] = tb ? tk[j] : tk[i];
        ti[i] = tb ? ti[j] : ti[i];
        ts[i] = tb ? ts[j] : ts[i];
      };
      // (one loop per level, each with a constant stride, so every index is static)
#pragma unroll
      for (int i = 0; i + 1 < VPL; i += 2) pick(i, i + 1);
#pragma unroll
      for (int i = 0; i + 2 < VPL; i += 4) pick(i, i + 2);
#pragma unroll
      for (int i = 0; i + 4 < VPL; i += 8) pick(i, i + 4);
#pragma unroll
      for (int i = 0; i + 8 < VPL; i += 16) pick(i, i + 8);
      static_assert(VPL <= 16, "experts per lane");
      bk = tk[0];
      bi = ti[0];
      bs = ts[0];
    };
    uint32_t hk;
    float hs;
    int hi;
    best(avail, hk, hi, hs);
    for (int r = 0; r < n_rounds; ++r) {
      uint32_t k2;
      float s2;
      int i2;
      best(avail & ~(1u << (hi & 31)), k2, i2, s2);
      const uint32_t m = wave_max_u32(hk);
      unsigned long long win = __ballot((hk > 0u) & (hk == m));
      win = win ? win : __ballot(hk > 0u);   // the fallback is unreachable while k <= E
      const int owner = static_cast<int>(__builtin_ctzll(win));
      const int id = __builtin_amdgcn_readlane(e_base + hi, owner);
      const float s_win = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hs), owner));
      // the owner drops its winner and takes its next candidate
      const bool own = lane == owner;
      avail = own ? (avail & ~(1u << (hi & 31))) : avail;
      hk = own ? k2 : hk;
      hi = own ? i2 : hi;
      hs = own ? s2 : hs;
      my_id = (lane == r) ? id : my_id;
      my_w = (lane == r) ? s_win : my_w;
    }
  } else {
    uint32_t hk = 0u;
    float hs = 0.f;
    int hi = -1;
    auto head = [&]() __attribute__((always_inline)) {
      hk = 0u;
      hi = -1;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const bool take = ((avail >> i) & 1u) & (key[i] > hk);
        hk = take ? key[i] : hk;
        hs = take ? sc[i] : hs;
        hi = take ? i : hi;
      }
    };
    head();
    for (int r = 0; r < n_rounds; ++r) {
      const uint32_t m = wave_max_u32(hk);
      unsigned long long win = __ballot((hi >= 0) & (hk == m));
      win = win ? win : __ballot(hi >= 0);   // the fallback is unreachable while k <= E
      const int owner = static_cast<int>(__builtin_ctzll(win));
      const int id = __builtin_amdgcn_readlane(e_base + hi, owner);
      const float s_win = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hs), owner));
      // the owner drops its winner and recomputes its best remaining candidate
      avail = (lane == owner) ? (avail & ~(1u << (hi & 31))) : avail;
      head();
      my_id = (lane == r) ? id : my_id;
      my_w = (lane == r) ? s_win : my_w;
    }
  }
  if (IDS_ONLY) {
    out_id = my_id;
    out_w = 0.f;
    return;
  }
  const float tot = wave_sum_f32(lane < P.k ? my_w : 0.f);
  // QMOE_NORM_ALWAYS, or QMOE_NORM_MULTI with more than one expert (a MoEGate keeps a single
  // expert's score as it is)
  if (P.norm_topk == 1 || (P.norm_topk == 2 && P.k > 1)) my_w = my_w / (tot + 1e-20f);
  out_id = my_id;
  out_w = my_w * P.scale;
}

// The routing tail of the router pair launch, for decode batches routed through the stable
// permute: the router workgroups store their logits with coherent stores and count their
// arrival; the last R to arrive rank the tokens (coherent loads of the logits; all but the last
// arrival first wait, bounded, for the count to complete), and the last ranker to finish runs
// the permute, in place of the top-k and permute launches. Each counter is a 64-bit workspace
// word holding (kRouteTailTag << 20) | count, counted with atomic adds; a workgroup that finds a
// word without the tag (a fresh workspace) replaces it by a tagged count, so the words need no
// clearing, and the last ranker resets both to a tagged 0 for the next call (or the next replay
// of a capture).
constexpr unsigned long long kRouteTailTag = 0xA5C3E1F7B9Dull;   // 44 bits
struct RouteTail {
  unsigned long long* ctr;    // two words: router workgroups arrived, rankers done
  uint32_t* timeouts;         // waits that ran out of their bound
  int total;                  // router workgroups of the launch
  int rankers;                // the last `rankers` arrivals rank the tokens (the launcher's choice)
  const float* logits;
  int ld;
  TopkParams P;
  int N;
  int32_t* idx;
  float* w;
  float* sg;
  int32_t* counts;
  int32_t* offsets;
  int32_t* tile_off;
  int32_t* sorted;
  int32_t* inv;
  int32_t* tile_map;
  int max_tiles;
  int words;                  // token bitmap words per expert, (N + 31) / 32
  int vpl;                    // experts per lane of the top-k wavefront (topk_vpl)
};
constexpr int kRouteTailMaxTokens = 64, kRouteTailMaxExperts = 512, kRouteTailMaxRankers = 32;
uint32_t* route_tail_timeouts_ptr();   // device address of the tail's timeout counter
uint32_t route_tail_timeouts();        // its value (synchronous)
// dynamic LDS of the tail: a 64-bit token mask, a count and an offset per expert, scan scratch
// and the ids of the N * k slots
inline size_t route_tail_lds_bytes(int E, int N, int k) {
  return 16 * static_cast<size_t>(E) + sizeof(int) * (34 + static_cast<size_t>(N) * k);
}
// The router pair launch (launch_qmm_pair_bf16) with the routing tail.
int launch_qmm_pair_route(const QmmArgs& a1, const QmmArgs& a2, hipStream_t stream, int fmt2,
                          const RouteTail& tail);

inline TopkParams topk_params(const float* bias, int E, int k, int scoring, int n_group,
                              int topk_group, int norm_topk, float scale, int has_sg) {
  TopkParams P;
  P.bias = bias;
  P.E = E;
  P.k = k;
  P.scoring = scoring;
  P.n_group = n_group;
  P.topk_group = topk_group;
  P.norm_topk = norm_topk;
  P.has_sg = has_sg;
  P.scale = scale;
  return P;
}

// Experts per lane of the top-k wavefront for E experts.
inline int topk_vpl(int E) {
  return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
}

// Top-k of token t by one wavefront, stored as idx/w rows of k and the shared-expert gate
// sigmoid(logit E); returns lane r's expert (r < k).
template <int VPL, bool COH = false>
__device__ __forceinline__ int topk_store(const float* __restrict__ logits, int ld,
                                           const TopkParams& P, int t, int lane,
                                           int32_t* __restrict__ idx_out,
                                           float* __restrict__ w_out, float* __restrict__ sg_out) {
  const float* row = logits + static_cast<int64_t>(t) * ld;
  int id;
  float w;
  topk_token<VPL, false, COH>(row, P, lane, id, w);
  if (lane < P.k) {
    idx_out[static_cast<int64_t>(t) * P.k + lane] = id;
    w_out[static_cast<int64_t>(t) * P.k + lane] = w;
  }
  if (P.has_sg && lane == 0) sg_out[t] = 1.0f / (1.0f + expf(-logit_ld<COH>(row + P.E)));
  return id;
}

// ---------------------------------------------------------------- stable permute body
// Stable permute of the (token, slot) list by expert: histogram, exclusive scans and scatter in
// LDS, with the stable rank taken from a per-expert token bitmap, so the result equals a stable
// argsort without ordered atomics. Stable rank of slot m = t*k + s routed to expert e = the
// number of earlier slots with the same expert; top-k routing selects distinct experts per
// token, so that equals the number of tokens t' < t that chose e: popcount of e's token bitmap
// below bit t. The workgroup owns experts [e0, e1) (their bitmaps in LDS), recomputes the full
// histogram for the offsets, and scatters only its own experts' slots. Workgroup 0 (is_first)
// writes counts, offsets, the m-tile prefix and the tile descriptors.
struct PermuteLds {
  int* hist;        // [1024]
  int* offs;        // [1025]
  int* scan_tmp;    // [40]
  uint32_t* bits;   // [(e1 - e0) * words_per_expert]
  uint32_t* pref;   // same size
  int* toffs;       // [1025] m-tile prefix per expert (the first workgroup's tile map)
  int* btoffs;      // [1025] the big-tile map's prefix (hybrid split)
};

// Exclusive scan across a 1024-thread workgroup (16 wavefronts of 64).
__device__ __forceinline__ int block_exclusive_scan(int v, int* warp_sums, int* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == 63) warp_sums[wid] = incl;
  __syncthreads();
  if (wid == 0) {
    int s = (lane < 16) ? warp_sums[lane] : 0;
    int si = s;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      int o = __shfl_up(si, off);
      if (lane >= off) si += o;
    }
    if (lane < 16) warp_sums[16 + lane] = si - s;   // exclusive prefix of wave totals
    if (lane == 15) *total = si;
  }
  __syncthreads();
  return warp_sums[16 + wid] + incl - v;
}

constexpr int kPermBatch = 8;   // expert ids loaded per thread before they are used

// Tile t's entry of a tile map whose expert m-tile prefix is toffs[0..E] (toffs[E] = tiles):
// the expert e with toffs[e] <= t < toffs[e + 1] (binary search; experts without tiles repeat
// the prefix and are never found), its i-th tile {e, first sorted position, rows, 0}.
__device__ __forceinline__ int4 tile_entry(const int* toffs, const int* offs, const int* hist, int E,
                                           int t, int m_tile) {
  int lo = 0, hi = E;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (toffs[mid] <= t) lo = mid; else hi = mid;
  }
  const int i = t - toffs[lo];
  return make_int4(lo, offs[lo] + i * m_tile, min(m_tile, hist[lo] - i * m_tile), 0);
}

// Optional split tile maps (hybrid regime): experts with more than `split_rows` rows get
// m-tiles of `m_tile_big` rows in tile_map_big; the others keep m_tile-row tiles in tile_map.
// RES > 0: every expert id is loaded once (RES per thread, all in flight together) and kept in
// registers for the scatter (lists of up to RES * 1024 slots); RES = 0: batches of kPermBatch,
// loaded again for the scatter.
// Must be called by all 1024 threads of the workgroup.
template <int RES>
__device__ __forceinline__ void permute_body(
    const int32_t* idx, int N, int k, int E, int m_tile, int e0, int e1, int words_per_expert,
    bool is_first, const PermuteLds& S, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ tile_off,
    int32_t* __restrict__ sorted_slot, int32_t* __restrict__ inv, int4* __restrict__ tile_map,
    int max_tiles, int split_rows, int m_tile_big, int4* __restrict__ tile_map_big,
    int max_tiles_big) {
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int mc = N * k;
  const int nbits = (e1 - e0) * words_per_expert;
  int* hist = S.hist;
  int* offs = S.offs;
  int* scan_tmp = S.scan_tmp;
  uint32_t* bits = S.bits;
  uint32_t* pref = S.pref;

  for (int i = tid; i < 1024; i += nthr) hist[i] = 0;
  for (int i = tid; i < nbits; i += nthr) bits[i] = 0u;
  __syncthreads();

  auto count_slot = [&](int m, int e) __attribute__((always_inline)) {
    if (e < 0 || e >= E) return;
    atomicAdd(&hist[e], 1);
    if (e >= e0 && e < e1) {
      const int t = m / k;
      atomicOr(&bits[(e - e0) * words_per_expert + (t >> 5)], 1u << (t & 31));
    }
  };
  int evr[RES > 0 ? RES : 1];   // RES: slot tid + j * nthr's expert (-1 past the list)
  if constexpr (RES > 0) {
#pragma unroll
    for (int j = 0; j < RES; ++j) {
      const int m = tid + j * nthr;
      const int v = idx[min(m, mc - 1)];
      evr[j] = (m < mc) ? v : -1;
    }
#pragma unroll
    for (int j = 0; j < RES; ++j) {
      const int m = tid + j * nthr;
      if (m < mc) count_slot(m, evr[j]);
    }
  } else {
    // (the expert ids are read kPermBatch per thread before any is used, so a long list costs
    // one global-load latency per batch rather than one per entry)
    for (int mb = tid; mb < mc; mb += kPermBatch * nthr) {
      int ev[kPermBatch];
#pragma unroll
      for (int j = 0; j < kPermBatch; ++j) {
        const int m = mb + j * nthr;
        ev[j] = (m < mc) ? idx[m] : -1;
      }
#pragma unroll
      for (int j = 0; j < kPermBatch; ++j) {
        const int m = mb + j * nthr;
        if (m < mc) count_slot(m, ev[j]);
      }
    }
  }
  __syncthreads();

  // Offsets (exclusive scan of counts) and the m-tile prefix.
  const int c = (tid < E) ? hist[tid] : 0;
  const int ex = block_exclusive_scan(c, scan_tmp, &scan_tmp[39]);
  const int total = scan_tmp[39];
  if (tid < E) offs[tid] = ex;
  if (tid == 0) offs[E] = total;
  __syncthreads();
  const int tiles = (c + m_tile - 1) / m_tile;
  const int tex = block_exclusive_scan(tiles, scan_tmp, &scan_tmp[38]);
  // hybrid split: small-tile map over the experts at or below split_rows, big-tile map over
  // the rest (block-uniform condition: tile_map_big is a kernel argument)
  int s_tiles = tiles, s_ex = tex, s_total = 0, b_tiles = 0, b_ex = 0, b_total = 0;
  if (tile_map_big) {
    const bool big = c > split_rows;
    s_tiles = big ? 0 : tiles;
    b_tiles = big ? (c + m_tile_big - 1) / m_tile_big : 0;
    s_ex = block_exclusive_scan(s_tiles, scan_tmp, &scan_tmp[37]);
    s_total = scan_tmp[37];
    b_ex = block_exclusive_scan(b_tiles, scan_tmp, &scan_tmp[36]);
    b_total = scan_tmp[36];
  }
  if (is_first) {
    if (tid < E) {
      counts[tid] = c;
      offsets[tid] = ex;
      tile_off[tid] = tex;
    }
    if (tid == 0) {
      offsets[E] = total;
      tile_off[E] = scan_tmp[38];
    }
    // Per-tile descriptors {expert, first sorted position, rows, 0} for the grouped-qmm grid,
    // and a -1 sentinel in every unused entry up to max_tiles, so a workgroup resolves its tile
    // with one 16-byte load. One thread per tile (a hot expert's hundreds of tiles would
    // otherwise be one thread's serial stores), its expert found in the tile prefix in LDS.
    if (tile_map && !tile_map_big) {
      const int nt = scan_tmp[38];
      if (tid < E) S.toffs[tid] = tex;
      if (tid == 0) S.toffs[E] = nt;
      __syncthreads();
      for (int t = tid; t < max_tiles; t += nthr)
        tile_map[t] = (t < nt) ? tile_entry(S.toffs, offs, hist, E, t, m_tile) : make_int4(-1, 0, 0, 0);
    }
    if (tile_map_big) {
      if (tid < E) {
        S.toffs[tid] = s_ex;
        S.btoffs[tid] = b_ex;
      }
      if (tid == 0) {
        S.toffs[E] = s_total;
        S.btoffs[E] = b_total;
      }
      __syncthreads();
      for (int t = tid; t < max_tiles; t += nthr)
        tile_map[t] = (t < s_total) ? tile_entry(S.toffs, offs, hist, E, t, m_tile) : make_int4(-1, 0, 0, 0);
      for (int t = tid; t < max_tiles_big; t += nthr)
        tile_map_big[t] =
            (t < b_total) ? tile_entry(S.btoffs, offs, hist, E, t, m_tile_big) : make_int4(-1, 0, 0, 0);
    }
  }

  // Per-expert exclusive popcount prefix over the token bitmap words: one thread per expert
  // for a few words; for long bitmaps 16 lanes per expert, each over a run of words, with the
  // run totals scanned across the 16 lanes.
  for (int i = tid; i < nbits; i += nthr) pref[i] = __popc(bits[i]);
  __syncthreads();
  if (words_per_expert <= 4) {
    for (int el = tid; el < e1 - e0; el += nthr) {
      uint32_t run = 0;
      uint32_t* p = pref + el * words_per_expert;
      for (int w = 0; w < words_per_expert; ++w) {
        const uint32_t v = p[w];
        p[w] = run;
        run += v;
      }
    }
  } else {
    const int l16 = tid & 15;
    const int per = (words_per_expert + 15) / 16;
    const int w0 = min(l16 * per, words_per_expert), w1 = min(w0 + per, words_per_expert);
    // the 16 lanes of a group share el, so the shuffles stay within active lanes
    for (int el = tid >> 4; el < e1 - e0; el += nthr >> 4) {
      uint32_t* p = pref + el * words_per_expert;
      uint32_t sum = 0;
      for (int w = w0; w < w1; ++w) sum += p[w];
      uint32_t incl = sum;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off, 16);
        if (l16 >= off) incl += o;
      }
      uint32_t run = incl - sum;
      for (int w = w0; w < w1; ++w) {
        const uint32_t v = p[w];
        p[w] = run;
        run += v;
      }
    }
  }
  // Own output segment starts as -1 so a malformed idx (duplicate experts within a token)
  // leaves detectable holes instead of stale data.
  if (e1 > e0)
    for (int p = offs[e0] + tid; p < offs[e1]; p += nthr) sorted_slot[p] = -1;
  __syncthreads();

  auto place_slot = [&](int m, int e) __attribute__((always_inline)) {
    if (e < 0 || e >= E) {
      if (is_first) inv[m] = -1;
      return;
    }
    if (e < e0 || e >= e1) return;
    const int t = m / k;
    const int wi = (e - e0) * words_per_expert + (t >> 5);
    const uint32_t below = bits[wi] & ((1u << (t & 31)) - 1u);
    const int pos = offs[e] + static_cast<int>(pref[wi]) + __popc(below);
    sorted_slot[pos] = m;
    inv[m] = pos;
  };
  if constexpr (RES > 0) {
#pragma unroll
    for (int j = 0; j < RES; ++j) {
      const int m = tid + j * nthr;
      if (m < mc) place_slot(m, evr[j]);
    }
  } else {
    for (int mb = tid; mb < mc; mb += kPermBatch * nthr) {
      int ev[kPermBatch];
#pragma unroll
      for (int j = 0; j < kPermBatch; ++j) {
        const int m = mb + j * nthr;
        ev[j] = (m < mc) ? idx[m] : E;
      }
#pragma unroll
      for (int j = 0; j < kPermBatch; ++j) {
        const int m = mb + j * nthr;
        if (m < mc) place_slot(m, ev[j]);
      }
    }
  }
}

}  // namespace qmoe
