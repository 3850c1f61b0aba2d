// Unpermute + weighted combine + gated shared expert + bf16 cast, and the C-ABI entry points
// for the grouped qmm and the whole-block forward.
//
// Reference: routed[t] = sum_s f32(d[t, s]) * w[t, s] (src/quanta/qwen35/moe.py:191; the sorted
// variant restores slot order with d[inv] first, src/quanta/modeling/moe.py:94-97);
// y = bf16(routed + f32(shared_out) * sigmoid(x . g)) (src/quanta/qwen35/moe.py:145-151,201-202).
// The combine gathers each slot's row through inv (no atomics), summing in slot order, so the
// output is deterministic.
#include <math.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <map>
#include <mutex>
#include <string>

#include "qmoe_internal.h"
#include "flow.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(const std::string& msg) {
  set_error(msg);
  return QMOE_EINVAL;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(err));
    return QMOE_EHIP;
  }
  return QMOE_OK;
}

// One 64-thread workgroup per (token, 512 features): the k slot rows are gathered through inv
// with their loads issued together (8 at a time), then summed in slot order.
// With resid (the block entry that carries the decoder layer's residual add), the bf16 block
// output is added to the residual row and rounded again: y = bf16(resid + bf16(moe)), the
// reference's bf16 `x + mlp(...)`; y may then alias resid (each element is read and written by
// the same thread).
__device__ __forceinline__ uint32_t add_resid(uint32_t packed_moe, uint32_t r) {
  return pack_bf16x2(bf16lo_to_f32(r) + bf16lo_to_f32(packed_moe),
                     bf16hi_to_f32(r) + bf16hi_to_f32(packed_moe));
}

__global__ void __launch_bounds__(64) combine_kernel(
    const uint16_t* __restrict__ d, const int32_t* __restrict__ inv, const float* __restrict__ w,
    int N, int k, int H, int64_t n_pos, const uint16_t* __restrict__ shared_out,
    const float* __restrict__ shared_gate, const uint16_t* resid, uint16_t* y) {
  const int t = blockIdx.y;
  const int h8 = (blockIdx.x * 64 + threadIdx.x) * 8;
  if (h8 >= H) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int64_t m0 = static_cast<int64_t>(t) * k;
  for (int s0 = 0; s0 < k; s0 += 8) {
    u32x4 v[8];
    float ws[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ws[j] = 0.f;
      v[j] = u32x4{0u, 0u, 0u, 0u};
      if (s0 + j < k) {
        const int pos = inv[m0 + s0 + j];
        if (pos >= 0 && pos < n_pos) {
          ws[j] = w[m0 + s0 + j];
          v[j] = *reinterpret_cast<const u32x4*>(d + static_cast<int64_t>(pos) * H + h8);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] += bf16lo_to_f32(v[j][q]) * ws[j];
        acc[2 * q + 1] += bf16hi_to_f32(v[j][q]) * ws[j];
      }
    }
  }
  if (shared_out) {
    const float g = shared_gate ? shared_gate[t] : 1.0f;
    const u32x4 v = *reinterpret_cast<const u32x4*>(shared_out + static_cast<int64_t>(t) * H + h8);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += bf16lo_to_f32(v[q]) * g;
      acc[2 * q + 1] += bf16hi_to_f32(v[q]) * g;
    }
  }
  u32x4 o;
  o[0] = pack_bf16x2(acc[0], acc[1]);
  o[1] = pack_bf16x2(acc[2], acc[3]);
  o[2] = pack_bf16x2(acc[4], acc[5]);
  o[3] = pack_bf16x2(acc[6], acc[7]);
  if (resid) {
    const u32x4 r = *reinterpret_cast<const u32x4*>(resid + static_cast<int64_t>(t) * H + h8);
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = add_resid(o[q], r[q]);
  }
  *reinterpret_cast<u32x4*>(y + static_cast<int64_t>(t) * H + h8) = o;
}

int launch_combine(const uint16_t* d, const int32_t* inv, const float* w, int N, int k, int H,
                   const uint16_t* shared_out, const float* shared_gate, uint16_t* y,
                   hipStream_t stream, const uint16_t* resid) {
  dim3 grid((H + 511) / 512, N);
  combine_kernel<<<grid, 64, 0, stream>>>(d, inv, w, N, k, H, static_cast<int64_t>(N) * k,
                                          shared_out, shared_gate, resid, y);
  return check_launch("combine");
}

// ------------------------------------------------------------------ combine + shared down
// Decode form of the combine with the shared expert's down projection fused in. A workgroup
// owns 16 output features f and a block of 16*MT tokens (MT m-tiles, each weight fragment
// feeding MT MFMAs):
//   sh[t, f] = bf16(sh_h[t] . Wd[f])                      (the reference's bf16 matmul output)
//   y[t, f]  = bf16(sum_s w[t,s] * f32(d[inv[t,s], f]) + g[t] * f32(sh[t, f]))
// sh is computed on v_mfma_f32_16x16x32_bf16 (16 tokens x 16 features per m-tile) with K cut
// into the same chunks as the standalone small-regime bf16 product (bf16_chunks, one wavefront
// each, summed from zero and added in chunk order; the other wavefronts add exact zeros), so
// the result is bit-identical to the unfused shared down and independent of the other tokens.
// Wd is the tiled bf16 [H/16][Is/32][64][8], or (FMT_INT8) the tiled int8 codes with their
// scale/bias, dequantized in registers to the same bf16 weights.
constexpr int kCsWaves = 8;
template <int MT, int FMT>
__global__ void __launch_bounds__(64 * kCsWaves) combine_shared_kernel(
    const uint16_t* __restrict__ d, const int32_t* __restrict__ inv, const float* __restrict__ w,
    int N, int k, int H, int64_t n_pos, const uint16_t* __restrict__ sh_h, int Is, int nch,
    const void* __restrict__ wd, const uint16_t* __restrict__ wd_sb,
    const float* __restrict__ shared_gate, const uint16_t* resid, uint16_t* y) {
  constexpr int TOK = 16 * MT;   // tokens per workgroup
  __shared__ f32x4_t part[kCsWaves][MT][64];
  __shared__ float sh[TOK][17];
  __shared__ float routed[TOK][17];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int fb = blockIdx.x;
  const int tm = blockIdx.y * TOK;
  const int nks = Is / 32;
  const int c0 = (wave < nch) ? wave * nks / nch : 0, c1 = (wave < nch) ? (wave + 1) * nks / nch : 0;
  DenseTile<FMT> wt;
  wt.init(wd, wd_sb, fb, Is, lane);
  // the routed gather-sum of (token tl, feature f) runs on wavefronts 4-7 while wavefronts 0-3
  // compute the shared down (when it has at most 4 chunks), else after it; 256 threads, MT
  // tokens each
  const int rt = threadIdx.x & 255;
  const int f = rt & 15;
  const int col = fb * 16 + f;
  const bool gather_early = nch <= 4;
  auto routed_sum = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < MT; ++u) {
      const int tl = (rt >> 4) + 16 * u;
      const int t = tm + tl;
      float acc1 = 0.f;
      if (t < N) {
        const int64_t m0 = static_cast<int64_t>(t) * k;
        // eight slots' positions, then their values, then the sums in slot order (one
        // dependent-load round trip per eight slots instead of one per slot)
        for (int s0 = 0; s0 < k; s0 += 8) {
          int pos[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) pos[j] = (s0 + j < k) ? inv[m0 + s0 + j] : -1;
          float dv[8], wv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const bool ok = pos[j] >= 0 && pos[j] < n_pos;
            dv[j] = ok ? bf16_to_f32(d[static_cast<int64_t>(pos[j]) * H + col]) : 0.f;
            wv[j] = ok ? w[m0 + s0 + j] : 0.f;
          }
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (pos[j] >= 0 && pos[j] < n_pos) acc1 = fmaf(dv[j], wv[j], acc1);
        }
      }
      routed[tl][f] = acc1;
    }
  };
  if (gather_early && wave >= 4) routed_sum();
  // shared down for tokens tm .. tm+TOK-1 (rows past N read token tm: computed, never used)
  {
    const uint16_t* xr[MT];
#pragma unroll
    for (int u = 0; u < MT; ++u) {
      const int tr = tm + 16 * u + (lane & 15);
      xr[u] = sh_h + static_cast<int64_t>(tr < N ? tr : tm) * Is + 8 * (lane >> 4);
    }
    f32x4_t acc[MT];
#pragma unroll
    for (int u = 0; u < MT; ++u) acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // batches of steps, all loads first (clamped indices), MFMAs in step order
    constexpr int BS = 8;
    for (int cb = c0; cb < c1; cb += BS) {
      DenseFrag<FMT> wv[BS];
      u32x4 xv[BS][MT];
#pragma unroll
      for (int i = 0; i < BS; ++i) {
        const int c = min(cb + i, c1 - 1);
        wv[i] = wt.load(c);
#pragma unroll
        for (int u = 0; u < MT; ++u) xv[i][u] = *reinterpret_cast<const u32x4*>(xr[u] + 32 * c);
      }
#pragma unroll
      for (int i = 0; i < BS; ++i)
        if (cb + i < c1) {
          const bf16x8_t B = as_bf16x8(dense_bf16<FMT>(wv[i]));
#pragma unroll
          for (int u = 0; u < MT; ++u) acc[u] = mfma16(as_bf16x8(xv[i][u]), B, acc[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < MT; ++u) part[wave][u][lane] = acc[u];
  }
  if (!gather_early && wave < 4) routed_sum();
  __syncthreads();
  if (wave < MT) {
    const int u = wave;
    f32x4_t s4 = part[0][u][lane];
#pragma unroll
    for (int q = 1; q < kCsWaves; ++q) {
      const f32x4_t o = part[q][u][lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) s4[j] += o[j];
    }
    // lane holds tokens 4*(lane/16) + j of m-tile u, feature lane%16
#pragma unroll
    for (int j = 0; j < 4; ++j)
      sh[16 * u + 4 * (lane >> 4) + j][lane & 15] = bf16_to_f32(f32_to_bf16(s4[j]));
  }
  __syncthreads();
  // routed sum (slot order) + gated shared, rounded once to bf16
  if (threadIdx.x < 16 * TOK) {
    const int tl = threadIdx.x >> 4;
    const int t = tm + tl;
    if (t < N) {
      const float g = shared_gate ? shared_gate[t] : 1.0f;
      const int64_t o = static_cast<int64_t>(t) * H + col;
      uint16_t v = f32_to_bf16(fmaf(sh[tl][f], g, routed[tl][f]));
      if (resid) v = f32_to_bf16(bf16_to_f32(resid[o]) + bf16_to_f32(v));   // see add_resid
      y[o] = v;
    }
  }
}

template <int FMT>
static void launch_cs(const uint16_t* d, const int32_t* inv, const float* w, int N, int k, int H,
                      const uint16_t* sh_h, int Is, int nch, const void* wd, const uint16_t* wd_sb,
                      const float* shared_gate, uint16_t* y, hipStream_t stream,
                      const uint16_t* resid) {
  // above 48 tokens, 32 per workgroup: the shared down weights are read once per 32 tokens
  // (below that the halved grid leaves CUs idle)
  if (N > 48) {
    dim3 grid(H / 16, (N + 31) / 32);
    combine_shared_kernel<2, FMT><<<grid, 64 * kCsWaves, 0, stream>>>(
        d, inv, w, N, k, H, static_cast<int64_t>(N) * k, sh_h, Is, nch, wd, wd_sb, shared_gate,
        resid, y);
  } else {
    dim3 grid(H / 16, (N + 15) / 16);
    combine_shared_kernel<1, FMT><<<grid, 64 * kCsWaves, 0, stream>>>(
        d, inv, w, N, k, H, static_cast<int64_t>(N) * k, sh_h, Is, nch, wd, wd_sb, shared_gate,
        resid, y);
  }
}

int launch_combine_shared(const uint16_t* d, const int32_t* inv, const float* w, int N, int k,
                          int H, const uint16_t* sh_h, int Is, const void* wd,
                          const uint16_t* wd_sb, int fmt, const float* shared_gate, uint16_t* y,
                          hipStream_t stream, const uint16_t* resid) {
  const int nch = bf16_chunks(Is);
  if (H % 16 || Is % 32 || Is <= 0 || nch > kCsWaves)
    return fail("combine: fused shared down needs H % 16 == 0, Is % 32 == 0, Is < 4096");
  if (fmt == FMT_INT8) {
    if (Is % 64 || !wd_sb) return fail("combine: int8 shared down needs Is % 64 == 0 and scale/bias");
    launch_cs<FMT_INT8>(d, inv, w, N, k, H, sh_h, Is, nch, wd, wd_sb, shared_gate, y, stream, resid);
  } else {
    launch_cs<FMT_BF16>(d, inv, w, N, k, H, sh_h, Is, nch, wd, wd_sb, shared_gate, y, stream, resid);
  }
  return check_launch("combine_shared");
}

int validate_routing(int N, int H, int E, int k, int scoring, int n_group, int topk_group);

// ------------------------------------------------------------------ auxiliary stream
// qmoe_forward runs independent work on a library-owned stream (created
// once per device, default priority) concurrently with the caller's stream:
//  * the shared expert, which depends only on x, beside the router -> top-k -> permute ->
//    routed chain (small decode batches instead fuse it into the router and combine launches:
//    there a join, which costs a launch that does not overlap the previous kernel, costs more
//    than the shared expert's bytes);
//  * in the hybrid regime, the cold experts' grouped matmuls (small kernel, bound by HBM)
//    beside the hot experts' (large kernel, bound by MFMA).
// A fork event records the caller's stream at entry, `perm` publishes the permute to the
// auxiliary stream, `cold` returns the cold gate_up (h complete), `hready` publishes the fp16
// copy of h, and the caller's stream waits on `join` right before the combine. The mutex is held
// from the fork record until the join wait is enqueued, so concurrent calls on different streams
// cannot exchange the events.
struct AuxStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr, perm = nullptr, cold = nullptr, hready = nullptr,
             xready = nullptr;
};
static std::mutex g_aux_mu;
constexpr int64_t kFuseSharedMaxTokens = 64;
// Slot-major routing (no permute launch) reads an expert once per slot that picks it, the
// permute once per call; the permute launch costs about as much as streaming this many bytes.
constexpr double kPermuteLaunchBytes = 24e6;
constexpr int64_t kSlotMajorCapTokens = 16;
// The routed gate_up ranks the logits in every workgroup: past ~2048 workgroups that costs more
// than the top-k launch it replaces (c2: N <= 3, 64 workgroups per slot; c1: N <= 8, 16).
constexpr int64_t kRouteMaxWorkgroups = 2048;

// The routing tail of the router pair launch (qmoe_set_route_tail): 1 (default) on, 0 off.
static std::atomic<int> g_route_tail{1};

// Routed expert bytes (gate_up + down) of one expert in the config's formats.
static double expert_bytes(const qmoe_config_t& c) {
  auto per_weight = [](int fmt) {
    return fmt == QMOE_FMT_BF16 ? 2.0 : fmt == QMOE_FMT_INT6_G64 ? 6.5 / 8 :
           fmt == QMOE_FMT_INT3_G64 ? 3.5 / 8 : 4.5 / 8;
  };
  const double iw = static_cast<double>(c.inter) * c.hidden;
  return 2.0 * iw * per_weight(c.expert_format) + iw * per_weight(c.down_format);
}

// Largest batch routed slot-major: at least 2 tokens; more while the expected number of
// duplicate expert reads under uniform routing, N*k - E*(1 - (1 - k/E)^N), costs fewer bytes
// than the permute launch (c1's shape: 8 tokens and more; c2's: 5).
static int64_t slot_major_max_tokens(const qmoe_config_t& c) {
  const double k = c.top_k, E = c.n_experts, be = expert_bytes(c);
  int64_t n = 2;
  for (int64_t t = 3; t <= kSlotMajorCapTokens; ++t) {
    const double dup = t * k - E * (1.0 - std::pow(1.0 - k / E, static_cast<double>(t)));
    if (dup * be > kPermuteLaunchBytes) break;
    n = t;
  }
  return n;
}
static std::map<int, AuxStream> g_aux;

static int aux_stream(hipStream_t caller, AuxStream** out) {
  int dev = 0;
  hipError_t err = hipStreamGetDevice(caller, &dev);
  if (err != hipSuccess) return fail(std::string("forward: stream device: ") + hipGetErrorString(err));
  AuxStream& a = g_aux[dev];
  if (!a.s) {
    int cur = 0;
    err = hipGetDevice(&cur);
    if (err == hipSuccess && cur != dev) err = hipSetDevice(dev);
    if (err == hipSuccess) err = hipStreamCreateWithFlags(&a.s, hipStreamNonBlocking);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&a.fork, hipEventDisableTiming);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&a.join, hipEventDisableTiming);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&a.perm, hipEventDisableTiming);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&a.cold, hipEventDisableTiming);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&a.hready, hipEventDisableTiming);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&a.xready, hipEventDisableTiming);
    if (cur != dev) (void)hipSetDevice(cur);
    if (err != hipSuccess) {
      a = AuxStream{};
      return fail(std::string("forward: auxiliary stream: ") + hipGetErrorString(err));
    }
  }
  *out = &a;
  return 0;
}

// Large-M tiles pay off once a batch gives experts tens of rows; they also need the output
// widths (hidden for the down projection) to be multiples of the 256-row tile.
static int dense_regime(const qmoe_config_t& c, int64_t N) {
  return (N > 256 && c.hidden % 256 == 0) ? QMOE_REGIME_LARGE : QMOE_REGIME_SMALL;
}

// Whether an int8 shared expert is expanded to bf16 for this call: the large-M kernel stages
// bf16 (or int4) weights only, and above the decode sizes the expansion (half the bf16 bytes
// read, all of them written once) is small beside the block.
static bool shared_expands(const qmoe_config_t& c, int64_t N) {
  return c.shared_inter > 0 && c.shared_format == QMOE_FMT_INT8_G64 &&
         dense_regime(c, N) == QMOE_REGIME_LARGE;
}

// ------------------------------------------------------------------ forward workspace layout
struct WsLayout {
  size_t logits, idx, w, sg, counts, offsets, tile_off, tile_map, tile_map_big, sorted, inv, h,
      d, sh_h, sh_out, sh_w16, x16, x_sinv, h16, h_sinv, awq_x, awq_gu, sync, route_ctr, total;
  int64_t max_tiles, max_tiles_big, sync_words;
};

static WsLayout ws_layout(const qmoe_config_t& c, int64_t N) {
  WsLayout L{};
  const int64_t mc = N * c.top_k;
  const int64_t ld = (c.router_format == QMOE_ROUTER_F32) ? c.n_experts + 1 : c.router_rows;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  L.logits = take(static_cast<size_t>(N) * ld * 4);
  L.idx = take(static_cast<size_t>(mc) * 4);
  L.w = take(static_cast<size_t>(mc) * 4);
  L.sg = take(static_cast<size_t>(N) * 4);
  L.counts = take(static_cast<size_t>(c.n_experts) * 4);
  L.offsets = take(static_cast<size_t>(c.n_experts + 1) * 4);
  L.tile_off = take(static_cast<size_t>(c.n_experts + 1) * 4);
  // tile descriptors for whichever m-tile the regime uses (16 needs the most entries); the
  // slot-major map of a few tokens has one tile per slot, which can exceed that bound when
  // k > E / 2
  L.max_tiles = mtile_upper_bound(mc, c.n_experts, kSmallMTile);
  if (N <= slot_major_max_tokens(c)) L.max_tiles = std::max<int64_t>(L.max_tiles, mc);
  L.tile_map = take(static_cast<size_t>(L.max_tiles) * 16);
  // large-M regime: 128-row tiles of the experts above the hybrid split
  L.max_tiles_big = mtile_upper_bound(mc, c.n_experts, kLargeMTile);
  L.tile_map_big = take(static_cast<size_t>(L.max_tiles_big) * 16);
  L.sorted = take(static_cast<size_t>(mc) * 4);
  L.inv = take(static_cast<size_t>(mc) * 4);
  L.h = take(static_cast<size_t>(mc) * c.inter * 2);
  L.d = take(static_cast<size_t>(mc) * c.hidden * 2);
  // (the shared expert's SwiGLU output, or with the decode dataflow launch its [gate | up] rows)
  L.sh_h = take(static_cast<size_t>(N) * (c.shared_inter > 0 ? 2 * c.shared_inter : 0) * 2);
  L.sh_out = take(static_cast<size_t>(N) * (c.shared_inter > 0 ? c.hidden : 0) * 2);
  // int8 shared expert above the decode sizes: its weights expanded to tiled bf16 for the
  // large-M kernel (gate|up [2 Is, H] then down [H, Is])
  L.sh_w16 = take(shared_expands(c, N) ? static_cast<size_t>(3) * c.shared_inter * c.hidden * 2 : 0);
  // fp16 per-row-scaled activation copies for the large-M int4 regime (AWQ: of the gate's and
  // the up projection's prescaled rows, [2][mc])
  const int64_t x16_rows = c.awq ? 2 * mc : N;
  L.x16 = take(static_cast<size_t>(x16_rows) * c.hidden * 2);
  L.x_sinv = take(static_cast<size_t>(x16_rows) * 4);
  L.h16 = take(static_cast<size_t>(mc) * c.inter * 2);
  L.h_sinv = take(static_cast<size_t>(mc) * 4);
  // AWQ: the gate and up projections' prescaled rows [2][mc][H] and their outputs [mc][2I]
  L.awq_x = take(c.awq ? static_cast<size_t>(2) * mc * c.hidden * 2 : 0);
  // (mixed widths also route gate and up through awq_gu)
  L.awq_gu = take((c.awq || c.mixed) ? static_cast<size_t>(mc) * 2 * c.inter * 2 : 0);
  // the decode dataflow kernel's counters (cleared by the router launch of every call)
  L.sync_words = decode_flow_sync_words(mc, c.hidden);
  L.sync = take(static_cast<size_t>(L.sync_words) * 4);
  // the routing tail's two counters (64-bit words; no clearing needed, RouteTail)
  L.route_ctr = take(16);
  L.total = o;
  return L;
}

// Gated activation of the SwiGLU epilogue: QMOE_ACT_SILU ignores alpha and limit; the clamped
// forms need limit > 0 (+inf: no clamp) and a finite alpha.
static int validate_glu(int act, float alpha, float limit) {
  if (act < QMOE_ACT_SILU || act > QMOE_ACT_SWIGLU_OAI) return fail("config: unknown act");
  if (act != QMOE_ACT_SILU && !(limit > 0.f)) return fail("config: act_limit must be > 0 (+inf: none)");
  if (act == QMOE_ACT_SWIGLU_OAI && !isfinite(alpha)) return fail("config: act_alpha must be finite");
  return 0;
}

// Kernel format of a QMOE_FMT_* value.
static int kernel_fmt(int f) {
  return f == QMOE_FMT_INT4_G64 ? FMT_INT4 : f == QMOE_FMT_INT6_G64 ? FMT_INT6
         : f == QMOE_FMT_INT3_G64 ? FMT_INT3 : f == QMOE_FMT_INT8_G64 ? FMT_INT8 : FMT_BF16;
}
// AWQ-scaled experts in the large regime: quantized weights (awq implies them), and gate and up
// halves that split at a whole 256-row block (the large kernels pick the activation copy per
// weight-row block)
static bool awq_large_ok(const qmoe_config_t& c) {
  return c.expert_format != QMOE_FMT_BF16 && c.down_format != QMOE_FMT_BF16 && c.inter % 256 == 0;
}

// formats the large-regime kernels dequantize to fp16 (an fp16 activation copy, row exponents)
static bool fp16_large_fmt(int kfmt) { return fmt_quant(kfmt); }
static bool fp16_large_fmt_q(int qfmt) {
  return qfmt == QMOE_FMT_INT4_G64 || qfmt == QMOE_FMT_INT6_G64 || qfmt == QMOE_FMT_INT3_G64;
}

static bool has_split(const qmoe_mixed_t& m) {
  for (int i = 0; i < m.n_stacks; ++i)
    if (m.stacks[i].proj == QMOE_PROJ_GATE || m.stacks[i].proj == QMOE_PROJ_UP) return true;
  return false;
}

static int validate_mixed(const qmoe_mixed_t& m) {
  if (m.n_stacks < 2 || m.n_stacks > QMOE_MAX_STACKS)
    return fail("mixed: 2 <= n_stacks <= QMOE_MAX_STACKS required");
  int seen[4] = {0, 0, 0, 0};
  for (int i = 0; i < m.n_stacks; ++i) {
    const qmoe_stack_t& st = m.stacks[i];
    if (st.proj < QMOE_PROJ_GATE || st.proj > QMOE_PROJ_GATE_UP) return fail("mixed: unknown proj");
    if (st.format != QMOE_FMT_INT4_G64 && st.format != QMOE_FMT_INT6_G64 && st.format != QMOE_FMT_INT3_G64)
      return fail("mixed: stack formats must be int3, int4 or int6");
    if (!st.codes || !st.sb || !st.expert_slot) return fail("mixed: null stack pointer");
    seen[st.proj] = 1;
  }
  const bool split = seen[QMOE_PROJ_GATE] || seen[QMOE_PROJ_UP];
  if (!seen[QMOE_PROJ_DOWN] || (split ? (!seen[QMOE_PROJ_GATE] || !seen[QMOE_PROJ_UP] || seen[QMOE_PROJ_GATE_UP])
                                      : !seen[QMOE_PROJ_GATE_UP]))
    return fail("mixed: every projection needs a stack (gate and up, or fused gate_up)");
  return 0;
}

static int validate_config(const qmoe_config_t& c) {
  const int rc = validate_routing(1, c.hidden, c.n_experts, c.top_k, c.scoring, c.n_group,
                                  c.topk_group);
  if (rc) return rc;
  if (c.hidden % 128) return fail("config: hidden % 128 == 0 required");
  if (c.norm_topk < QMOE_NORM_NONE || c.norm_topk > QMOE_NORM_MULTI)
    return fail("config: norm_topk must be QMOE_NORM_NONE, _ALWAYS or _MULTI");
  if (c.regime == QMOE_REGIME_LARGE && c.hidden % 256)
    return fail("config: the large-M regime needs hidden % 256 == 0");
  if (c.inter <= 0 || c.inter % 128) return fail("config: inter % 128 == 0 required");
  if (c.shared_inter < 0 || c.shared_inter % 128) return fail("config: shared_inter % 128 == 0 required");
  if (c.shared_format != QMOE_FMT_BF16 && c.shared_format != QMOE_FMT_INT8_G64)
    return fail("config: shared_format must be QMOE_FMT_BF16 (1) or QMOE_FMT_INT8_G64 (4)");
  if (c.expert_format < QMOE_FMT_INT4_G64 || c.expert_format > QMOE_FMT_INT3_G64 ||
      c.down_format < QMOE_FMT_INT4_G64 || c.down_format > QMOE_FMT_INT3_G64)
    return fail("config: expert_format / down_format must be int4-g64 (0), bf16 (1), int6-g64 (2) or int3-g64 (3)");
  if ((c.expert_format == QMOE_FMT_BF16) != (c.down_format == QMOE_FMT_BF16))
    return fail("config: gate_up and down must both be quantized or both bf16");
  if (c.awq != 0 && c.awq != 1) return fail("config: awq must be 0 or 1");
  if (c.awq && c.expert_format == QMOE_FMT_BF16)
    return fail("config: awq scales need quantized experts");
  if (c.awq && c.regime == QMOE_REGIME_LARGE && !awq_large_ok(c))
    return fail("config: awq scales in the large regime need inter % 256 == 0");
  if (c.mixed != 0 && c.mixed != 1) return fail("config: mixed must be 0 or 1");
  if (c.mixed && c.awq) return fail("config: mixed-width experts run without awq scales");
  if (c.router_format == QMOE_ROUTER_BF16_TILED) {
    if (c.router_rows < c.n_experts + (c.shared_gated ? 1 : 0) || c.router_rows % 256)
      return fail("config: router_rows must cover E (+1 shared gate row) and be a multiple of 256");
  } else if (c.router_format != QMOE_ROUTER_F32) {
    return fail("config: unknown router_format");
  }
  if (c.regime < QMOE_REGIME_AUTO || c.regime > QMOE_REGIME_LARGE) return fail("config: bad regime");
  return validate_glu(c.act, c.act_alpha, c.act_limit);
}

}  // namespace qmoe

using namespace qmoe;

extern "C" const char* qmoe_last_error(void) { return g_last_error.c_str(); }

extern "C" int qmoe_abi_version(void) { return QMOE_ABI_VERSION; }

extern "C" int qmoe_combine(const uint16_t* d, const int32_t* inv, const float* w, int64_t N, int k,
                            int H, const uint16_t* shared_out, const float* shared_gate,
                            uint16_t* y, void* stream) {
  if (N <= 0 || N > 65535 || k <= 0 || H <= 0 || H % 8) return fail("qmoe_combine: need 0 < N <= 65535, H % 8 == 0");
  if (!d || !inv || !w || !y) return fail("qmoe_combine: null pointer");
  return launch_combine(d, inv, w, static_cast<int>(N), k, H, shared_out, shared_gate, y,
                        static_cast<hipStream_t>(stream));
}

extern "C" size_t qmoe_grouped_qmm_workspace(int64_t act_rows, int K, int weight_format,
                                             int regime) {
  if (act_rows <= 0 || K <= 0) return 0;
  if (regime == QMOE_REGIME_LARGE && fp16_large_fmt_q(weight_format))
    return act16_ws_bytes(act_rows, K);
  return 0;
}

extern "C" int qmoe_grouped_qmm(const uint16_t* act, int64_t act_rows, const int32_t* slot_of,
                                int slot_div, int64_t n_slots, const int32_t* offsets,
                                const int32_t* tile_off, const int32_t* tile_map, int n_experts,
                                int64_t dense_rows, int K, int n_rows, int weight_format,
                                const void* codes, const uint16_t* sb, const int8_t* row_exp,
                                int epilogue, int glu,
                                float glu_alpha, float glu_limit, void* out,
                                int ld_out, int regime, void* ws, size_t ws_bytes, void* stream) {
  if (!act || !codes || !out) return fail("qmoe_grouped_qmm: null pointer");
  if (epilogue == QMOE_EPI_SWIGLU) {
    const int rc = validate_glu(glu, glu_alpha, glu_limit);
    if (rc) return rc;
  }
  if (weight_format < QMOE_FMT_INT4_G64 || weight_format > QMOE_FMT_INT8_G64)
    return fail("qmoe_grouped_qmm: bad weight_format");
  if (weight_format != QMOE_FMT_BF16 && !sb) return fail("qmoe_grouped_qmm: quantized weights need sb");
  if (epilogue < QMOE_EPI_SWIGLU || epilogue > QMOE_EPI_F32) return fail("qmoe_grouped_qmm: bad epilogue");
  if (regime != QMOE_REGIME_SMALL && regime != QMOE_REGIME_LARGE)
    return fail("qmoe_grouped_qmm: regime must be small (1) or large (2)");
  if (slot_of && slot_div <= 0) return fail("qmoe_grouped_qmm: slot_div must be positive");
  if (regime == QMOE_REGIME_LARGE && fp16_large_fmt_q(weight_format) && !row_exp)
    return fail("qmoe_grouped_qmm: int4 weights in the large regime need row_exp (qmoe_row_exponents)");
  const int out_cols = (epilogue == QMOE_EPI_SWIGLU) ? n_rows / 2 : n_rows;
  if (ld_out < out_cols) return fail("qmoe_grouped_qmm: ld_out too small");
  QmmArgs a{};
  a.act = act;
  a.act_rows = act_rows;
  a.slot_of = slot_of;
  a.slot_div = slot_div > 0 ? slot_div : 1;
  a.n_slots = n_slots;
  a.offsets = offsets;
  a.tile_off = tile_off;
  a.tile_map = offsets ? reinterpret_cast<const int4*>(tile_map) : nullptr;
  a.dense_rows = dense_rows;
  a.n_experts = offsets ? n_experts : 1;
  a.K = K;
  a.n_rows = n_rows;
  a.codes = codes;
  a.sb = sb;
  a.row_exp = fp16_large_fmt_q(weight_format) ? row_exp : nullptr;
  a.out = out;
  a.ld_out = ld_out;
  a.glu = glu;
  a.glu_alpha = glu_alpha;
  a.glu_limit = glu_limit;
  const int m_tile = (regime == QMOE_REGIME_SMALL) ? kSmallMTile : kLargeMTile;
  int64_t bound;
  if (offsets) {
    if (!tile_off || n_experts <= 0) return fail("qmoe_grouped_qmm: segmented mode needs tile_off");
    bound = mtile_upper_bound(n_slots, n_experts, m_tile);
  } else {
    if (dense_rows <= 0) return fail("qmoe_grouped_qmm: dense_rows must be positive");
    bound = (dense_rows + m_tile - 1) / m_tile;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (regime == QMOE_REGIME_LARGE && fp16_large_fmt_q(weight_format)) {
    const size_t need = act16_ws_bytes(act_rows, K);
    if (!ws || ws_bytes < need) return fail("qmoe_grouped_qmm: workspace too small for the fp16 copy");
    uint16_t* act16 = static_cast<uint16_t*>(ws);
    float* sinv = reinterpret_cast<float*>(static_cast<char*>(ws) +
                                           align256(static_cast<size_t>(act_rows) * K * 2));
    const int rc = launch_act_to_f16(act, act_rows, K, act16, sinv, st);
    if (rc) return rc;
    a.act16 = act16;
    a.row_sinv = sinv;
  }
  return launch_qmm(a, weight_format, epilogue, regime, bound, st);
}

extern "C" size_t qmoe_forward_workspace(const qmoe_config_t* cfg, int64_t N) {
  if (!cfg || N <= 0) return 0;
  return ws_layout(*cfg, N).total;
}

extern "C" int qmoe_set_route_tail(int on) {
  if (on < 0 || on > 1) return qmoe::g_route_tail.load();
  return qmoe::g_route_tail.exchange(on);
}

static int pick_regime(const qmoe_config_t& c, int64_t N) {
  if (c.regime != QMOE_REGIME_AUTO) return c.regime;
  if (c.awq && !awq_large_ok(c)) return QMOE_REGIME_SMALL;
  return dense_regime(c, N);
}

// The block on x; with resid, the combine adds the decoder layer's residual row.
// single_stream: every launch on the caller's stream (no auxiliary stream or events, which are
// created on first use), for the entry point that allocates nothing.
// norm_w: the decoder layer's RMSNorm in front of the block (qmoe_forward_residual): x is the raw
// residual row, the block runs on xn = rmsnorm(x) (written to `xn`, outside ws), and the combine
// adds x back. For small decode batches the norm runs inside the router launch; otherwise it is
// a launch of its own, first.
static int forward_impl(const qmoe_config_t* cfg, const qmoe_weights_t* wts, const uint16_t* x_in,
                        int64_t N, uint16_t* y, void* ws, size_t ws_bytes, void* stream_,
                        const qmoe_mixed_t* mixed = nullptr, bool single_stream = false,
                        const uint16_t* norm_w = nullptr, float norm_eps = 0.f,
                        uint16_t* xn = nullptr) {
  if (!cfg || !wts || !x_in || !y || !ws || (norm_w && !xn)) return fail("qmoe_forward: null pointer");
  const qmoe_config_t& c = *cfg;
  int rc = validate_config(c);
  if (rc) return rc;
  if (c.mixed != (mixed != nullptr))
    return fail("qmoe_forward: mixed-width experts go through qmoe_forward_mixed (config mixed = 1)");
  if (mixed) {
    rc = validate_mixed(*mixed);
    if (rc) return rc;
  }
  if (N <= 0 || N > 65535) return fail("qmoe_forward: 0 < N <= 65535 tokens per call");
  const WsLayout L = ws_layout(c, N);
  if (ws_bytes < L.total) return fail("qmoe_forward: workspace too small");
  if (!wts->router_w || (!mixed && (!wts->gu_codes || !wts->dn_codes)))
    return fail("qmoe_forward: missing weights");
  if (!mixed && c.expert_format != QMOE_FMT_BF16 && (!wts->gu_sb || !wts->dn_sb))
    return fail("qmoe_forward: quantized experts need scale/bias");
  if (c.shared_inter > 0 && (!wts->sh_gu || !wts->sh_dn)) return fail("qmoe_forward: missing shared expert");
  if (c.shared_inter > 0 && c.shared_format == QMOE_FMT_INT8_G64 && (!wts->sh_gu_sb || !wts->sh_dn_sb))
    return fail("qmoe_forward: an int8 shared expert needs sh_gu_sb and sh_dn_sb");
  if (c.router_format == QMOE_ROUTER_F32 && c.shared_gated && !wts->shared_gate_w)
    return fail("qmoe_forward: fp32 router with a gated shared expert needs shared_gate_w");
  if (c.awq && (!wts->awq_gu || !wts->awq_dn)) return fail("qmoe_forward: awq needs awq_gu and awq_dn");
  if (mixed && pick_regime(c, N) == QMOE_REGIME_LARGE) {
    for (int i = 0; i < mixed->n_stacks; ++i)
      if (!mixed->stacks[i].row_exp)
        return fail("qmoe_forward_mixed: stacks in the large regime (N > 256) need row_exp "
                    "(qmoe_row_exponents)");
  }
  if (!mixed && pick_regime(c, N) == QMOE_REGIME_LARGE &&
      ((fp16_large_fmt(kernel_fmt(c.expert_format)) && !wts->gu_rexp) ||
       (fp16_large_fmt(kernel_fmt(c.down_format)) && !wts->dn_rexp)))
    return fail("qmoe_forward: quantized experts in the large regime (N > 256) need gu_rexp and "
                "dn_rexp (qmoe_row_exponents)");

  hipStream_t stream = static_cast<hipStream_t>(stream_);
  char* base = static_cast<char*>(ws);
  float* logits = reinterpret_cast<float*>(base + L.logits);
  int32_t* idx = reinterpret_cast<int32_t*>(base + L.idx);
  float* wv = reinterpret_cast<float*>(base + L.w);
  float* sg = reinterpret_cast<float*>(base + L.sg);
  int32_t* counts = reinterpret_cast<int32_t*>(base + L.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(base + L.offsets);
  int32_t* tile_off = reinterpret_cast<int32_t*>(base + L.tile_off);
  int32_t* tile_map = reinterpret_cast<int32_t*>(base + L.tile_map);
  int32_t* sorted = reinterpret_cast<int32_t*>(base + L.sorted);
  int32_t* inv = reinterpret_cast<int32_t*>(base + L.inv);
  uint16_t* h = reinterpret_cast<uint16_t*>(base + L.h);
  uint16_t* d = reinterpret_cast<uint16_t*>(base + L.d);
  uint16_t* sh_h = reinterpret_cast<uint16_t*>(base + L.sh_h);
  uint16_t* sh_out = reinterpret_cast<uint16_t*>(base + L.sh_out);
  uint16_t* x16 = reinterpret_cast<uint16_t*>(base + L.x16);
  float* x_sinv = reinterpret_cast<float*>(base + L.x_sinv);
  uint16_t* h16 = reinterpret_cast<uint16_t*>(base + L.h16);
  float* h_sinv = reinterpret_cast<float*>(base + L.h_sinv);

  const int n = static_cast<int>(N);
  const int64_t mc = N * c.top_k;
  const int regime = pick_regime(c, N);
  // Large-M regime = hybrid: experts with more than kHybridSplitRows rows run on the large
  // kernel (128-row tiles), the rest on the small kernel (16-row tiles). A handful of rows
  // cannot amortise a 128-row tile's weight dequant; under skewed routing most experts are
  // that small while a few carry thousands of rows.
  const bool hybrid = (regime == QMOE_REGIME_LARGE);
  int32_t* tile_map_big = reinterpret_cast<int32_t*>(base + L.tile_map_big);
  const int64_t bound_small = mtile_upper_bound(mc, c.n_experts, kSmallMTile);
  const int64_t cold_bound =
      std::min<int64_t>(bound_small, static_cast<int64_t>(c.n_experts) *
                                         ((kHybridSplitRows + kSmallMTile - 1) / kSmallMTile));
  const int64_t hot_bound = (mc + kLargeMTile - 1) / kLargeMTile +
                            std::min<int64_t>(c.n_experts, mc / (kHybridSplitRows + 1));
  const int gfmt = kernel_fmt(c.expert_format), dfmt = kernel_fmt(c.down_format);
  const int has_sg = (c.shared_inter > 0 && c.shared_gated) ? 1 : 0;

  const int sreg = dense_regime(c, N);
  const bool decode = (sreg == QMOE_REGIME_SMALL);
  // Small decode batches: the shared expert rides in the neighbouring launches, its gate_up with
  // the router logits and its down projection in the combine, so no launch or stream event of
  // its own. Otherwise the shared expert and, in the hybrid regime, the cold experts' grouped
  // matmuls run on the auxiliary stream (held until its join is enqueued below).
  const bool shared = c.shared_inter > 0;
  // (the fused launches give bit-identical results; above kFuseSharedMaxTokens the shared
  // expert's re-read weights cost more than the auxiliary stream's join)
  const bool fuse = decode && shared && N <= kFuseSharedMaxTokens;
  const bool fuse_gu = fuse && c.router_format == QMOE_ROUTER_BF16_TILED;
  // the block's input rows: x itself, or its RMSNorm (made inside the router launch when that is
  // the fused pair, else by a launch of its own ahead of everything)
  const uint16_t* resid = norm_w ? x_in : nullptr;
  const uint16_t* x = norm_w ? xn : x_in;
  // (the router launch normalises the rows when its shape allows, pair_norm_fusable)
  const bool fuse_norm = norm_w && fuse_gu && pair_norm_fusable(c.hidden, N);
  if (norm_w && !fuse_norm) {
    rc = launch_rmsnorm(x_in, norm_w, N, c.hidden, norm_eps, xn, static_cast<hipStream_t>(stream_));
    if (rc) return rc;
  }
  const bool fuse_dn = fuse && bf16_chunks(c.shared_inter) <= 8;
  // a few tokens: slot-major routing written by the top-k, no permute launch (each slot
  // its own m-tile; an expert two tokens share is read twice, cheaper than the launch)
  // (AWQ prescaling finds each row's expert from the permute's segment offsets)
  const bool slot_major = !hybrid && N <= slot_major_max_tokens(c) && !c.awq;
  // m-tiles of the small-kernel launches: one per slot when slot-major
  const int64_t tiles_small = slot_major ? std::max<int64_t>(bound_small, mc) : bound_small;
  std::unique_lock<std::mutex> aux_lock;
  AuxStream* aux = nullptr;
  hipStream_t sstream = stream;
  const bool shared_aux = shared && !fuse;
  auto link = [&](hipEvent_t ev, hipStream_t from, hipStream_t to, const char* what) {
    hipError_t err = hipEventRecord(ev, from);
    if (err == hipSuccess) err = hipStreamWaitEvent(to, ev, 0);
    return err == hipSuccess ? 0 : fail(std::string("forward: ") + what + ": " + hipGetErrorString(err));
  };
  if ((shared_aux || hybrid) && !single_stream) {
    aux_lock = std::unique_lock<std::mutex>(g_aux_mu);
    rc = aux_stream(stream, &aux);
    if (rc) return rc;
    rc = link(aux->fork, stream, aux->s, "fork");
    if (rc) return rc;
    if (shared_aux) sstream = aux->s;
  }
  // hybrid prefill with int4 experts: the hot experts' gate_up reads an fp16 copy of x, made
  // first on the auxiliary stream, beside the routing chain (hybrid implies int4 or bf16 experts;
  // AWQ: copies of the prescaled rows instead, made after the permute), and their down an fp16
  // copy of h. A mixed-width layer's stacks are all int3, int4 or int6 (validate_mixed), whatever
  // placeholder formats the config carries, so its prefill kernels always read the copies.
  const bool f16_acts = hybrid && !c.awq && (mixed || fp16_large_fmt(gfmt));
  const bool f16_h = hybrid && (mixed || fp16_large_fmt(dfmt));
  if (f16_acts) {
    rc = launch_act_to_f16(x, N, c.hidden, x16, x_sinv, aux ? aux->s : stream);
    if (rc) return rc;
    if (aux) {
      const hipError_t err = hipEventRecord(aux->xready, aux->s);
      if (err != hipSuccess) return fail(std::string("forward: x16 record: ") + hipGetErrorString(err));
    }
  }

  // 1. shared expert gate_up + SwiGLU -> sh_h (fused with the router below when decoding)
  const int st = decode ? kSmallMTile : kLargeMTile;
  QmmArgs sgu{};
  // the shared expert's weights as the kernels read them: int8 codes dequantized in registers,
  // or (large regime) expanded to bf16 in the workspace first
  int sfmt = (c.shared_format == QMOE_FMT_INT8_G64) ? FMT_INT8 : FMT_BF16;
  const void* sh_gu_w = wts->sh_gu;
  const void* sh_dn_w = wts->sh_dn;
  if (shared && shared_expands(c, N)) {
    uint16_t* w16 = reinterpret_cast<uint16_t*>(base + L.sh_w16);
    const int64_t gu_elems = static_cast<int64_t>(2) * c.shared_inter * c.hidden;
    rc = launch_expand_int8(reinterpret_cast<const uint32_t*>(wts->sh_gu), wts->sh_gu_sb,
                            2 * c.shared_inter, c.hidden, w16, sstream);
    if (!rc)
      rc = launch_expand_int8(reinterpret_cast<const uint32_t*>(wts->sh_dn), wts->sh_dn_sb,
                              c.hidden, c.shared_inter, w16 + gu_elems, sstream);
    if (rc) return rc;
    sh_gu_w = w16;
    sh_dn_w = w16 + gu_elems;
    sfmt = FMT_BF16;
  }
  const bool sh8 = (sfmt == FMT_INT8);
  if (shared) {
    sgu.act = x; sgu.act_rows = N; sgu.slot_div = 1; sgu.dense_rows = N; sgu.n_experts = 1;
    sgu.K = c.hidden; sgu.n_rows = 2 * c.shared_inter; sgu.codes = sh_gu_w; sgu.out = sh_h;
    sgu.sb = sh8 ? wts->sh_gu_sb : nullptr;
    sgu.ld_out = c.shared_inter;
    sgu.glu = c.act; sgu.glu_alpha = c.act_alpha; sgu.glu_limit = c.act_limit;
    if (!fuse_gu) {
      rc = launch_qmm(sgu, sfmt, EPI_SWIGLU, sreg, (N + st - 1) / st, sstream);
      if (rc) return rc;
    }
  }
  // shared down -> sh_out (fused into the combine when decoding). In the hybrid regime it is
  // enqueued on the auxiliary stream after the cold experts' launches, so it runs beside the hot
  // experts' down projection (where the auxiliary stream has slack) rather than their gate_up.
  auto shared_down_args = [&]() {
    QmmArgs b{};
    b.act = sh_h; b.act_rows = N; b.slot_div = 1; b.dense_rows = N; b.n_experts = 1;
    b.K = c.shared_inter; b.n_rows = c.hidden; b.codes = sh_dn_w; b.out = sh_out;
    b.sb = sh8 ? wts->sh_dn_sb : nullptr;
    b.ld_out = c.hidden;
    return b;
  };
  auto shared_down = [&]() -> int {
    return launch_qmm(shared_down_args(), sfmt, EPI_BF16, sreg, (N + st - 1) / st, sstream);
  };
  // decode batches whose shared down would ride in the combine: with int8 shared weights and
  // int4 routed experts it rides in the routed gate_up's launch instead (the combine then only
  // gathers), when that launch pair has a compiled shape
  bool sdn_in_gate_up = false;
  const bool shared_down_late = shared && !fuse_dn && hybrid && aux && sstream == aux->s;
  // (a shared gate_up in the router pair launch: its down product follows that launch)
  const bool shared_down_after_router = shared && !fuse_dn && !shared_down_late && fuse_gu;
  if (shared && !fuse_dn && !shared_down_late && !fuse_gu) {
    rc = shared_down();
    if (rc) return rc;
  }

  // Decode batches with int4 experts whose shared expert rides in the router launch: everything
  // after that launch (top-k, permute, routed gate_up and down, shared down, combine) runs as one
  // dataflow launch (flow.hip), whose counters the router launch clears. Same outputs, bit for bit.
  const bool use_flow = fuse_gu && slot_major && !mixed && gfmt == FMT_INT4 && dfmt == FMT_INT4 &&
                        decode_flow_enabled(n) &&
                        decode_flow_fits(n, c.top_k, c.n_experts, c.hidden, c.inter, c.shared_inter);
  uint32_t* sync = reinterpret_cast<uint32_t*>(base + L.sync);
  // Decode batches routed through the permute, with the router in the pair launch: that launch's
  // last router workgroups also rank the tokens (one per workgroup, up to 32 workgroups) and the
  // last of them sorts the slots by expert (RouteTail), in place of the top-k and permute
  // launches. Same outputs, bit for bit; 3 us saved per call at c1's shape from 12 to 64 tokens
  // and at c2's with 8, 12 and 48, level elsewhere.
  const bool route_tail = fuse_gu && !use_flow && !slot_major && !hybrid &&
                          c.n_experts <= kRouteTailMaxExperts && c.top_k <= 64 &&
                          N <= kRouteTailMaxTokens && g_route_tail.load(std::memory_order_relaxed) != 0;

  // 2. router logits (+ the shared-expert gate logit in column E)
  int ld = 0;
  if (c.router_format == QMOE_ROUTER_F32) {
    ld = c.n_experts + 1;
    rc = launch_router_f32(x, static_cast<const float*>(wts->router_w),
                           has_sg ? wts->shared_gate_w : nullptr, n, c.hidden, c.n_experts, logits,
                           ld, stream);
  } else {
    ld = c.router_rows;
    QmmArgs a{};
    // the decode kernel stops at the 16-row tile holding logit E (the rows up to router_rows
    // are padding for the large kernel's 256-row tiles)
    const int live_rows = (c.n_experts + has_sg + 15) / 16 * 16;
    a.act = x; a.act_rows = N; a.slot_div = 1; a.dense_rows = N; a.n_experts = 1;
    a.K = c.hidden; a.n_rows = decode ? std::min(live_rows, c.router_rows) : c.router_rows;
    a.codes = wts->router_w; a.out = logits; a.ld_out = ld;
    if (fuse_norm) {   // both products read the raw rows and normalise them; the router writes xn
      a.act = x_in; a.norm_w = norm_w; a.norm_eps = norm_eps; a.norm_out = xn;
      sgu.act = x_in; sgu.norm_w = norm_w; sgu.norm_eps = norm_eps;
    }
    // (large regime: 64-token m-tiles, so the few row blocks of the router still give twice
    // as many workgroups)
    const int rt = decode ? st : 64;
    if (!decode) a.dense_mtile = rt;
    if (use_flow) {
      a.zero_words = sync;
      a.n_zero = static_cast<int>(L.sync_words / kSyncStride);
    }
    if (route_tail) {
      RouteTail T{};
      T.ctr = reinterpret_cast<unsigned long long*>(base + L.route_ctr);
      T.timeouts = route_tail_timeouts_ptr();
      T.logits = logits; T.ld = ld; T.N = n;
      T.P = topk_params(wts->router_bias, c.n_experts, c.top_k, c.scoring, c.n_group, c.topk_group,
                        c.norm_topk, c.routed_scale, has_sg);
      T.idx = idx; T.w = wv; T.sg = sg;
      T.counts = counts; T.offsets = offsets; T.tile_off = tile_off; T.sorted = sorted; T.inv = inv;
      T.tile_map = tile_map; T.max_tiles = static_cast<int>(bound_small);
      T.words = (n + 31) / 32;
      T.vpl = topk_vpl(c.n_experts);
      rc = launch_qmm_pair_route(a, sgu, stream, sfmt, T);
    } else if (fuse_gu) {
      // (where the dataflow launch forms the shared expert's gated activation itself, the pair
      // launch writes its gate and up halves, each tile a job of its own)
      const bool split = use_flow && decode_flow_split_shared(c.hidden, c.inter, c.shared_inter);
      if (split) sgu.ld_out = 2 * c.shared_inter;
      rc = launch_qmm_pair_bf16(a, sgu, stream, sfmt, split);
    } else {
      rc = launch_qmm(a, FMT_BF16, EPI_F32, sreg, (N + rt - 1) / rt, stream);
    }
  }
  if (rc) return rc;
  if (shared_down_after_router) {
    rc = shared_down();
    if (rc) return rc;
  }
  if (use_flow) {
    FlowLaunch F{};
    F.x = x; F.N = n; F.k = c.top_k; F.H = c.hidden; F.I = c.inter; F.Is = c.shared_inter;
    F.logits = logits; F.ld = ld;
    F.P = topk_params(wts->router_bias, c.n_experts, c.top_k, c.scoring, c.n_group, c.topk_group,
                      c.norm_topk, c.routed_scale, has_sg);
    F.gu_codes = wts->gu_codes; F.gu_sb = wts->gu_sb; F.dn_codes = wts->dn_codes; F.dn_sb = wts->dn_sb;
    F.glu = c.act; F.glu_alpha = c.act_alpha; F.glu_limit = c.act_limit;
    F.sh_h = sh_h; F.sh_dn = sh_dn_w; F.sh_dn_sb = sh8 ? wts->sh_dn_sb : nullptr; F.sfmt = sfmt;
    F.w = wv; F.sg = sg;
    F.h = h; F.d = d; F.sh_out = sh_out; F.sync = sync;
    F.resid = resid; F.y = y;
    return launch_decode_flow(F, stream);
  }
  // slot-major int4 SwiGLU experts: the top-k runs inside the routed gate_up launch (one
  // wavefront per workgroup ranks its slot's token), while the launch has few enough workgroups
  const bool route_in_gate_up =
      slot_major && !mixed && gfmt == FMT_INT4 && route_gate_up_fits(c.n_experts, c.top_k) &&
      route_gate_up_workgroups(c.hidden, 2 * c.inter, mc) <= kRouteMaxWorkgroups;
  if (route_in_gate_up || route_tail) {
    // (the routed gate_up below ranks the logits itself; the routing tail has written the
    // routing and the permute's outputs)
  } else if (slot_major) {
    // 3-4. top-k with the slot-major tile map
    rc = launch_topk(logits, ld, wts->router_bias, n, c.n_experts, c.top_k, c.scoring, c.n_group,
                     c.topk_group, c.norm_topk, c.routed_scale, has_sg, idx, wv, sg, stream,
                     tile_map, tiles_small, sorted, inv);
    if (rc) return rc;
  } else {
    // 3. top-k
    rc = launch_topk(logits, ld, wts->router_bias, n, c.n_experts, c.top_k, c.scoring, c.n_group,
                     c.topk_group, c.norm_topk, c.routed_scale, has_sg, idx, wv, sg, stream);
    if (rc) return rc;
    // 4. stable permute by expert (16-row tiles; hybrid: hot experts' 128-row tiles separately)
    rc = launch_permute(idx, n, c.top_k, c.n_experts, kSmallMTile, counts, offsets, tile_off,
                        sorted, inv, tile_map, bound_small, stream, kHybridSplitRows, kLargeMTile,
                        hybrid ? tile_map_big : nullptr, L.max_tiles_big);
    if (rc) return rc;
  }
  // AWQ: each sorted row divided by its expert's gate and up scales (and, for the hybrid
  // regime's hot experts, the fp16 copies of both row sets)
  uint16_t* awq_xg = reinterpret_cast<uint16_t*>(base + L.awq_x);
  if (c.awq && hybrid && c.hidden <= kAwqSplitMaxH) {
    // (hot experts' rows only as their fp16 copies, cold experts' only as bf16)
    rc = launch_awq_prescale_split(x, sorted, offsets, c.n_experts, c.top_k, mc, c.hidden,
                                   wts->awq_gu, kHybridSplitRows, awq_xg, x16, x_sinv, stream);
    if (rc) return rc;
  } else if (c.awq) {
    rc = launch_awq_prescale(x, sorted, offsets, c.n_experts, c.top_k, mc, c.hidden, wts->awq_gu,
                             awq_xg, awq_xg + mc * c.hidden, stream);
    if (!rc && hybrid) rc = launch_act_to_f16(awq_xg, 2 * mc, c.hidden, x16, x_sinv, stream);
    if (rc) return rc;
  }
  // the cold experts' tiles wait for the permute on the auxiliary stream
  hipStream_t cstream = stream;
  if (hybrid && aux) {
    rc = link(aux->perm, stream, aux->s, "permute to auxiliary stream");
    if (rc) return rc;
    cstream = aux->s;
  }
  // routed grouped matmul over the permuted rows: small kernel over the (cold) 16-row tiles,
  // large kernel over the hot experts' tiles (hybrid: the two on different streams; hot and
  // cold experts own disjoint rows of the output)
  auto routed = [&](QmmArgs a, int fmt, int epi, const uint16_t* act16, const float* sinv) {
    a.tile_map = reinterpret_cast<const int4*>(tile_map);
    int r = launch_qmm(a, fmt, epi, QMOE_REGIME_SMALL, hybrid ? cold_bound : tiles_small, cstream);
    if (r || !hybrid) return r;
    a.tile_map = reinterpret_cast<const int4*>(tile_map_big);
    a.act16 = act16;
    a.row_sinv = sinv;
    return launch_qmm(a, fmt, epi, QMOE_REGIME_LARGE, hot_bound, stream);
  };
  if (f16_acts && aux) {   // the fp16 copy of x, made on the auxiliary stream at the fork
    const hipError_t err = hipStreamWaitEvent(stream, aux->xready, 0);
    if (err != hipSuccess) return fail(std::string("forward: x16 wait: ") + hipGetErrorString(err));
  }
  // 5. routed gate_up + SwiGLU -> h (sorted order)
  if (mixed && !has_split(*mixed)) {
    // fused gate_up stacks by width: SwiGLU in the epilogue, straight into h
    for (int i = 0; i < mixed->n_stacks; ++i) {
      const qmoe_stack_t& st = mixed->stacks[i];
      if (st.proj != QMOE_PROJ_GATE_UP) continue;
      QmmArgs a{};
      a.act = x; a.act_rows = N; a.slot_of = sorted; a.slot_div = c.top_k; a.n_slots = mc;
      a.offsets = offsets; a.tile_off = tile_off; a.n_experts = c.n_experts;
      a.K = c.hidden; a.n_rows = 2 * c.inter; a.codes = st.codes; a.sb = st.sb;
      a.expert_map = st.expert_slot; a.out = h; a.ld_out = c.inter;
      a.row_exp = st.row_exp;
      a.glu = c.act; a.glu_alpha = c.act_alpha; a.glu_limit = c.act_limit;
      rc = routed(a, kernel_fmt(st.format), EPI_SWIGLU, x16, x_sinv);
      if (rc) return rc;
    }
    if (hybrid && aux) {   // h complete (cold rows from the auxiliary stream)
      rc = link(aux->cold, aux->s, stream, "cold gate_up");
      if (rc) return rc;
    }
  } else if (mixed) {
    // widths per (expert, projection): gate and up by width into awq_gu, then h = bf16(glu)
    uint16_t* gu = reinterpret_cast<uint16_t*>(base + L.awq_gu);
    for (int i = 0; i < mixed->n_stacks; ++i) {
      const qmoe_stack_t& st = mixed->stacks[i];
      if (st.proj != QMOE_PROJ_GATE && st.proj != QMOE_PROJ_UP) continue;
      QmmArgs a{};
      a.act = x; a.act_rows = N; a.slot_of = sorted; a.slot_div = c.top_k; a.n_slots = mc;
      a.offsets = offsets; a.tile_off = tile_off; a.n_experts = c.n_experts;
      a.K = c.hidden; a.n_rows = c.inter; a.codes = st.codes; a.sb = st.sb;
      a.expert_map = st.expert_slot; a.row_exp = st.row_exp;
      a.out = gu + (st.proj == QMOE_PROJ_UP ? c.inter : 0); a.ld_out = 2 * c.inter;
      rc = routed(a, kernel_fmt(st.format), EPI_BF16, x16, x_sinv);
      if (rc) return rc;
    }
    if (hybrid && aux) {   // all of gu (cold rows from the auxiliary stream) before the glu pass
      rc = link(aux->cold, aux->s, stream, "cold gate_up");
      if (rc) return rc;
    }
    rc = launch_awq_glu(gu, offsets, c.n_experts, mc, c.inter, nullptr, c.act, c.act_alpha,
                        c.act_limit, h, stream);
    if (rc) return rc;
  } else if (c.awq) {
    // AWQ: gate and up on their own prescaled rows (one launch over all 2I rows of each expert,
    // the up half's tiles reading the up rows) into awq_gu, then h = bf16(glu / s_dn)
    uint16_t* gu = reinterpret_cast<uint16_t*>(base + L.awq_gu);
    QmmArgs a{};
    a.act = awq_xg; a.act_hi = awq_xg + mc * c.hidden; a.split_tile = c.inter / 16;
    a.act_rows = mc; a.slot_div = 1; a.n_slots = mc;
    a.offsets = offsets; a.tile_off = tile_off; a.n_experts = c.n_experts;
    a.K = c.hidden; a.n_rows = 2 * c.inter; a.codes = wts->gu_codes; a.sb = wts->gu_sb;
    a.row_exp = fp16_large_fmt(gfmt) ? wts->gu_rexp : nullptr;
    a.out = gu; a.ld_out = 2 * c.inter;
    if (hybrid) { a.act16_hi = x16 + mc * c.hidden; a.row_sinv_hi = x_sinv + mc; }
    rc = routed(a, gfmt, EPI_BF16, x16, x_sinv);
    if (rc) return rc;
    if (hybrid && aux) {   // all of gu (cold rows from the auxiliary stream) before the glu pass
      rc = link(aux->cold, aux->s, stream, "cold gate_up");
      if (rc) return rc;
    }
    rc = launch_awq_glu(gu, offsets, c.n_experts, mc, c.inter, wts->awq_dn, c.act, c.act_alpha,
                        c.act_limit, h, stream);
    if (rc) return rc;
  } else {
    QmmArgs a{};
    a.act = x; a.act_rows = N; a.slot_of = sorted; a.slot_div = c.top_k; a.n_slots = mc;
    a.offsets = offsets; a.tile_off = tile_off; a.n_experts = c.n_experts;
    a.K = c.hidden; a.n_rows = 2 * c.inter; a.codes = wts->gu_codes; a.sb = wts->gu_sb;
    a.row_exp = fp16_large_fmt(gfmt) ? wts->gu_rexp : nullptr;
    a.out = h; a.ld_out = c.inter;
    a.glu = c.act; a.glu_alpha = c.act_alpha; a.glu_limit = c.act_limit;
    // (the fused tail below computes the shared down itself)
    const bool tail = slot_major && dfmt == FMT_INT4 &&
                      down_combine_fits(n, c.top_k, c.hidden, c.inter, c.shared_inter);
    if (route_in_gate_up) {
      a.slot_of = nullptr; a.slot_div = 1; a.n_slots = 0; a.offsets = nullptr; a.tile_off = nullptr;
      const QmmArgs sdn = shared_down_args();
      // (the fused tail then adds the computed shared output instead of its shared units)
      const bool with_sdn = fuse_dn && sh8;
      rc = launch_route_gate_up(a, n, logits, ld, wts->router_bias, c.n_experts, c.top_k, c.scoring,
                                c.n_group, c.topk_group, c.norm_topk, c.routed_scale, has_sg, idx,
                                wv, sg, tile_map, tiles_small, sorted, inv, stream,
                                with_sdn ? &sdn : nullptr);
      if (rc == 1)
        rc = launch_route_gate_up(a, n, logits, ld, wts->router_bias, c.n_experts, c.top_k,
                                  c.scoring, c.n_group, c.topk_group, c.norm_topk, c.routed_scale,
                                  has_sg, idx, wv, sg, tile_map, tiles_small, sorted, inv, stream);
      else
        sdn_in_gate_up = with_sdn && rc == 0;
    } else if (fuse_dn && sh8 && !hybrid && gfmt == FMT_INT4 && !tail) {
      a.tile_map = reinterpret_cast<const int4*>(tile_map);
      rc = launch_gate_up_shared_down(a, tiles_small, shared_down_args(), stream);
      if (rc == 1) rc = routed(a, gfmt, EPI_SWIGLU, x16, x_sinv);
      else sdn_in_gate_up = (rc == 0);
    } else {
      rc = routed(a, gfmt, EPI_SWIGLU, x16, x_sinv);
    }
    if (rc) return rc;
    if (hybrid && aux) {   // h complete (cold rows from the auxiliary stream) before its fp16 copy
      rc = link(aux->cold, aux->s, stream, "cold gate_up");
      if (rc) return rc;
    }
  }
  // 6-7. slot-major decode with a shared expert and one int4 down stack: routed down, shared
  // down and combine in one launch per 16 output features (the down output stays on chip)
  if (slot_major && fuse_dn && !mixed && dfmt == FMT_INT4 &&
      down_combine_fits(n, c.top_k, c.hidden, c.inter, c.shared_inter)) {
    if (sdn_in_gate_up)
      return launch_down_combine(h, idx, wv, has_sg ? sg : nullptr, n, c.top_k, c.hidden, c.inter,
                                 wts->dn_codes, wts->dn_sb, nullptr, 0, nullptr, nullptr, sfmt,
                                 resid, y, stream, sh_out);
    return launch_down_combine(h, idx, wv, has_sg ? sg : nullptr, n, c.top_k, c.hidden, c.inter,
                               wts->dn_codes, wts->dn_sb, sh_h, c.shared_inter, sh_dn_w,
                               sh8 ? wts->sh_dn_sb : nullptr, sfmt, resid, y, stream);
  }
  // 6. routed down -> d (sorted order)
  {
    QmmArgs a{};
    a.act = h; a.act_rows = mc; a.slot_div = 1; a.n_slots = mc;
    a.offsets = offsets; a.tile_off = tile_off; a.n_experts = c.n_experts;
    a.K = c.inter; a.n_rows = c.hidden; a.codes = wts->dn_codes; a.sb = wts->dn_sb;
    a.row_exp = fp16_large_fmt(dfmt) ? wts->dn_rexp : nullptr;
    a.out = d; a.ld_out = c.hidden;
    if (f16_h) {
      rc = launch_act_to_f16(h, mc, c.inter, h16, h_sinv, stream);
      if (rc) return rc;
    }
    if (hybrid && aux) {   // the cold down reads bf16 h, complete since the cold gate_up join
      rc = link(aux->hready, stream, aux->s, "h to auxiliary stream");
      if (rc) return rc;
    }
    if (mixed) {
      for (int i = 0; i < mixed->n_stacks; ++i) {
        const qmoe_stack_t& st = mixed->stacks[i];
        if (st.proj != QMOE_PROJ_DOWN) continue;
        a.codes = st.codes; a.sb = st.sb; a.expert_map = st.expert_slot; a.row_exp = st.row_exp;
        rc = routed(a, kernel_fmt(st.format), EPI_BF16, h16, h_sinv);
        if (rc) return rc;
      }
    } else {
      rc = routed(a, dfmt, EPI_BF16, h16, h_sinv);
      if (rc) return rc;
    }
  }
  if (shared_down_late) {
    rc = shared_down();
    if (rc) return rc;
  }
  if (aux) {
    rc = link(aux->join, aux->s, stream, "join");
    if (rc) return rc;
  }
  // 7. unpermute + weighted combine + gated shared (its down projection fused when decoding) + bf16
  if (fuse_dn && !sdn_in_gate_up)
    return launch_combine_shared(d, inv, wv, n, c.top_k, c.hidden, sh_h, c.shared_inter, sh_dn_w,
                                 sh8 ? wts->sh_dn_sb : nullptr, sfmt, has_sg ? sg : nullptr, y,
                                 stream, resid);
  return launch_combine(d, inv, wv, n, c.top_k, c.hidden, shared ? sh_out : nullptr,
                        has_sg ? sg : nullptr, y, stream, resid);
}

extern "C" int qmoe_forward(const qmoe_config_t* cfg, const qmoe_weights_t* wts, const uint16_t* x,
                            int64_t N, uint16_t* y, void* ws, size_t ws_bytes, void* stream) {
  return forward_impl(cfg, wts, x, N, y, ws, ws_bytes, stream);
}

extern "C" int qmoe_forward_mixed(const qmoe_config_t* cfg, const qmoe_weights_t* wts,
                                  const qmoe_mixed_t* mixed, const uint16_t* x, int64_t N,
                                  uint16_t* y, void* ws, size_t ws_bytes, void* stream) {
  if (!mixed) return fail("qmoe_forward_mixed: null pointer");
  return forward_impl(cfg, wts, x, N, y, ws, ws_bytes, stream, mixed);
}

// The block with the decoder layer's steps either side of it: the normalised rows go to the
// end of the workspace, the block runs on them, and the combine adds the residual.
extern "C" size_t qmoe_forward_residual_workspace(const qmoe_config_t* cfg, int64_t N) {
  if (!cfg || N <= 0 || N > 65535 || cfg->hidden <= 0) return 0;
  return ws_layout(*cfg, N).total + align256(static_cast<size_t>(N) * cfg->hidden * 2);
}

extern "C" int qmoe_forward_residual(const qmoe_config_t* cfg, const qmoe_weights_t* wts,
                                     const uint16_t* x, const uint16_t* norm_w, float eps,
                                     int64_t N, uint16_t* y, void* ws, size_t ws_bytes,
                                     void* stream) {
  if (!cfg || !wts || !x || !norm_w || !y || !ws) return fail("qmoe_forward_residual: null pointer");
  int rc = validate_config(*cfg);
  if (rc) return rc;
  if (N <= 0 || N > 65535) return fail("qmoe_forward_residual: 0 < N <= 65535 tokens per call");
  const size_t main = ws_layout(*cfg, N).total;
  if (ws_bytes < qmoe_forward_residual_workspace(cfg, N))
    return fail("qmoe_forward_residual: workspace too small");
  if (!(eps >= 0.f) || !isfinite(eps)) return fail("qmoe_forward_residual: eps must be finite and >= 0");
  uint16_t* xn = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + main);
  return forward_impl(cfg, wts, x, N, y, ws, main, stream, nullptr, false, norm_w, eps, xn);
}

// ------------------------------------------------------------------ allocation-free entry point
// qmoe_forward for callers that cannot allocate (HIP graph capture, serving loops, harnesses that
// forbid hipMalloc): the per-call workspace is a file-scope device array of fixed size, one copy
// per GPU the library runs on, held until the process ends, and every launch goes on the
// caller's stream (no auxiliary stream or events, which qmoe_forward creates on first use).
// The array's host-side name is not a device address: its address on each device comes from
// hipGetSymbolAddress, taken once per device with that device current, and only that pointer is
// handed to kernels. Calls on one GPU share the array, so calls that overlap on one GPU race;
// nothing in it needs to start at zero (qmoe_forward takes uninitialised workspace too).
constexpr size_t kScratchBytes = static_cast<size_t>(QMOE_NOALLOC_SCRATCH_BYTES);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kScratchMaxDevices = 64;
static void* g_scratch_ptr[kScratchMaxDevices];   // per device: scratch's device address
static std::mutex g_scratch_mu;

static int scratch_on(hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t err = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (err != hipSuccess) return fail(std::string("qmoe_forward_noalloc: stream device: ") + hipGetErrorString(err));
  if (dev < 0 || dev >= kScratchMaxDevices) return fail("qmoe_forward_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    err = hipGetDevice(&cur);
    if (err == hipSuccess && cur != dev) err = hipSetDevice(dev);
    void* p = nullptr;
    if (err == hipSuccess) err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (err != hipSuccess || !p)
      return fail(std::string("qmoe_forward_noalloc: hipGetSymbolAddress(scratch): ") +
                  (err != hipSuccess ? hipGetErrorString(err) : "null address"));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

extern "C" int qmoe_forward_noalloc(const qmoe_config_t* cfg, const qmoe_weights_t* wts,
                                    const uint16_t* x, int64_t N, uint16_t* y, void* stream) {
  if (!cfg || !wts || !x || !y) return fail("qmoe_forward_noalloc: null pointer");
  int rc = validate_config(*cfg);
  if (rc) return rc;
  if (N <= 0 || N > 65535) return fail("qmoe_forward_noalloc: 0 < N <= 65535 tokens per call");
  const size_t need = ws_layout(*cfg, N).total;
  if (need > kScratchBytes)
    return fail("qmoe_forward_noalloc: " + std::to_string(N) + " tokens need " +
                std::to_string(need) + " bytes of workspace, more than the fixed " +
                std::to_string(kScratchBytes) + "-byte scratch; call qmoe_forward with a "
                "workspace, or pass fewer tokens per call");
  void* ws = nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = scratch_on(st, &ws);
  if (rc) return rc;
  return forward_impl(cfg, wts, x, N, y, ws, kScratchBytes, stream, nullptr, true);
}
