// Router: logits for fp32 router weights (VALU), and the per-token top-k selection in
// wavefront registers (softmax or sigmoid scores, optional correction bias and group-limited
// selection, renormalisation and routed scaling).
//
// Reference: src/quanta/qwen35/moe.py:36-56 (softmax top-k, renorm with +1e-20),
// src/quanta/modeling/moe.py:33-44 and src/quanta/glm/moe.py:44-55 (sigmoid + correction bias,
// bias-free weights, routed_scaling_factor). Group-limited selection (absent from the reference,
// which asserts n_group == 1) follows transformers' DeepseekV3TopkRouter
// (models/deepseek_v3/modeling_deepseek_v3.py:144-170).
//
// Output order is canonical: choice value descending, expert id ascending on ties. The
// reference's argpartition returns the same set in an unspecified order.
#include <math.h>

#include "qmoe_internal.h"
#include "route_common.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

// ---------------------------------------------------------------- fp32-weight router logits
// One wavefront per (expert row, 16-token block). Row E (when shared_gate != null) is the
// shared-expert sigmoid gate logit x . g, computed alongside the router rows.
__global__ void __launch_bounds__(256) router_f32_kernel(const uint16_t* __restrict__ x,
                                                         const float* __restrict__ wr,
                                                         const float* __restrict__ shared_gate,
                                                         int N, int H, int E, int rows,
                                                         float* __restrict__ logits, int ld) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= rows) return;
  const int t0 = blockIdx.y * 16;
  const bool is_gate = (e == E);
  for (int tt = 0; tt < 16; ++tt) {
    const int t = t0 + tt;
    if (t >= N) break;
    const uint16_t* xr = x + static_cast<int64_t>(t) * H;
    float acc = 0.f;
    if (is_gate) {
      for (int h = lane; h < H; h += 64) acc = fmaf(bf16_to_f32(xr[h]), shared_gate[h], acc);
    } else {
      const float* w = wr + static_cast<int64_t>(e) * H;
      for (int h = lane; h < H; h += 64) acc = fmaf(bf16_to_f32(xr[h]), w[h], acc);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) logits[static_cast<int64_t>(t) * ld + e] = acc;
  }
}

// ---------------------------------------------------------------- one-call router logits
// Logits from the router weight as stored, bf16 or fp32 [E, H] row-major, for qmoe_router.
// One wavefront per (expert row, 4-token group): lanes take 8 consecutive columns per step
// (16-byte loads of bf16 x and bf16 weights, two 16-byte loads of fp32 weights), fp32 FMAs, and
// the fixed-order DPP wavefront sum. Row E (shared_gate != null) is the shared-expert gate
// logit. bf16 x bf16 products are exact in fp32, so the logits equal xf.f32 @ gate.f32^T up to
// the fp32 summation order.
template <bool F32W>
__global__ void __launch_bounds__(256) router_rows_kernel(const uint16_t* __restrict__ x,
                                                          const void* __restrict__ wr,
                                                          const void* __restrict__ shared_gate,
                                                          int N, int H, int E, int rows,
                                                          float* __restrict__ logits, int ld) {
  constexpr int TT = 4;
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= rows) return;  // whole wavefronts exit together; no block barriers below
  const int t0 = blockIdx.y * TT;
  const int nt = min(TT, N - t0);
  const size_t row_elems = static_cast<size_t>(e < E ? e : 0) * H;
  const void* wbase = (e < E) ? wr : shared_gate;
  float acc[TT] = {0.f, 0.f, 0.f, 0.f};
  for (int h = lane * 8; h < H; h += 512) {
    float wv[8];
    if (F32W) {
      const float4* wp = reinterpret_cast<const float4*>(static_cast<const float*>(wbase) + row_elems + h);
      const float4 a = wp[0], b = wp[1];
      wv[0] = a.x; wv[1] = a.y; wv[2] = a.z; wv[3] = a.w;
      wv[4] = b.x; wv[5] = b.y; wv[6] = b.z; wv[7] = b.w;
    } else {
      const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(wbase) + row_elems + h);
      const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wv[2 * i] = __uint_as_float(u[i] << 16);
        wv[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
      }
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      if (tt < nt) {
        const uint4 q = *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t0 + tt) * H + h);
        const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[tt] = fmaf(__uint_as_float(u[i] << 16), wv[2 * i], acc[tt]);
          acc[tt] = fmaf(__uint_as_float(u[i] & 0xFFFF0000u), wv[2 * i + 1], acc[tt]);
        }
      }
    }
  }
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const float v = wave_sum_f32(acc[tt]);
    if (tt < nt && lane == 0) logits[static_cast<int64_t>(t0 + tt) * ld + e] = v;
  }
}

int launch_router_f32(const uint16_t* x, const float* wr, const float* shared_gate, int N, int H,
                      int E, float* logits, int ld, hipStream_t stream) {
  int rows = E + (shared_gate ? 1 : 0);
  dim3 grid((rows + 3) / 4, (N + 15) / 16);
  router_f32_kernel<<<grid, 256, 0, stream>>>(x, wr, shared_gate, N, H, E, rows, logits, ld);
  return check_launch("router_f32");
}

// ---------------------------------------------------------------- top-k
// One wavefront per token (topk_token in route_common.h).
// With tile_map (SlotMap), also the slot-major routing of a few tokens: slot m = t*k + s is its
// own one-row m-tile {idx[m], m, 1, 0} and sorted/inv are the identity, in place of the stable
// permute. Every output row is computed independently of the other rows of its m-tile, so the
// results equal those of the sorted order; an expert chosen by two tokens is read twice.
struct SlotMap {
  int4* tile_map;
  int max_tiles;
  int32_t* sorted;
  int32_t* inv;
};

template <int VPL>
__global__ void __launch_bounds__(256) topk_kernel(const float* __restrict__ logits, int ld,
                                                   TopkParams P, int N,
                                                   int32_t* __restrict__ idx_out,
                                                   float* __restrict__ w_out,
                                                   float* __restrict__ sg_out, SlotMap sm) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;  // whole wavefront exits together; no block barriers below
  const int id = topk_store<VPL>(logits, ld, P, t, lane, idx_out, w_out, sg_out);
  if (sm.tile_map) {
    const int m = t * P.k + lane;
    if (lane < P.k) {
      sm.tile_map[m] = make_int4(id, m, 1, 0);
      sm.sorted[m] = m;
      sm.inv[m] = m;
    }
    if (t == 0)
      for (int i = N * P.k + lane; i < sm.max_tiles; i += 64) sm.tile_map[i] = make_int4(-1, 0, 0, 0);
  }
}

int launch_topk(const float* logits, int ld, const float* bias, int N, int E, int k, int scoring,
                int n_group, int topk_group, int norm_topk, float scale, int has_sg,
                int32_t* idx, float* w, float* sg_out, hipStream_t stream, int32_t* tile_map,
                int64_t max_tiles, int32_t* sorted, int32_t* inv) {
  const TopkParams P = topk_params(bias, E, k, scoring, n_group, topk_group, norm_topk, scale, has_sg);
  SlotMap sm{};
  if (tile_map) {
    if (!sorted || !inv || max_tiles < static_cast<int64_t>(N) * k || max_tiles > (int64_t(1) << 30))
      return fail("topk: slot-major routing needs sorted, inv and N*k tiles");
    sm = SlotMap{reinterpret_cast<int4*>(tile_map), static_cast<int>(max_tiles), sorted, inv};
  }
  dim3 grid((N + 3) / 4);
#define QMOE_TOPK(V) topk_kernel<V><<<grid, 256, 0, stream>>>(logits, ld, P, N, idx, w, sg_out, sm)
  switch (topk_vpl(E)) {
    case 1: QMOE_TOPK(1); break;
    case 2: QMOE_TOPK(2); break;
    case 4: QMOE_TOPK(4); break;
    case 8: QMOE_TOPK(8); break;
    default: QMOE_TOPK(16); break;
  }
#undef QMOE_TOPK
  return check_launch("topk");
}

int validate_routing(int N, int H, int E, int k, int scoring, int n_group, int topk_group) {
  if (N <= 0 || H <= 0) return fail("router: N and H must be positive");
  if (E < 1 || E > 1024) return fail("router: 1 <= E <= 1024 required");
  if (k < 1 || k > E || k > 64) return fail("router: 1 <= k <= min(E, 64) required");
  if (scoring != QMOE_SCORE_SOFTMAX && scoring != QMOE_SCORE_SIGMOID &&
      scoring != QMOE_SCORE_SQRTSOFTPLUS)
    return fail("router: scoring must be softmax (0), sigmoid (1) or sqrtsoftplus (2)");
  if (n_group < 1 || n_group > 64 || E % n_group) return fail("router: E % n_group == 0, n_group <= 64");
  if (n_group > 1) {
    if (E / n_group < 2) return fail("router: group-limited routing needs >= 2 experts per group");
    if (topk_group < 1 || topk_group > n_group) return fail("router: 1 <= topk_group <= n_group");
    if (k > topk_group * (E / n_group)) return fail("router: k exceeds experts in kept groups");
  }
  return 0;
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int qmoe_router_topk(const float* logits, int64_t ld_logits, const float* bias,
                                int64_t N, int E, int k, int scoring, int n_group, int topk_group,
                                int norm_topk, float routed_scale, int has_shared_gate,
                                int32_t* idx, float* w, float* shared_gate_out, void* stream) {
  int rc = validate_routing(static_cast<int>(N), 1, E, k, scoring, n_group, topk_group);
  if (rc) return rc;
  if (N > (int64_t(1) << 30)) return fail("qmoe_router_topk: N too large");
  if (norm_topk < QMOE_NORM_NONE || norm_topk > QMOE_NORM_MULTI)
    return fail("qmoe_router_topk: norm_topk must be QMOE_NORM_NONE, _ALWAYS or _MULTI");
  if (ld_logits < E + (has_shared_gate ? 1 : 0)) return fail("qmoe_router_topk: ld_logits too small");
  if (!logits || !idx || !w || (has_shared_gate && !shared_gate_out))
    return fail("qmoe_router_topk: null pointer");
  return launch_topk(logits, static_cast<int>(ld_logits), bias, static_cast<int>(N), E, k, scoring,
                     n_group, topk_group, norm_topk, routed_scale, has_shared_gate, idx, w,
                     shared_gate_out, static_cast<hipStream_t>(stream));
}

extern "C" int qmoe_router_logits_f32(const uint16_t* x, const float* wr,
                                      const float* shared_gate, int64_t N, int H, int E,
                                      float* logits, int64_t ld_logits, void* stream) {
  if (N <= 0 || N > (int64_t(1) << 30) || H <= 0 || E <= 0) return fail("qmoe_router_logits_f32: bad dims");
  if (ld_logits < E + (shared_gate ? 1 : 0)) return fail("qmoe_router_logits_f32: ld_logits too small");
  if (!x || !wr || !logits) return fail("qmoe_router_logits_f32: null pointer");
  return launch_router_f32(x, wr, shared_gate, static_cast<int>(N), H, E, logits,
                           static_cast<int>(ld_logits), static_cast<hipStream_t>(stream));
}

extern "C" size_t qmoe_router_workspace(int64_t N, int E) {
  if (N <= 0 || E <= 0) return 0;
  return align256(static_cast<size_t>(N) * (E + 1) * sizeof(float));
}

extern "C" int qmoe_router(const uint16_t* x, const void* wr, int wr_is_f32, const void* shared_gate,
                           const float* bias, int64_t N, int H, int E, int k, int scoring,
                           int n_group, int topk_group, int norm_topk, float routed_scale,
                           int32_t* idx, float* w, float* shared_gate_out, void* ws,
                           size_t ws_bytes, void* stream) {
  if (N <= 0 || N > (int64_t(1) << 30)) return fail("qmoe_router: 0 < N <= 2^30 required");
  int rc = validate_routing(static_cast<int>(N), H, E, k, scoring, n_group, topk_group);
  if (rc) return rc;
  if (H % 8) return fail("qmoe_router: H % 8 == 0 required");
  if (wr_is_f32 != 0 && wr_is_f32 != 1) return fail("qmoe_router: wr_is_f32 must be 0 or 1");
  if (norm_topk < QMOE_NORM_NONE || norm_topk > QMOE_NORM_MULTI)
    return fail("qmoe_router: norm_topk must be QMOE_NORM_NONE, _ALWAYS or _MULTI");
  if (!x || !wr || !idx || !w || !ws || (shared_gate && !shared_gate_out))
    return fail("qmoe_router: null pointer");
  if (ws_bytes < qmoe_router_workspace(N, E)) return fail("qmoe_router: workspace too small");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(wr) |
       reinterpret_cast<uintptr_t>(shared_gate)) % 16)
    return fail("qmoe_router: x, wr and shared_gate must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* logits = static_cast<float*>(ws);
  const int ld = E + 1;
  const int rows = E + (shared_gate ? 1 : 0);
  const dim3 grid((rows + 3) / 4, static_cast<unsigned>((N + 3) / 4));
  if (grid.y > 65535u) return fail("qmoe_router: N <= 262140 tokens per call");
  if (wr_is_f32)
    router_rows_kernel<true><<<grid, 256, 0, st>>>(x, wr, shared_gate, static_cast<int>(N), H, E,
                                                   rows, logits, ld);
  else
    router_rows_kernel<false><<<grid, 256, 0, st>>>(x, wr, shared_gate, static_cast<int>(N), H, E,
                                                    rows, logits, ld);
  if ((rc = check_launch("qmoe_router logits"))) return rc;
  return launch_topk(logits, ld, bias, static_cast<int>(N), E, k, scoring, n_group, topk_group,
                     norm_topk, routed_scale, shared_gate ? 1 : 0, idx, w, shared_gate_out, st);
}
