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

int launch_router_f32(const uint16_t* x, const float* wr, const float* shared_gate, int N, int H,
                      int E, float* logits, int ld, hipStream_t stream) {
  int rows = E + (shared_gate ? 1 : 0);
  dim3 grid((rows + 3) / 4, (N + 15) / 16);
  router_f32_kernel<<<grid, 256, 0, stream>>>(x, wr, shared_gate, N, H, E, rows, logits, ld);
  return check_launch("router_f32");
}

// ---------------------------------------------------------------- top-k in wavefront registers
// Wavefront reductions from ROCm's device library (declared by HIP's own headers only under an
// opt-in macro). They return the reduction over all active lanes to every lane.
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_max_u64(
    unsigned long long);
extern "C" __device__ __attribute__((const)) float __ockl_wfred_max_f32(float);
extern "C" __device__ __attribute__((const)) float __ockl_wfred_add_f32(float);

// Order-preserving map of a float onto uint32 (larger float -> larger integer).
__device__ __forceinline__ uint32_t orderable(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// Selection key: value first, then the lower id wins a tie.
__device__ __forceinline__ unsigned long long sel_key(float v, int id) {
  return (static_cast<unsigned long long>(orderable(v)) << 32) |
         static_cast<unsigned long long>(0xFFFFFFFFu - static_cast<uint32_t>(id));
}
__device__ __forceinline__ int key_id(unsigned long long key) {
  return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key));
}

// One wavefront per token. Lane l holds experts l*VPL .. l*VPL+VPL-1 (contiguous, so a group
// of E/n_group experts spans whole lanes when VPL divides the group size). Each lane keeps the
// key of its best remaining expert; every round takes one wavefront max-reduction, and only the
// winning lane rescans its VPL values.
template <int VPL>
__global__ void __launch_bounds__(256) topk_kernel(
    const float* __restrict__ logits, int ld, const float* __restrict__ bias, int N, int E, int k,
    int scoring, int n_group, int topk_group, int norm_topk, float scale, int has_sg,
    int32_t* __restrict__ idx_out, float* __restrict__ w_out, float* __restrict__ sg_out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;  // whole wavefront exits together; no block barriers below
  const float NEG_INF = -INFINITY;
  const float* row = logits + static_cast<int64_t>(t) * ld;
  const int e_base = lane * VPL;

  float lg[VPL], sc[VPL], ch[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) lg[i] = (e_base + i < E) ? row[e_base + i] : NEG_INF;
  if (scoring == QMOE_SCORE_SOFTMAX) {
    float m = NEG_INF;
#pragma unroll
    for (int i = 0; i < VPL; ++i) m = fmaxf(m, lg[i]);
    m = __ockl_wfred_max_f32(m);
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      sc[i] = (e_base + i < E) ? expf(lg[i] - m) : 0.f;
      z += sc[i];
    }
    z = __ockl_wfred_add_f32(z);
    const float inv = 1.0f / z;
#pragma unroll
    for (int i = 0; i < VPL; ++i) sc[i] *= inv;
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      sc[i] = (e_base + i < E) ? 1.0f / (1.0f + expf(-lg[i])) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = e_base + i;
    if (e >= E) {
      ch[i] = NEG_INF;
    } else if (bias) {
      ch[i] = sc[i] + bias[e];
    } else {
      // Without a bias, softmax selection by probability equals selection by logit (monotone);
      // the logit avoids ties manufactured by rounding exp(). Sigmoid selects on the score.
      ch[i] = (scoring == QMOE_SCORE_SOFTMAX) ? lg[i] : sc[i];
    }
  }

  if (n_group > 1) {
    const int gsize = E / n_group;
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
      for (int gam = 0; gam < n_group; ++gam) {
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
    for (int r = 0; r < topk_group; ++r) {
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

  // lane's best remaining candidate
  unsigned long long keys[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) keys[i] = (e_base + i < E) ? sel_key(ch[i], e_base + i) : 0ull;
  unsigned long long mine = 0ull;
#pragma unroll
  for (int i = 0; i < VPL; ++i) mine = keys[i] > mine ? keys[i] : mine;

  int my_id = 0;
  float my_w = 0.f;
  for (int r = 0; r < k; ++r) {
    const unsigned long long best = __ockl_wfred_max_u64(mine);
    const int id = key_id(best);
    const int owner = id / VPL;
    float s_win = 0.f;
    if (lane == owner) {
      unsigned long long nb = 0ull;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        if (e_base + i == id) {
          s_win = sc[i];
          keys[i] = 0ull;
        }
        nb = keys[i] > nb ? keys[i] : nb;
      }
      mine = nb;
    }
    s_win = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s_win), owner));
    if (lane == r) { my_id = id; my_w = s_win; }
  }
  const float tot = __ockl_wfred_add_f32(lane < k ? my_w : 0.f);
  if (norm_topk) my_w = my_w / (tot + 1e-20f);
  my_w *= scale;
  if (lane < k) {
    idx_out[static_cast<int64_t>(t) * k + lane] = my_id;
    w_out[static_cast<int64_t>(t) * k + lane] = my_w;
  }
  if (has_sg && lane == 0) sg_out[t] = 1.0f / (1.0f + expf(-row[E]));
}

int launch_topk(const float* logits, int ld, const float* bias, int N, int E, int k, int scoring,
                int n_group, int topk_group, int norm_topk, float scale, int has_sg,
                int32_t* idx, float* w, float* sg_out, hipStream_t stream) {
  dim3 grid((N + 3) / 4);
#define QMOE_TOPK(V)                                                                         \
  topk_kernel<V><<<grid, 256, 0, stream>>>(logits, ld, bias, N, E, k, scoring, n_group,       \
                                           topk_group, norm_topk, scale, has_sg, idx, w, sg_out)
  if (E <= 64) QMOE_TOPK(1);
  else if (E <= 128) QMOE_TOPK(2);
  else if (E <= 256) QMOE_TOPK(4);
  else if (E <= 512) QMOE_TOPK(8);
  else QMOE_TOPK(16);
#undef QMOE_TOPK
  return check_launch("topk");
}

int validate_routing(int N, int H, int E, int k, int scoring, int n_group, int topk_group) {
  if (N <= 0 || H <= 0) return fail("router: N and H must be positive");
  if (E < 1 || E > 1024) return fail("router: 1 <= E <= 1024 required");
  if (k < 1 || k > E || k > 64) return fail("router: 1 <= k <= min(E, 64) required");
  if (scoring != QMOE_SCORE_SOFTMAX && scoring != QMOE_SCORE_SIGMOID)
    return fail("router: scoring must be softmax (0) or sigmoid (1)");
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
