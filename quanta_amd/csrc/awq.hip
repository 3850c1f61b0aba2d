// Activation-aware (AWQ) expert scales around the routed grouped matmuls.
//
// Reference: DeepSeek-V4's packed experts hold the codes of W·diag(s) with a per-expert,
// per-input-channel awq_scale s for each projection; the routed SwiGLU divides the gathered
// activation by s before each quantized matmul: g = qmm(x / s_w1), u = qmm(x / s_w3),
// h = silu(clamp(g)) * clamp(u), d = qmm(h / s_w2), the divisions in fp32 and the quotients
// rounded to bf16 by the matmul's bf16 input (src/quanta/dsv4/moe.py:112-137; the scales come
// from the artifact's {key}.awq_scale, src/quanta/dsv4/artifact.py:252-290, all ones for RTN
// experts).
//
// The gate and up projections of one row then read different activations, so they cannot share
// the decode kernel's activation fragments: the block runs gate_up with the bf16 epilogue, the
// gate half's wavefronts reading the rows prescaled for the gate and the up half's those for the
// up projection (QmmArgs::act_hi), and the gated activation with the down projection's division
// as one pass between gate_up and down.
#include "qmoe_internal.h"

namespace qmoe {

// Owner of sorted row m: the last expert e with offsets[e] <= m (empty experts share their
// offset with the next one, which is the owner).
__device__ __forceinline__ int expert_of_row(const int32_t* __restrict__ offsets, int E, int64_t m) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[mid] <= m) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// One workgroup per sorted row; each thread 8 channels at a time.
__global__ void __launch_bounds__(256) awq_prescale_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ offsets, int E, int k, int H, const uint16_t* __restrict__ s_gu,
    uint16_t* __restrict__ xg, uint16_t* __restrict__ xu) {
  const int64_t m = blockIdx.x;
  const int e = expert_of_row(offsets, E, m);
  const int64_t tok = sorted[m] / k;
  const u32x4* xs = reinterpret_cast<const u32x4*>(x + tok * H);
  const u32x4* sg = reinterpret_cast<const u32x4*>(s_gu + static_cast<int64_t>(e) * 2 * H);
  const u32x4* su = sg + H / 8;
  u32x4* og = reinterpret_cast<u32x4*>(xg + m * H);
  u32x4* ou = reinterpret_cast<u32x4*>(xu + m * H);
  for (int i = threadIdx.x; i < H / 8; i += 256) {
    const u32x4 v = xs[i], a = sg[i], b = su[i];
    u32x4 rg, ru;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = bf16lo_to_f32(v[j]), hi = bf16hi_to_f32(v[j]);
      // correctly rounded fp32 quotients (hipcc's default division), then one bf16 rounding
      rg[j] = pack_bf16x2(lo / bf16lo_to_f32(a[j]), hi / bf16hi_to_f32(a[j]));
      ru[j] = pack_bf16x2(lo / bf16lo_to_f32(b[j]), hi / bf16hi_to_f32(b[j]));
    }
    og[i] = rg;
    ou[i] = ru;
  }
}

// Hybrid (prefill) regime: one wavefront per (sorted row, projection), the row's quotients
// bf16(x / s) held in registers (RPL 16-byte pieces per lane). A cold expert's row (at most
// split_rows rows, read by the decode kernel) is written as bf16 into xgu [2][mc][H]; a hot
// expert's row only as the fp16 copy that the prefill kernels read, x16 [2][mc][H] with its
// inverse scale x_sinv [2][mc]: fp16(q * 2^(14 - e)) with 2^(e-1) <= max|q| < 2^e, the conversion
// of act_to_f16 (qmm.hip) applied to the same bf16 quotients, so both paths give the same bits.
// Hot and cold follow the permute's split: more than split_rows rows.
template <int RPL>
__global__ void __launch_bounds__(256) awq_prescale_split_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ offsets, int E, int k, int H, int64_t mc,
    const uint16_t* __restrict__ s_gu, int split_rows, uint16_t* __restrict__ xgu,
    uint16_t* __restrict__ x16, float* __restrict__ x_sinv) {
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t m = w >> 1;
  const int proj = static_cast<int>(w & 1);   // 0: gate, 1: up
  if (m >= mc) return;   // whole wavefront
  const int e = expert_of_row(offsets, E, m);
  const bool hot = offsets[e + 1] - offsets[e] > split_rows;
  const int64_t tok = sorted[m] / k;
  const u32x4* xs = reinterpret_cast<const u32x4*>(x + tok * H);
  const u32x4* sc = reinterpret_cast<const u32x4*>(s_gu + (static_cast<int64_t>(e) * 2 + proj) * H);
  const int n8 = H / 8;
  const int64_t orow = proj * mc + m;
  u32x4 v[RPL];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = u32x4{0u, 0u, 0u, 0u};
    if (c < n8) {
      const u32x4 xv = xs[c], sv = sc[c];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // correctly rounded fp32 quotients, one bf16 rounding (as awq_prescale_kernel)
        v[i][j] = pack_bf16x2(bf16lo_to_f32(xv[j]) / bf16lo_to_f32(sv[j]),
                              bf16hi_to_f32(xv[j]) / bf16hi_to_f32(sv[j]));
        amax = fmaxf(amax, fabsf(bf16lo_to_f32(v[i][j])));
        amax = fmaxf(amax, fabsf(bf16hi_to_f32(v[i][j])));
      }
    }
  }
  if (!hot) {
    u32x4* dst = reinterpret_cast<u32x4*>(xgu + orow * H);
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      const int c = lane + 64 * i;
      if (c < n8) dst[c] = v[i];
    }
    return;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  int ex = 0;
  const bool fin = amax > 0.f && amax <= 3.4e38f;
  if (fin) frexpf(amax, &ex);   // amax = f * 2^ex, f in [0.5, 1)
  const int sh = fin ? 14 - ex : 0;
  if (lane == 0) x_sinv[orow] = ldexpf(1.0f, -sh);
  u32x4* dst = reinterpret_cast<u32x4*>(x16 + orow * H);
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int c = lane + 64 * i;
    if (c < n8) {
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f16x2_t hv = {static_cast<_Float16>(ldexpf(bf16lo_to_f32(v[i][j]), sh)),
                            static_cast<_Float16>(ldexpf(bf16hi_to_f32(v[i][j]), sh))};
        o[j] = __builtin_bit_cast(uint32_t, hv);
      }
      dst[c] = o;
    }
  }
}

__global__ void __launch_bounds__(256) awq_glu_kernel(
    const uint16_t* __restrict__ gu, const int32_t* __restrict__ offsets, int E, int I,
    const uint16_t* __restrict__ s_dn, int act, float alpha, float limit, uint16_t* __restrict__ h) {
  const int64_t m = blockIdx.x;
  const u32x4* g4 = reinterpret_cast<const u32x4*>(gu + m * 2 * I);
  const u32x4* u4 = g4 + I / 8;
  u32x4* o4 = reinterpret_cast<u32x4*>(h + m * I);
  if (!s_dn) {   // no down-projection scales (experts of mixed widths): h = bf16(glu(g, u))
    for (int i = threadIdx.x; i < I / 8; i += 256) {
      const u32x4 g = g4[i], u = u4[i];
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(glu_f(bf16lo_to_f32(g[j]), bf16lo_to_f32(u[j]), act, alpha, limit),
                           glu_f(bf16hi_to_f32(g[j]), bf16hi_to_f32(u[j]), act, alpha, limit));
      o4[i] = o;
    }
    return;
  }
  const int e = expert_of_row(offsets, E, m);
  const u32x4* s4 = reinterpret_cast<const u32x4*>(s_dn + static_cast<int64_t>(e) * I);
  for (int i = threadIdx.x; i < I / 8; i += 256) {
    const u32x4 g = g4[i], u = u4[i], s = s4[i];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = glu_f(bf16lo_to_f32(g[j]), bf16lo_to_f32(u[j]), act, alpha, limit);
      const float hi = glu_f(bf16hi_to_f32(g[j]), bf16hi_to_f32(u[j]), act, alpha, limit);
      o[j] = pack_bf16x2(lo / bf16lo_to_f32(s[j]), hi / bf16hi_to_f32(s[j]));
    }
    o4[i] = o;
  }
}

int launch_awq_prescale(const uint16_t* x, const int32_t* sorted, const int32_t* offsets, int E,
                        int k, int64_t mc, int H, const uint16_t* s_gu, uint16_t* xg, uint16_t* xu,
                        hipStream_t stream) {
  if (mc <= 0) return 0;
  if (H <= 0 || H % 8) return fail("awq prescale: H % 8 == 0 required");
  if (E <= 0 || k <= 0) return fail("awq prescale: E, k > 0 required");
  if (mc > 0x7fffffff) return fail("awq prescale: too many rows");
  awq_prescale_kernel<<<static_cast<unsigned>(mc), 256, 0, stream>>>(x, sorted, offsets, E, k, H,
                                                                      s_gu, xg, xu);
  return check_launch("awq prescale");
}

int launch_awq_prescale_split(const uint16_t* x, const int32_t* sorted, const int32_t* offsets,
                              int E, int k, int64_t mc, int H, const uint16_t* s_gu,
                              int split_rows, uint16_t* xgu, uint16_t* x16, float* x_sinv,
                              hipStream_t stream) {
  if (mc <= 0) return 0;
  if (H <= 0 || H % 8 || H > kAwqSplitMaxH) return fail("awq prescale: H % 8 == 0, H <= 8192 required");
  if (E <= 0 || k <= 0) return fail("awq prescale: E, k > 0 required");
  if (mc > (int64_t(1) << 30)) return fail("awq prescale: too many rows");
  const unsigned grid = static_cast<unsigned>((2 * mc + 3) / 4);
  const int rpl = (H / 8 + 63) / 64;   // 16-byte pieces per lane
#define QMOE_AWQ(R)                                                                      \
  awq_prescale_split_kernel<R><<<grid, 256, 0, stream>>>(x, sorted, offsets, E, k, H, mc, s_gu, \
                                                         split_rows, xgu, x16, x_sinv)
  if (rpl <= 4) QMOE_AWQ(4);
  else if (rpl <= 8) QMOE_AWQ(8);
  else if (rpl <= 12) QMOE_AWQ(12);
  else QMOE_AWQ(16);
#undef QMOE_AWQ
  return check_launch("awq prescale");
}

int launch_awq_glu(const uint16_t* gu, const int32_t* offsets, int E, int64_t mc, int I,
                   const uint16_t* s_dn, int act, float alpha, float limit, uint16_t* h,
                   hipStream_t stream) {
  if (mc <= 0) return 0;
  if (I <= 0 || I % 8) return fail("awq glu: I % 8 == 0 required");
  if (mc > 0x7fffffff) return fail("awq glu: too many rows");
  awq_glu_kernel<<<static_cast<unsigned>(mc), 256, 0, stream>>>(gu, offsets, E, I, s_dn, act, alpha,
                                                                 limit, h);
  return check_launch("awq glu");
}

}  // namespace qmoe
