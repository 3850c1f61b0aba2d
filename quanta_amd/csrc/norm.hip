// RMSNorm of the block's input (the decoder layer's post_attention_layernorm), for the block
// entry that also carries the residual add after it.
//
// Reference: the decoder layer runs x = x + mlp(post_attention_layernorm(x))
// (src/quanta/qwen35/model.py:104-105; the batched decode step src/quanta/qwen35/
// batched_runtime.py:304-306). post_attention_layernorm is nn.RMSNorm whose resident weight is
// source + 1 (src/quanta/qwen35/runtime.py:57-63); the reference restates its norms as fp32
// math rounded once to the input dtype: (w * (x * rsqrt(mean(x^2) + eps))).astype(x.dtype)
// (src/quanta/qwen35/attention.py:113-117; src/quanta/qwen35/mtp.py:40-42, "matching the
// model's norms").
//
// One wavefront per row. The sum of squares is accumulated in fp32 in a fixed order, so a row's
// result does not depend on the other rows. For H % 32 == 0 (every block shape) it is the
// canonical order that the router launch with the norm fused in also follows (qmm.hip, the bf16
// pair launch): K cut into bf16_chunks(H) chunks of 32-wide steps, lane group g (0..3) of a chunk
// summing elements 32 s + 8 g + j (steps in order, j = 0..7 in order), the group sums combined as
// (g0 + g1) + (g2 + g3), and the chunk sums added in chunk order; so the block gives the same
// bits with the norm fused or launched on its own. Other widths: lanes over strided 8-element
// pieces and a butterfly.
#include <math.h>

#include "qmoe_internal.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w, int64_t N,
                                                      int H, int nch, float eps,
                                                      uint16_t* __restrict__ out) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= N) return;   // the whole wavefront
  const u32x4* src = reinterpret_cast<const u32x4*>(x + row * H);
  const u32x4* wv = reinterpret_cast<const u32x4*>(w);
  const int n8 = H / 8;
  float ss;
  if (nch > 0) {   // canonical order: lane 4c + g sums lane group g of chunk c
    const int nks = H / 32, c = lane >> 2, g = lane & 3;
    float p = 0.f;
    if (c < nch) {
      const int s0 = c * nks / nch, s1 = (c + 1) * nks / nch;
      // batches of 8 steps, every load issued before the first sum (clamped indices)
      for (int b = s0; b < s1; b += 8) {
        u32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = src[min(b + i, s1 - 1) * 4 + g];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (b + i < s1) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float lo = bf16lo_to_f32(v[i][j]), hi = bf16hi_to_f32(v[i][j]);
              p = fmaf(lo, lo, p);
              p = fmaf(hi, hi, p);
            }
          }
      }
    }
    p += __shfl_xor(p, 1);
    p += __shfl_xor(p, 2);
    ss = __shfl(p, 0);
    for (int cc = 1; cc < nch; ++cc) ss += __shfl(p, 4 * cc);
  } else {
    float p = 0.f;
    for (int i = lane; i < n8; i += 64) {
      const u32x4 v = src[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16lo_to_f32(v[j]), hi = bf16hi_to_f32(v[j]);
        p = fmaf(lo, lo, p);
        p = fmaf(hi, hi, p);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) p += __shfl_xor(p, off);
    ss = p;
  }
  const float r = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  u32x4* dst = reinterpret_cast<u32x4*>(out + row * H);
  for (int i0 = lane; i0 < n8; i0 += 4 * 64) {   // four 16-byte pieces per lane in flight
    u32x4 v[4], g[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = min(i0 + 64 * q, n8 - 1);
      v[q] = src[i];
      g[q] = wv[i];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (i0 + 64 * q >= n8) break;
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2_rne(bf16lo_to_f32(g[q][j]) * (bf16lo_to_f32(v[q][j]) * r),
                               bf16hi_to_f32(g[q][j]) * (bf16hi_to_f32(v[q][j]) * r));
      dst[i0 + 64 * q] = o;
    }
  }
}

int launch_rmsnorm(const uint16_t* x, const uint16_t* w, int64_t N, int H, float eps, uint16_t* out,
                   hipStream_t stream) {
  if (N <= 0) return 0;
  if (H <= 0 || H % 8) return fail("rmsnorm: H % 8 == 0 required");
  if (N > (int64_t(0x7fffffff) * 4)) return fail("rmsnorm: too many rows");
  if (!(eps >= 0.f) || !isfinite(eps)) return fail("rmsnorm: eps must be finite and >= 0");
  const int nch = (H % 32 == 0) ? bf16_chunks(H) : 0;
  rmsnorm_kernel<<<static_cast<unsigned>((N + 3) / 4), 256, 0, stream>>>(x, w, N, H, nch, eps, out);
  return check_launch("rmsnorm");
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int qmoe_rmsnorm(const uint16_t* x, const uint16_t* w, int64_t N, int H, float eps,
                            uint16_t* out, void* stream) {
  if (!x || !w || !out) return fail("qmoe_rmsnorm: null pointer");
  if (N < 0) return fail("qmoe_rmsnorm: N must be >= 0");
  return launch_rmsnorm(x, w, N, H, eps, out, static_cast<hipStream_t>(stream));
}
