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
// One workgroup per row. The sum of squares is accumulated in fp32 in a fixed order (each
// thread over its strided 8-element chunks, then a fixed butterfly within the wavefront, then
// the four wavefront sums in order), so a row's result does not depend on the other rows.
#include <math.h>

#include "qmoe_internal.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w, int H,
                                                      float eps, uint16_t* __restrict__ out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(x + row * H);
  const u32x4* wv = reinterpret_cast<const u32x4*>(w);
  const int n8 = H / 8;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n8; i += 256) {
    const u32x4 v = src[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf16lo_to_f32(v[j]), b = bf16hi_to_f32(v[j]);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = ((red[0] + red[1]) + red[2]) + red[3];
  const float r = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  u32x4* dst = reinterpret_cast<u32x4*>(out + row * H);
  for (int i = threadIdx.x; i < n8; i += 256) {
    const u32x4 v = src[i], g = wv[i];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = bf16lo_to_f32(g[j]) * (bf16lo_to_f32(v[j]) * r);
      const float hi = bf16hi_to_f32(g[j]) * (bf16hi_to_f32(v[j]) * r);
      o[j] = pack_bf16x2(lo, hi);
    }
    dst[i] = o;
  }
}

int launch_rmsnorm(const uint16_t* x, const uint16_t* w, int64_t N, int H, float eps, uint16_t* out,
                   hipStream_t stream) {
  if (N <= 0) return 0;
  if (H <= 0 || H % 8) return fail("rmsnorm: H % 8 == 0 required");
  if (N > 0x7fffffff) return fail("rmsnorm: too many rows");
  if (!(eps >= 0.f) || !isfinite(eps)) return fail("rmsnorm: eps must be finite and >= 0");
  rmsnorm_kernel<<<static_cast<unsigned>(N), 256, 0, stream>>>(x, w, H, eps, out);
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
