// Slot-major decode tail: routed down projection, shared-expert down projection and the weighted
// combine in one launch, for batches routed slot-major (a few tokens, every slot its own row).
//
// Reference: the down gather_qmm src/quanta/qwen35/moe.py:121-123, the combine
// src/quanta/qwen35/moe.py:191, the shared expert and its sigmoid gate
// src/quanta/qwen35/moe.py:145-151,201-202.
//
// One workgroup owns 16 output features f and every slot of the batch. Its wavefronts take
// units of work round-robin:
//   * shared unit c (c < nch): chunk c of the shared expert's down product for the 16 features
//     and all tokens (the chunking and step order of combine_shared_kernel);
//   * routed unit (m, c): chunk c of slot m's down product, one 16-row tile of its expert's
//     int4 down stack (the chunking and per-superblock arithmetic of the decode kernel:
//     MFMA on the raw codes as bf16 128 + q, affine fix-up per 64-wide group).
// Partial sums meet in LDS, are added in chunk order, rounded to bf16 (the down output d and
// the shared output, bf16 tensors in the reference), then summed over each token's slots in
// slot order in fp32: y = bf16(fmaf(sh, g, sum_s w * d)) (+ the residual row). With sh_out the
// shared output comes computed (by the routed gate_up's launch) and no shared units run. Every value
// equals the unfused path's (decode kernel, combine_shared_kernel) bit for bit, and the down
// output never round-trips HBM.
//
// A wavefront streams its units with two register stages: the loads of its next unit are in
// flight while the current one is multiplied.
#include "qmoe_internal.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

constexpr int kDcSpu = 4;          // superblocks per routed unit (one K chunk)
constexpr int kDcMaxSlots = 96;    // slots per call (N * k)
constexpr int kDcMaxChunks = 2;    // K chunks of the routed down product
constexpr int kDcMaxTokens = 16;   // tokens per call (one m-tile of the shared product)
constexpr int kDcSharedWaves = 8;  // the shared product's chunk partials, as combine_shared_kernel
// Units per workgroup (8 wavefronts): beyond about three per wavefront the workgroup's serial
// stream costs more than the separate down and combine launches (measured at c1 and c2, N >= 4).
constexpr int kDcMaxUnits = 24;

struct DcArgs {
  const uint16_t* h;        // [N*k][I] bf16, slot order
  const int32_t* idx;       // [N*k] expert of each slot
  const float* w;           // [N*k] routing weight of each slot
  const float* sg;          // [N] shared-expert gate (nullable: 1)
  const void* codes;        // tiled int4 down stack [E][H/16][I/128][64][4 u32]
  const uint16_t* sb;       // tiled scale/bias
  const uint16_t* sh_h;     // [N][Is] bf16 (nullable: no shared expert)
  const void* wd;           // shared down, tiled bf16 or int8
  const uint16_t* wd_sb;    // shared down scale/bias (int8)
  const uint16_t* resid;    // nullable residual rows [N][H]
  const uint16_t* sh_out;   // [N][H] bf16 shared output computed earlier (with sh_h null), or null
  uint16_t* y;              // [N][H]
  int N, k, H, I, Is, nch, chd;
};

struct DcUnit {
  u32x4 q[kDcSpu];
  uint2 sb[kDcSpu];
  u32x4 x[kDcSpu][4];
};

template <int SFMT, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) down_combine_kernel(DcArgs a) {
  __shared__ float part_r[kDcMaxSlots][kDcMaxChunks][16];
  __shared__ f32x4_t spart[kDcSharedWaves][64];
  __shared__ float sh[kDcMaxTokens][17];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int fb = blockIdx.x;
  const int lg = lane >> 4;
  const int mc = a.N * a.k;
  const int nsb = a.I / 128;
  const int tiles_per_expert = a.H / 16;

  // ---- shared expert: chunk `wave` of the down product (waves past nch contribute zeros)
  if (a.sh_h && wave < kDcSharedWaves) {
    const int nks = a.Is / 32;
    const int c0 = (wave < a.nch) ? wave * nks / a.nch : 0;
    const int c1 = (wave < a.nch) ? (wave + 1) * nks / a.nch : 0;
    DenseTile<SFMT> wt;
    wt.init(a.wd, a.wd_sb, fb, a.Is, lane);
    const int tr = lane & 15;
    const uint16_t* xr = a.sh_h + static_cast<int64_t>(tr < a.N ? tr : 0) * a.Is + 8 * lg;
    f32x4_t acc{0.f, 0.f, 0.f, 0.f};
    constexpr int BS = 8;
    for (int cb = c0; cb < c1; cb += BS) {
      DenseFrag<SFMT> wv[BS];
      u32x4 xv[BS];
#pragma unroll
      for (int i = 0; i < BS; ++i) {
        const int c = min(cb + i, c1 - 1);
        wv[i] = wt.load(c);
        xv[i] = *reinterpret_cast<const u32x4*>(xr + 32 * c);
      }
#pragma unroll
      for (int i = 0; i < BS; ++i)
        if (cb + i < c1) acc = mfma16(as_bf16x8(xv[i]), as_bf16x8(dense_bf16<SFMT>(wv[i])), acc);
    }
    spart[wave][lane] = acc;
  }

  // ---- routed units (m, c), round-robin after the shared chunks
  const int n_units = mc * a.chd;
  const int nsh = a.sh_h ? a.nch : 0;
  int r = ((wave - nsh) % WAVES + WAVES) % WAVES;
  const uint32_t lane_c = static_cast<uint32_t>(lane) * 16u;
  const uint32_t lane_s = static_cast<uint32_t>(lane & 15) * 8u;
  auto load_unit = [&](DcUnit& U, int ru) __attribute__((always_inline)) {
    const int m = ru / a.chd, c = ru - m * a.chd;
    const int e = a.idx[m];
    const int64_t tb = (static_cast<int64_t>(e) * tiles_per_expert + fb) * nsb + c * kDcSpu;
    const char* cp = static_cast<const char*>(a.codes) + tb * 1024 + lane_c;
    const char* sp = reinterpret_cast<const char*>(a.sb) + tb * 128 + lane_s;
    const u32x4* xp = reinterpret_cast<const u32x4*>(a.h + static_cast<int64_t>(m) * a.I +
                                                      c * kDcSpu * 128) + 2 * lg;
#pragma unroll
    for (int p = 0; p < kDcSpu; ++p) {
      U.q[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cp + p * 1024));
      const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(sp + p * 128));
      U.sb[p] = uint2{v.x, v.y};
      U.x[p][0] = xp[p * 16 + 0];
      U.x[p][1] = xp[p * 16 + 1];
      U.x[p][2] = xp[p * 16 + 8];
      U.x[p][3] = xp[p * 16 + 9];
    }
  };
  bf16x8_t ones;
  {
    uint32_t* o = reinterpret_cast<uint32_t*>(&ones);
    o[0] = o[1] = o[2] = o[3] = 0x3F803F80u;
  }
  const f32x4_t zero4{0.f, 0.f, 0.f, 0.f};
  // one chunk's sum from zero, superblocks in order (the decode kernel's compute, one tile)
  auto compute_unit = [&](const DcUnit& U, int ru) __attribute__((always_inline)) {
    f32x4_t acc = zero4;
#pragma unroll
    for (int p = 0; p < kDcSpu; ++p) {
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const bf16x8_t A0 = as_bf16x8(U.x[p][2 * gg]);
        const bf16x8_t A1 = as_bf16x8(U.x[p][2 * gg + 1]);
        f32x4_t xs = mfma16(A0, ones, zero4);
        xs = mfma16(A1, ones, xs);
        const uint32_t w0 = gg ? U.q[p].z : U.q[p].x;
        const uint32_t w1 = gg ? U.q[p].w : U.q[p].y;
        f32x4_t rr = mfma16(A0, unpack_q128(w0), zero4);
        rr = mfma16(A1, unpack_q128(w1), rr);
        const uint32_t sbw = gg ? U.sb[p].y : U.sb[p].x;
        const float sc = bf16lo_to_f32(sbw);
        const float bi = bf16hi_to_f32(sbw) - 128.0f * sc;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = fmaf(sc, rr[j], fmaf(bi, xs[j], acc[j]));
      }
    }
    // row 0 of the product (the slot's row): lanes 0-15, element 0
    const int m = ru / a.chd, c = ru - m * a.chd;
    if (lane < 16) part_r[m][c][lane] = acc[0];
  };
  if (r < n_units) {
    // two register stages, unrolled; loads past the wavefront's last unit re-read that unit
    // (cache hits), so no load sits under a branch
    const int last = r + (n_units - 1 - r) / WAVES * WAVES;
    DcUnit s0, s1;
    load_unit(s0, r);
    for (;;) {
      const int r1 = r + WAVES;
      load_unit(s1, min(r1, last));
      compute_unit(s0, r);
      if (r1 > last) break;
      const int r2 = r1 + WAVES;
      load_unit(s0, min(r2, last));
      compute_unit(s1, r1);
      if (r2 > last) break;
      r = r2;
    }
  }
  __syncthreads();

  // ---- shared output for the 16 features: chunk partials added in order, rounded to bf16
  if (a.sh_h && wave == 0) {
    f32x4_t s4 = spart[0][lane];
#pragma unroll
    for (int q = 1; q < kDcSharedWaves; ++q) {
      const f32x4_t o = spart[q][lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) s4[j] += o[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) sh[4 * lg + j][lane & 15] = bf16_to_f32(f32_to_bf16(s4[j]));
  }
  __syncthreads();

  // ---- combine: token tl, feature f
  const int tid = threadIdx.x;
  if (tid < 16 * a.N) {
    const int tl = tid >> 4, f = tid & 15;
    float routed = 0.f;
    for (int s = 0; s < a.k; ++s) {
      const int m = tl * a.k + s;
      float dsum = part_r[m][0][f];
      for (int c = 1; c < a.chd; ++c) dsum += part_r[m][c][f];
      routed = fmaf(bf16_to_f32(f32_to_bf16(dsum)), a.w[m], routed);
    }
    const int64_t o = static_cast<int64_t>(tl) * a.H + fb * 16 + f;
    uint16_t v;
    if (a.sh_h) {
      const float g = a.sg ? a.sg[tl] : 1.0f;
      v = f32_to_bf16(fmaf(sh[tl][f], g, routed));
    } else if (a.sh_out) {
      const float g = a.sg ? a.sg[tl] : 1.0f;
      v = f32_to_bf16(fmaf(bf16_to_f32(a.sh_out[o]), g, routed));
    } else {
      v = f32_to_bf16(routed);
    }
    if (a.resid) v = f32_to_bf16(bf16_to_f32(a.resid[o]) + bf16_to_f32(v));
    a.y[o] = v;
  }
}

bool down_combine_fits(int N, int k, int H, int I, int Is) {
  const int nsb = I / 128;
  const int chd = (nsb >= 32) ? 4 : (nsb >= 8) ? 2 : 1;
  const int nch = (Is > 0) ? bf16_chunks(Is) : 0;
  return I % 128 == 0 && nsb == chd * kDcSpu && chd <= kDcMaxChunks && N <= kDcMaxTokens &&
         N * k <= kDcMaxSlots && N * k * chd + nch <= kDcMaxUnits && H % 16 == 0 &&
         (Is == 0 || (Is % 64 == 0 && nch <= kDcSharedWaves));
}

int launch_down_combine(const uint16_t* h, const int32_t* idx, const float* w, const float* sg,
                        int N, int k, int H, int I, const void* codes, const uint16_t* sb,
                        const uint16_t* sh_h, int Is, const void* wd, const uint16_t* wd_sb,
                        int sfmt, const uint16_t* resid, uint16_t* y, hipStream_t stream,
                        const uint16_t* sh_out) {
  if (sh_h && sh_out) return fail("down_combine: the shared output is computed here or given");
  if (!down_combine_fits(N, k, H, I, sh_h ? Is : 0))
    return fail("down_combine: shape outside the slot-major fused tail");
  const int nsb = I / 128;
  DcArgs a{h, idx, w, sg, codes, sb, sh_h, wd, wd_sb, resid, sh_out, y,
           N, k, H, I, sh_h ? Is : 0, sh_h ? bf16_chunks(Is) : 0, (nsb >= 8) ? 2 : 1};
  const dim3 grid(H / 16);
  if (sfmt == FMT_INT8) down_combine_kernel<FMT_INT8, 8><<<grid, 512, 0, stream>>>(a);
  else down_combine_kernel<FMT_BF16, 8><<<grid, 512, 0, stream>>>(a);
  return check_launch("down_combine");
}

}  // namespace qmoe
