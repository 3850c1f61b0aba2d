// Decode dataflow kernel: the MoE block after the router logits in one launch, for batches of a
// few tokens routed slot-major (every slot its own one-row m-tile), int4 routed experts and a
// shared expert.
//
// Reference: top-k routing src/quanta/qwen35/moe.py:36-56 (and src/quanta/modeling/moe.py:33-44);
// the routed gate_up gather_qmm + SwiGLU and the down gather_qmm src/quanta/qwen35/moe.py:117-123;
// the weighted combine src/quanta/qwen35/moe.py:191; the gated shared expert
// src/quanta/qwen35/moe.py:145-151,201-202.
//
// The launch before it (the router logits and the shared expert's gate_up, qmm_small_pair_kernel)
// clears this kernel's counters. The grid is a list of units; a unit only ever waits for units
// with smaller workgroup ids:
//   T  ranks tokens (one wavefront per token, topk_token) and stores each slot's weight and the
//      shared gate; the last T unit to finish arms the combine counters;
//   G  the routed gate_up + SwiGLU of slot m for one job block: it ranks the slot's token itself
//      (the ids of the top-k, as the multi-launch path's routed gate_up does), so it waits for
//      nothing, and counts itself done on slot m's counter;
//   S  the shared expert's down projection (needs only the router launch's output; after G, so
//      the routed stream starts first);
//   D  the routed down of slot m for one block of output features: it ranks the token too,
//      issues every weight load of its K chunk, and only then waits for slot m's G units before
//      it reads the slot's h row; the last of a feature block's D and S units (its counter was
//      armed to wrap to zero then) sums the block's slots in slot order, adds the gated shared
//      output and rounds: the combine, with no unit of its own.
//
// Every product runs small_body with the chunking and summation order of its standalone launch,
// and the combine sums as combine_kernel does, so the output equals the multi-launch path's bit
// for bit. Data handed between units goes through agent-coherent loads and stores (small_body.h);
// a producer waits for its stores before it counts itself done, and a consumer reads only after
// it has seen the count. Units start in workgroup-id order on each XCD, so the lowest unfinished
// unit's dependencies are always done: no unit can wait forever. Waits are still bounded
// (poll_geq); one that runs out counts a timeout in a device counter (qmoe_flow_timeouts) and the
// unit goes on, so every workgroup exits.
#include <math.h>

#include "qmoe_internal.h"
#include "route_common.h"
#include "small_body.h"
#include "flow.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

__device__ uint32_t g_flow_timeouts;

constexpr int kFlowMaxFb = 256;   // feature blocks (combine counters) per launch
constexpr int kFlowMaxK = 16;     // experts per token

struct FlowArgs {
  const float* logits;   // [N][ld] router logits (+ the shared gate's in column E)
  int ld;
  TopkParams P;
  int N, k, mc;
  float* w;              // [mc] routing weight of each slot (written here)
  float* sg;             // [N] shared-expert gate
  QmmArgs g, d, s;       // routed gate_up, routed down, shared down
  const uint16_t* dout;  // [mc][H] down output (d.out)
  const uint16_t* sh_out;   // [N][H] shared output (s.out)
  const uint16_t* resid;    // [N][H] residual rows or null
  uint16_t* y;
  int H;
  uint32_t* sync;        // counters kSyncStride words apart, zero at launch: T units done,
                         // then per slot its G units done, then per feature block its arrivals
  int nH, nT, nG, nS, nD;  // units of each kind, in that order in the grid
  int Is;                // the shared expert's width (H unit: [gate | up] rows of 2 Is)
  int gx_g, gx_d, gx_s;  // job blocks (workgroups) per slot (G, D) or token m-tile (S)
  int n_gjobs, n_djobs, n_sjobs;
  int fb_tiles;          // 16-feature output tiles per feature block (one D workgroup's)
  int s_per_fb;          // S workgroups per feature block
  int n_fb;              // feature blocks
};


// This workgroup's stores are complete; thread 0 adds one to *p and the workgroup learns whether
// that made the counter wrap to zero (it was the last of an armed count).
__device__ __forceinline__ bool flow_arrive(uint32_t* p, int* bcast) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *bcast = (old == 0xFFFFFFFFu) ? 1 : 0;
  }
  __syncthreads();
  return *bcast != 0;
}

// Combine of feature block fb: y[t, f] = bf16(sum_s fma(d[t*k+s, f], w[t,s]) then
// fma(sh[t, f], g[t])) for every token, the arithmetic of combine_kernel (slot order, one
// rounding), plus the residual row when given.
__device__ void flow_combine(const FlowArgs& a, int fb) {
  const int F = a.fb_tiles * 16, groups = F / 8;
  const int units = a.N * groups;
  for (int u = threadIdx.x; u < units; u += 256) {
    const int t = u / groups, gi = u - t * groups;
    const int f0 = fb * F + 8 * gi;
    // every slot's weight and down row, and the shared output, loaded before any is summed
    float ws[kFlowMaxK];
    u32x4 v[kFlowMaxK];
#pragma unroll
    for (int s = 0; s < kFlowMaxK; ++s) {
      const int m = t * a.k + min(s, a.k - 1);
      ws[s] = __uint_as_float(coh_ld32(a.w + m));
      v[s] = coh_ld128(a.dout + static_cast<int64_t>(m) * a.H + f0);
    }
    const float g = a.P.has_sg ? __uint_as_float(coh_ld32(a.sg + t)) : 1.0f;
    const u32x4 sh = coh_ld128(a.sh_out + static_cast<int64_t>(t) * a.H + f0);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kFlowMaxK; ++s) {
      if (s < a.k) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = fmaf(bf16lo_to_f32(v[s][q]), ws[s], acc[2 * q]);
          acc[2 * q + 1] = fmaf(bf16hi_to_f32(v[s][q]), ws[s], acc[2 * q + 1]);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] = fmaf(bf16lo_to_f32(sh[q]), g, acc[2 * q]);
      acc[2 * q + 1] = fmaf(bf16hi_to_f32(sh[q]), g, acc[2 * q + 1]);
    }
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
    const int64_t off = static_cast<int64_t>(t) * a.H + f0;
    if (a.resid) {   // y = bf16(resid + bf16(block)), as combine_kernel's add_resid
      const u32x4 r = *reinterpret_cast<const u32x4*>(a.resid + off);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack_bf16x2(bf16lo_to_f32(r[q]) + bf16lo_to_f32(o[q]),
                           bf16hi_to_f32(r[q]) + bf16hi_to_f32(o[q]));
    }
    *reinterpret_cast<u32x4*>(a.y + off) = o;
  }
}

template <int A, int B> struct CMax { static constexpr int v = A > B ? A : B; };

// VPL: experts per lane of the top-k. G: routed gate_up (GW wavefronts per job, one tile pair
// each, 8 superblocks per chunk staged deep); D: routed down (DW wavefronts per job, DJPW tiles
// each, 4 superblocks per chunk); S: shared down (SW chunks, weights SFMT).
// The router launch writes the shared expert's gate_up as [gate | up] rows (split: each tile a
// job of its own, so that launch ends with its router workgroups); one H unit forms the gated
// activation once, in place of the gate half (coherent stores, the SwiGLU epilogue's arithmetic
// on the same bf16 values), and the shared-down units wait for it.
template <int VPL, int GW, int DW, int DJPW, int SW, int SFMT>
__global__ void __launch_bounds__(256) decode_flow_kernel(FlowArgs a) {
  constexpr int RG = SmallCfg<FMT_INT4, EPI_SWIGLU, GW, 1, 1, 1>::RED;
  constexpr int RD = SmallCfg<FMT_INT4, EPI_BF16, DW, 1, DJPW, 1>::RED;
  constexpr int RS = SmallCfg<SFMT, EPI_BF16, SW, 1, 1, 1>::RED;
  constexpr int RR = CMax<CMax<RG, RD>::v, RS>::v;
  __shared__ f32x4_t red[RR];
  __shared__ u32x4 xlds[4 * 8 * 16];
  __shared__ int bcast, route_e;
  uint32_t* const gdone = a.sync + kSyncStride;                  // [m * kSyncStride]
  uint32_t* const cnt = a.sync + (1 + a.mc) * kSyncStride;       // [fb * kSyncStride]
  SlotRoute route{};
  route.logits = a.logits;
  route.ld = a.ld;
  route.P = a.P;
  route.mc = a.mc;
  route.store = 0;
  int b = blockIdx.x;
  uint32_t* const hdone = a.sync + (1 + a.mc + a.H / 16) * kSyncStride;

  // ---- H: the shared expert's gated activation, once per row element
  if (b < a.nH) {
    const int per = a.Is / 8;   // 16-byte groups of a half row
    for (int v = threadIdx.x; v < a.N * per; v += 256) {
      const int t = v / per, j = v - t * per;
      u32x4* row = reinterpret_cast<u32x4*>(const_cast<uint16_t*>(a.s.act) + static_cast<int64_t>(t) * 2 * a.Is);
      const u32x4 g = row[j], up = row[j + per];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        coh_st32(reinterpret_cast<uint32_t*>(row + j) + q,
                 pack_bf16x2_rne(glu_f(bf16lo_to_f32(g[q]), bf16lo_to_f32(up[q]), a.s.glu, a.s.glu_alpha, a.s.glu_limit),
                                 glu_f(bf16hi_to_f32(g[q]), bf16hi_to_f32(up[q]), a.s.glu, a.s.glu_alpha, a.s.glu_limit)));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(hdone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  b -= a.nH;

  // ---- T: each slot's routing weight and each token's shared gate, for the combine
  if (b < a.nT) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = b * 4 + wave;
    if (t < a.N) {
      const float* row = a.logits + static_cast<int64_t>(t) * a.ld;
      int id;
      float wsel;
      topk_token<VPL>(row, a.P, lane, id, wsel);
      if (lane < a.k) coh_st32(a.w + t * a.k + lane, __float_as_uint(wsel));
      if (a.P.has_sg && lane == 0) coh_st32(a.sg + t, __float_as_uint(1.0f / (1.0f + expf(-row[a.P.E]))));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      bcast = (__hip_atomic_fetch_add(a.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               static_cast<uint32_t>(a.nT - 1)) ? 1 : 0;
    __syncthreads();
    if (!bcast) return;
    // the last T unit: arm the combine counters (each wraps to zero at its block's last D or S
    // arrival); a block whose units all arrived already completes here
    __shared__ int done_fb[kFlowMaxFb];
    const uint32_t arm = 0u - static_cast<uint32_t>(a.mc + a.s_per_fb);
    for (int fb = threadIdx.x; fb < a.n_fb; fb += 256)
      done_fb[fb] = (__hip_atomic_fetch_add(cnt + fb * kSyncStride, arm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) +
                     arm == 0u) ? 1 : 0;
    __syncthreads();
    for (int fb = 0; fb < a.n_fb; ++fb)
      if (done_fb[fb]) flow_combine(a, fb);
    return;
  }
  b -= a.nT;

  // ---- G: routed gate_up + SwiGLU of slot m
  if (b < a.nG) {
    const int m = b / a.gx_g, bx = b - m * a.gx_g;
    small_body<FMT_INT4, EPI_SWIGLU, GW, 1, 1, 1, false, VPL, 8, kCohOut>(a.g, a.n_gjobs, bx, m, red,
                                                                         &route, xlds, &route_e);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_fetch_add(gdone + m * kSyncStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  b -= a.nG;

  // ---- S: shared expert down projection
  if (b < a.nS) {
    const int tm = b / a.gx_s, bx = b - tm * a.gx_s;
    small_body<SFMT, EPI_BF16, SW, 1, 1, 1, false, 0, 0, kCohOut | kCohAct | kCohWaitAct>(a.s, a.n_sjobs, bx, tm, red);
    const int fb = (bx * (4 / SW)) / a.fb_tiles;
    if (flow_arrive(cnt + fb * kSyncStride, &bcast)) flow_combine(a, fb);
    return;
  }
  b -= a.nS;

  // ---- D: routed down of slot m, feature block bx; the block's last arrival combines it
  {
    const int m = b / a.gx_d, bx = b - m * a.gx_d;
    small_body<FMT_INT4, EPI_BF16, DW, 1, DJPW, 1, false, VPL, 4,
               kCohAct | kCohOut | kCohRowSlot | kCohWaitAct>(a.d, a.n_djobs, bx, m, red, &route,
                                                               xlds, &route_e);
    if (flow_arrive(cnt + bx * kSyncStride, &bcast)) flow_combine(a, bx);
  }
}

// ------------------------------------------------------------------ host side
struct FlowShape {
  bool ok = false;
  int vpl = 0, gw = 0, dw = 0, djpw = 0, sw = 0;
};

static int int4_chunks(int K) {
  const int nsb = K / 128;
  return (nsb >= 32) ? 4 : (nsb >= 8) ? 2 : 1;   // launch_qmm's int4 chunk rule
}

// The shapes the kernel is compiled for: c2-like (gate_up K chunks 4, down 2, shared down 4) and
// c1-like (2, 1, 2), every gate_up chunk 8 superblocks and every down chunk 4 (the deep staging),
// top-k over 129-512 experts, a bf16 or int8 shared expert.
static FlowShape flow_shape(int N, int k, int E, int H, int I, int Is) {
  FlowShape f;
  if (N < 1 || N > 16 || N * k > 256 || E > 512 || k > kFlowMaxK || H % 128 || I % 128 || Is <= 0 ||
      Is % 64)
    return f;
  f.vpl = topk_vpl(E);
  if (f.vpl != 4 && f.vpl != 8) return f;
  f.gw = int4_chunks(H);
  f.dw = int4_chunks(I);
  f.sw = bf16_chunks(Is);
  const bool c2 = (f.gw == 4 && f.dw == 2 && f.sw == 4), c1 = (f.gw == 2 && f.dw == 1 && f.sw == 2);
  if (!c2 && !c1) return f;
  if (H / 128 != 8 * f.gw || I / 128 != 4 * f.dw) return f;
  f.djpw = 4;
  const int gjobs = I / 16, djobs = H / 16 / f.djpw;
  if (gjobs % (4 / f.gw) || djobs % (4 / f.dw) || (H / 16) % (4 / f.sw)) return f;
  const int fb_tiles = (4 / f.dw) * f.djpw;
  if (fb_tiles % (4 / f.sw) || (H / 16) / fb_tiles > kFlowMaxFb) return f;
  f.ok = true;
  return f;
}

bool decode_flow_fits(int N, int k, int E, int H, int I, int Is) {
  return flow_shape(N, k, E, H, I, Is).ok;
}

// sync words the kernel needs for mc slots (cleared by the launch before it): the T count, a
// count per slot, per feature block, and the H unit's
int64_t decode_flow_sync_words(int64_t mc, int H) { return (2 + mc + H / 16) * kSyncStride; }

static int g_flow_mode = 1;
}  // namespace qmoe

extern "C" int qmoe_set_decode_flow(int mode) {
  const int prev = qmoe::g_flow_mode;
  if (mode >= 0 && mode <= 2) qmoe::g_flow_mode = mode;
  return prev;
}

// (the decode dataflow launch's waits and the routing tail's)
extern "C" uint32_t qmoe_flow_timeouts(void) {
  uint32_t v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(qmoe::g_flow_timeouts), sizeof(v), 0, hipMemcpyDeviceToHost) !=
      hipSuccess)
    return 0xFFFFFFFFu;
  const uint32_t r = qmoe::route_tail_timeouts();
  return r == 0xFFFFFFFFu ? r : v + r;
}

namespace qmoe {

// Mode 1 (default) takes the dataflow launch up to kFlowAutoTokens tokens: measured on MI355X
// (c2 shape, 200-step loops) it beats the separate launches at one token (33.3 vs 36.1 us) and
// two (49.2 vs 52.9 us), and loses from four (81.8 vs 76.9 us), where every gate_up workgroup
// ranking its own token costs more than the one top-k launch. Mode 2 takes it wherever the shape
// fits (tests, measurements); mode 0 never.
constexpr int kFlowAutoTokens = 2;
bool decode_flow_enabled(int N) {
  return g_flow_mode == 2 || (g_flow_mode == 1 && N <= kFlowAutoTokens);
}

template <int VPL, int GW, int DW, int DJPW, int SW, int SFMT>
static void flow_go(const FlowArgs& a, hipStream_t stream) {
  const int64_t grid = static_cast<int64_t>(a.nH) + a.nT + a.nG + a.nS + a.nD;
  decode_flow_kernel<VPL, GW, DW, DJPW, SW, SFMT><<<dim3(static_cast<unsigned>(grid)), 256, 0, stream>>>(a);
}

template <int VPL, int SFMT>
static void flow_dispatch_shape(const FlowArgs& a, const FlowShape& f, hipStream_t stream) {
  if (f.gw == 4) flow_go<VPL, 4, 2, 4, 4, SFMT>(a, stream);   // c2-like
  else flow_go<VPL, 2, 1, 4, 2, SFMT>(a, stream);             // c1-like
}

// Whether the dataflow launch for this shape takes the shared expert's [gate | up] rows (the
// router launch then runs the shared gate_up's tiles as separate jobs, launch_qmm_pair_bf16
// split): every compiled shape does. Measured on MI355X (300-step loops, µs, SwiGLU rows ->
// split with the H unit): c2 one token 33.0 -> 32.4, two 49.3 -> 46.2; c1 21.9 -> 20.5 and
// 25.7 -> 24.1. (Forming the activation in every shared-down unit instead, 256 per m-tile at
// c2, each for the whole row: c2 38.2 and 58.7.)
bool decode_flow_split_shared(int H, int I, int Is) { return flow_shape(1, 1, 256, H, I, Is).ok; }

int launch_decode_flow(const FlowLaunch& L, hipStream_t stream) {
  const FlowShape f = flow_shape(L.N, L.k, L.P.E, L.H, L.I, L.Is);
  if (!f.ok) return fail("decode flow: shape outside the compiled decode dataflow kernel");
  if (!L.gu_codes || !L.gu_sb || !L.dn_codes || !L.dn_sb || !L.sh_dn || (L.sfmt == FMT_INT8 && !L.sh_dn_sb))
    return fail("decode flow: missing weights");
  uint32_t* timeouts = nullptr;
  if (hipGetSymbolAddress(reinterpret_cast<void**>(&timeouts), HIP_SYMBOL(g_flow_timeouts)) != hipSuccess)
    return fail("decode flow: timeout counter address");
  FlowArgs a{};
  a.logits = L.logits;
  a.ld = L.ld;
  a.P = L.P;
  a.N = L.N;
  a.k = L.k;
  a.mc = L.N * L.k;
  a.w = L.w;
  a.sg = L.sg;
  a.H = L.H;
  a.y = L.y;
  a.resid = L.resid;
  a.sync = L.sync;
  // routed gate_up + SwiGLU -> h, rows by slot (each unit ranks its slot's token itself)
  QmmArgs& g = a.g;
  g.act = L.x; g.act_rows = L.N; g.slot_div = 1; g.n_experts = L.P.E;
  g.K = L.H; g.n_rows = 2 * L.I; g.codes = L.gu_codes; g.sb = L.gu_sb; g.out = L.h; g.ld_out = L.I;
  g.glu = L.glu; g.glu_alpha = L.glu_alpha; g.glu_limit = L.glu_limit;
  // routed down -> d, rows by slot, each unit reading its slot's h row once slot m's G units
  // have counted themselves done
  QmmArgs& d = a.d;
  d.act = L.h; d.act_rows = a.mc; d.slot_div = 1; d.n_experts = L.P.E;
  d.K = L.I; d.n_rows = L.H; d.codes = L.dn_codes; d.sb = L.dn_sb; d.out = L.d; d.ld_out = L.H;
  d.act_ready = L.sync + kSyncStride;
  d.timeouts = timeouts;
  a.dout = L.d;
  // shared down -> sh_out, from the router launch's [gate | up] rows of the shared expert (the
  // gated activation formed as the fragments are loaded)
  QmmArgs& s = a.s;
  s.act = L.sh_h; s.act_rows = L.N; s.slot_div = 1; s.dense_rows = L.N; s.n_experts = 1;
  s.K = L.Is; s.n_rows = L.H; s.codes = L.sh_dn; s.sb = L.sh_dn_sb; s.out = L.sh_out; s.ld_out = L.H;
  s.glu = L.glu; s.glu_alpha = L.glu_alpha; s.glu_limit = L.glu_limit;
  a.Is = L.Is;
  a.nH = 1;
  // the H unit's rows: [h | up], h in place of the gate half, complete once it counts
  s.act_stride = 2 * L.Is;
  s.act_ready = L.sync + (1 + L.N * L.k + L.H / 16) * kSyncStride;
  s.act_ready_target = 1;
  s.timeouts = timeouts;
  a.sh_out = L.sh_out;
  // units
  a.n_gjobs = L.I / 16;
  a.n_djobs = L.H / 16 / f.djpw;
  a.n_sjobs = L.H / 16;
  a.gx_g = a.n_gjobs / (4 / f.gw);
  a.gx_d = a.n_djobs / (4 / f.dw);
  a.gx_s = a.n_sjobs / (4 / f.sw);
  d.act_ready_target = static_cast<uint32_t>(a.gx_g);
  a.fb_tiles = (4 / f.dw) * f.djpw;
  a.n_fb = a.gx_d;
  const int s_mtiles = (L.N + kSmallMTile - 1) / kSmallMTile;
  a.s_per_fb = s_mtiles * (a.fb_tiles / (4 / f.sw));
  a.nT = (L.N + 3) / 4;
  a.nS = s_mtiles * a.gx_s;
  a.nG = a.mc * a.gx_g;
  a.nD = a.mc * a.gx_d;
  if (f.vpl == 8) {
    if (L.sfmt == FMT_INT8) flow_dispatch_shape<8, FMT_INT8>(a, f, stream);
    else flow_dispatch_shape<8, FMT_BF16>(a, f, stream);
  } else {
    if (L.sfmt == FMT_INT8) flow_dispatch_shape<4, FMT_INT8>(a, f, stream);
    else flow_dispatch_shape<4, FMT_BF16>(a, f, stream);
  }
  return check_launch("decode flow");
}

}  // namespace qmoe
